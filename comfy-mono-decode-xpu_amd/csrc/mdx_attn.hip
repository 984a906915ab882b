// Tree-verify / draft decode attention over a bf16 KV cache, split along the context (flash decoding)
// with bf16 MFMA on gfx950, and the chunk merge in the same launch.
//
// Reference semantics (comfy-mono-decode-xpu): csrc/attn_dpas.sycl:269-342 (contract: rows of one kv
// head attend the committed prefix [0, L) of the cache and, for tree verify, the tree rows their mask
// admits from xk / xv; the softmax is scaled by 1/sqrt(D); P is rounded to bf16 for the P.V product,
// partials merge in fp32; a row with no admitted token writes 0). Tolerance-level parity (fp64 bound),
// as the reference's own kernel is not bit-identical to the chain it replaces.
//
// Query rows of kv head kh: r = (h % groups) * S + s for the heads h of that kv head, 16 rows per
// row tile (rt). Work-group = (kv head, row tile, chunk) of 4 waves; each wave owns a quarter of the
// chunk's tokens and runs, per 32-token step:
//   S^T = K Q^T   v_mfma_f32_16x16x32_bf16, A = 16 K rows (tokens) x 32 dims from HBM, B = Q^T held in
//                 registers; the accumulator gives each lane 4 tokens of one query row (lane % 16), so
//                 the online softmax state of a row lives in its lanes;
//   O^T += V^T P^T   A = V^T from LDS (the wave transposes its 32 x D V tile into [dim][token] order,
//                 tokens permuted so a lane's 8 k-slots are the 8 tokens its S^T accumulators hold),
//                 B = bf16(P^T) straight from the S^T registers -- no shuffle of P.
// The 4 waves merge in LDS; the work-group's partial (m, l, O) goes to the workspace; the last
// work-group of a (kv head, row tile) (device-scope counter, reset by it) merges the chunks and writes
// the bf16 rows. Every work-group increments the counter, also those whose chunk is empty for the
// current context length (read from device memory, so a captured graph replays for any length).
// Work-group ids are laid out so the row tiles of one (kv head, chunk) share an XCD (ids are dealt
// round-robin over the 8 XCDs): the 4x re-read of a K/V chunk hits that XCD's L2.
#include <math.h>

#include "mdx_common.hpp"

namespace mdx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int AT_WAVES = 4;
constexpr int AT_STEP = 32;        // tokens per MFMA step
constexpr int AT_VT_ROW = 72;      // bytes per [dim] row of the transposed V tile (64 + 8: conflict-free writes)
constexpr int AT_MIN_TPW = 128;    // at least this many tokens per wave per chunk
constexpr float LOG2E = 1.4426950408889634f;

struct AttnArgs {
    const uint16_t* q;       // [H, S, D] with strides qh, qs
    int64_t qh, qs;
    const uint16_t* key;     // [Hk, cap, D]
    const uint16_t* value;
    const int32_t* seqlen;   // [1]
    const uint16_t* xk;      // [Hk, S, D] with strides xh, xs (tree rows)
    const uint16_t* xv;
    int64_t xh, xs, vh, vs;
    const int32_t* mask;     // [S] or null (draft row)
    uint16_t* out;           // [S, H, D]
    float* part;             // [Hk][RT][C + 1][2 * 16 + 16 * D]
    unsigned* counter;       // [Hk * RT]
    int H, Hk, S, cap, groups, rows, RT, C;
    float zscale;            // 1/sqrt(D) * log2(e)
};

__device__ __forceinline__ unsigned bf16pair(float a, float b) { return unsigned(f2bf(a)) | (unsigned(f2bf(b)) << 16); }

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

// the column of token t (0..31) in a transposed V row: lane group g's 8 k-slots are tokens
// {4g..4g+3} (first S^T tile) and {16+4g..16+4g+3} (second tile), stored contiguously at 8g
__device__ __forceinline__ int vt_col(int t) { return t < 16 ? 8 * (t >> 2) + (t & 3) : 8 * ((t - 16) >> 2) + 4 + (t & 3); }

// per-device context split: chunks of at least AT_MIN_TPW tokens per wave
__device__ __forceinline__ void split(int L, int C, int& tpw, int& active) {
    int c = (L + AT_WAVES * AT_MIN_TPW - 1) / (AT_WAVES * AT_MIN_TPW);
    c = c < 1 ? 1 : (c > C ? C : c);
    tpw = (L + AT_WAVES * c - 1) / (AT_WAVES * c);
    tpw = (tpw + AT_STEP - 1) / AT_STEP * AT_STEP;
    active = L > 0 ? (L + AT_WAVES * tpw - 1) / (AT_WAVES * tpw) : 0;
}

template <int D>
__global__ __launch_bounds__(64 * AT_WAVES) void attn_kernel(AttnArgs a) {
    constexpr int KK = D / 32;   // MFMA k-steps over the head dim
    constexpr int DT = D / 16;   // 16-dim output tiles
    constexpr int NV = D / 16;   // 16-byte V loads per lane per step
    constexpr int WREG = 72 * D; // LDS bytes per wave: the transposed V tile, later the wave's (m, l, O)
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int last_s;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, c16 = lane & 15;
    const int units = a.Hk * (a.C + 1);
    const int bid = blockIdx.x;
    const int unit = (bid % 8) + 8 * ((bid / 8) / a.RT);
    const int rt = (bid / 8) % a.RT;
    if (unit >= units) return;  // padding ids of the last group of 8 (not counted)
    const int kh = unit / (a.C + 1), cslot = unit % (a.C + 1);
    const bool tree = cslot == a.C;
    int L = a.seqlen[0];
    L = L < 0 ? 0 : (L > a.cap ? a.cap : L);
    int tpw, active;
    split(L, a.C, tpw, active);

    // this lane's query row: the column of S^T and O^T it holds
    const int r = rt * 16 + c16;
    const bool rvalid = r < a.rows;
    const int rr = rvalid ? r : 0;
    const int hq = kh * a.groups + rr / a.S, sq = rr % a.S;
    // the tree work-group of a draft launch (no mask) has no tokens and must not read the mask
    const uint32_t rmask = (tree && rvalid && a.mask != nullptr) ? uint32_t(a.mask[sq]) : 0u;

    // the wave's tokens
    int t_begin = 0, t_end = 0;
    const uint16_t *kb, *vb;
    int64_t kstride, vstride;
    if (tree) {
        if (a.mask && w == 0) t_end = a.S;
        kb = a.xk + kh * a.xh;
        vb = a.xv + kh * a.vh;
        kstride = a.xs;
        vstride = a.vs;
    } else {
        if (cslot < active) {
            t_begin = (cslot * AT_WAVES + w) * tpw;
            t_end = min(L, t_begin + tpw);
        }
        kb = a.key + int64_t(kh) * a.cap * D;
        vb = a.value + int64_t(kh) * a.cap * D;
        kstride = vstride = D;
    }

    u32x4 qf[KK];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
        qf[kk] = rvalid ? ld16(a.q + hq * a.qh + sq * a.qs + 32 * kk + 8 * g) : u32x4{0, 0, 0, 0};

    f32x4 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;
    unsigned char* vt = smem + w * WREG;

    for (int t0 = t_begin; t0 < t_end; t0 += AT_STEP) {
        // K rows (A of S^T) and this lane's V pieces, clamped into the wave's range
        u32x4 kf[2][KK], vr[NV];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int tok = min(t0 + 16 * tt + c16, t_end - 1);
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) kf[tt][kk] = ld16(kb + tok * kstride + 32 * kk + 8 * g);
        }
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int tok = min(t0 + 2 * c16 + (j & 1), t_end - 1);
            vr[j] = ld16(vb + tok * vstride + 8 * (4 * (j >> 1) + g));
        }
        // S^T: lane holds tokens t0 + 16 tt + 4 g + i of query row c16
        f32x4 st[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            st[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KK; ++kk)
                st[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kf[tt][kk]), as_bf16x8(qf[kk]), st[tt], 0, 0, 0);
        }
        float z[2][4], mx = -INFINITY;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tok = t0 + 16 * tt + 4 * g + i;
                bool ok = tok < t_end;
                if (tree) ok = ok && ((rmask >> tok) & 1u);
                z[tt][i] = ok ? st[tt][i] * a.zscale : -INFINITY;
                mx = fmaxf(mx, z[tt][i]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mnew = fmaxf(m, mx);
        const float alpha = (m == -INFINITY) ? 0.f : exp2f(m - mnew);
        float p[2][4], ps = 0.f;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                p[tt][i] = z[tt][i] == -INFINITY ? 0.f : bfround(exp2f(z[tt][i] - mnew));
                ps += p[tt][i];
            }
        ps += __shfl_xor(ps, 16, 64);
        ps += __shfl_xor(ps, 32, 64);
        l = l * alpha + ps;
        m = mnew;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
        const u32x4 pf = {bf16pair(p[0][0], p[0][1]), bf16pair(p[0][2], p[0][3]), bf16pair(p[1][0], p[1][1]),
                          bf16pair(p[1][2], p[1][3])};
        // V^T into LDS: tokens 2 c16 and 2 c16 + 1, dims 8 (4 jj + g) .. + 8, one dword per dim
        const int col = 2 * vt_col(2 * c16);
#pragma unroll
        for (int jj = 0; jj < NV / 2; ++jj) {
            const int d0 = 8 * (4 * jj + g);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const unsigned va = vr[2 * jj][e >> 1], vb2 = vr[2 * jj + 1][e >> 1];
                const unsigned pr = __builtin_amdgcn_perm(vb2, va, (e & 1) ? 0x07060302u : 0x05040100u);
                *reinterpret_cast<unsigned*>(vt + (d0 + e) * AT_VT_ROW + col) = pr;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const unsigned char* src = vt + (16 * dt + c16) * AT_VT_ROW + 16 * g;
            const uint2 lo = *reinterpret_cast<const uint2*>(src), hi = *reinterpret_cast<const uint2*>(src + 8);
            const u32x4 vf = {lo.x, lo.y, hi.x, hi.y};
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(vf), as_bf16x8(pf), acc[dt], 0, 0, 0);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // merge the 4 waves in LDS: per wave m[16], l[16], O[16][D]
    __syncthreads();
    float* wr = reinterpret_cast<float*>(smem + w * WREG);
    if (g == 0) {
        wr[c16] = m;
        wr[16 + c16] = l;
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4*>(wr + 32 + c16 * D + 16 * dt + 4 * g) = acc[dt];
    __syncthreads();
    const bool has = tree ? (a.mask != nullptr) : (cslot < active);
    float* rec = a.part + (int64_t(kh * a.RT + rt) * (a.C + 1) + cslot) * (32 + 16 * D);
    if (has) {
        for (int e = threadIdx.x; e < 16 * D; e += 64 * AT_WAVES) {
            const int row = e / D, d = e % D;
            float M = -INFINITY;
#pragma unroll
            for (int v = 0; v < AT_WAVES; ++v) M = fmaxf(M, reinterpret_cast<const float*>(smem + v * WREG)[row]);
            float o = 0.f, s = 0.f;
#pragma unroll
            for (int v = 0; v < AT_WAVES; ++v) {
                const float* wv = reinterpret_cast<const float*>(smem + v * WREG);
                const float mv = wv[row];
                const float f = mv == -INFINITY ? 0.f : exp2f(mv - M);
                o += wv[32 + row * D + d] * f;
                s += wv[16 + row] * f;
            }
            rec[32 + e] = o;
            if (d == 0) {
                rec[row] = M;
                rec[16 + row] = s;
            }
        }
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0)
        last_s = __hip_atomic_fetch_add(a.counter + kh * a.RT + rt, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) ==
                 unsigned(a.C);
    __syncthreads();
    if (!last_s) return;
    __threadfence();
    // the last work-group of (kv head, row tile): merge the chunks and the tree partial, write bf16 rows
    const float* base = a.part + int64_t(kh * a.RT + rt) * (a.C + 1) * (32 + 16 * D);
    const bool use_tree = a.mask != nullptr;
    for (int e = threadIdx.x; e < 16 * D; e += 64 * AT_WAVES) {
        const int row = e / D, d = e % D;
        const int rr2 = rt * 16 + row;
        if (rr2 >= a.rows) continue;
        float M = -INFINITY;
        for (int c = 0; c <= a.C; ++c) {
            if (c < a.C ? c >= active : !use_tree) continue;
            M = fmaxf(M, base[c * (32 + 16 * D) + row]);
        }
        float o = 0.f, s = 0.f;
        for (int c = 0; c <= a.C; ++c) {
            if (c < a.C ? c >= active : !use_tree) continue;
            const float* rc = base + c * (32 + 16 * D);
            const float mc = rc[row];
            const float f = mc == -INFINITY ? 0.f : exp2f(mc - M);
            o += rc[32 + e] * f;
            s += rc[16 + row] * f;
        }
        const int h = kh * a.groups + rr2 / a.S, sr = rr2 % a.S;
        a.out[(int64_t(sr) * a.H + h) * D + d] = f2bf(s > 0.f ? __fdiv_rn(o, s) : 0.f);
    }
    if (threadIdx.x == 0) __hip_atomic_store(a.counter + kh * a.RT + rt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

int plan_chunks(int Hk, int RT, int cap) {
    int c = (512 + Hk * RT - 1) / (Hk * RT);
    const int by_cap = (cap + AT_WAVES * AT_MIN_TPW - 1) / (AT_WAVES * AT_MIN_TPW);
    c = c > by_cap ? by_cap : c;
    return c < 1 ? 1 : (c > 64 ? 64 : c);
}

size_t workspace_bytes(int Hk, int RT, int C, int D) {
    return 256 + size_t(Hk) * RT * (C + 1) * (32 + 16 * size_t(D)) * sizeof(float);
}

template <int D>
int launch(const AttnArgs& a, hipStream_t st) {
    const int units = a.Hk * (a.C + 1);
    const int grid = (units + 7) / 8 * 8 * a.RT;
    const size_t lds = size_t(AT_WAVES) * 72 * D;
    allow_smem(reinterpret_cast<const void*>(&attn_kernel<D>), lds);
    hipLaunchKernelGGL(attn_kernel<D>, dim3(grid), dim3(64 * AT_WAVES), lds, st, a);
    MDX_LAUNCHED();
    return MDX_OK;
}

}  // namespace
}  // namespace mdx

using namespace mdx;

extern "C" size_t mdx_attn_workspace(int64_t H, int64_t Hk, int64_t S, int64_t D, int64_t cap) {
    if (Hk <= 0 || H % Hk != 0 || S <= 0) return 0;
    const int RT = int((H / Hk * S + 15) / 16);
    return workspace_bytes(int(Hk), RT, plan_chunks(int(Hk), RT, int(cap)), int(D));
}

extern "C" int mdx_attn_decode(const uint16_t* q, int64_t q_head_stride, int64_t q_row_stride, const uint16_t* key,
                               const uint16_t* value, const int32_t* seqlen, const uint16_t* xk, const uint16_t* xv,
                               int64_t x_head_stride, int64_t x_row_stride, const int32_t* mask, uint16_t* out,
                               int64_t H, int64_t Hk, int64_t S, int64_t D, int64_t cap, void* workspace,
                               size_t workspace_bytes_, void* stream) {
    MDX_CHECK(q && key && value && seqlen && xk && xv && out, "null pointer");
    MDX_CHECK(D == 64 || D == 128 || D == 256, "head_dim must be 64, 128 or 256");
    MDX_CHECK(Hk >= 1 && H % Hk == 0 && S >= 1 && S <= 16, "heads / 1..16 rows");
    MDX_CHECK(mask || S == 1, "a draft (no mask) has one row");
    MDX_CHECK(H / Hk * S <= 64, "at most 64 query rows per kv head");
    MDX_CHECK(cap >= 1 && cap < (int64_t(1) << 30) / D, "cache capacity");
    MDX_CHECK(aligned(q, 16) && aligned(key, 16) && aligned(value, 16) && aligned(xk, 16) && aligned(xv, 16) &&
                  q_head_stride % 8 == 0 && q_row_stride % 8 == 0 && x_head_stride % 8 == 0 && x_row_stride % 8 == 0,
              "16-byte aligned rows");
    const int RT = int((H / Hk * S + 15) / 16);
    const int C = plan_chunks(int(Hk), RT, int(cap));
    MDX_CHECK(workspace && aligned(workspace, 256) && workspace_bytes_ >= workspace_bytes(int(Hk), RT, C, int(D)),
              "workspace: %zu bytes, 256-byte aligned, zeroed once", workspace_bytes(int(Hk), RT, C, int(D)));
    AttnArgs a{};
    a.q = q;
    a.qh = q_head_stride;
    a.qs = q_row_stride;
    a.key = key;
    a.value = value;
    a.seqlen = seqlen;
    a.xk = xk;
    a.xv = xv;
    a.xh = a.vh = x_head_stride;
    a.xs = a.vs = x_row_stride;
    a.mask = mask;
    a.out = out;
    a.counter = static_cast<unsigned*>(workspace);
    a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + 256);
    a.H = int(H);
    a.Hk = int(Hk);
    a.S = int(S);
    a.cap = int(cap);
    a.groups = int(H / Hk);
    a.rows = int(H / Hk * S);
    a.RT = RT;
    a.C = C;
    a.zscale = float(1.0 / sqrt(double(D)) * 1.4426950408889634);
    MDX_CHECK(Hk * RT <= 64, "counter table");
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (D == 64) return launch<64>(a, st);
    if (D == 128) return launch<128>(a, st);
    return launch<256>(a, st);
}
