// Tree-verify / draft decode attention over a bf16 KV cache, split along the context (flash decoding)
// with bf16 MFMA on gfx950, then a wide merge of the chunk partials.
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
// Each wave prefetches its next step's K and V into a second register set while the current step
// computes (head_dim <= 128). The 4 waves merge in LDS; the work-group's partial (m, l, O) goes to
// the workspace; attn_merge_kernel (one work-group per query row, one thread per dim) combines the
// chunks and the tree-row partial and writes bf16. The context split is recomputed on the device
// from seqlen in both kernels, so a captured graph replays for any context length.
// Work-group ids are laid out so the row tiles of one (kv head, chunk) share an XCD (ids are dealt
// round-robin over the 8 XCDs): the 4x re-read of a K/V chunk hits that XCD's L2.
#include <math.h>
#include <stdlib.h>

#include "mdx_common.hpp"

namespace mdx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int AT_WAVES = 4;
constexpr int AT_STEP = 32;        // tokens per MFMA step
constexpr int AT_VT_ROW = 72;      // bytes per [dim] row of the transposed V tile (64 + 8: conflict-free writes)
constexpr int AT_MIN_TPW = 64;     // default: at least this many tokens per wave per chunk (swept: 32, 64, 128)
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
    int H, Hk, S, cap, groups, rows, RT, C;
    int min_tpw;             // a chunk gives each wave at least this many tokens
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

// per-device context split: at most C chunks of at least min_tpw tokens per wave
__device__ __forceinline__ void split(int L, int C, int min_tpw, int& tpw, int& active) {
    int c = (L + AT_WAVES * min_tpw - 1) / (AT_WAVES * min_tpw);
    c = c < 1 ? 1 : (c > C ? C : c);
    tpw = (L + AT_WAVES * c - 1) / (AT_WAVES * c);
    tpw = (tpw + AT_STEP - 1) / AT_STEP * AT_STEP;
    active = L > 0 ? (L + AT_WAVES * tpw - 1) / (AT_WAVES * tpw) : 0;
}

template <int D, bool PINGPONG>
__global__ __launch_bounds__(64 * AT_WAVES) void attn_kernel(AttnArgs a) {
    constexpr int KK = D / 32;   // MFMA k-steps over the head dim
    constexpr int DT = D / 16;   // 16-dim output tiles
    constexpr int NV = D / 16;   // 16-byte V loads per lane per step
    constexpr int WREG = 72 * D; // LDS bytes per wave: the transposed V tile, later the wave's (m, l, O)
    extern __shared__ __align__(16) unsigned char smem[];
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
    split(L, a.C, a.min_tpw, tpw, active);

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

    // one 32-token step: S^T, online softmax, V^T through LDS, O^T
    auto step = [&](int t0, const u32x4 (&kf)[2][KK], const u32x4 (&vr)[NV]) {
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
        mx = max_x32(max_x16(mx));
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
        ps = sum_x32(sum_x16(ps));
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
    };
    // K rows (A of S^T) and this lane's V pieces of the step at t0, clamped into the wave's range
    // (loads past the range repeat its last token, so every load is unconditional)
    auto load = [&](int t0, u32x4 (&kf)[2][KK], u32x4 (&vr)[NV]) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int tok = max(min(t0 + 16 * tt + c16, t_end - 1), 0);
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) kf[tt][kk] = ld16(kb + tok * kstride + 32 * kk + 8 * g);
        }
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int tok = max(min(t0 + 2 * c16 + (j & 1), t_end - 1), 0);
            vr[j] = ld16(vb + tok * vstride + 8 * (4 * (j >> 1) + g));
        }
    };
    if (t_begin < t_end) {
        u32x4 kA[2][KK], vA[NV];
        load(t_begin, kA, vA);
        if (PINGPONG) {
            // two register sets: the next step's loads are in flight while this step computes
            u32x4 kB[2][KK], vB[NV];
            for (int t0 = t_begin; t0 < t_end; t0 += 2 * AT_STEP) {
                load(t0 + AT_STEP, kB, vB);
                step(t0, kA, vA);
                load(t0 + 2 * AT_STEP, kA, vA);
                if (t0 + AT_STEP < t_end) step(t0 + AT_STEP, kB, vB);
            }
        } else {
            for (int t0 = t_begin; t0 < t_end; t0 += AT_STEP) {
                if (t0 > t_begin) load(t0, kA, vA);
                step(t0, kA, vA);
            }
        }
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
        // the rows' maxima and the waves' weights once per row (threads 0..15), then each output
        // element is four products; the same arithmetic, in the same order, as per element
        __shared__ float fw[16][AT_WAVES];
        if (threadIdx.x < 16) {
            const int row = threadIdx.x;
            float M = -INFINITY;
#pragma unroll
            for (int v = 0; v < AT_WAVES; ++v) M = fmaxf(M, reinterpret_cast<const float*>(smem + v * WREG)[row]);
            float s = 0.f;
#pragma unroll
            for (int v = 0; v < AT_WAVES; ++v) {
                const float* wv = reinterpret_cast<const float*>(smem + v * WREG);
                const float mv = wv[row];
                const float f = mv == -INFINITY ? 0.f : exp2f(mv - M);
                fw[row][v] = f;
                s += wv[16 + row] * f;
            }
            rec[row] = M;
            rec[16 + row] = s;
        }
        __syncthreads();
        for (int e = threadIdx.x; e < 16 * D; e += 64 * AT_WAVES) {
            const int row = e / D, d = e % D;
            float o = 0.f;
#pragma unroll
            for (int v = 0; v < AT_WAVES; ++v) o += reinterpret_cast<const float*>(smem + v * WREG)[32 + row * D + d] * fw[row][v];
            rec[32 + e] = o;
        }
    }
}

// Merge of the chunk partials and the tree partial: one work-group per (kv head, row tile, row), one
// thread per output dim; the partials' weights are computed once in LDS, the O loads are independent.
template <int D>
__global__ __launch_bounds__(D) void attn_merge_kernel(AttnArgs a) {
    __shared__ float wgt[72], lsum[72];
    const int row = blockIdx.x % 16, rt = (blockIdx.x / 16) % a.RT, kh = blockIdx.x / (16 * a.RT);
    const int r = rt * 16 + row;
    if (r >= a.rows) return;
    int L = a.seqlen[0];
    L = L < 0 ? 0 : (L > a.cap ? a.cap : L);
    int tpw, active;
    split(L, a.C, a.min_tpw, tpw, active);
    const bool use_tree = a.mask != nullptr;
    const int np = active + (use_tree ? 1 : 0);
    const float* base = a.part + int64_t(kh * a.RT + rt) * (a.C + 1) * (32 + 16 * D);
    auto slot = [&](int i) { return i < active ? i : a.C; };
    const int t = threadIdx.x, lane = t % 64;
    // every wave takes the partials' maximum itself (lane i: partials i and i + 64, np <= 65), then
    // the weights go to LDS (both waves write the same values): one barrier
    const float m0 = lane < np ? base[slot(lane) * (32 + 16 * D) + row] : -INFINITY;
    const float m1 = lane + 64 < np ? base[slot(lane + 64) * (32 + 16 * D) + row] : -INFINITY;
    float M = fmaxf(m0, m1);
    M = max_x32(max_x16(M));
    M = fmaxf(M, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(M), 0x128, 0xF, 0xF, false)));  // row_ror:8
    M = fmaxf(M, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(M), 0x124, 0xF, 0xF, false)));  // row_ror:4
    M = fmaxf(M, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(M), 0x122, 0xF, 0xF, false)));  // row_ror:2
    M = fmaxf(M, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(M), 0x121, 0xF, 0xF, false)));  // row_ror:1
    if (t < 64 || D <= 64) {
        if (lane < np) {
            wgt[lane] = m0 == -INFINITY ? 0.f : exp2f(m0 - M);
            lsum[lane] = base[slot(lane) * (32 + 16 * D) + 16 + row];
        }
        if (lane + 64 < np) {
            wgt[lane + 64] = m1 == -INFINITY ? 0.f : exp2f(m1 - M);
            lsum[lane + 64] = base[slot(lane + 64) * (32 + 16 * D) + 16 + row];
        }
    }
    __syncthreads();
    float o = 0.f, s = 0.f;
#pragma unroll 8
    for (int i = 0; i < np; ++i) {
        o += base[slot(i) * (32 + 16 * D) + 32 + row * D + t] * wgt[i];
        s += lsum[i] * wgt[i];
    }
    const int h = kh * a.groups + r / a.S, sr = r % a.S;
    a.out[(int64_t(sr) * a.H + h) * D + t] = f2bf(s > 0.f ? __fdiv_rn(o, s) : 0.f);
}

// the context split's tuning (MDX_ATTN_TPW: minimum tokens per wave of a chunk; MDX_ATTN_UNITS: the
// work-group count the chunk count aims at), read once; sweeps only
int env_int(const char* name, int dflt, int lo, int hi) {
    const char* e = getenv(name);
    const int v = e ? atoi(e) : dflt;
    return v < lo ? lo : (v > hi ? hi : v);
}
int min_tpw_default() {
    static const int v = env_int("MDX_ATTN_TPW", AT_MIN_TPW, AT_STEP, 4096) / AT_STEP * AT_STEP;
    return v;
}
int target_units() {
    static const int v = env_int("MDX_ATTN_UNITS", 512, 8, 65536);
    return v;
}

int plan_chunks(int Hk, int RT, int cap, int hint) {
    if (hint > 0) return hint > 64 ? 64 : hint;
    const int tpw = min_tpw_default();
    int c = (target_units() + Hk * RT - 1) / (Hk * RT);
    const int by_cap = (cap + AT_WAVES * tpw - 1) / (AT_WAVES * tpw);
    c = c > by_cap ? by_cap : c;
    return c < 1 ? 1 : (c > 64 ? 64 : c);  // the merge holds at most 64 + 1 partial weights
}

size_t workspace_bytes(int Hk, int RT, int C, int D) {
    return 256 + size_t(Hk) * RT * (C + 1) * (32 + 16 * size_t(D)) * sizeof(float);
}

template <int D>
int launch(const AttnArgs& a, hipStream_t st) {
    constexpr bool PP = D <= 128;  // register ping-pong fits below 256 VGPRs up to head_dim 128
    const int units = a.Hk * (a.C + 1);
    const int grid = (units + 7) / 8 * 8 * a.RT;
    const size_t lds = size_t(AT_WAVES) * 72 * D;
    allow_smem(reinterpret_cast<const void*>(&attn_kernel<D, PP>), lds);
    hipLaunchKernelGGL((attn_kernel<D, PP>), dim3(grid), dim3(64 * AT_WAVES), lds, st, a);
    MDX_LAUNCHED();
    hipLaunchKernelGGL(attn_merge_kernel<D>, dim3(a.Hk * a.RT * 16), dim3(D), 0, st, a);
    MDX_LAUNCHED();
    return MDX_OK;
}

}  // namespace
}  // namespace mdx

using namespace mdx;

extern "C" size_t mdx_attn_workspace(int64_t H, int64_t Hk, int64_t S, int64_t D, int64_t cap, int64_t chunks_hint) {
    if (Hk <= 0 || H % Hk != 0 || S <= 0) return 0;
    const int RT = int((H / Hk * S + 15) / 16);
    return workspace_bytes(int(Hk), RT, plan_chunks(int(Hk), RT, int(cap), int(chunks_hint)), int(D));
}

extern "C" int mdx_attn_decode(const uint16_t* q, int64_t q_head_stride, int64_t q_row_stride, const uint16_t* key,
                               const uint16_t* value, const int32_t* seqlen, const uint16_t* xk, int64_t xk_head_stride,
                               int64_t xk_row_stride, const uint16_t* xv, int64_t xv_head_stride, int64_t xv_row_stride,
                               const int32_t* mask, uint16_t* out,
                               int64_t H, int64_t Hk, int64_t S, int64_t D, int64_t cap, int64_t chunks_hint,
                               void* workspace, size_t workspace_bytes_, void* stream) {
    MDX_CHECK(q && key && value && seqlen && xk && xv && out, "null pointer");
    MDX_CHECK(D == 64 || D == 128 || D == 256, "head_dim must be 64, 128 or 256");
    MDX_CHECK(Hk >= 1 && H % Hk == 0 && S >= 1 && S <= 16, "heads / 1..16 rows");
    MDX_CHECK(mask || S == 1, "a draft (no mask) has one row");
    MDX_CHECK(H / Hk * S <= 64, "at most 64 query rows per kv head");
    MDX_CHECK(cap >= 1 && cap < (int64_t(1) << 30) / D, "cache capacity");
    MDX_CHECK(aligned(q, 16) && aligned(key, 16) && aligned(value, 16) && aligned(xk, 16) && aligned(xv, 16) &&
                  q_head_stride % 8 == 0 && q_row_stride % 8 == 0 && xk_head_stride % 8 == 0 &&
                  xk_row_stride % 8 == 0 && xv_head_stride % 8 == 0 && xv_row_stride % 8 == 0,
              "16-byte aligned rows");
    const int RT = int((H / Hk * S + 15) / 16);
    const int C = plan_chunks(int(Hk), RT, int(cap), int(chunks_hint));
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
    a.xh = xk_head_stride;
    a.xs = xk_row_stride;
    a.vh = xv_head_stride;
    a.vs = xv_row_stride;
    a.mask = mask;
    a.out = out;
    a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + 256);
    a.H = int(H);
    a.Hk = int(Hk);
    a.S = int(S);
    a.cap = int(cap);
    a.groups = int(H / Hk);
    a.rows = int(H / Hk * S);
    a.RT = RT;
    a.C = C;
    a.min_tpw = chunks_hint > 0 ? AT_STEP : min_tpw_default();
    a.zscale = float(1.0 / sqrt(double(D)) * 1.4426950408889634);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (D == 64) return launch<64>(a, st);
    if (D == 128) return launch<128>(a, st);
    return launch<256>(a, st);
}
