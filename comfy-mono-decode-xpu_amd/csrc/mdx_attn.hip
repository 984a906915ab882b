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
// row tile (rt). Both forms below compute, per 32-token step of a query row tile:
//   S^T = K Q^T   v_mfma_f32_16x16x32_bf16, A = 16 K rows (tokens) x 32 dims, B = Q^T held in
//                 registers; the accumulator gives each lane 4 tokens of one query row (lane % 16), so
//                 the online softmax state of a row lives in its lanes;
//   O^T += V^T P^T   A = V^T, its 8 k-slots per lane in the token order the S^T accumulators hold,
//                 B = bf16(P^T) straight from the S^T registers -- no shuffle of P.
// Each work-group stores a chunk partial (m, l, O in fp32); attn_merge_kernel (one work-group per
// query row, one thread per dim) combines the chunks and the tree-row partial and writes bf16. The
// context split is recomputed on the device from seqlen in both launches, so a captured graph
// replays for any context length.
//
// The streaming form (attn2_kernel, head_dim 64 / 128): one work-group per (kv head, chunk) over all
// of the kv head's row tiles, K/V read once from HBM into an LDS ring (see the layout note at
// stage_k). The register form (attn_kernel, head_dim 256): work-group = (kv head, row tile, chunk) of
// 4 waves, each owning a quarter of the chunk; K rows straight from HBM as the A operand, V transposed
// into LDS per wave, the next step's K and V prefetched into a second register set (head_dim <= 128);
// work-group ids dealt so that the row tiles of one (kv head, chunk) share an XCD and re-read the
// chunk from its L2.
//
// The tree-verify form with the Q/K prep (attn2_kernel<.., PREP>, head_dim 128): the launch also does the
// RoPE/KV kernel's work for these rows (mdx_rope.hpp: per-head RMSNorm, split-half RoPE), so the step
// needs no launch for it. Every work-group computes its kv head's query rows itself (64 rows x 128, into
// LDS) while its first ring stages stream in; the tree work-group also computes the tree rows' k, writes
// them (k_out, and the cache at their positions, which lie past the prefix the chunks read) with the v
// rows, and only then streams them back as its tree stage. Bit-identical to qk_norm_rope_kv + the
// streaming form.
#include <math.h>
#include <stdlib.h>

#include "mdx_common.hpp"
#include "mdx_rope.hpp"

namespace mdx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

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
    int p2;                  // the streaming form's token parts per chunk (0: the register form)
    float zscale;            // 1/sqrt(D) * log2(e)
    // the Q/K prep (PREP launches): raw q / k rows [S][H][D] with strides (row, head), the per-head norm
    // weights (null: no norm), the rows' rotation matrices [S][rd / 2][2][2] (row stride fs floats), the
    // caches the tree rows' k / v are written to at pos, k_out = xk [Hk][S][D], q_out [H][S][D] or null
    const uint16_t* rq;
    int64_t rqs, rqh;
    const uint16_t* rk;
    int64_t rks, rkh;
    const uint16_t* wq;
    const uint16_t* wk;
    float epsq, epsk;
    const float* freqs;
    int64_t fs;
    int rd;
    uint16_t* kc;
    uint16_t* vc;
    const int64_t* pos;
    uint16_t* k_out;
    uint16_t* q_out;
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

// ---- The streaming form (head_dim 64 and 128) ---------------------------------------------------
// One work-group per (kv head, chunk): all of the kv head's query rows (up to 4 row tiles) in one
// work-group, so each K/V byte leaves HBM once and is read from LDS by every row tile. Wave w of NWV
// owns row tile w % RTW and token part w / RTW of the chunk (P = NWV / RTW parts; eight waves, two per
// SIMD, wherever each part still gets two ring stages). A part's K and V stream through its share of
// a 128 KiB LDS ring of 32-token stages by direct-to-LDS loads (1 KiB per wave instruction, the ring's
// stages in flight from the prologue). Per stage a wave reads its S^T and V^T operands from LDS in two
// batches (layouts at stage_k), computes S^T = K Q^T, the online softmax in its lanes, and
// O^T += V^T P^T; the P parts of a row tile merge in LDS. The grid is at most 256 work-groups (one
// round on the chip's 256 CUs: the ring takes most of a CU's LDS).
constexpr int A2_STEP = 32;
constexpr int A2_RING = 128 * 1024;  // K/V ring bytes per work-group
constexpr int A2_MAX_WG = 256;

// LDS layout of a ring stage (32 tokens; no swizzle: every read below covers contiguous bytes)
//   K: [kk < D/32][token 32][g 4][16 B]  -- unit 4 kk + g of each token row; the S^T operand of
//      (16-token tile tt, kk) is one contiguous KiB: lane (c16, g) at kk * 2048 + (16 tt + c16) * 64 + g * 16
//   V: [dt < D/16][token 32][2][16 B]    -- dims 16 dt .. 16 dt + 15 of each token row; a transposing
//      read of (dt, tokens 16 h ..) is 512 contiguous bytes at dt * 1024 + h * 512
// so one base address per lane and immediate offsets reach every operand of the stage. The reads are
// inline asm: the builtins make the compiler wait for every outstanding direct-to-LDS load (vmcnt(0))
// before them, which would drain the ring each stage. Each asm statement ends with its lgkmcnt(0)
// wait, so its results exist (for the compiler) only after the wait. ds_read_b64_tr_b16 (gfx950): in
// each 16-lane group, lane i receives element i % 4 of the 8-byte runs that lanes i / 4 + 4 j point
// at (j = 0..3).
__device__ __forceinline__ uint32_t lds_addr(const unsigned char* p) {
    return uint32_t(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const unsigned char*)p));
}
template <int D>
__device__ __forceinline__ void stage_k(u32x4 (&kf)[2][D / 32], uint32_t base) {
    if constexpr (D == 128) {
        asm volatile(
            "ds_read_b128 %0, %8\n\tds_read_b128 %1, %8 offset:2048\n\tds_read_b128 %2, %8 offset:4096\n\t"
            "ds_read_b128 %3, %8 offset:6144\n\tds_read_b128 %4, %8 offset:1024\n\tds_read_b128 %5, %8 offset:3072\n\t"
            "ds_read_b128 %6, %8 offset:5120\n\tds_read_b128 %7, %8 offset:7168\n\ts_waitcnt lgkmcnt(0)"
            : "=&v"(kf[0][0]), "=&v"(kf[0][1]), "=&v"(kf[0][2]), "=&v"(kf[0][3]), "=&v"(kf[1][0]), "=&v"(kf[1][1]),
              "=&v"(kf[1][2]), "=&v"(kf[1][3])
            : "v"(base));
    } else {
        static_assert(D == 64, "head_dim 64 or 128");
        asm volatile(
            "ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:2048\n\tds_read_b128 %2, %4 offset:1024\n\t"
            "ds_read_b128 %3, %4 offset:3072\n\ts_waitcnt lgkmcnt(0)"
            : "=&v"(kf[0][0]), "=&v"(kf[0][1]), "=&v"(kf[1][0]), "=&v"(kf[1][1])
            : "v"(base));
    }
}
template <int D>
__device__ __forceinline__ void stage_v(u32x2 (&va)[D / 16], u32x2 (&vb)[D / 16], uint32_t base) {
    if constexpr (D == 128) {
        asm volatile(
            "ds_read_b64_tr_b16 %0, %16\n\tds_read_b64_tr_b16 %1, %16 offset:1024\n\t"
            "ds_read_b64_tr_b16 %2, %16 offset:2048\n\tds_read_b64_tr_b16 %3, %16 offset:3072\n\t"
            "ds_read_b64_tr_b16 %4, %16 offset:4096\n\tds_read_b64_tr_b16 %5, %16 offset:5120\n\t"
            "ds_read_b64_tr_b16 %6, %16 offset:6144\n\tds_read_b64_tr_b16 %7, %16 offset:7168\n\t"
            "ds_read_b64_tr_b16 %8, %16 offset:512\n\tds_read_b64_tr_b16 %9, %16 offset:1536\n\t"
            "ds_read_b64_tr_b16 %10, %16 offset:2560\n\tds_read_b64_tr_b16 %11, %16 offset:3584\n\t"
            "ds_read_b64_tr_b16 %12, %16 offset:4608\n\tds_read_b64_tr_b16 %13, %16 offset:5632\n\t"
            "ds_read_b64_tr_b16 %14, %16 offset:6656\n\tds_read_b64_tr_b16 %15, %16 offset:7680\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(va[0]), "=&v"(va[1]), "=&v"(va[2]), "=&v"(va[3]), "=&v"(va[4]), "=&v"(va[5]), "=&v"(va[6]),
              "=&v"(va[7]), "=&v"(vb[0]), "=&v"(vb[1]), "=&v"(vb[2]), "=&v"(vb[3]), "=&v"(vb[4]), "=&v"(vb[5]),
              "=&v"(vb[6]), "=&v"(vb[7])
            : "v"(base));
    } else {
        asm volatile(
            "ds_read_b64_tr_b16 %0, %8\n\tds_read_b64_tr_b16 %1, %8 offset:1024\n\t"
            "ds_read_b64_tr_b16 %2, %8 offset:2048\n\tds_read_b64_tr_b16 %3, %8 offset:3072\n\t"
            "ds_read_b64_tr_b16 %4, %8 offset:512\n\tds_read_b64_tr_b16 %5, %8 offset:1536\n\t"
            "ds_read_b64_tr_b16 %6, %8 offset:2560\n\tds_read_b64_tr_b16 %7, %8 offset:3584\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(va[0]), "=&v"(va[1]), "=&v"(va[2]), "=&v"(va[3]), "=&v"(vb[0]), "=&v"(vb[1]), "=&v"(vb[2]),
              "=&v"(vb[3])
            : "v"(base));
    }
}

// chunk length (tokens, a multiple of 32 P) and active chunk count for context L over C chunks
__device__ __forceinline__ void split2(int L, int C, int P, int& T, int& active) {
    const int per = (L + C - 1) / C, q = A2_STEP * P;
    T = per < 1 ? q : (per + q - 1) / q * q;
    active = L > 0 ? (L + T - 1) / T : 0;
}

template <int D, int RTW, int NWV, bool PREP = false>
__global__ __launch_bounds__(64 * NWV) void attn2_kernel(AttnArgs a) {
    constexpr int P = NWV / RTW;
    constexpr int KK = D / 32, DT = D / 16;
    constexpr int RB = 2 * D;                    // bytes per token row
    constexpr int STAGE = A2_STEP * RB;          // bytes of K (or V) per stage
    constexpr int NS = A2_RING / (2 * STAGE * P);  // ring stages per part
    constexpr int PER = STAGE / 1024 / RTW;      // DMA instructions per wave, stage and matrix
    static_assert(NS >= 2 && PER >= 1 && (NS - 2) * 2 * PER <= 63, "ring geometry");
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, c16 = lane & 15;
    const int rt = w % RTW, part = w / RTW;
    const int kh = blockIdx.x / (a.C + 1), cslot = blockIdx.x % (a.C + 1);
    const bool tree = cslot == a.C;
    int L = a.seqlen[0];
    L = L < 0 ? 0 : (L > a.cap ? a.cap : L);
    int T, active;
    split2(L, a.C, P, T, active);
    if (tree ? a.mask == nullptr : cslot >= active) return;  // no tokens: no partial (the merge skips it)
    const int nst = tree ? 1 : T / (A2_STEP * P);  // stages per part

    // this lane's query row
    const int r = rt * 16 + c16;
    const bool rvalid = r < a.rows;
    const int rr = rvalid ? r : 0;
    const int hq = kh * a.groups + rr / a.S, sq = rr % a.S;
    // the tree rows' masks by scalar loads (the tree work-group only): a vector load here would be waited
    // for with vmcnt(0) at its first use, i.e. behind every stage of the ring issued below
    uint32_t rmask = 0u;
    if (tree) {  // (uniform)
        typedef __attribute__((address_space(4))) const int32_t* const_i32p;
        const const_i32p mc = (const_i32p)(a.mask);
        for (int i = 0; i < a.S; ++i) {
            const uint32_t mi = uint32_t(mc[i]);
            rmask = (rvalid && sq == i) ? mi : rmask;
        }
    }

    // the part's tokens and sources (element strides)
    int t_begin, t_end;
    const uint16_t *kb, *vb;
    int64_t ks, vs;
    if (tree) {
        t_begin = 0;
        t_end = part == 0 ? a.S : 0;
        kb = a.xk + kh * a.xh;
        vb = a.xv + kh * a.vh;
        ks = a.xs;
        vs = a.vs;
    } else {
        t_begin = cslot * T + part * (T / P);
        t_end = min(L, t_begin + T / P);
        kb = a.key + int64_t(kh) * a.cap * D;
        vb = a.value + int64_t(kh) * a.cap * D;
        ks = vs = D;
    }
    const int t_last = t_end > t_begin ? t_end - 1 : (tree ? 0 : min(t_begin, L - 1));
    const int t_clamp = t_last < 0 ? 0 : t_last;  // a token every load may read (in bounds)

    // The query rows reach the MFMA operands through LDS, read by inline asm: the compiler waits for every
    // direct-to-LDS load in flight before it uses a vector register that a load wrote, so query rows loaded
    // into registers would drain the ring at every stage. Rows D + 8 elements apart with the Q/K prep
    // (written by asm), D apart otherwise (direct loads of whole rows).
    u32x4 qf[KK];
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qf[kk] = u32x4{0, 0, 0, 0};
    static_assert(!PREP || (D == 128 && NWV == 8), "the Q/K prep: head_dim 128, eight waves");
    constexpr int QROW = D + (PREP ? 8 : 0);
    __shared__ __align__(16) uint16_t qst[64 * QROW];
    const uint32_t qbase = lds_addr(reinterpret_cast<const unsigned char*>(qst));
    if constexpr (!PREP) {
        // part 0's wave of each row tile brings the tile's 16 rows (D / 32 loads of 1 KiB, ahead of the ring:
        // the first stage's wait covers them, its barrier every tile's)
        if (part == 0) {
            constexpr int LPR = D / 8, RPI = 64 / LPR;  // lanes per row, rows per load
#pragma unroll
            for (int j = 0; j < D / 32; ++j) {
                const int rr_ = min(rt * 16 + j * RPI + lane / LPR, a.rows - 1);  // (clamped: in bounds)
                const uint16_t* src = a.q + (kh * a.groups + rr_ / a.S) * a.qh + (rr_ % a.S) * a.qs + (lane % LPR) * 8;
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                                 (__attribute__((address_space(3))) void*)(qst + (rt * 16 + j * RPI) * D),
                                                 16, 0, 0);
            }
        }
    }
    auto read_q = [&]() {  // lane (row c16 of tile rt, k-group g): 8 elements at 32 kk + 8 g of its row
        const uint32_t ar = qbase + uint32_t((rvalid ? r : 0) * QROW + 8 * g) * 2;
        if constexpr (KK == 4)
            asm volatile("ds_read_b128 %0, %4\n\tds_read_b128 %1, %4 offset:64\n\tds_read_b128 %2, %4 offset:128\n\t"
                         "ds_read_b128 %3, %4 offset:192\n\ts_waitcnt lgkmcnt(0)"
                         : "=&v"(qf[0]), "=&v"(qf[1]), "=&v"(qf[2]), "=&v"(qf[3])
                         : "v"(ar));
        else
            asm volatile("ds_read_b128 %0, %2\n\tds_read_b128 %1, %2 offset:64\n\ts_waitcnt lgkmcnt(0)"
                         : "=&v"(qf[0]), "=&v"(qf[1])
                         : "v"(ar));
        if (!rvalid)
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) qf[kk] = u32x4{0, 0, 0, 0};
    };

    // (the tree work-group of a PREP launch writes its one stage itself, into part 0's first slot, which all
    // of its parts read: the other parts have no tokens there)
    unsigned char* ring = smem + ((PREP && tree) ? 0 : part) * NS * 2 * STAGE;
    // stage s of this part into ring slot s % NS: the wave's PER instructions of K and of V (instruction
    // i of a matrix writes LDS bytes [1024 i, 1024 i + 1024) of the stage's block in the layouts above;
    // lane -> (token within the stage, byte offset within the token row)). Byte offsets fit 32 bits
    // (cap * D * 2 < 2^31).
    const unsigned char* kbase = reinterpret_cast<const unsigned char*>(kb);
    const unsigned char* vbase = reinterpret_cast<const unsigned char*>(vb);
    const int ksb = int(ks) * 2, vsb = int(vs) * 2;
    int ktok[PER], kofs[PER], vtok[PER], vofs[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int i = rt * PER + j;
        ktok[j] = 16 * (i & 1) + (lane >> 2);
        kofs[j] = (4 * (i >> 1) + (lane & 3)) * 16;
        vtok[j] = lane >> 1;
        vofs[j] = (2 * i + (lane & 1)) * 16;
    }
    auto issue = [&](int s) {
        unsigned char* kd = ring + (s % NS) * 2 * STAGE;
        const int t0 = t_begin + s * A2_STEP;
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int o0 = (rt * PER + j) * 1024;
            const int tk = min(t0 + ktok[j], t_clamp), tv = min(t0 + vtok[j], t_clamp);
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(kbase + (tk * ksb + kofs[j])),
                                             (__attribute__((address_space(3))) void*)(kd + o0), 16, 0, 0);
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)(vbase + (tv * vsb + vofs[j])),
                                             (__attribute__((address_space(3))) void*)(kd + STAGE + o0), 16, 0, 0);
        }
    };

    f32x4 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;

    if constexpr (!PREP) {
        for (int s = 0; s < NS - 1 && s < nst; ++s) issue(s);
    } else {
        // The chunk work-groups issue the ring's first round, then the raw query rows (this wave's rows w,
        // w + NWV, ...; lane l: elements l and l + 64), their rotation matrices and norm weights: the wait
        // for these also waits for that round (loads return in order), which the first stage needs
        // anyway. The compiler waits for every direct-to-LDS load before it uses a vector register that a
        // load issued after them wrote, so no loaded register may be live into the stage loop: the query
        // rows go through LDS (inline asm, which the compiler does not track).
        if (!tree)
            for (int s = 0; s < NS - 1 && s < nst; ++s) issue(s);
        constexpr int QPW = 64 / NWV;
        float rx0[QPW], rx1[QPW];
        float4 rm[QPW];
        // the rotation pair of element l (a lane past the rotated elements reads pair 0, unused)
        const int jj = lane >= a.rd ? 0 : (lane < a.rd / 2 ? lane : lane - a.rd / 2);
#pragma unroll
        for (int i = 0; i < QPW; ++i) {
            const int rc = min(w + NWV * i, a.rows - 1);  // (clamped: every load in bounds)
            const int s_ = rc % a.S;
            const uint16_t* src = a.rq + s_ * a.rqs + (kh * a.groups + rc / a.S) * a.rqh;
            rx0[i] = bf2f(src[lane]);
            rx1[i] = bf2f(src[lane + 64]);
            rm[i] = *reinterpret_cast<const float4*>(a.freqs + s_ * a.fs + jj * 4);
        }
        const uint16_t* wsrc = a.wq ? a.wq : a.rq;  // (no norm: any valid row, the values unused)
        const float wq0 = bf2f(wsrc[lane]), wq1 = bf2f(wsrc[lane + 64]);
        // the query rows into LDS (rows D + 8 elements apart: no bank conflicts)
        uint16_t qo0[QPW], qo1[QPW];
        qk_rope128_n<QPW>(rx0, rx1, a.wq != nullptr, wq0, wq1, a.epsq, a.rd, rm, lane, qo0, qo1);
#pragma unroll
        for (int i = 0; i < QPW; ++i) {
            const int r_ = w + NWV * i;
            if (r_ < a.rows) {  // (uniform)
                const uint32_t ad = qbase + uint32_t(r_ * QROW + lane) * 2;
                asm volatile("ds_write_b16 %0, %1\n\tds_write_b16 %0, %2 offset:128" ::"v"(ad), "v"(uint32_t(qo0[i])),
                             "v"(uint32_t(qo1[i])));
                if (tree && a.q_out) {
                    uint16_t* qo = a.q_out + ((kh * a.groups + r_ / a.S) * a.S + r_ % a.S) * D;
                    qo[lane] = qo0[i];
                    qo[lane + 64] = qo1[i];
                }
            }
        }
        if (tree) {
            // the tree rows' k (normed, rotated) and v straight into the stage this work-group reads, in the
            // layouts the ring's loads produce (K: block 2 (d / 32) + t / 16, row t % 16, 64 bytes; V: block
            // d / 16, row t, 32 bytes), and to k_out and the caches (stores nothing waits for); the V rows past
            // the tree rows zeroed (their P is 0, which a non-finite V would turn into NaN)
            const uint32_t kl = lds_addr(smem), vl = kl + STAGE;
            if ((threadIdx.x & 63) / 2 >= a.S)
                asm volatile("ds_write_b128 %0, %1" ::"v"(vl + threadIdx.x * 16), "v"(u32x4{0u, 0u, 0u, 0u}));
            for (int s_ = w; s_ < a.S; s_ += NWV) {
                const uint16_t* src = a.rk + s_ * a.rks + kh * a.rkh;
                const uint16_t* vsrc = a.xv + kh * a.vh + s_ * a.vs;
                const float x0 = bf2f(src[lane]), x1 = bf2f(src[lane + 64]);
                const uint16_t v0 = vsrc[lane], v1 = vsrc[lane + 64];
                const float4 m = *reinterpret_cast<const float4*>(a.freqs + s_ * a.fs + jj * 4);
                const float w0 = a.wk ? bf2f(a.wk[lane]) : 1.f, w1 = a.wk ? bf2f(a.wk[lane + 64]) : 1.f;
                uint16_t o0, o1;
                qk_rope128(x0, x1, a.wk != nullptr, w0, w1, a.epsk, a.rd, m, lane, o0, o1);
                asm volatile("ds_write_b16 %0, %1\n\tds_write_b16 %0, %2 offset:4096" ::"v"(
                                 kl + uint32_t((2 * (lane >> 5)) * 1024 + s_ * 64 + (lane & 31) * 2)),
                             "v"(uint32_t(o0)), "v"(uint32_t(o1)));
                asm volatile("ds_write_b16 %0, %1\n\tds_write_b16 %0, %2 offset:4096" ::"v"(
                                 vl + uint32_t((lane >> 4) * 1024 + s_ * 32 + (lane & 15) * 2)),
                             "v"(uint32_t(v0)), "v"(uint32_t(v1)));
                uint16_t* ko = a.k_out + (kh * a.S + s_) * D;
                ko[lane] = o0;
                ko[lane + 64] = o1;
                const int64_t p = a.pos[s_];
                if (p >= 0 && p < a.cap) {  // (a position outside the cache writes nothing)
                    uint16_t* kd = a.kc + (int64_t(kh) * a.cap + p) * D;
                    uint16_t* vd = a.vc + (int64_t(kh) * a.cap + p) * D;
                    kd[lane] = o0;
                    kd[lane + 64] = o1;
                    vd[lane] = v0;
                    vd[lane + 64] = v1;
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's rows are in LDS (the ring stays in flight)
        __builtin_amdgcn_s_barrier();
        read_q();
    }
    for (int s = 0; s < nst; ++s) {
        // stage s landed (this wave's share), then everyone's share and everyone done with stage s - 1 (the
        // PREP tree stage was written to LDS before the barrier that precedes the loop: no wait)
        if (PREP && tree) {
        } else if (s + NS - 2 < nst) {
            __builtin_amdgcn_s_waitcnt(((((NS - 2) * 2 * PER) & 15)) | ((((NS - 2) * 2 * PER) >> 4) << 14) | (7 << 4) | (15 << 8));
        } else {
            __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0): the ring's tail
        }
        // s_barrier alone: __syncthreads' release fence would wait for the whole ring (vmcnt(0))
        __builtin_amdgcn_s_barrier();
        if constexpr (!PREP)
            if (s == 0) read_q();
        if (s + NS - 1 < nst) issue(s + NS - 1);
        const unsigned char* kd = ring + (s % NS) * 2 * STAGE;
        const unsigned char* vd = kd + STAGE;
        const int t0 = t_begin + s * A2_STEP;
        // the S^T operands of the stage: lane (token 16 tt + c16, k-group g) reads unit 4 kk + g
        u32x4 kf[2][KK];
        stage_k<D>(kf, lds_addr(kd) + c16 * 64 + g * 16);
        f32x4 st[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            st[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KK; ++kk)
                st[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kf[tt][kk]), as_bf16x8(qf[kk]), st[tt], 0, 0, 0);
        }
        // V^T operands by transposing reads (issued while the S^T MFMAs run): lane s of group g points at token 4 g + s / 4 (+ 16 for the
        // second read), dims 16 dt + 4 (s % 4) .. + 3, so lane (dim 16 dt + c16, g) receives the 8 tokens
        // of its k-slots (4 g .. 4 g + 3, then 16 + 4 g ..), the order its S^T accumulators give P^T
        u32x2 va[DT], vb2[DT];
        stage_v<D>(va, vb2, lds_addr(vd) + (4 * g + (c16 >> 2)) * 32 + (c16 & 3) * 8);
        // the stage's admitted tokens (bit j: token t0 + j); whole stages of the prefix skip the mask
        const int nvalid = t_end - t0;
        uint32_t mbits = nvalid >= 32 ? ~0u : (nvalid > 0 ? (1u << nvalid) - 1u : 0u);
        if (tree) mbits &= rmask;
        float z[2][4], mx = -INFINITY;
        if (__builtin_amdgcn_ballot_w64(mbits != ~0u) == 0) {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    z[tt][i] = st[tt][i] * a.zscale;
                    mx = fmaxf(mx, z[tt][i]);
                }
        } else {
            const uint32_t lb = mbits >> (4 * g);
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    z[tt][i] = ((lb >> (16 * tt + i)) & 1u) ? st[tt][i] * a.zscale : -INFINITY;
                    mx = fmaxf(mx, z[tt][i]);
                }
        }
        mx = max_x32(max_x16(mx));
        const float mnew = fmaxf(m, mx);
        // v_exp_f32 directly (2^-inf = 0; a result below 2^-126 flushes to 0, far inside the bound);
        // a row with nothing admitted yet subtracts 0, so -inf - -inf never forms
        const float msub = mnew == -INFINITY ? 0.f : mnew;
        const float alpha = __builtin_amdgcn_exp2f(m - msub);
        float p[2][4], ps = 0.f;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; i += 2) {
                p[tt][i] = __builtin_amdgcn_exp2f(z[tt][i] - msub);
                p[tt][i + 1] = __builtin_amdgcn_exp2f(z[tt][i + 1] - msub);
                bfround2(p[tt][i], p[tt][i + 1]);
                ps += p[tt][i];
                ps += p[tt][i + 1];
            }
        ps = sum_x32(sum_x16(ps));
        l = l * alpha + ps;
        m = mnew;
        // O^T is rescaled only when some row's maximum moved (x * 1 == x: skipping changes no bit)
        if (__builtin_amdgcn_ballot_w64(alpha != 1.f) != 0) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
        }
        // p holds bf16 values: their top halves are the MFMA operand
        auto top2 = [](float lo, float hi) { return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u); };
        const u32x4 pf = {top2(p[0][0], p[0][1]), top2(p[0][2], p[0][3]), top2(p[1][0], p[1][1]), top2(p[1][2], p[1][3])};
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const u32x4 vf = {va[dt].x, va[dt].y, vb2[dt].x, vb2[dt].y};
            acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(vf), as_bf16x8(pf), acc[dt], 0, 0, 0);
        }
    }

    // the work-group's partial per row tile: (m, l, O) of its rows; P parts merge through LDS first
    float* rec = a.part + (int64_t(kh * a.RT + rt) * (a.C + 1) + cslot) * (32 + 16 * D);
    if (P == 1) {
        if (rt >= a.RT) return;
        if (g == 0) {
            rec[c16] = m;
            rec[16 + c16] = l;
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4*>(rec + 32 + c16 * D + 16 * dt + 4 * g) = acc[dt];
        return;
    }
    __syncthreads();  // the ring is free
    // a wave's (m, l, O) in LDS with O's rows D + 4 floats apart (rows D apart would put the 16 rows a
    // store or load instruction touches in the same banks)
    constexpr int OR = D + 4;
    constexpr int WREG = (32 + 16 * OR) * 4;
    float* wr = reinterpret_cast<float*>(smem + w * WREG);
    if (g == 0) {
        wr[c16] = m;
        wr[16 + c16] = l;
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4*>(wr + 32 + c16 * OR + 16 * dt + 4 * g) = acc[dt];
    __syncthreads();
    // the row tile's P waves (w = rt + RTW * p) merged in part order by the RTW * 64 threads of part 0
    if (part != 0 || rt >= a.RT) return;
    auto part_reg = [&](int p_) { return reinterpret_cast<const float*>(smem + (rt + RTW * p_) * WREG); };
    float fw[P];
    float M = -INFINITY;
#pragma unroll
    for (int p_ = 0; p_ < P; ++p_) M = fmaxf(M, part_reg(p_)[c16]);
    float sl = 0.f;
#pragma unroll
    for (int p_ = 0; p_ < P; ++p_) {
        const float mv = part_reg(p_)[c16];
        fw[p_] = mv == -INFINITY ? 0.f : exp2f(mv - M);
        sl += part_reg(p_)[16 + c16] * fw[p_];
    }
    if (g == 0) {
        rec[c16] = M;
        rec[16 + c16] = sl;
    }
    // lane (row c16, group g): dims 4g + 16 dt .. + 3 of its row
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
        f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int p_ = 0; p_ < P; ++p_) {
            const f32x4 v = *reinterpret_cast<const f32x4*>(part_reg(p_) + 32 + c16 * OR + 16 * dt + 4 * g);
            o += v * fw[p_];
        }
        *reinterpret_cast<f32x4*>(rec + 32 + c16 * D + 16 * dt + 4 * g) = o;
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
    if (a.p2)
        split2(L, a.C, a.p2, tpw, active);
    else
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

// the streaming form for head_dim 64 / 128 (its ring needs two stages per part; 256 does not fit),
// unless MDX_ATTN_V1=1 (A/B sweeps only)
bool use_stream(int D) {
    static const int v1 = env_int("MDX_ATTN_V1", 0, 0, 1);
    return !v1 && (D == 64 || D == 128);
}
int stream_rtw(int RT) { return RT <= 1 ? 1 : (RT == 2 ? 2 : 4); }
// token parts per chunk: eight waves per work-group (two per SIMD, so one wave's LDS and MFMA waits
// overlap the other's work) where each part still gets two ring stages, else four waves (head_dim 128
// with one row tile)
int stream_parts(int D, int RT) {
    const int rtw = stream_rtw(RT);
    if (D == 128) return rtw == 4 ? 2 : 4;
    return 8 / rtw;
}
// chunks per kv head of the streaming form: one work-group per (kv head, chunk) plus the tree
// work-group within one round of 256, at least 32 tokens per part, at most 64 chunks (the merge)
int plan_chunks2(int Hk, int RT, int D, int cap, int hint) {
    const int P = stream_parts(D, RT);
    int c = A2_MAX_WG / Hk - 1;
    const int by_cap = (cap + A2_STEP * P - 1) / (A2_STEP * P);
    c = c > by_cap ? by_cap : c;
    if (hint > 0 && c > hint) c = hint;
    return c < 1 ? 1 : (c > 64 ? 64 : c);
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

template <int D, int RTW, int NWV, bool PREP = false>
int launch2(const AttnArgs& a, hipStream_t st) {
    allow_smem(reinterpret_cast<const void*>(&attn2_kernel<D, RTW, NWV, PREP>), A2_RING);
    hipLaunchKernelGGL((attn2_kernel<D, RTW, NWV, PREP>), dim3(a.Hk * (a.C + 1)), dim3(64 * NWV), A2_RING, st, a);
    MDX_LAUNCHED();
    hipLaunchKernelGGL(attn_merge_kernel<D>, dim3(a.Hk * a.RT * 16), dim3(D), 0, st, a);
    MDX_LAUNCHED();
    return MDX_OK;
}

template <int D>
int launch(const AttnArgs& a, hipStream_t st) {
    if (a.p2) {
        if constexpr (D == 64 || D == 128) {
            const int rtw = stream_rtw(a.RT);
            if (rtw == 1) return launch2<D, 1, (D == 128 ? 4 : 8)>(a, st);
            if (rtw == 2) return launch2<D, 2, 8>(a, st);
            return launch2<D, 4, 8>(a, st);
        }
    }
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
    const int C = use_stream(int(D)) ? plan_chunks2(int(Hk), RT, int(D), int(cap), int(chunks_hint))
                                     : plan_chunks(int(Hk), RT, int(cap), int(chunks_hint));
    return workspace_bytes(int(Hk), RT, C, int(D));
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
    const bool v2 = use_stream(int(D));
    const int C = v2 ? plan_chunks2(int(Hk), RT, int(D), int(cap), int(chunks_hint))
                     : plan_chunks(int(Hk), RT, int(cap), int(chunks_hint));
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
    a.p2 = v2 ? stream_parts(int(D), RT) : 0;
    a.zscale = float(1.0 / sqrt(double(D)) * 1.4426950408889634);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (D == 64) return launch<64>(a, st);
    if (D == 128) return launch<128>(a, st);
    return launch<256>(a, st);
}

// Tree-verify attention with the RoPE/KV kernel's Q/K prep in the same launch: see the note at the top of
// this file. Raw rows as mdx_qk_norm_rope_kv takes them, the cache written at position[s] as it writes it,
// k_out [Hk, S, D] (also the tree rows' k the launch attends), q_out [H, S, D] optional.
extern "C" int mdx_attn_decode_rope(const uint16_t* q, int64_t q_row_stride, int64_t q_head_stride, const uint16_t* k,
                                    int64_t k_row_stride, int64_t k_head_stride, const uint16_t* v, int64_t v_row_stride,
                                    int64_t v_head_stride, const uint16_t* weight_q, const uint16_t* weight_k, float eps_q,
                                    float eps_k, const float* freqs, int64_t freqs_row_stride, int64_t rd, uint16_t* key,
                                    uint16_t* value, const int64_t* position, const int32_t* seqlen, const int32_t* mask,
                                    uint16_t* k_out, uint16_t* q_out, uint16_t* out, int64_t H, int64_t Hk, int64_t S,
                                    int64_t D, int64_t cap, int64_t chunks_hint, void* workspace, size_t workspace_bytes_,
                                    void* stream) {
    MDX_CHECK(q && k && v && freqs && key && value && position && seqlen && mask && k_out && out, "null pointer");
    MDX_CHECK((weight_q == nullptr) == (weight_k == nullptr), "norm weights: both or neither");
    MDX_CHECK(D == 128 && use_stream(int(D)), "the Q/K prep form: head_dim 128 (streaming form)");
    MDX_CHECK(rd == 32 || rd == 64 || rd == 128, "rotary dimension 32, 64 or 128");
    MDX_CHECK(Hk >= 1 && H % Hk == 0 && S >= 1 && S <= 16, "heads / 1..16 rows");
    const int64_t rows = H / Hk * S;
    MDX_CHECK(rows > 16 && rows <= 64, "17..64 query rows per kv head (fewer: the separate launches)");
    MDX_CHECK(cap >= 1 && cap < (int64_t(1) << 30) / D, "cache capacity");
    MDX_CHECK(aligned(key, 16) && aligned(value, 16) && aligned(k_out, 16) && aligned(v, 16) && aligned(freqs, 16) &&
                  v_row_stride % 8 == 0 && v_head_stride % 8 == 0 && freqs_row_stride % 4 == 0,
              "16-byte aligned cache, k_out, v rows and rotation rows");
    const int RT = int((rows + 15) / 16);
    const int C = plan_chunks2(int(Hk), RT, int(D), int(cap), int(chunks_hint));
    MDX_CHECK(workspace && aligned(workspace, 256) && workspace_bytes_ >= workspace_bytes(int(Hk), RT, C, int(D)),
              "workspace: %zu bytes, 256-byte aligned, zeroed once", workspace_bytes(int(Hk), RT, C, int(D)));
    AttnArgs a{};
    a.key = key;
    a.value = value;
    a.seqlen = seqlen;
    a.xk = k_out;
    a.xh = S * D;
    a.xs = D;
    a.xv = v;
    a.vh = v_head_stride;
    a.vs = v_row_stride;
    a.mask = mask;
    a.out = out;
    a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + 256);
    a.H = int(H);
    a.Hk = int(Hk);
    a.S = int(S);
    a.cap = int(cap);
    a.groups = int(H / Hk);
    a.rows = int(rows);
    a.RT = RT;
    a.C = C;
    a.min_tpw = chunks_hint > 0 ? AT_STEP : min_tpw_default();
    a.p2 = stream_parts(int(D), RT);
    a.zscale = float(1.0 / sqrt(double(D)) * 1.4426950408889634);
    a.rq = q;
    a.rqs = q_row_stride;
    a.rqh = q_head_stride;
    a.rk = k;
    a.rks = k_row_stride;
    a.rkh = k_head_stride;
    a.wq = weight_q;
    a.wk = weight_k;
    a.epsq = eps_q;
    a.epsk = eps_k;
    a.freqs = freqs;
    a.fs = freqs_row_stride;
    a.rd = int(rd);
    a.kc = key;
    a.vc = value;
    a.pos = position;
    a.k_out = k_out;
    a.q_out = q_out;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (stream_rtw(RT) == 2) return launch2<128, 2, 8, true>(a, st);
    return launch2<128, 4, 8, true>(a, st);
}
