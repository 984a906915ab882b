// The second stage of the two-stage draft lm_head ("draft pick"), one launch: from approximate scores
// of the whole vocabulary, the exact top-n (torch XPU topk order) and argmax of the exact logits, and
// the draft's outputs.
//
// Reference semantics (comfy-mono-decode-xpu): csrc/draft_lmhead.sycl:82-291 (contract: exact int8
// logits bf16((float(acc) * x_scale) * w_scale[n]) with acc the int32 dot of the rotated, quantised
// activation and the int8 row; torch topk's tie order and argmax rules; outputs top[:n], the rank row,
// the draft token (the argmax, or top[0]) and the children's verify tokens; a call counter; with no
// weight the scores are the logits), comfy_mono_decode_xpu/draft_lmhead.py:1-20,134-149.
// The bf16 form (mdx_draft_pick_bf16) is this library's own: the exact logits are those of its bf16
// lm_head (mdx_bf16_linear) for the candidates, recomputed with the same MFMA chain, so the pick equals
// the one-stage head (bf16_linear + fast_topk) whenever the exact top-n lies within the candidates.
//
// Launch: PK_WG work-groups of 256, each owning a contiguous segment of the vocabulary.
//   1. candidates: the work-group's S best approximate scores (ties: the smaller index), selected as
//      in the top-k kernel: theta = the S-th largest of the 256 thread maxima; every element >= theta
//      belongs to a thread whose maximum is >= theta (at most S of them), then counting ranks;
//   2. the candidates' exact logits: int8 (the 32 candidate rows and the activation land in LDS by DMA
//      in K blocks of 4 KiB, then v_dot4 and a wave sum per candidate; integer, so any order), bf16
//      (the 16 candidate rows land in LDS by DMA in the MFMA
//      A-operand layout, then one wave runs the lm_head kernel's chain: v_mfma_f32_16x16x32_bf16 per
//      32-k chunk over each K slice, the slices added in slice order), or the scores themselves;
//   3. the work-group's top 8 by topk rank and its best argmax rank go to the workspace (coherent
//      stores); the last work-group (device-scope counter, reset by it) takes the nout-th largest list
//      head as a floor, ranks the entries at or above it (at most 8 nout) by counting and writes the
//      outputs.
#include <algorithm>

#include "mdx_common.hpp"
#include "mdx_rank.hpp"

namespace mdx {
namespace {

constexpr int PK_WG = 32;
constexpr int PK_T = 256;
constexpr int PK_MAXN = 8;
constexpr int PK_MAXCH = 8;
constexpr int PK_E = 32;      // elements per thread (segments of at most 8192)
constexpr int PK_MAXS = 32;   // candidates per work-group at most
constexpr int PK_CAP = PK_MAXS * PK_E;
constexpr int PK_KB = 4096;  // int8 head: K bytes per LDS block

enum PickMode : int { PICK_EXACT = 0, PICK_I8 = 1, PICK_BF16 = 2 };

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

#define PK_G __attribute__((address_space(1)))
#define PK_LDS(p) ((__attribute__((address_space(3))) void*)(p))

struct PickArgs {
    const uint16_t* approx;  // [N] bf16 scores
    int64_t N;
    int seg;                 // segment length (<= PK_T * PK_E)
    int mode, S;
    const int8_t* qx;        // PICK_I8: int8 [K], f32 x_scale [1], int8 [N, K], f32 [N]
    const float* sx;
    const int8_t* w8;
    const float* sw;
    const uint16_t* xb;      // PICK_BF16: bf16 [K] row, bf16 [N, K] head (tile-major or row-major), K slices
    const uint16_t* wb;
    int layout, KS;
    int K;
    int nout, argmax_first, nch;
    int ch[PK_MAXCH];
    int64_t* top;            // [nout] or null
    int64_t* ranks_row;      // [nout] or null
    uint16_t* top_vals;      // [nout] bf16 or null
    int64_t* token;          // [1]
    int64_t* vtok;           // verify tokens (children written)
    int64_t* calls;          // [1] or null
    uint64_t* lists;         // workspace [PK_WG][PK_MAXN] topk ranks, [PK_WG] argmax ranks, counter
    uint64_t* amax;
    unsigned* counter;
};

__device__ __forceinline__ void st_c64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_c64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// approximate-score selection key: the bf16 value order, then the smaller index; unique per element
__device__ __forceinline__ uint64_t sel_key(uint16_t b, uint32_t i) {
    return (uint64_t(key_bf16(b)) << 32) | (0xFFFFFFFFu - i);
}

// bf16 bits of a topk rank's value (inverse of key_bf16; a NaN comes back as 0x7FFF)
__device__ __forceinline__ uint16_t bits_of_rank(uint64_t r) {
    const uint32_t k = uint32_t(r >> 32);
    return uint16_t(k >= 0x8000u ? k ^ 0x8000u : k ^ 0xFFFFu);
}

__device__ __forceinline__ int count_above(const uint64_t* buf, int n, uint64_t v) {
    int c = 0;
    for (int f0 = 0; f0 < n; f0 += 8) {
        uint64_t x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = buf[min(f0 + j, n - 1)];
#pragma unroll
        for (int j = 0; j < 8; ++j) c += (f0 + j < n && x[j] > v) ? 1 : 0;
    }
    return c;
}

// The bf16 lm_head kernel's MFMA chain over the candidate rows in LDS: chunk j's A operand at
// w + j * WSTEP, its B operand (the activation) at x + 64 j, zero in the lanes of activation rows past the
// first (zero_b). Each K slice (chunks [ks NC / KS, (ks + 1) NC / KS)) is one chain and the slices are
// added in order. The chain runs in groups of 8 chunks: the next group's operand reads are issued before
// this group's MFMAs (scheduling barriers keep the two apart), so the MFMAs wait on no LDS latency.
template <int WSTEP>
__device__ __forceinline__ f32x4 pick_chain(const uint8_t* w, const uint8_t* x, int NC, int KS, bool zero_b) {
    constexpr int PD = 8;
    auto mfma = [&](f32x4 acc, u32x4 wv, u32x4 xv) {
        if (zero_b) xv = u32x4{0u, 0u, 0u, 0u};
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wv), __builtin_bit_cast(bf16x8, xv), acc,
                                                       0, 0, 0);
    };
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    for (int ks = 0; ks < KS; ++ks) {
        const int c0 = ks * NC / KS, c1 = (ks + 1) * NC / KS, cf = c0 + (c1 - c0) / PD * PD;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        if (cf > c0) {
            u32x4 wv[PD], xv[PD];
#pragma unroll
            for (int i = 0; i < PD; ++i) {
                wv[i] = *reinterpret_cast<const u32x4*>(w + (c0 + i) * WSTEP);
                xv[i] = *reinterpret_cast<const u32x4*>(x + (c0 + i) * 64);
            }
            for (int j = c0; j < cf; j += PD) {
                const int jn = j + PD < cf ? j + PD : j;  // the last group reads itself again (in bounds)
                u32x4 wn[PD], xn[PD];
#pragma unroll
                for (int i = 0; i < PD; ++i) {
                    wn[i] = *reinterpret_cast<const u32x4*>(w + (jn + i) * WSTEP);
                    xn[i] = *reinterpret_cast<const u32x4*>(x + (jn + i) * 64);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < PD; ++i) acc = mfma(acc, wv[i], xv[i]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < PD; ++i) {
                    wv[i] = wn[i];
                    xv[i] = xn[i];
                }
            }
        }
        for (int j = cf; j < c1; ++j)
            acc = mfma(acc, *reinterpret_cast<const u32x4*>(w + j * WSTEP), *reinterpret_cast<const u32x4*>(x + j * 64));
        if (ks == 0) s = acc;
        else s += acc;
    }
    return s;
}

__global__ __launch_bounds__(PK_T) void draft_pick_kernel(PickArgs a) {
    extern __shared__ __align__(16) uint8_t rows_lds[];  // PICK_BF16: [K / 32][64 lanes][16 B] rows, then x [K]
    __shared__ uint64_t cand[PK_CAP];
    __shared__ uint64_t tmax[PK_T];
    __shared__ uint64_t theta;
    __shared__ int ncand;
    __shared__ int sel[PK_MAXS];
    __shared__ uint16_t logit[PK_MAXS];
    __shared__ uint64_t rk[PK_MAXS], ra[PK_MAXS];
    __shared__ uint64_t mlist[PK_WG * PK_MAXN + PK_WG];
    __shared__ uint64_t m2[PK_MAXN * PK_MAXN];
    __shared__ uint64_t theta2;
    __shared__ int is_last, nm2;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int w = blockIdx.x;
    const int64_t s0 = int64_t(w) * a.seg;
    const int len = int(min(int64_t(a.seg), a.N - s0));  // >= PK_T (host check)

    // 1. candidates: this thread's elements s0 + t + 256 j, all loads first
    uint16_t v[PK_E];
#pragma unroll
    for (int j = 0; j < PK_E; ++j) v[j] = a.approx[s0 + min(t + PK_T * j, len - 1)];
    uint64_t m = 0;
#pragma unroll
    for (int j = 0; j < PK_E; ++j)
        if (t + PK_T * j < len) {
            const uint64_t k = sel_key(v[j], uint32_t(s0 + t + PK_T * j));
            m = k > m ? k : m;
        }
    tmax[t] = m;
    if (t == 0) ncand = 0;
    __syncthreads();
    // theta: the S-th largest thread maximum (maxima are unique and every thread holds an element)
    if (count_above(tmax, PK_T, m) == a.S - 1) theta = m;
    __syncthreads();
    const uint64_t th = theta;
#pragma unroll
    for (int j = 0; j < PK_E; ++j)
        if (t + PK_T * j < len) {
            const uint64_t k = sel_key(v[j], uint32_t(s0 + t + PK_T * j));
            if (k >= th) {
                const int slot = atomicAdd(&ncand, 1);
                cand[slot] = k;  // (at most S threads hold such elements: slot < S * PK_E)
            }
        }
    __syncthreads();
    const int nc = ncand;
    for (int i = t; i < nc; i += PK_T) {
        const int pos = count_above(cand, nc, cand[i]);
        if (pos < a.S) sel[pos] = int(0xFFFFFFFFu - uint32_t(cand[i]));
    }
    __syncthreads();

    // 2. the candidates' exact logits
    if (a.mode == PICK_EXACT) {
        if (t < a.S) logit[t] = a.approx[sel[t]];
    } else if (a.mode == PICK_I8) {
        // K blocks of at most PK_KB bytes: the S candidate rows' block and the activation's land in LDS by
        // DMA (every load in flight at once), then wave q sums candidates q, q + 4, ... (int32: any order)
        uint8_t* xq = rows_lds + size_t(a.S) * min(a.K, PK_KB);
        int acc[PK_MAXS / 4];
#pragma unroll
        for (int i = 0; i < PK_MAXS / 4; ++i) acc[i] = 0;
        for (int kb0 = 0; kb0 < a.K; kb0 += PK_KB) {
            const int kb = min(PK_KB, a.K - kb0), per = kb / 16, pieces = a.S * per;
            for (int p0 = wave * 64; p0 < pieces; p0 += PK_T) {
                const int p = p0 + lane, c = p / per, o = (p - c * per) * 16;  // (pieces: a multiple of 64)
                __builtin_amdgcn_global_load_lds((const PK_G uint8_t*)(a.w8 + int64_t(sel[c]) * a.K + kb0 + o),
                                                 PK_LDS(rows_lds + size_t(p0) * 16), 16, 0, 0);
            }
            for (int p0 = wave * 64; p0 < per; p0 += PK_T)
                if (p0 + lane < per)  // (a lane past the block would write past the LDS block)
                    __builtin_amdgcn_global_load_lds((const PK_G uint8_t*)(a.qx + kb0 + (p0 + lane) * 16),
                                                     PK_LDS(xq + size_t(p0) * 16), 16, 0, 0);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            for (int r = 0; 16 * lane + 1024 * r < kb; ++r) {
                const int k = 16 * lane + 1024 * r;
                const uint4 xv = *reinterpret_cast<const uint4*>(xq + k);
#pragma unroll
                for (int i = 0; i < PK_MAXS / 4; ++i) {
                    const int q = wave + 4 * i;
                    if (q < a.S) {
                        const uint4 wv = *reinterpret_cast<const uint4*>(rows_lds + size_t(q) * kb + k);
                        acc[i] = sdot4(int(wv.x), int(xv.x), acc[i]);
                        acc[i] = sdot4(int(wv.y), int(xv.y), acc[i]);
                        acc[i] = sdot4(int(wv.z), int(xv.z), acc[i]);
                        acc[i] = sdot4(int(wv.w), int(xv.w), acc[i]);
                    }
                }
            }
            __syncthreads();  // (the next block reuses the LDS)
        }
        const float xs = a.sx[0];
#pragma unroll
        for (int i = 0; i < PK_MAXS / 4; ++i) {
            int v = acc[i];
            for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
            const int q = wave + 4 * i;
            if (lane == 0 && q < a.S) logit[q] = f2bf(__fmul_rn(__fmul_rn(float(v), xs), a.sw[sel[q]]));
        }
    } else {
        // PICK_BF16, S = 16. Row-major head with K % 512 == 0: each candidate row lands in LDS contiguously
        // (1 KiB contiguous per DMA instruction), rows 2 K + 16 bytes apart (the 16 rows of one MFMA operand
        // read fall on different banks); otherwise piece (chunk j, lane 16 g + c) = candidate c's k
        // [32 j + 8 g, + 8) in the MFMA A-operand layout. Then x.
        const int NC = a.K / 32;
        const bool rowl = a.layout == MDX_LAYOUT_ROW && a.K % 512 == 0;
        const int rstride = 2 * a.K + 16;
        const size_t rows_bytes = rowl ? size_t(16) * rstride : size_t(NC) * 64 * 16;
        uint8_t* xl = rows_lds + rows_bytes;
        if (rowl) {
            const int per = a.K / 8;  // 16-byte pieces per row (a multiple of 64)
            for (int p0 = wave * 64; p0 < 16 * per; p0 += PK_T) {
                const int c = p0 / per, q0 = p0 - c * per;
                __builtin_amdgcn_global_load_lds((const PK_G uint8_t*)(a.wb + int64_t(sel[c]) * a.K + 8 * (q0 + lane)),
                                                 PK_LDS(rows_lds + size_t(c) * rstride + size_t(q0) * 16), 16, 0, 0);
            }
        } else {
            const int pieces = NC * 64;
            for (int p0 = wave * 64; p0 < pieces; p0 += PK_T) {
                const int p = p0 + lane, j = p >> 6, l = p & 63, g = l >> 4, c = l & 15;
                const int64_t n = sel[c];
                const uint16_t* src = a.layout == MDX_LAYOUT_TILE
                                          ? a.wb + ((n >> 4) * int64_t(NC) + j) * 512 + (16 * g + (n & 15)) * 8
                                          : a.wb + n * a.K + 32 * j + 8 * g;
                __builtin_amdgcn_global_load_lds((const PK_G uint8_t*)(src), PK_LDS(rows_lds + size_t(p0) * 16), 16, 0, 0);
            }
        }
        for (int p0 = wave * 64; p0 < a.K / 8; p0 += PK_T)
            if (p0 + lane < a.K / 8)  // (a lane past the row would write past the LDS block)
                __builtin_amdgcn_global_load_lds((const PK_G uint8_t*)(a.xb) + size_t(p0 + lane) * 16,
                                                 PK_LDS(xl + size_t(p0) * 16), 16, 0, 0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (wave == 0) {
            const int g = lane >> 4, c = lane & 15;
            const uint8_t* wbase = rowl ? rows_lds + size_t(c) * rstride + 16 * g : rows_lds + size_t(lane) * 16;
            const f32x4 s = rowl ? pick_chain<64>(wbase, xl + 16 * g, NC, a.KS, c != 0)
                                 : pick_chain<1024>(wbase, xl + 16 * g, NC, a.KS, c != 0);
            // D: lane 16 g + c holds outputs 4 g + i of activation row c (row 0 is the real one)
            if (c == 0)
#pragma unroll
                for (int i = 0; i < 4; ++i) logit[4 * g + i] = f2bf(s[i]);
        }
    }
    __syncthreads();

    // 3. the work-group's top 8 (topk ranks) and best argmax rank, published; the last work-group merges
    if (t < a.S) {
        const uint32_t n = uint32_t(sel[t]);
        rk[t] = rank_raw<ORDER_BF16>(logit[t], n);
        ra[t] = rank_raw<ORDER_ARGMAX>(logit[t], n);
    }
    __syncthreads();
    if (t < a.S) {
        const int pos = count_above(rk, a.S, rk[t]);
        if (pos < PK_MAXN) st_c64(a.lists + w * PK_MAXN + pos, rk[t]);
    }
    if (t == 0) {
        uint64_t b = 0;
        for (int q = 0; q < a.S; ++q) b = ra[q] > b ? ra[q] : b;
        st_c64(a.amax + w, b);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t == 0) is_last = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == PK_WG - 1;
    __syncthreads();
    if (!is_last) return;
    if (t < PK_WG * PK_MAXN) mlist[t] = ld_c64(a.lists + t);
    if (t < PK_WG) mlist[PK_WG * PK_MAXN + t] = ld_c64(a.amax + t);
    if (t == 0) nm2 = 0;
    __syncthreads();
    // theta2 = the nout-th largest list head (lists are descending and full, ranks unique): the nout lists
    // with the largest heads hold nout entries >= theta2, so the top nout are all >= theta2, and only
    // those nout lists hold such entries (at most 8 nout of them)
    if (t < PK_WG) {
        const uint64_t hd = mlist[t * PK_MAXN];
        int above = 0;
        for (int q = 0; q < PK_WG; ++q) above += mlist[q * PK_MAXN] > hd ? 1 : 0;
        if (above == a.nout - 1) theta2 = hd;
    }
    __syncthreads();
    if (t < PK_WG * PK_MAXN && mlist[t] >= theta2) m2[atomicAdd(&nm2, 1)] = mlist[t];
    __syncthreads();
    if (t < nm2) {
        const uint64_t r = m2[t];
        const int pos = count_above(m2, nm2, r);
        if (pos < a.nout) {
            const int64_t idx = int64_t(index_of<ORDER_BF16>(r));
            if (a.top) a.top[pos] = idx;
            if (a.ranks_row) a.ranks_row[pos] = idx;
            if (a.top_vals) a.top_vals[pos] = bits_of_rank(r);
            if (pos >= 1 && pos < a.nch) a.vtok[a.ch[pos]] = idx;
            if (pos == 0 && !a.argmax_first) {
                a.token[0] = idx;
                a.vtok[a.ch[0]] = idx;
            }
        }
    }
    if (t == 0) {
        if (a.argmax_first) {
            uint64_t b = 0;
            for (int q = 0; q < PK_WG; ++q) b = mlist[PK_WG * PK_MAXN + q] > b ? mlist[PK_WG * PK_MAXN + q] : b;
            const int64_t idx = int64_t(index_of<ORDER_ARGMAX>(b));
            a.token[0] = idx;
            a.vtok[a.ch[0]] = idx;
        }
        if (a.calls) a.calls[0] += 1;
        __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

size_t pick_ws_bytes() { return size_t(PK_WG * PK_MAXN + PK_WG) * 8 + 256; }

int launch_pick(PickArgs& a, const int64_t* children, int64_t nch, int64_t nvtok, void* ws, size_t ws_bytes,
                hipStream_t st) {
    MDX_CHECK(a.approx && a.token && a.vtok && children && ws, "null pointer");
    MDX_CHECK(ws_bytes >= pick_ws_bytes() && aligned(ws, 256), "workspace: mdx_draft_pick_workspace() bytes, 256-byte aligned");
    MDX_CHECK(a.N >= int64_t(PK_WG) * PK_T && a.N < (int64_t(1) << 31), "N must be in [8192, 2^31)");
    const int64_t seg = (a.N + PK_WG - 1) / PK_WG;
    MDX_CHECK(seg <= int64_t(PK_T) * PK_E && a.N - seg * (PK_WG - 1) >= PK_T, "N too large for the segment size (at most %d)",
              PK_WG * PK_T * PK_E);
    MDX_CHECK(a.nout >= 1 && a.nout <= PK_MAXN, "1 <= nout <= 8");
    MDX_CHECK(nch >= 1 && nch <= PK_MAXCH && nch <= a.nout, "1 <= children <= min(8, nout)");
    for (int64_t j = 0; j < nch; ++j) MDX_CHECK(children[j] >= 0 && children[j] < nvtok, "child row out of range");
    a.seg = int(seg);
    a.nch = int(nch);
    for (int j = 0; j < PK_MAXCH; ++j) a.ch[j] = j < nch ? int(children[j]) : 0;
    uint64_t* base = static_cast<uint64_t*>(ws);
    a.lists = base;
    a.amax = base + PK_WG * PK_MAXN;
    a.counter = reinterpret_cast<unsigned*>(base + PK_WG * PK_MAXN + PK_WG);
    size_t lds = 0;
    if (a.mode == PICK_BF16)
        lds = (a.layout == MDX_LAYOUT_ROW && a.K % 512 == 0 ? size_t(16) * (2 * a.K + 16) : size_t(a.K / 32) * 64 * 16) +
              size_t(a.K) * 2;
    if (a.mode == PICK_I8) lds = size_t(a.S + 1) * std::min(a.K, PK_KB);
    if (lds > 64 * 1024) allow_smem(reinterpret_cast<const void*>(&draft_pick_kernel), lds);
    hipLaunchKernelGGL(draft_pick_kernel, dim3(PK_WG), dim3(PK_T), lds, st, a);
    MDX_LAUNCHED();
    return MDX_OK;
}

}  // namespace
}  // namespace mdx

using namespace mdx;

extern "C" size_t mdx_draft_pick_workspace(void) { return pick_ws_bytes(); }

extern "C" int mdx_draft_pick(const uint16_t* approx, int64_t N, const int8_t* qx, const float* x_scale,
                              const int8_t* w, const float* w_scale, int64_t K, int64_t nout, int32_t argmax_first,
                              int64_t* top, int64_t* ranks_row, int64_t* token, int64_t* vtok, int64_t nvtok,
                              const int64_t* children, int64_t nchildren, int64_t* calls, void* workspace,
                              size_t workspace_bytes, void* stream) {
    PickArgs a{};
    a.approx = approx;
    a.N = N;
    a.mode = w ? PICK_I8 : PICK_EXACT;
    a.S = PK_MAXS;
    if (w) {
        MDX_CHECK(qx && x_scale && w_scale, "int8 head: qx, x_scale and w_scale");
        MDX_CHECK(K >= 64 && K % 64 == 0 && K <= 16384, "K must be a multiple of 64 in 64..16384");
        MDX_CHECK(aligned(w, 16) && aligned(qx, 16), "16-byte aligned w / qx");
    }
    a.qx = qx;
    a.sx = x_scale;
    a.w8 = w;
    a.sw = w_scale;
    a.K = int(K);
    a.nout = int(nout);
    a.argmax_first = argmax_first ? 1 : 0;
    a.top = top;
    a.ranks_row = ranks_row;
    a.token = token;
    a.vtok = vtok;
    a.calls = calls;
    return launch_pick(a, children, nchildren, nvtok, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int mdx_draft_pick_bf16(const uint16_t* approx, const uint16_t* x, const uint16_t* w, int32_t layout, int64_t N,
                                   int64_t K, int64_t nout, int32_t argmax_first, int64_t* top, uint16_t* top_values,
                                   int64_t* token, int64_t* vtok, int64_t nvtok, const int64_t* children, int64_t nchildren,
                                   int64_t* calls, void* workspace, size_t workspace_bytes, void* stream) {
    MDX_CHECK(x && w, "null pointer");
    MDX_CHECK(layout == MDX_LAYOUT_ROW || layout == MDX_LAYOUT_TILE, "layout");
    MDX_CHECK(K >= 32 && K % 32 == 0 && K <= 4096, "K must be a multiple of 32 in 32..4096 (the rows in LDS)");
    MDX_CHECK(N % 16 == 0, "N % 16 == 0");
    MDX_CHECK(aligned(x, 16) && aligned(w, 16), "16-byte aligned x / w");
    PickArgs a{};
    a.approx = approx;
    a.N = N;
    a.mode = PICK_BF16;
    a.S = 16;
    a.xb = x;
    a.wb = w;
    a.layout = layout;
    a.K = int(K);
    // the K split of mdx_bf16_linear for this shape (its chain is replayed slice by slice)
    const int tiles = int(N / 16), NC = int(K / 32);
    int KS = 1;
    for (int d = 1; d <= 16; ++d)
        if (NC % d == 0) {
            KS = d;
            if (int64_t(tiles) * d >= 3072) break;
        }
    a.KS = KS;
    a.nout = int(nout);
    a.argmax_first = argmax_first ? 1 : 0;
    a.top = top;
    a.top_vals = top_values;
    a.token = token;
    a.vtok = vtok;
    a.calls = calls;
    return launch_pick(a, children, nchildren, nvtok, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}
