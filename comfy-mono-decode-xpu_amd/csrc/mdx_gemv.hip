// W4A8 decode GEMV engine, row activation prep (norm / rotate / quantise) and the fused MLP.
//
// Reference semantics (comfy-mono-decode-xpu):
//   w4a8_decode_linear  csrc/w4a8_decode.sycl:4-11, 33-45, 139-166
//   rot_quant           csrc/act_prep.sycl:4-10, 70-91
//   mono_mlp            csrc/mono_mlp.sycl:109-167
//
// Scales are always the row-major [N, K/G] array (both layouts); a work-group stages its tiles'
// scale rows in LDS once (at one row with caller-asserted integral G128 scales, each wave stages its
// own tile's groups of its own slice, and its own activation run, and waits for no other wave). Weight stream: a wave owns one 16-column tile and a K slice; its unit of
// work is a "chunk", 16 columns x 128 k = 1 KiB of codes, fetched with ONE 16-byte load per lane
// (lane l: column l % 16, quarter kq = l / 16 of the chunk, 32 consecutive k). In the tile-major
// layout the 64 lanes' pieces are adjacent, so every chunk is one contiguous 1 KiB burst, and each
// code dword holds k 0..3 in its low nibbles and k 4..7 in its high ones (natural activation
// order); in the checkpoint (row-major) layout the pieces are 16 runs of 64 B and a dword's low /
// high nibbles are its even / odd k (two byte permutes put them in natural order). All per-chunk
// address math is 32-bit pointer increments; group indices are shifts (G is a power of two).
//
// Activation. The int8 rows of the unit's K range are staged in LDS (natural order) by DMA, or
// quantised there in the prologue from bf16 rows (Src).
//
// Decode. Per-weight form: a 16-entry int8 table per (lane, scale) is built with the reference
// formula w8 = clamp(rint(cb[c] * s), +-127) (NaN -> 0), and codes are mapped through it with
// v_perm_b32 byte selects. Integral form, taken by a unit under MDX_DECODE_AUTO when the codebook
// is c - 8 and every staged scale is an integer in [-15, 15] (checked in the prologue), and under
// MDX_DECODE_INTEGRAL (asserted by the caller, no check): then w8 = (c - 8) * s exactly; the
// codes become the int8 bytes 16 (c - 8), whose products give 16 sum_k x (c - 8) exactly, and an
// arithmetic shift by 4 and the scale finish each group. Both forms give the same int32
// accumulator (mod 2^32) as the reference.
//
// Products. One row: v_dot4_i32_i8 on the VALU. Rows 2..16: v_mfma_i32_16x16x32_i8 with the
// activation rows as A (rows past the last read zeros) and the decoded tile as B; lane l's dword j
// of codes is exactly its B fragment for the j-th MFMA of the chunk.
//
// Split-K partial sums of the waves of a work-group are int32 and are added through LDS:
// integer addition is associative, so every split gives the same bits.
#include <algorithm>
#include <stdio.h>
#include <vector>
#include <stdlib.h>

#include "mdx_common.hpp"
#include "mdx_gdn_ops.hpp"
#include "mdx_row.hpp"

namespace mdx {
namespace {

constexpr int WAVE = 64;
constexpr int CHUNK_K = 128;
constexpr int MAX_PREP_K = 16384;

typedef int v4i __attribute__((ext_vector_type(4)));

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

// global-memory pointers as such (accesses through generic pointers are "flat" ones, which also
// wait for outstanding LDS traffic)
#define MDX_G __attribute__((address_space(1)))

// streamed-once weights: a non-temporal 16-byte load (does not displace reused data in L2)
__device__ __forceinline__ uint4 ldg_stream(const void* p) {
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint4 ldg_stream(const MDX_G uint8_t* p) {
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const MDX_G v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// =================================================================================================
// Row prep: [sigmoid gate] -> [RMSNorm] -> [rotation] -> absmax -> int8 quantisation, one
// work-group per row (layout below, at the kernel).
// =================================================================================================
struct PrepArgs {
    const uint16_t* x;     // bf16 [rows, K]
    const uint16_t* nw;    // RMSNorm weight bf16 [K] or null (no norm)
    float eps;
    uint16_t* xn_out;      // bf16 [rows, K] normalised row (optional)
    const uint16_t* h;     // bf16 [256, 256] for MDX_ROT_MATRIX
    int rot;
    int8_t* q;             // int8 [rows, K]
    float* scale;          // f32 [rows]
    int K;
    // optional sigmoid gate: x[i] <- bf16(x[i] * sig[gate[row * g_row + (i / g_head) * g_hstride + g_off +
    // i % g_head]]) before the rotation (the gated attention output of layer_post)
    const uint16_t* gate = nullptr;
    const uint16_t* sig = nullptr;
    int64_t g_row = 0;
    int g_head = 0, g_hstride = 0, g_off = 0;
    // optional gated RMSNorm per 128-element head (the Gated-DeltaNet output): x <- bf16(bf16(x * hw *
    // rsqrt(mean_head(x^2) + heps)) * bf16(silu(hz))), hw bf16 [128] shared by the heads, hz bf16 [rows, K]
    const uint16_t* hw = nullptr;
    const uint16_t* hz = nullptr;
    float heps = 0.f;
    int hz_gated = 0;  // hz holds the gate factors gnorm_gate(z) instead of z
};

// Row prep. One work-group per row, one wave per 256-element group (wave w takes groups w, w + W, ...,
// W = min(16, K / 256)); lane l holds elements 4 l .. 4 l + 3 of each of its groups in registers.
// Canonical RMSNorm sum: per group, lane partial ((sq0 + sq1) + sq2) + sq3 of its four squares, the
// halving tree over the 64 lanes (l + 32, + 16, ..., + 1), then the group sums added in group order.
// The work-group's waves (any count) share the row; gsum holds K / 256 floats, wmax one per wave.
template <int GPW>
__device__ __forceinline__ void prep_row(const PrepArgs& a, const int row, float* gsum, float* wmax) {
    const int W = blockDim.x / WAVE, w = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    const int K = a.K, G = K / 256;
    const uint16_t* x = a.x + int64_t(row) * K + 4 * lane;
    float v[GPW][4];
    uint2 raw[GPW], wraw[GPW], graw[GPW];
    // all loads first (group index clamped: no branches around loads)
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) {
        const int g = min(w + W * gi, G - 1);
        raw[gi] = *reinterpret_cast<const uint2*>(x + 256 * g);
        if (a.nw) wraw[gi] = *reinterpret_cast<const uint2*>(a.nw + 256 * g + 4 * lane);
        if (a.gate) {
            const int i0 = 256 * g + 4 * lane;
            graw[gi] = *reinterpret_cast<const uint2*>(a.gate + row * a.g_row + (i0 / a.g_head) * a.g_hstride + a.g_off +
                                                       i0 % a.g_head);
        }
        if (a.hw) graw[gi] = *reinterpret_cast<const uint2*>(a.hz + int64_t(row) * K + 256 * g + 4 * lane);
    }
    uint2 hwraw = make_uint2(0u, 0u);
    if (a.hw) hwraw = *reinterpret_cast<const uint2*>(a.hw + 4 * (lane & 31));
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) unpack4(raw[gi], v[gi]);
    if (a.gate) {
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
            const uint16_t gb[4] = {uint16_t(graw[gi].x), uint16_t(graw[gi].x >> 16), uint16_t(graw[gi].y),
                                    uint16_t(graw[gi].y >> 16)};
#pragma unroll
            for (int e = 0; e < 4; ++e) v[gi][e] = bfround(__fmul_rn(v[gi][e], bf2f(a.sig[gb[e]])));
        }
    }
    if (a.hw) {
        // lanes 0..31 hold head 2 g of group g, lanes 32..63 head 2 g + 1: lane partial ((sq0 + sq1) + sq2)
        // + sq3, a halving tree within each half (l + 16, ..., + 1), read back from lane 0 / 32
        float hwf[4];
        unpack4(hwraw, hwf);
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
            float zf[4];
            unpack4(graw[gi], zf);
            if (a.hz_gated) gnorm_pair_g(v[gi], hwf, zf, a.heps, lane);
            else gnorm_pair(v[gi], hwf, zf, a.heps, lane);
        }
    }
    if (a.nw) {
        const float r = row_rms_factor<GPW>(v, K, a.eps, gsum);
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
            float wv[4];
            unpack4(wraw[gi], wv);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[gi][e] = bfround(__fmul_rn(__fmul_rn(v[gi][e], r), wv[e]));
        }
    }
    if (a.xn_out) {
        // the normalised row (may be x itself: every lane has read its elements above)
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
            const int g = w + W * gi;
            if (g < G) *reinterpret_cast<uint2*>(a.xn_out + int64_t(row) * K + 256 * g + 4 * lane) = pack4(v[gi]);
        }
    }
    if (!a.q) return;  // RMSNorm only (xn_out)
    if (a.rot == MDX_ROT_H256) {
        // fp64 FWHT, then * 1/16, rounded once to fp32 and once to bf16
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
            double d[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) d[e] = double(v[gi][e]);
            fwht256_lane(d, lane);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[gi][e] = bfround(float(__dmul_rn(d[e], 0.0625)));
        }
    } else if (a.rot == MDX_ROT_MATRIX) {
        // generic bf16 [256, 256] matrix: out_j = fp64 sum over k (in order, from 0.0) of the exact
        // products x_k * h[k][j], then fp32, then bf16
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
            double acc[4] = {0.0, 0.0, 0.0, 0.0};
            for (int k4 = 0; k4 < 64; ++k4) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float xk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[gi][e]), k4));
                    float hv[4];
                    unpack4(*reinterpret_cast<const uint2*>(a.h + (4 * k4 + e) * 256 + 4 * lane), hv);
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc[j] = __dadd_rn(acc[j], __dmul_rn(double(xk), double(hv[j])));
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) v[gi][j] = bfround(float(acc[j]));
        }
    }
    // absmax (exact, order-free), scale, quantise
    float m = 0.f;
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi)
        if (w + W * gi < G)
#pragma unroll
            for (int e = 0; e < 4; ++e) m = fmaxf(m, fabsf(v[gi][e]));
    m = wave_max_nn(m);
    if (lane == 0) wmax[w] = m;
    __syncthreads();
    const float rm = wave_max_nn(lane < W ? wmax[lane] : 0.f);
    const float s = fmaxf(__fdiv_rn(rm, 127.0f), 1e-30f);
    if (threadIdx.x == 0) a.scale[row] = s;
    // quant_rcp: the code of v is rint(bf16(v / sb)), the quotient rounded to fp32, then bf16. It is
    // computed as bf16(v * r) with r = fl32(1 / sb): for bf16 v and sb (8-bit significands m_v, m_s)
    // the exact quotient is never a tie of the bf16 rounding (a tie has a 9-bit odd significand, which
    // m_v / m_s cannot produce) and lies at least 1 / (255 * 511) > 2^-17 (relative) from every tie,
    // while the two fp32 roundings of v * r move it by less than 2^-23; r is finite for every sb >=
    // 2^-126, and quotients below the fp32 normal range quantise to 0 either way. (Checked over every
    // bf16 v against 3,256 scales.)
    const float rr = quant_rcp(s);
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) {
        const int g = w + W * gi;
        if (g < G) {
            uint32_t* qp = reinterpret_cast<uint32_t*>(a.q + int64_t(row) * K + 256 * g + 4 * lane);
            *qp = quant4(v[gi], rr);
        }
    }
}

template <int GPW>
__global__ __launch_bounds__(1024) void prep_rows_kernel(PrepArgs a) {
    __shared__ float gsum[MAX_PREP_K / 256];
    __shared__ float wmax[16];
    prep_row<GPW>(a, blockIdx.x, gsum, wmax);
}

int launch_prep(const PrepArgs& a, int64_t rows, hipStream_t st) {
    // waves per row (MDX_PREP_WAVES overrides for sweeps; the result does not depend on it: the norm adds
    // the group sums in group order and the maximum is order-free)
    static const int pw = [] {
        const char* e = getenv("MDX_PREP_WAVES");
        return e ? std::max(1, std::min(16, atoi(e))) : 16;
    }();
    const int G = a.K / 256, W = std::min(G, std::max(pw, (G + 3) / 4)), gpw = (G + W - 1) / W;
    MDX_CHECK(gpw <= 4, "row prep: %d groups over %d waves exceeds 4 per wave", G, W);
    const dim3 grid{unsigned(rows)}, block{unsigned(W * WAVE)};
    switch (gpw) {
        case 1: hipLaunchKernelGGL(prep_rows_kernel<1>, grid, block, 0, st, a); break;
        case 2: hipLaunchKernelGGL(prep_rows_kernel<2>, grid, block, 0, st, a); break;
        case 3: hipLaunchKernelGGL(prep_rows_kernel<3>, grid, block, 0, st, a); break;
        default: hipLaunchKernelGGL(prep_rows_kernel<4>, grid, block, 0, st, a); break;
    }
    MDX_LAUNCHED();
    return MDX_OK;
}

// =================================================================================================
// GEMV engine
// =================================================================================================
enum Epi : int { EPI_STORE = 0, EPI_SILU = 1 };

struct MatArg {
    const uint8_t* q;
    const uint8_t* s;
    const float* sch;
    int n;
    int tiles;
};

// A Gated-DeltaNet projection launch (matrices qkv, z): the tiles of matrix 0 run the deferred causal conv
// of their 16 channels in the epilogue, and `nside` work-groups after the GEMV's `units` compute the step's
// gates (buffers as in mdx_gdn.hip).
struct GdnFold {
    int on;
    const uint16_t* conv_w;  // [C, 4]
    uint16_t* conv_state;    // [C, 3]
    uint16_t* pb;            // [2][slots][C]
    uint16_t* qb;            // [2][slots][C]
    const int32_t* ctl;      // [2 + 3 slots]
    const uint16_t* xn;      // [rows, K]
    const uint16_t* wa;      // [HV, K]
    const uint16_t* wb;      // [HV, K]
    const float* dt_bias;    // [HV]
    const float* g_decay;    // [HV]
    float* gates;            // [2][slots][HV][2]
    uint16_t* zg;            // [rows, HV * 128] or null: the gate factors gnorm_gate(z) of the z outputs
    int HV, slots, units, nside;
};

struct GemvArgs {
    MatArg m[3];
    int nm;
    int pair;             // gate/up interleaved tile list (nm == 2)
    int K;
    int lgG;              // log2(group size)
    int layout;
    const float* cb;      // codebook or null (code - 8)
    const int8_t* xq;     // int8 [rows, K]
    const float* xs;      // f32 [rows]
    int rows;
    int KS, TPW;          // K slices per tile, tiles per work-group
    int force_exact;      // MDX_DECODE_EXACT: never take the integral form
    int assume_int;       // MDX_DECODE_INTEGRAL (every matrix): the integral form without the check
    int pwo;              // per-wave one-shots (one int8 row, G128, assume_int): no work-group barrier
    int tbl;              // per-weight decode tables built once per work-group into LDS: 1 16-byte, 2 8-byte (gemv_table_bytes)
    int red_alias;        // table-only variants with int8 rows: the split-K partials reuse the table region after the loop
    int epi;
    void* out[3];
    const void* res[3];
    int out_dt;
    const uint16_t* lut;  // EPI_SILU
    // EPI_SILU with hmax_out: each gate/up pair (tile) also stores its rows' |h| maxima (fp32 bits) at
    // hmax_out[row * (number of pairs) + pair]
    uint32_t* hmax_out;
    // SRC_HR units: the activation is hr (bf16 [rows, K]) quantised in the prologue with the row
    // scale max(absmax / 127, 1e-30), absmax = the maximum of hmax[row * hmax_n + w] over w < hmax_n
    const uint16_t* hr;
    const uint32_t* hmax;
    int hmax_n;
    // SRC_XP units (one row): the activation is the bf16 row xp_x, RMSNorm'd with xp_nw / xp_eps
    // (xp_nw may be null) and quantised (no rotation) in the prologue: the row prep's arithmetic in
    // its order
    const uint16_t* xp_x;
    const uint16_t* xp_nw;
    float xp_eps;
    // SRC_GN units (one or two rows): the activation is the gated RMSNorm per 128-element head of gn_y
    // (weight gn_w, gate input gn_z; gnorm_pair) quantised in the prologue (no rotation); work-group 0
    // also stores the normalised rows in gn_out (optional, not aliasing gn_y)
    const uint16_t* gn_y;
    const uint16_t* gn_z;
    const uint16_t* gn_w;
    float gn_eps;
    uint16_t* gn_out;
    int gn_gated;  // gn_z holds the gate factors gnorm_gate(z)
    GdnFold gf;
};

// Where a unit's activation comes from: int8 rows a.xq (DMA to LDS), bf16 rows quantised with
// given maxima (SRC_HR), one bf16 row prepared from scratch (SRC_XP), or one or two rows of a
// Gated-DeltaNet's raw outputs gated-normed and quantised (SRC_GN).
enum Src : int { SRC_Q8 = 0, SRC_HR = 1, SRC_XP = 2, SRC_GN = 3 };
constexpr int GN_PASSES = 4;  // SRC_GN: head rows per lane (rows x K / 128 <= 8 x waves)
// Added to a source: the kernel variant with the integral decode only (scales asserted integral, the
// default codebook, groups the integral form takes). Without the per-weight decode's code the
// integral path keeps its registers and schedule (the 1-row MLP 24.6 -> 23.x us).
constexpr int SRC_INT_ONLY = 4;
// Added to a source (MFMA kernels only): the per-weight table decode only, for groups of at least one
// chunk with their (tile row, group) tables in LDS: 16-byte tables (SRC_TBL) or the default codebook's
// eight magnitudes (SRC_TBL8). No per-launch scale check and no scale reads in the loop; the tables ride
// a ring beside the weights at scalar offsets.
constexpr int SRC_TBL = 8;
constexpr int SRC_TBL8 = 16;
// Added to an int8-row source: a Gated-DeltaNet projection launch (GdnFold), its conv epilogue and gate
// work-groups compiled into these variants only (the gate rows' loads would raise every other variant's
// registers).
constexpr int SRC_GDN = 32;
constexpr int XP_GPW = 4;
constexpr int HMW = 16;  // SRC_HR: maxima per lane when every wave reads them all (<= 1024 work-groups)  // SRC_XP: 256-groups per wave (K <= 1024 x waves)

struct Lut {
    uint32_t w[4];
};

__device__ __forceinline__ Lut make_lut(float s, const float* cb) {
    Lut L;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        uint32_t v = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const float r = rintf(__fmul_rn(cb[d * 4 + b], s));
            const int q = (r != r) ? 0 : int(fminf(fmaxf(r, -127.f), 127.f));
            v |= (uint32_t(q) & 0xFFu) << (8 * b);
        }
        L.w[d] = v;
    }
    return L;
}

// The table of the default codebook (c - 8) from its eight magnitudes: rint and the clamp are odd
// functions and (-k) s = -(k s) exactly, so entry 8 - k is the negation of q(k s) = clamp(rint(k s),
// +-127) (NaN -> 0) and entry 8 is 0 (0 * s rounds to 0, or is NaN -> 0): eight products instead of
// sixteen, the same bytes as make_lut.
__device__ __forceinline__ Lut make_lut_c8(float s) {
    int q[9];
    q[0] = 0;
#pragma unroll
    for (int k = 1; k <= 8; ++k) {
        const float r = rintf(__fmul_rn(float(k), s));
        q[k] = (r != r) ? 0 : int(fminf(fmaxf(r, -127.f), 127.f));
    }
    auto pk = [](int b0, int b1, int b2, int b3) {
        return (uint32_t(b0) & 0xFFu) | ((uint32_t(b1) & 0xFFu) << 8) | ((uint32_t(b2) & 0xFFu) << 16) | (uint32_t(b3) << 24);
    };
    Lut L;
    L.w[0] = pk(-q[8], -q[7], -q[6], -q[5]);
    L.w[1] = pk(-q[4], -q[3], -q[2], -q[1]);
    L.w[2] = pk(0, q[1], q[2], q[3]);
    L.w[3] = pk(q[4], q[5], q[6], q[7]);
    return L;
}

// The eight magnitudes q(k s), k = 1..8, of the default codebook's table as int8 bytes (q1..q4, q5..q8).
__device__ __forceinline__ uint2 make_q8(float s) {
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int k = 1; k <= 8; ++k) {
        const float r = rintf(__fmul_rn(float(k), s));
        const int q = (r != r) ? 0 : int(fminf(fmaxf(r, -127.f), 127.f));
        w[(k - 1) >> 2] |= (uint32_t(q) & 0xFFu) << (8 * ((k - 1) & 3));
    }
    return make_uint2(w[0], w[1]);
}

// make_q8 for an fp16 scale |s| <= 127 / 8 (bits & 0x7FFF <= 0x4BF0; every fp16-ratio GPTQ scale): four packed
// half-precision FMAs k s + 1536 (k = 1..8). Each forms k s exactly and rounds once; in [1024, 2048) the
// spacing of half precision is 1, so the result is 1536 + rint(k s) (ties to even, 1536 being even), and
// its low byte is rint(k s) as int8. |k s| <= 127: no clamp. Two byte permutes gather the eight bytes.
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
constexpr uint32_t F16_FAST_MAX = 0x4BF0u;  // fp16 15.875

__device__ __forceinline__ uint2 make_q8_f16(uint32_t sbits) {
    const half2_t s2 = __builtin_bit_cast(half2_t, sbits | (sbits << 16));
    const half2_t magic = {(_Float16)1536.0f, (_Float16)1536.0f};
    uint32_t r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const half2_t kk = {(_Float16)float(2 * i + 1), (_Float16)float(2 * i + 2)};
        r[i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(kk, s2, magic));
    }
    return make_uint2(__builtin_amdgcn_perm(r[1], r[0], 0x06040200u), __builtin_amdgcn_perm(r[3], r[2], 0x06040200u));
}

// The default codebook's 16-byte table from its magnitudes (make_lut_c8's bytes): byte reversal and
// a carry-free negation of four int8 at once (~b + 1 per byte; no byte is -128 after the clamp).
__device__ __forceinline__ Lut lut_from_q8(uint32_t qa, uint32_t qb) {
    auto neg4 = [](uint32_t b) {
        const uint32_t n = ~b;
        return ((n & 0x7F7F7F7Fu) + 0x01010101u) ^ (n & 0x80808080u);
    };
    Lut L;
    L.w[0] = neg4(__builtin_amdgcn_perm(0u, qb, 0x00010203u));  // -q8, -q7, -q6, -q5
    L.w[1] = neg4(__builtin_amdgcn_perm(0u, qa, 0x00010203u));  // -q4 .. -q1
    L.w[2] = __builtin_amdgcn_perm(0u, qa, 0x0201000Cu);        // 0, q1, q2, q3
    L.w[3] = __builtin_amdgcn_perm(qb, qa, 0x06050403u);        // q4 .. q7
    return L;
}

// four codes (one per byte, values 0..15) -> four int8 via the 16-byte table
__device__ __forceinline__ uint32_t lut4(const Lut& L, uint32_t c) {
    const uint32_t sel = c & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(L.w[1], L.w[0], sel);
    const uint32_t hi = __builtin_amdgcn_perm(L.w[3], L.w[2], sel);
    const uint32_t pick = ((c >> 1) & 0x04040404u) | 0x03020100u;
    return __builtin_amdgcn_perm(hi, lo, pick);
}

// per-weight decode of one chunk's four code dwords (two scales: dwords 0-1 and 2-3; one when the
// group spans the lane's 32 k, `one`, uniform); cbdef (uniform): the default codebook c - 8
__device__ __forceinline__ void decode_exact(const uint32_t* wd, float s0, float s1, bool one, bool cbdef,
                                             const float* cb, uint32_t* lo, uint32_t* hi) {
    const Lut L0 = cbdef ? make_lut_c8(s0) : make_lut(s0, cb);
    Lut L1 = L0;
    if (!one) L1 = (__float_as_uint(s1) == __float_as_uint(s0)) ? L0 : (cbdef ? make_lut_c8(s1) : make_lut(s1, cb));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const Lut& L = j < 2 ? L0 : L1;
        lo[j] = lut4(L, wd[j] & 0x0F0F0F0Fu);
        hi[j] = lut4(L, (wd[j] >> 4) & 0x0F0F0F0Fu);
    }
}

// per-weight decode of one chunk's four code dwords through one table (a group spans the chunk)
// (q8: T holds the default codebook's eight magnitudes in .x, .y)
__device__ __forceinline__ void decode_tbl(const uint32_t* wd, const uint4 T, bool q8, uint32_t* lo, uint32_t* hi) {
    Lut L;
    if (q8) {
        L = lut_from_q8(T.x, T.y);
    } else {
        L.w[0] = T.x;
        L.w[1] = T.y;
        L.w[2] = T.z;
        L.w[3] = T.w;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        lo[j] = lut4(L, wd[j] & 0x0F0F0F0Fu);
        hi[j] = lut4(L, (wd[j] >> 4) & 0x0F0F0F0Fu);
    }
}

// The table-only decode of one chunk's four code dwords (tile-major nibble order: k 8j..8j+3 in the low
// nibbles of dword j, k 8j+4..8j+7 in the high ones). Per four codes: the byte selectors (c & 7) index
// both 8-byte halves of the table by v_perm_b32, and a third v_perm_b32 picks per byte by bit 3 of the
// code (selector i or 4 + i, built by one bitop3 from the shifted codes): 13 VALU per code dword.
// Q8: T.x, T.y hold the default codebook's eight magnitudes (expanded once per chunk).
template <bool Q8>
__device__ __forceinline__ void decode_tb(const uint4 w, const uint4 T, uint32_t* lo, uint32_t* hi) {
    Lut L;
    if (Q8) {
        L = lut_from_q8(T.x, T.y);
    } else {
        L.w[0] = T.x;
        L.w[1] = T.y;
        L.w[2] = T.z;
        L.w[3] = T.w;
    }
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    const uint32_t m4 = 0x04040404u, id = 0x03020100u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t v = wd[j];
        const uint32_t sl = v & 0x07070707u, sh = (v >> 4) & 0x07070707u;
        // (a & b) | c: bitop3 truth table 0xEA (index 4 a + 2 b + c)
        const uint32_t pl = __builtin_amdgcn_bitop3_b32(v >> 1, m4, id, 0xEA);
        const uint32_t ph = __builtin_amdgcn_bitop3_b32(v >> 5, m4, id, 0xEA);
        lo[j] = __builtin_amdgcn_perm(__builtin_amdgcn_perm(L.w[3], L.w[2], sl), __builtin_amdgcn_perm(L.w[1], L.w[0], sl), pl);
        hi[j] = __builtin_amdgcn_perm(__builtin_amdgcn_perm(L.w[3], L.w[2], sh), __builtin_amdgcn_perm(L.w[1], L.w[0], sh), ph);
    }
}

// global tile -> (matrix, local tile)
__device__ __forceinline__ int which_mat(const GemvArgs& a, int g, int& tile) {
    if (a.pair) { tile = g >> 1; return g & 1; }
    if (a.nm < 2 || g < a.m[0].tiles) { tile = g; return 0; }
    if (a.nm < 3 || g < a.m[0].tiles + a.m[1].tiles) { tile = g - a.m[0].tiles; return 1; }
    tile = g - a.m[0].tiles - a.m[1].tiles;
    return 2;
}

template <int SDT>
__device__ __forceinline__ float rd_scale(const uint8_t* p) {
    if (SDT == MDX_DT_F32) return *reinterpret_cast<const float*>(p);
    if (SDT == MDX_DT_F16) return fp16_to_f32(*reinterpret_cast<const uint16_t*>(p));
    return fp8_to_f32(*p);
}

// -------------------------------------------------------------------------------------------------
// epilogue
// -------------------------------------------------------------------------------------------------
// Per-matrix fields for a run-time matrix index. The three values are loaded at fixed offsets and
// passed through an empty asm before the select: otherwise the compiler folds the select of loads
// into one load at a run-time offset, which needs an addressable copy of the whole argument struct
// (scratch memory, a round trip before every use).
template <typename T>
__device__ __forceinline__ T opaque(T v) {
    asm volatile("" : "+s"(v));
    return v;
}
template <typename T>
__device__ __forceinline__ T pick3(int i, T v0, T v1, T v2) {
    v0 = opaque(v0);
    v1 = opaque(v1);
    v2 = opaque(v2);
    return i == 0 ? v0 : (i == 1 ? v1 : v2);
}
// a pointer into global memory again (the asm hid where it came from)
template <typename T>
__device__ __forceinline__ MDX_G T* as_global(T* p) {
    return (MDX_G T*)p;
}
__device__ __forceinline__ int mat_n(const GemvArgs& a, int mi) { return pick3(mi, a.m[0].n, a.m[1].n, a.m[2].n); }
__device__ __forceinline__ int mat_tiles(const GemvArgs& a, int mi) {
    return pick3(mi, a.m[0].tiles, a.m[1].tiles, a.m[2].tiles);
}
__device__ __forceinline__ MDX_G void* mat_out(const GemvArgs& a, int mi) {
    return as_global(pick3(mi, a.out[0], a.out[1], a.out[2]));
}
__device__ __forceinline__ const MDX_G void* mat_res(const GemvArgs& a, int mi) {
    return as_global(pick3(mi, a.res[0], a.res[1], a.res[2]));
}
__device__ __forceinline__ const MDX_G uint8_t* mat_q(const GemvArgs& a, int mi) {
    return as_global(pick3(mi, a.m[0].q, a.m[1].q, a.m[2].q));
}
__device__ __forceinline__ const MDX_G uint8_t* mat_s(const GemvArgs& a, int mi) {
    return as_global(pick3(mi, a.m[0].s, a.m[1].s, a.m[2].s));
}
__device__ __forceinline__ const MDX_G float* mat_sch(const GemvArgs& a, int mi) {
    return as_global(pick3(mi, a.m[0].sch, a.m[1].sch, a.m[2].sch));
}

__device__ __forceinline__ void store_out(const GemvArgs& a, int mi, int n, int r, int32_t acc, float xs, float sc) {
    const float f = scaleback(acc, xs, sc);
    const int o = r * mat_n(a, mi) + n;
    const MDX_G void* res = mat_res(a, mi);
    MDX_G void* out = mat_out(a, mi);
    if (a.out_dt == MDX_DT_BF16) {
        uint16_t v = f2bf(f);
        if (res) v = f2bf(__fadd_rn(bf2f(static_cast<const MDX_G uint16_t*>(res)[o]), bf2f(v)));
        static_cast<MDX_G uint16_t*>(out)[o] = v;
    } else {
        float v = f;
        if (res) v = __fadd_rn(static_cast<const MDX_G float*>(res)[o], v);
        static_cast<MDX_G float*>(out)[o] = v;
    }
}

__device__ __forceinline__ uint16_t silu_h(const GemvArgs& a, int32_t ag, int32_t au, float xs, float scg, float scu) {
    const uint16_t g = f2bf(scaleback(ag, xs, scg));
    const uint16_t u = f2bf(scaleback(au, xs, scu));
    const float act = bf2f(a.lut[g]);
    return f2bf(__fmul_rn(act, bf2f(u)));
}

// red layout: [TPW][KS][16 columns][rows] (VALU) or [TPW][KS][64 lanes][4] (MFMA); sums the slices
template <bool MFMA>
__device__ __forceinline__ int32_t reduced(const GemvArgs& a, const int32_t* red, int ts, int r, int c) {
    // the slices' partials four at a time (reads clamped to the last slice, masked; int32 sums are
    // associative, so any order gives the same bits): one LDS round trip per four slices
    uint32_t s = 0;
    for (int k0 = 0; k0 < a.KS; k0 += 4) {
        uint32_t v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = min(k0 + j, a.KS - 1);
            v[j] = MFMA ? uint32_t(red[((ts * a.KS + k) * 64 + (r >> 2) * 16 + c) * 4 + (r & 3)])
                        : uint32_t(red[((ts * a.KS + k) * 16 + c) * a.rows + r]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) s += k0 + j < a.KS ? v[j] : 0u;
    }
    return int32_t(s);
}

template <bool MFMA>
__device__ void epilogue(const GemvArgs& a, const int wg, const int32_t* red, const float* prml) {
    const int per = 16 * a.rows;
    const float* xsl = prml + a.TPW * 16;
    if (a.epi == EPI_SILU) {
        // pairs: tile slots 2 p / 2 p + 1 hold gate / up tile wg TPW / 2 + p; a thread stores two
        // adjacent columns
        const int np = a.TPW / 2, half = per / 2;
        for (int e = threadIdx.x; e < np * half; e += blockDim.x) {
            const int p = e / half, rem = e - p * half, r = rem >> 3, c = 2 * (rem & 7);
            const int tile = wg * np + p;
            if (tile >= a.m[0].tiles) continue;
            const int sg = 2 * p, su = 2 * p + 1;
            const uint32_t v = uint32_t(silu_h(a, reduced<MFMA>(a, red, sg, r, c), reduced<MFMA>(a, red, su, r, c), xsl[r],
                                               prml[sg * 16 + c], prml[su * 16 + c])) |
                               (uint32_t(silu_h(a, reduced<MFMA>(a, red, sg, r, c + 1), reduced<MFMA>(a, red, su, r, c + 1),
                                                xsl[r], prml[sg * 16 + c + 1], prml[su * 16 + c + 1]))
                                << 16);
            uint32_t* o = reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.out[0]) + r * a.m[0].n + tile * 16 + c);
            *o = v;
            if (a.hmax_out) {
                // the row's |h| maximum over the 8 threads that hold this pair's 16 columns of the row (NaN
                // counts as 0, as in the row prep's fmaxf from 0), stored as this pair's entry
                float m = fmaxf(fabsf(bf2f(uint16_t(v))), fabsf(bf2f(uint16_t(v >> 16))));
                m = fmaxf(m, __shfl_xor(m, 1, 8));
                m = fmaxf(m, __shfl_xor(m, 2, 8));
                m = fmaxf(m, __shfl_xor(m, 4, 8));
                if ((rem & 7) == 0) a.hmax_out[r * a.m[0].tiles + tile] = __float_as_uint(m != m ? 0.f : m);
            }
        }
        return;
    }
    for (int ts = 0; ts < a.TPW; ++ts) {  // one tile slot at a time: the matrix choice stays uniform
        int tile;
        const int mi = which_mat(a, wg * a.TPW + ts, tile);
        if (tile >= mat_tiles(a, mi)) continue;
        for (int e = threadIdx.x; e < per; e += blockDim.x) {
            const int r = e >> 4, c = e & 15;
            store_out(a, mi, tile * 16 + c, r, reduced<MFMA>(a, red, ts, r, c), xsl[r], prml[ts * 16 + c]);
        }
    }
}

// The Gated-DeltaNet projection epilogue: both matrices' outputs stored (bf16, no residual), matrix 0's
// also staged in LDS (stage [TPW][rows][16], in the activation region, dead after the loop) with the
// control words (gctl: thread t's word, loaded in the prologue), then one lane per (qkv channel, row)
// runs the conv (gdn_conv_row: the rows' LDS taps and the history loads overlap, no row waits on the
// previous one). The channel's tile owns it: no other work-group reads or writes the channel's conv
// state or buffers in this launch.
template <bool MFMA>
__device__ void gdn_epilogue(const GemvArgs& a, const int wg, const int32_t* red, const float* prml, uint8_t* xl,
                             int gctl) {
    const GdnFold& g = a.gf;
    const int per = 16 * a.rows, t = threadIdx.x;
    const float* xsl = prml + a.TPW * 16;
    uint16_t* stage = reinterpret_cast<uint16_t*>(xl);
    int* sctl = reinterpret_cast<int*>(xl + ((a.TPW * per * 2 + 15) & ~15));
    for (int ts = 0; ts < a.TPW; ++ts) {  // (the matrix choice stays uniform)
        int tile;
        const int mi = which_mat(a, wg * a.TPW + ts, tile);
        if (tile >= mat_tiles(a, mi)) continue;
        uint16_t* out = static_cast<uint16_t*>(mi == 0 ? a.out[0] : a.out[1]);
        const int n = mi == 0 ? a.m[0].n : a.m[1].n;
        for (int e = t; e < per; e += blockDim.x) {
            const int r = e >> 4, c = e & 15;
            const uint16_t v = f2bf(scaleback(reduced<MFMA>(a, red, ts, r, c), xsl[r], prml[ts * 16 + c]));
            out[r * n + tile * 16 + c] = v;
            if (mi == 0) stage[(ts * a.rows + r) * 16 + c] = v;
            else if (g.zg) g.zg[r * n + tile * 16 + c] = f2bf(gnorm_gate(bf2f(v)));
        }
    }
    const int S = g.slots, R = a.rows;
    if (t < 2 + 3 * S) sctl[t] = gctl;
    __syncthreads();
    const int pending = sctl[0], p = sctl[1];
    if (!gdn_ctl_ok(pending, p, S)) return;  // (uniform)
    // one lane per (channel, row): a channel's rows on the 2^lp >= S consecutive lanes of one wave (2^lp
    // divides the wave), which gdn_conv_row needs for its state write-back
    const int lp = S <= 1 ? 0 : (S <= 2 ? 1 : (S <= 4 ? 2 : (S <= 8 ? 3 : 4)));
    for (int e = t; e < (a.TPW * 16) << lp; e += blockDim.x) {
        const int row = e & ((1 << lp) - 1), ch = e >> lp;
        const int ts = ch >> 4, c16 = ch & 15;
        int tile;
        if (row >= S || which_mat(a, wg * a.TPW + ts, tile) != 0 || tile >= a.m[0].tiles) continue;
        const uint16_t* st = stage + ts * R * 16 + c16;
        gdn_conv_row(tile * 16 + c16, a.m[0].n, row, R, S, pending, p, sctl + 2, sctl + 2 + S,
                     [&](int r) { return st[r * 16]; }, g.conv_w, g.conv_state, g.pb, g.qb);
    }
}

// The RMSNorm of a row-prep launch's one row into LDS (xnl, bf16 [K]) by a gate work-group: the row
// prep's arithmetic (row_rms_factor's order, then bf16((v r) w)), wave w taking the 256-groups w, w +
// waves, ... (K <= 1024 x waves).
__device__ void side_row_norm(const GemvArgs& a, uint16_t* xnl, float* gsum) {
    const int K = a.K, G = K / 256, W = blockDim.x / 64, w = threadIdx.x / 64, lane = threadIdx.x % 64;
    float v[XP_GPW][4];
    uint2 wr[XP_GPW];
#pragma unroll
    for (int gi = 0; gi < XP_GPW; ++gi) {
        const int g = min(w + W * gi, G - 1);
        unpack4(*reinterpret_cast<const uint2*>(a.xp_x + 256 * g + 4 * lane), v[gi]);
        wr[gi] = *reinterpret_cast<const uint2*>(a.xp_nw + 256 * g + 4 * lane);
    }
    const float r = row_rms_factor<XP_GPW>(v, K, a.xp_eps, gsum);
#pragma unroll
    for (int gi = 0; gi < XP_GPW; ++gi) {
        const int g = w + W * gi;
        if (g < G) {
            float wv[4];
            unpack4(wr[gi], wv);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[gi][e] = bfround(__fmul_rn(__fmul_rn(v[gi][e], r), wv[e]));
            *reinterpret_cast<uint2*>(xnl + 256 * g + 4 * lane) = pack4(v[gi]);
        }
    }
    __syncthreads();
}

// The gates of a Gated-DeltaNet projection launch, by side work-group b (< nside): wave w computes row ts,
// value head h of pair b * waves + w (rows < R; gdn_gate_row); rows R .. slots - 1 get zeros. A row-prep
// launch (one bf16 row, a.xp_x) has no normalised row in memory: each gate work-group computes it into
// LDS first.
__device__ void gdn_gates_side(const GemvArgs& a, int b, uint8_t* lds) {
    const GdnFold& g = a.gf;
    const int t = threadIdx.x, lane = t & 63, nw = blockDim.x >> 6, nthr = blockDim.x;
    const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
    const int R = a.rows, S = g.slots, HV = g.HV;
    const int pending = g.ctl[0], p = g.ctl[1];
    const bool ok = gdn_ctl_ok(pending, p, S);
    const uint16_t* xn = g.xn;
    if (a.xp_x) {  // (uniform)
        uint16_t* xnl = reinterpret_cast<uint16_t*>(lds);
        side_row_norm(a, xnl, reinterpret_cast<float*>(lds + 2 * a.K));
        xn = xnl;
    }
    const int pair = b * nw + wv;
    if (pair < R * HV) {
        const int ts = pair / HV, h = pair - ts * HV;
        float decay, beta;
        gdn_gate_row<2>(xn + int64_t(ts) * a.K, g.wa + int64_t(h) * a.K, g.wb + int64_t(h) * a.K, a.K, g.dt_bias[h],
                        g.g_decay[h], lane, decay, beta);
        if (lane == 0 && ok) {
            g.gates[((p * S + ts) * HV + h) * 2] = decay;
            g.gates[((p * S + ts) * HV + h) * 2 + 1] = beta;
        }
    }
    if (ok)
        for (int i = b * nthr + t; i < (S - R) * HV * 2; i += g.nside * nthr) g.gates[(p * S + R) * HV * 2 + i] = 0.f;
}

// -------------------------------------------------------------------------------------------------
// the kernel
// -------------------------------------------------------------------------------------------------
// 16 (c - 8) as int8 for the four low / high nibbles c of a code dword: c ^ 8 moved into the byte's
// high half reads, as a signed byte, as 16 (c - 8) (c < 8: c + 8 - 16; c >= 8: c - 8), without a
// borrow between bytes; products against these bytes are 16 times the integral form's
// sum x (c - 8), exactly (an arithmetic shift by 4 recovers it)
__device__ __forceinline__ uint32_t sx16_lo(uint32_t w) { return ((w << 4) & 0xF0F0F0F0u) ^ 0x80808080u; }
__device__ __forceinline__ uint32_t sx16_hi(uint32_t w) { return (w & 0xF0F0F0F0u) ^ 0x80808080u; }

// natural-order code bytes of a code dword: [c0 c1 c2 c3], [c4 c5 c6 c7] from its low / high nibbles
__device__ __forceinline__ void nat_order(uint32_t lo, uint32_t hi, uint32_t& n0, uint32_t& n1) {
    n0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
    n1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
}

#define MDX_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// Copy `rows` runs of `bytes` (a multiple of 16) spaced `stride` apart in global memory into one
// packed LDS block (row r at dst + r * bytes), 16 bytes per lane with direct-to-LDS loads (the LDS
// side of one wave instruction is 64 x 16 contiguous bytes). The caller waits and barriers.
__device__ __forceinline__ void dma_rows_to_lds(const MDX_G uint8_t* src, int stride, int bytes, int rows, uint8_t* dst,
                                                int nthr) {
    const int lane = threadIdx.x % WAVE, nw = nthr / WAVE, w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
    const int per = bytes / 16, pieces = rows * per;
    for (int i0 = w * WAVE; i0 < pieces; i0 += nw * WAVE) {
        const int i = i0 + lane;
        if (i < pieces) {
            const int r = i / per;
            __builtin_amdgcn_global_load_lds(src + size_t(r) * stride + (i - r * per) * 16, MDX_LDS(dst + i0 * 16), 16, 0, 0);
        }
    }
}

// The scale bytes a unit stages per tile row: the groups [g0, g1) that its chunk range touches when
// those are whole 16-byte runs of every row, else the whole row.
__device__ __forceinline__ void unit_groups(int cu0, int ncu, int lgG, int ng, int esz, int& g0, int& g1) {
    g0 = (cu0 * CHUNK_K) >> lgG;
    g1 = ((cu0 + ncu) * CHUNK_K + (1 << lgG) - 1) >> lgG;
    if ((ng * esz) % 16 || (g0 * esz) % 16 || ((g1 - g0) * esz) % 16) {
        g0 = 0;
        g1 = ng;
    }
}

// One work unit of the GEMV engine: work unit `wg` (TPW tiles, KS waves per tile) over the chunk
// range [cu0, cu0 + ncu) of K.
//
// Issue order matters more than anything else here. Vector memory results return in issue order
// and the wait instruction counts outstanding operations, so: first the one-shot operands (the
// activation rows and the scales, straight to LDS, and the channel scales), then the weight ring
// (RING loads in flight per wave), and only then a wait that lets the ring stay in flight. The
// main loop runs whole ring rounds without conditions around the loads (a load under a condition
// is merged at the join and waited for at once, which leaves one load in flight per wave): a chunk
// past the slice re-reads the slice's last chunk and adds nothing. Everything that selects a
// matrix or a tile is wave-uniform (scalar registers).
// SRC: where the activation comes from (Src).
template <bool MFMA, int R, int SDT, int RING, int SRC = SRC_Q8>
__device__ __forceinline__ void gemv_unit(const GemvArgs& a, const int wg, const int cu0, const int ncu, uint8_t* lds) {
    constexpr int ESZ = SDT == MDX_DT_F32 ? 4 : (SDT == MDX_DT_F16 ? 2 : 1);
    const int K = a.K;
    const int ng = K >> a.lgG;
    const int Kr = ncu * CHUNK_K;
    const int nthr = a.TPW * a.KS * WAVE;
    int g0, g1;
    unit_groups(cu0, ncu, a.lgG, ng, ESZ, g0, g1);
    const int seg = (g1 - g0) * ESZ;  // scale bytes per tile row in LDS
    // LDS: activation rows of the K range | scales [TPW][16][seg] | reduction | parameters [128] |
    // flag | 32 zero bytes (the activation of MFMA rows past the last)
    uint8_t* xl = lds;
    uint8_t* sl = xl + ((a.rows * Kr + 1023) & ~1023);
    // (table-only variants with int8 rows may keep the split-K partials in the table region, which is dead
    // after the loop: no region of their own)
    const bool ralias = (SRC & (SRC_TBL | SRC_TBL8)) != 0 && (SRC & 3) == SRC_Q8 && a.red_alias;
    int32_t* red = reinterpret_cast<int32_t*>(sl + ((a.TPW * 16 * seg + 1023) & ~1023));
    float* prml = reinterpret_cast<float*>(red + (ralias ? 0 : (MFMA ? a.TPW * a.KS * 64 * 4 : a.TPW * a.KS * 16 * a.rows)));
    int* mixed = reinterpret_cast<int*>(prml + 128);
    uint8_t* zeros = reinterpret_cast<uint8_t*>(mixed + 4);

    const int t = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(t / WAVE), lane = t % WAVE;
    const int ts = wave / a.KS, slice = wave - ts * a.KS;
    int tile;
    const int mi = which_mat(a, wg * a.TPW + ts, tile);
    const MDX_G uint8_t* mq = mat_q(a, mi);
    const int mtiles = mat_tiles(a, mi);
    const bool live = tile < mtiles;
    const int NC = K / CHUNK_K;
    const int c0 = live ? cu0 + slice * ncu / a.KS : 0, c1 = live ? cu0 + (slice + 1) * ncu / a.KS : 0;
    const int nch = c1 - c0;
    const int c = lane & 15, kq = lane >> 4;
    const int klane = 32 * kq;
    const int lgG = a.lgG;

    // 1. one-shot operands: activation rows (unless produced in this launch), tile scales, channel scales
    constexpr int SRCK = SRC & 3;
    constexpr bool IO = (SRC & SRC_INT_ONLY) != 0;  // the integral decode only
    constexpr bool HR = SRCK == SRC_HR, XP = SRCK == SRC_XP;
    constexpr bool TB = (SRC & (SRC_TBL | SRC_TBL8)) != 0;  // the table decode only
    constexpr bool TB8 = (SRC & SRC_TBL8) != 0;
    static_assert(!TB || (MFMA && !IO), "the table-only variants are MFMA kernels");
    const bool own_x = SRCK == SRC_Q8;  // int8 rows a.xq staged by this prologue
    // Per-wave one-shots (a.pwo): each wave stages only what it reads, its slice's activation run
    // (the TPW waves of a slice write the same bytes) and its tile's scales of its slice's groups
    // into a region of its own, so no wave waits for another before its loop.
    const bool pwo = a.pwo && !MFMA;  // (uniform)
    const int sbw = (ncu / a.KS) * ESZ;                               // pwo: scale bytes per tile row
    uint8_t* swv = sl + wave * 16 * sbw;                              // pwo: [16][sbw]
    if (pwo && SRCK == SRC_Q8) {
        const MDX_G uint8_t* xsrc = as_global(reinterpret_cast<const uint8_t*>(a.xq)) + c0 * CHUNK_K;
        const int xp = nch * (CHUNK_K / 16);
        for (int i0 = 0; i0 < xp; i0 += WAVE)
            if (i0 + lane < xp)
                __builtin_amdgcn_global_load_lds(xsrc + (i0 + lane) * 16, MDX_LDS(xl + (c0 - cu0) * CHUNK_K + i0 * 16), 16, 0, 0);
    }
    if (pwo) {
        const int per = sbw / 16, sp = 16 * per;
        const MDX_G uint8_t* ssrc = mat_s(a, mi) + size_t(live ? tile : 0) * 16 * ng * ESZ + c0 * ESZ;  // (G128: group = chunk)
        for (int i0 = 0; i0 < sp; i0 += WAVE)
            if (i0 + lane < sp) {
                const int i = i0 + lane, r = i / per;
                __builtin_amdgcn_global_load_lds(ssrc + size_t(r) * ng * ESZ + (i - r * per) * 16, MDX_LDS(swv + i0 * 16), 16, 0, 0);
            }
    }
    if (own_x && !pwo) dma_rows_to_lds(as_global(reinterpret_cast<const uint8_t*>(a.xq)) + cu0 * CHUNK_K, K, Kr, a.rows, xl, nthr);
    for (int tsi = 0; tsi < (pwo ? 0 : a.TPW); ++tsi) {
        int tl;
        const int mm = which_mat(a, wg * a.TPW + tsi, tl);
        const MDX_G uint8_t* sb = mat_s(a, mm);
        if (tl >= mat_tiles(a, mm)) continue;
        const MDX_G uint8_t* tb = sb + size_t(tl) * 16 * ng * ESZ;
        if (seg % 16) dma_rows_to_lds(tb, 0, 16 * seg, 1, sl + tsi * 16 * seg, nthr);  // whole block at once
        else dma_rows_to_lds(tb + g0 * ESZ, ng * ESZ, seg, 16, sl + tsi * 16 * seg, nthr);
    }
    // channel scales: slice 0 of each tile slot loads its own tile's (wave-uniform matrix choice)
    float prm = 0.f;
    if (slice == 0 && lane < 16) {
        const MDX_G float* sc = mat_sch(a, mi);
        prm = sc[(live ? tile : 0) * 16 + lane];
    } else if (own_x && wave == a.TPW * a.KS - 1 && lane >= 16 && lane < 16 + a.rows) {
        prm = a.xs[lane - 16];
    }
    // a Gated-DeltaNet projection's control words (the epilogue's conv reads them from LDS)
    constexpr bool GDN = (SRC & SRC_GDN) != 0;
    static_assert(!GDN || (SRC & 3) == SRC_Q8 || (SRC & 3) == SRC_XP, "Gated-DeltaNet projections take int8 rows or one bf16 row");
    int gctl = 0;
    if (GDN && t < 2 + 3 * a.gf.slots) gctl = a.gf.ctl[t];
    // SRC_HR: the bf16 rows (HRP 16-byte pieces per thread at most) and the maxima entries (thread t:
    // entries t, t + threads, ... of both rows) are one-shot operands too
    constexpr int HRP = HR ? 16 : 1;
    constexpr int HMV = HR ? HMW : 1;
    uint4 hraw[HRP];
    float hmx[2] = {0.f, 0.f};
    float hv[2][HMV];  // SRC_HR with every maximum per wave: this lane's maxima (reduced behind the ring)
    const int nwv = a.TPW * a.KS;
    if (HR) {
        const int total = a.rows * (Kr / 8), per_row = Kr / 8;
#pragma unroll
        for (int k = 0; k < HRP; ++k) {
            // (one or two rows: the row index is a comparison, not a division per piece)
            const int i = k * nthr + t, r = i >= per_row ? 1 : 0, j = i - r * per_row;
            hraw[k] = make_uint4(0u, 0u, 0u, 0u);
            if (i < total) hraw[k] = *reinterpret_cast<const uint4*>(a.hr + r * K + cu0 * CHUNK_K + 8 * j);
        }
        // every wave reads the maxima itself (HMW per lane in 16-byte pieces, issued at once; all of
        // them when hmax_n <= WAVE * HMW, so that the rows' maxima need no exchange between the
        // waves; hmax_n is a multiple of 4). They are reduced after the weight ring is issued, so
        // that its first round does not wait for them.
#pragma unroll
        for (int j = 0; j < HMV / 4; ++j)
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const uint4 m4 = *reinterpret_cast<const uint4*>(
                    a.hmax + min(r, a.rows - 1) * a.hmax_n + min(4 * lane + 4 * WAVE * j, a.hmax_n - 4));
                hv[r][4 * j] = __uint_as_float(m4.x);
                hv[r][4 * j + 1] = __uint_as_float(m4.y);
                hv[r][4 * j + 2] = __uint_as_float(m4.z);
                hv[r][4 * j + 3] = __uint_as_float(m4.w);
            }
    }
    // SRC_GN: lane l of wave w takes head rows 2 w + l / 32 + 2 waves p (p < GN_PASSES; head row i: row
    // i / (K / 128), head i % (K / 128)), elements 4 (l % 32) .. + 3: the raw values, the gate inputs and
    // the norm weights are one-shot operands
    constexpr bool GN = SRCK == SRC_GN;
    constexpr int GNP = GN ? GN_PASSES : 1;
    uint2 gyr[GNP], gzr[GNP], gwr = make_uint2(0u, 0u);
    if (GN) {
        const int H = K / 128, nhr = a.rows * H, npass = (nhr + 2 * nwv - 1) / (2 * nwv);
#pragma unroll
        for (int p = 0; p < GNP; ++p) {
            if (p >= npass) break;  // (uniform)
            const int hr = min(p * 2 * nwv + 2 * wave + (lane >> 5), nhr - 1), row = hr >= H ? 1 : 0;  // (one or two rows)
            const int64_t off = int64_t(row) * K + (hr - row * H) * 128 + 4 * (lane & 31);
            gyr[p] = *reinterpret_cast<const uint2*>(a.gn_y + off);
            gzr[p] = *reinterpret_cast<const uint2*>(a.gn_z + off);
        }
        gwr = *reinterpret_cast<const uint2*>(a.gn_w + 4 * (lane & 31));
    }
    // SRC_XP: the bf16 row and its norm weights land in LDS by DMA with the other one-shot operands,
    // ahead of the weight ring (requested behind it, they would queue behind the whole chip's first
    // round of weights); the prep runs from LDS while that round streams in
    uint8_t* xs_l = zeros + 32;  // SRC_XP: [K] bf16 row, then [K] bf16 norm weights
    // per-weight decode tables [g1 - g0][TPW x 16 rows] x 16 bytes (after the SRC_XP region; the rows of
    // a group adjacent, so the 16 rows a wave reads at once fall in distinct banks)
    uint4* tbl = reinterpret_cast<uint4*>(xs_l + (XP ? 4 * K : 0));
    if (ralias) red = reinterpret_cast<int32_t*>(tbl);
    const bool tbl_on = TB || a.tbl != 0;  // (uniform; groups of at least one chunk, scales not asserted integral)
    const bool tbl8 = TB ? TB8 : a.tbl == 2;  // (uniform) 8-byte tables: the default codebook's magnitudes
    const int ngr = g1 - g0;
    if (XP && pwo) {
        // per wave: the 256-groups its prep reads (group g: 512 bytes of the row, 512 of the weights)
        const int G = K / 256, nw4 = a.TPW * a.KS;
#pragma unroll
        for (int gi = 0; gi < XP_GPW; ++gi) {
            const int g = wave + nw4 * gi;
            if (g < G && lane < 32) {
                __builtin_amdgcn_global_load_lds(as_global(reinterpret_cast<const uint8_t*>(a.xp_x)) + 512 * g + lane * 16,
                                                 MDX_LDS(xs_l + 512 * g), 16, 0, 0);
                if (a.xp_nw)
                    __builtin_amdgcn_global_load_lds(as_global(reinterpret_cast<const uint8_t*>(a.xp_nw)) + 512 * g + lane * 16,
                                                     MDX_LDS(xs_l + 2 * K + 512 * g), 16, 0, 0);
            }
        }
    } else if (XP) {
        dma_rows_to_lds(as_global(reinterpret_cast<const uint8_t*>(a.xp_x)), 0, 2 * K, 1, xs_l, nthr);
        if (a.xp_nw) dma_rows_to_lds(as_global(reinterpret_cast<const uint8_t*>(a.xp_nw)), 0, 2 * K, 1, xs_l + 2 * K, nthr);
    }

    // the codebook by scalar loads (it is read-only for the whole launch): one instruction instead
    // of sixteen vector loads per wave in the memory pipeline ahead of the ring
    typedef __attribute__((address_space(4))) const float* const_f32p;
    float cb[16];
    bool cbdef = true;  // (uniform) the codebook is code - 8: a null one, or loaded values that equal it
    if (a.cb) {
        const const_f32p cbc = (const_f32p)(a.cb);
#pragma unroll
        for (int i = 0; i < 16; ++i) cb[i] = cbc[i];
#pragma unroll
        for (int i = 0; i < 16; ++i) cbdef = cbdef && cb[i] == float(i - 8);
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) cb[i] = float(i - 8);
    }

    // 2. the weight ring: every slot issues one load; reads past the slice repeat its last chunk. A
    // tile slot past the matrix's last tile (a work-group's share can end inside its tile slots)
    // reads tile 0 and adds nothing: its addresses must stay inside the matrix all the same.
    const int tl = live ? tile : 0;
    const MDX_G uint8_t* wp;
    int wstride;
    if (a.layout == MDX_LAYOUT_TILE) {
        wp = mq + (tl * NC + c0) * 1024 + lane * 16;
        wstride = 1024;
    } else {
        wp = mq + (tl * 16 + c) * (K / 2) + c0 * 64 + kq * 16;
        wstride = 64;
    }
    const int last = nch > 0 ? nch - 1 : 0;
    uint4 buf[RING];
#pragma unroll
    for (int p = 0; p < RING; ++p) buf[p] = ldg_stream(wp + (live ? min(p, last) : 0) * wstride);
    const bool can_int = !a.force_exact && cbdef && (lgG >= (MFMA ? 7 : 5));
    const bool one_scale = lgG >= 5;  // (uniform) a lane's 32-k run lies in one group
    if (t == 0) *mixed = 0;
    if (t < 8) reinterpret_cast<uint32_t*>(zeros)[t] = 0u;

    if (pwo) {
        // this wave's one-shots are complete once at most RING loads remain; no other wave's matter
        __builtin_amdgcn_s_waitcnt((RING & 15) | ((RING >> 4) << 14) | (7 << 4) | (15 << 8));
    } else {
        // the one-shot loads (issued before the ring) are complete once at most RING loads remain
        static_assert(RING <= 63, "vmcnt field");  // vmcnt: bits 3:0 and 15:14
        __builtin_amdgcn_s_waitcnt((RING & 15) | ((RING >> 4) << 14) | (7 << 4) | (15 << 8));  // vmcnt(RING) only
        __builtin_amdgcn_s_waitcnt(0xC07F);                        // lgkmcnt(0): LDS writes of this wave
        __builtin_amdgcn_s_barrier();
    }
    // a (tile row, group) table from the staged scales: 16 bytes (make_lut's), or the default codebook's eight
    // magnitudes (8 bytes)
    auto build_table = [&](int rw, int gg) {
        const int j = gg * (a.TPW * 16) + rw;
        const uint8_t* sp = sl + rw * seg + gg * ESZ;
        uint2 q8;
        bool have = false;
        if (SDT == MDX_DT_F16 && cbdef) {
            const uint32_t sb = *reinterpret_cast<const uint16_t*>(sp);
            if ((sb & 0x7FFFu) <= F16_FAST_MAX) {
                q8 = make_q8_f16(sb);
                have = true;
            }
        }
        if (tbl8) {
            reinterpret_cast<uint2*>(tbl)[j] = have ? q8 : make_q8(rd_scale<SDT>(sp));
        } else {
            const Lut L = have ? lut_from_q8(q8.x, q8.y) : (cbdef ? make_lut_c8(rd_scale<SDT>(sp)) : make_lut(rd_scale<SDT>(sp), cb));
            tbl[j] = make_uint4(L.w[0], L.w[1], L.w[2], L.w[3]);
        }
    };
    if (TB) {
        // each wave builds the tables it reads itself (its tile's 16 rows x its slice's groups: lane l takes
        // row l % 16 of every fourth group), so no work-group barrier follows; a group shared by two slices
        // is built by both with the same bytes
        if (nch > 0) {
            const int gsh = lgG - 7, ga = c0 >> gsh, gb = ((c1 - 1) >> gsh) + 1;
            for (int gg = ga + (lane >> 4); gg < gb; gg += 4) build_table(ts * 16 + c, gg - g0);
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's table writes are done before its reads
    }
    if (HR) {
        // the rows' scales (the row prep's formula), then the rows quantised into LDS while the ring
        // stays in flight: bf16(v / sb) as bf16(v * fl32(1 / sb)) (quant_rcp)
        float* wm = reinterpret_cast<float*>(red);  // [2][16 waves] (the reduction block is free here)
        const bool whole = a.hmax_n <= WAVE * HMW;  // (uniform) each wave holds every maximum
#pragma unroll
        for (int j = 0; j < HMV; ++j)
#pragma unroll
            for (int r = 0; r < 2; ++r) hmx[r] = fmaxf(hmx[r], hv[r][j]);
        if (!whole) {
            for (int w = t; w < a.hmax_n; w += nthr)
#pragma unroll
                for (int r = 0; r < 2; ++r)
                    if (r < a.rows) hmx[r] = fmaxf(hmx[r], __uint_as_float(a.hmax[r * a.hmax_n + w]));
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const float m = wave_max_nn(hmx[r]);
                if (lane == 0) wm[r * 16 + wave] = m;
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);
            __builtin_amdgcn_s_barrier();
        }
        // every wave takes the rows' maxima over the waves itself (no second hand-off); the first
        // stores the scales for the epilogue
        float rcp[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const float m = whole ? wave_max_nn(hmx[r]) : wave_max_nn(lane < nwv ? wm[r * 16 + lane] : 0.f);
            const float s = fmaxf(__fdiv_rn(m, 127.0f), 1e-30f);
            uint16_t sb = f2bf(s);
            if ((sb & 0x7FFFu) == 0) sb = 0x0080u;
            if (t == 0 && r < a.rows) prml[a.TPW * 16 + r] = s;
            rcp[r] = __fdiv_rn(1.f, bf2f(sb));
        }
        const int total = a.rows * (Kr / 8), per_row = Kr / 8;
#pragma unroll
        for (int k = 0; k < HRP; ++k) {
            const int i = k * nthr + t;
            if (i < total) {
                const int r = i >= per_row ? 1 : 0, j = i - r * per_row;  // (one or two rows)
                const float rr = r ? rcp[1] : rcp[0];
                const uint32_t w[4] = {hraw[k].x, hraw[k].y, hraw[k].z, hraw[k].w};
                uint32_t o[2] = {0u, 0u};
                float d[8];
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    d[e] = __fmul_rn(__uint_as_float((e & 1) ? (w[e >> 1] & 0xFFFF0000u) : (w[e >> 1] << 16)), rr);
#pragma unroll
                for (int e = 0; e < 8; e += 2) bfround2(d[e], d[e + 1]);
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    o[e >> 2] |= (uint32_t(int(fminf(fmaxf(rintf(d[e]), -128.f), 127.f))) & 0xFFu) << (8 * (e & 3));
                *reinterpret_cast<uint2*>(xl + r * Kr + 8 * j) = make_uint2(o[0], o[1]);
            }
        }
    }
    if (GN) {
        // the gated RMSNorm of every head row (gnorm_pair), the rows' maxima across the waves (the
        // reduction block holds them), then the row prep's scale and codes into LDS while the ring stays in
        // flight
        float* wm = reinterpret_cast<float*>(red);  // [2][16 waves]
        const int H = K / 128, nhr = a.rows * H, npass = (nhr + 2 * nwv - 1) / (2 * nwv);
        float hw[4], v[GNP][4], mx[2] = {0.f, 0.f};
        unpack4(gwr, hw);
#pragma unroll
        for (int p = 0; p < GNP; ++p) {
            if (p >= npass) break;  // (uniform)
            float z4[4];
            unpack4(gyr[p], v[p]);
            unpack4(gzr[p], z4);
            if (a.gn_gated) gnorm_pair_g(v[p], hw, z4, a.gn_eps, lane);
            else gnorm_pair(v[p], hw, z4, a.gn_eps, lane);
            const int hr = p * 2 * nwv + 2 * wave + (lane >> 5);
            if (hr < nhr) {
                float m = 0.f;
#pragma unroll
                for (int e = 0; e < 4; ++e) m = fmaxf(m, fabsf(v[p][e]));
                if (hr < H) mx[0] = fmaxf(mx[0], m);
                else mx[1] = fmaxf(mx[1], m);
            }
        }
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const float m = wave_max_nn(mx[r]);
            if (lane == 0) wm[r * 16 + wave] = m;
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
        float rr[2];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const float m = wave_max_nn(lane < nwv ? wm[r * 16 + lane] : 0.f);
            const float s = fmaxf(__fdiv_rn(m, 127.0f), 1e-30f);
            if (t == 0 && r < a.rows) prml[a.TPW * 16 + r] = s;
            rr[r] = quant_rcp(s);
        }
#pragma unroll
        for (int p = 0; p < GNP; ++p) {
            const int hr = p * 2 * nwv + 2 * wave + (lane >> 5);
            if (p < npass && hr < nhr) {
                const int row = hr >= H ? 1 : 0, o = (hr - row * H) * 128 + 4 * (lane & 31);  // (one or two rows)
                *reinterpret_cast<uint32_t*>(xl + row * Kr + o) = quant4(v[p], row ? rr[1] : rr[0]);
                if (wg == 0 && a.gn_out) *reinterpret_cast<uint2*>(a.gn_out + int64_t(row) * K + o) = pack4(v[p]);
            }
        }
    }
    if (XP) {
        // the row prep of one row (prep_row's arithmetic and order), the barriers without memory
        // waits so that the ring stays in flight; the reduction block holds the group sums / maxima
        const int G = K / 256;
        float* gsum = reinterpret_cast<float*>(red);  // [G] group sums, then [waves] maxima
        // lane l of wave w: elements 4 l .. 4 l + 3 of the groups w, w + waves, ...
        float v[XP_GPW][4];
#pragma unroll
        for (int gi = 0; gi < XP_GPW; ++gi)
            unpack4(reinterpret_cast<const uint2*>(xs_l)[64 * min(wave + nwv * gi, G - 1) + lane], v[gi]);
        if (a.xp_nw) {
#pragma unroll
            for (int gi = 0; gi < XP_GPW; ++gi) {
                float q = __fmul_rn(v[gi][0], v[gi][0]);
#pragma unroll
                for (int e = 1; e < 4; ++e) q = __fadd_rn(q, __fmul_rn(v[gi][e], v[gi][e]));
                q = tree_sum64(q);
                const int g = wave + nwv * gi;
                if (lane == 0 && g < G) gsum[g] = q;
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);
            __builtin_amdgcn_s_barrier();
            // the group sums in group order (one LDS read per lane, then lane by lane)
            const float gv = lane < G ? gsum[lane] : 0.f;
            float ss = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(gv)));
            for (int g = 1; g < G; ++g) ss = __fadd_rn(ss, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gv), g)));
            const float rr = __fdiv_rn(1.f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, float(K)), a.xp_eps)));
#pragma unroll
            for (int gi = 0; gi < XP_GPW; ++gi) {
                float wv[4];
                unpack4(reinterpret_cast<const uint2*>(xs_l + 2 * K)[64 * min(wave + nwv * gi, G - 1) + lane], wv);
#pragma unroll
                for (int e = 0; e < 4; ++e) v[gi][e] = __fmul_rn(__fmul_rn(v[gi][e], rr), wv[e]);
                bfround2(v[gi][0], v[gi][1]);
                bfround2(v[gi][2], v[gi][3]);
            }
        }
        float m = 0.f;
#pragma unroll
        for (int gi = 0; gi < XP_GPW; ++gi)
            if (wave + nwv * gi < G)
#pragma unroll
                for (int e = 0; e < 4; ++e) m = fmaxf(m, fabsf(v[gi][e]));
        m = wave_max_nn(m);
        if (lane == 0) gsum[G + wave] = m;
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
        const float rm = wave_max_nn(lane < nwv ? gsum[G + lane] : 0.f);
        const float s = fmaxf(__fdiv_rn(rm, 127.0f), 1e-30f);
        if (t == 0) prml[a.TPW * 16] = s;
        uint16_t sb = f2bf(s);
        if ((sb & 0x7FFFu) == 0) sb = 0x0080u;
        const float rr = __fdiv_rn(1.f, bf2f(sb));  // (quant_rcp)
#pragma unroll
        for (int gi = 0; gi < XP_GPW; ++gi) {
            const int g = wave + nwv * gi;
            if (g < G) {
                uint32_t o = 0;
                float d[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) d[e] = __fmul_rn(v[gi][e], rr);
                bfround2(d[0], d[1]);
                bfround2(d[2], d[3]);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    o |= (uint32_t(int(fminf(fmaxf(rintf(d[e]), -128.f), 127.f))) & 0xFFu) << (8 * e);
                *reinterpret_cast<uint32_t*>(xl + 256 * g + 4 * lane) = o;
            }
        }
    }
    // Whether every staged scale is an integer in [-15, 15]: then the unit takes the integral form
    // throughout (both forms give the same int32 sums, so the choice is free). Under
    // MDX_DECODE_INTEGRAL the caller asserts it: no check, and no barrier unless this prologue wrote
    // the activation rows to LDS itself (SRC_HR, SRC_XP).
    bool integ;
    if (TB) {
        if (HR || XP || GN) {  // (the rows this prologue wrote to LDS)
            __builtin_amdgcn_s_waitcnt(0xC07F);
            __builtin_amdgcn_s_barrier();
        }
        integ = false;
    } else if (IO) {
        if (HR || XP || GN) {  // (the rows this prologue wrote to LDS)
            __builtin_amdgcn_s_waitcnt(0xC07F);
            __builtin_amdgcn_s_barrier();
        }
        integ = true;
    } else if (pwo) {
        if (HR || XP || GN) {  // (the rows this prologue wrote to LDS)
            __builtin_amdgcn_s_waitcnt(0xC07F);
            __builtin_amdgcn_s_barrier();
        }
        integ = true;  // (pwo implies assume_int with the default codebook and G128)
    } else if (a.assume_int && can_int) {
        if (HR || XP || GN) {
            __builtin_amdgcn_s_waitcnt(0xC07F);
            __builtin_amdgcn_s_barrier();
        }
        integ = true;
    } else {
        if (can_int) {
            bool bad = false;
            for (int j = t; j < a.TPW * 16 * (seg / ESZ); j += nthr) {
                const float s = rd_scale<SDT>(sl + j * ESZ);
                bad = bad || !(s == rintf(s) && fabsf(s) <= 15.f);
            }
            if (bad) *mixed = 1;
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS writes are done (the ring stays in flight)
        __builtin_amdgcn_s_barrier();
        integ = can_int && *mixed == 0;  // uniform over the unit
    }
    if (!TB && !integ && tbl_on) {
        // every (tile row, group) table once, from the staged scales: thread t takes row t % nr of groups
        // t / nr, t / nr + nthr / nr, ... (nthr is a multiple of nr = 16 TPW)
        const int nr = a.TPW * 16, gstep = nthr / nr;
        for (int gg = t / nr; gg < ngr; gg += gstep) build_table(t % nr, gg);
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
    }
    // the tile-major layout keeps k 0..3 of a code word in its low nibbles and k 4..7 in its high
    // ones (natural activation order); the checkpoint layout interleaves them (even k low, odd k high)
    const bool split = a.layout == MDX_LAYOUT_TILE;
    const uint8_t* scol = pwo ? swv + c * sbw - c0 * ESZ : sl + (ts * 16 + c) * seg - g0 * ESZ;
    // the tables travel in a ring beside the weights: slot p's table is read from LDS when the slot's
    // weights are requested, a round ahead of its use (an LDS read right before the lookups would
    // expose its latency at every chunk)
    const bool tring = !integ && tbl_on;  // (uniform)
    auto tbl_of = [&](int i) {
        // (TB: groups of at least one chunk, so a chunk's group is a uniform shift of its index and the
        // offset a scalar; the generic path also serves smaller groups through klane)
        const int o = TB ? (ts * 16 + c) + (((c0 + min(i, last)) >> (lgG - 7)) - g0) * (a.TPW * 16)
                         : (ts * 16 + c) + ((((c0 + min(i, last)) * CHUNK_K + klane) >> lgG) - g0) * (a.TPW * 16);
        if (tbl8) {
            const uint2 q = reinterpret_cast<const uint2*>(tbl)[o];
            return make_uint4(q.x, q.y, 0u, 0u);
        }
        return tbl[o];
    };
    uint4 tq[RING];
#pragma unroll
    for (int p = 0; p < RING; ++p) tq[p] = tring ? tbl_of(p) : make_uint4(0u, 0u, 0u, 0u);

    if constexpr (TB) {
        // the table decode only: per chunk the lane's four code dwords through its (row, group) table,
        // four MFMAs against the activation rows (rows past the last repeat the last row: their sums are
        // never stored); a chunk past the slice adds nothing (a uniform branch)
        v4i acc = {0, 0, 0, 0};
        const uint8_t* xrow = xl + min(lane & 15, a.rows - 1) * Kr + klane - cu0 * CHUNK_K;
        auto chunk = [&](int p, int i, bool refill) {
            const int ch = c0 + min(i, last);
            const uint4* x4 = reinterpret_cast<const uint4*>(xrow + ch * CHUNK_K);
            const uint4 xa = x4[0], xb = x4[1];
            const uint32_t xd[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
            uint32_t lo[4], hi[4];
            decode_tb<TB8>(buf[p], tq[p], lo, hi);
            if (!split)
#pragma unroll
                for (int j = 0; j < 4; ++j) nat_order(lo[j], hi[j], lo[j], hi[j]);
            if (i < nch) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(long(uint64_t(xd[2 * j]) | (uint64_t(xd[2 * j + 1]) << 32)),
                                                                long(uint64_t(lo[j]) | (uint64_t(hi[j]) << 32)), acc, 0, 0, 0);
            }
            if (refill) {  // refill after use
                buf[p] = ldg_stream(wp + min(i + RING, last) * wstride);
                tq[p] = tbl_of(i + RING);
            }
            __builtin_amdgcn_sched_barrier(0);
        };
        // whole rounds that refill their slots, then the last round without refills: no load past the
        // slice is in flight when the wave leaves its loop
        int i0 = 0;
        for (; i0 + RING < nch; i0 += RING)
#pragma unroll
            for (int p = 0; p < RING; ++p) chunk(p, i0 + p, true);
#pragma unroll
        for (int p = 0; p < RING; ++p) chunk(p, i0 + p, false);
        if (ralias) __syncthreads();  // every wave is past its last table read
        int32_t* dst = red + ((ts * a.KS + slice) * 64 + lane) * 4;
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[r] = acc[r];
    } else if (MFMA) {
        v4i accE = {0, 0, 0, 0};        // per-weight decoded chunks: one running MFMA sum
        int32_t tot[4] = {0, 0, 0, 0};  // integral chunks: sum of s * (chunk dot - 8 sum x)
        // rows past the last read 32 zero bytes at every chunk (stride 0)
        const bool xlive = (lane & 15) < a.rows;
        const uint8_t* xrow = xlive ? xl + (lane & 15) * Kr + klane - cu0 * CHUNK_K : zeros;
        const int xstride = xlive ? CHUNK_K : 0;
        for (int i0 = 0; i0 < nch; i0 += RING) {
#pragma unroll
            for (int p = 0; p < RING; ++p) {
                // whole rounds: a chunk past the slice re-reads the last one and adds nothing
                const int i = i0 + p;
                const bool valid = i < nch;
                const uint4 w = buf[p];
                const int ch = c0 + min(i, last);
                const int k0 = ch * CHUNK_K + klane;
                const float s0 = rd_scale<SDT>(scol + (k0 >> lgG) * ESZ);
                const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
                const uint4* x4 = reinterpret_cast<const uint4*>(xrow + ch * xstride);
                const uint4 xa = x4[0], xb = x4[1];
                uint32_t xd[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
                if (integ) {
                    v4i dacc = {0, 0, 0, 0};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        uint32_t n0 = sx16_lo(wd[j]), n1 = sx16_hi(wd[j]);
                        if (!split) nat_order(n0, n1, n0, n1);
                        dacc = __builtin_amdgcn_mfma_i32_16x16x32_i8(long(uint64_t(xd[2 * j]) | (uint64_t(xd[2 * j + 1]) << 32)),
                                                                     long(uint64_t(n0) | (uint64_t(n1) << 32)), dacc, 0, 0, 0);
                    }
                    // D rows 4 kq + r: 16 * sum x (c - 8), exactly; times the chunk's scale (0 past the slice)
                    const int sv = valid ? int(s0) : 0;
                    tot[0] += __mul24(sv, dacc[0] >> 4);
                    tot[1] += __mul24(sv, dacc[1] >> 4);
                    tot[2] += __mul24(sv, dacc[2] >> 4);
                    tot[3] += __mul24(sv, dacc[3] >> 4);
                } else {
                    if (!valid)
#pragma unroll
                        for (int j = 0; j < 8; ++j) xd[j] = 0;
                    uint32_t lo[4], hi[4];
                    if (tbl_on)
                        decode_tbl(wd, tq[p], tbl8, lo, hi);
                    else
                        decode_exact(wd, s0, rd_scale<SDT>(scol + ((k0 + 16) >> lgG) * ESZ), one_scale, cbdef, cb, lo, hi);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        uint32_t n0 = lo[j], n1 = hi[j];
                        if (!split) nat_order(n0, n1, n0, n1);
                        accE = __builtin_amdgcn_mfma_i32_16x16x32_i8(long(uint64_t(xd[2 * j]) | (uint64_t(xd[2 * j + 1]) << 32)),
                                                                     long(uint64_t(n0) | (uint64_t(n1) << 32)), accE, 0, 0, 0);
                    }
                }
                // refill the slot only now: its old and new contents never live at once, so the ring
                // keeps its registers across rounds (no copies, and no wait, at the loop end)
                buf[p] = ldg_stream(wp + min(i + RING, last) * wstride);
                if (tring) tq[p] = tbl_of(i + RING);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        int32_t* dst = red + ((ts * a.KS + slice) * 64 + lane) * 4;
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[r] = int32_t(uint32_t(tot[r]) + uint32_t(accE[r]));
    } else {
        int32_t tot[R];
#pragma unroll
        for (int r = 0; r < R; ++r) tot[r] = 0;
        for (int i0 = 0; i0 < nch; i0 += RING) {
#pragma unroll
            for (int p = 0; p < RING; ++p) {
                const int i = i0 + p;
                const bool valid = i < nch;
                const uint4 w = buf[p];
                const int ch = c0 + min(i, last);
                const int k0 = ch * CHUNK_K + klane;
                const float s0 = rd_scale<SDT>(scol + (k0 >> lgG) * ESZ);
                const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
                uint32_t lo[4], hi[4];  // weights of k 8 j + [0, 4) and + [4, 8) (16 (c - 8) in the integral form)
                if (integ) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        lo[j] = sx16_lo(wd[j]);
                        hi[j] = sx16_hi(wd[j]);
                    }
                } else {
                    if (tbl_on)
                        decode_tbl(wd, tq[p], tbl8, lo, hi);
                    else
                        decode_exact(wd, s0, rd_scale<SDT>(scol + ((k0 + 16) >> lgG) * ESZ), one_scale, cbdef, cb, lo, hi);
                }
                if (!split)
#pragma unroll
                    for (int j = 0; j < 4; ++j) nat_order(lo[j], hi[j], lo[j], hi[j]);
                const int sv = valid ? (integ ? int(s0) : 1) : 0;
                const int sg = (ch - cu0) * 4 + kq;  // this lane's 32-k run within the unit
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    if (r < a.rows) {
                        const uint4* x4 = reinterpret_cast<const uint4*>(xl + r * Kr + sg * 32);
                        const uint4 xa = x4[0], xb = x4[1];
                        const uint32_t xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
                        int d = 0;
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            d = sdot4(int(lo[j]), int(xv[2 * j]), d);
                            d = sdot4(int(hi[j]), int(xv[2 * j + 1]), d);
                        }
                        tot[r] += __mul24(sv, integ ? (d >> 4) : d);
                    }
                }
                buf[p] = ldg_stream(wp + min(i + RING, last) * wstride);  // refill after use (see above)
                if (tring) tq[p] = tbl_of(i + RING);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // fold the four k quarters of each column (lanes c, c + 16, c + 32, c + 48)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            tot[r] = isum_x32(isum_x16(tot[r]));
        }
        if (lane < 16)
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (r < a.rows) red[((ts * a.KS + slice) * 16 + lane) * a.rows + r] = tot[r];
    }
    // the epilogue's parameters (only the epilogue reads them; written this late, their loads need no
    // wait that would also wait for the ring)
    if (slice == 0 && lane < 16) prml[ts * 16 + lane] = prm;
    else if (own_x && wave == a.TPW * a.KS - 1 && lane >= 16 && lane < 16 + a.rows) prml[a.TPW * 16 + lane - 16] = prm;
    __syncthreads();
    if constexpr (GDN) gdn_epilogue<MFMA>(a, wg, red, prml, xl, gctl);
    else epilogue<MFMA>(a, wg, red, prml);
}

// SRC_HR work-groups have at most 12 waves: their staged pieces need the registers of 3 waves per
// SIMD.
template <bool MFMA, int R, int SDT, int RING, int SRC = SRC_Q8>
__global__ __launch_bounds__((SRC & 3) == SRC_HR ? 768 : 1024) void gemv_kernel(GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    if constexpr ((SRC & SRC_GDN) != 0) {
        if (int(blockIdx.x) >= a.gf.units) {  // (uniform) a gate work-group
            gdn_gates_side(a, int(blockIdx.x) - a.gf.units, lds);
            return;
        }
    }
    gemv_unit<MFMA, R, SDT, RING, SRC>(a, blockIdx.x, 0, a.K / CHUNK_K, lds);
}

// Bytes of a per-weight decode table in LDS (0: none): 16 (the table), 8 (the default codebook's
// eight magnitudes, expanded per chunk by four byte permutes and two carry-free negations).
int gemv_table_bytes(const GemvArgs& a) { return a.tbl == 1 ? 16 : (a.tbl == 2 ? 8 : 0); }

// LDS bytes of a unit over `ncu` chunks starting at chunk cu0 (the layout of gemv_unit)
size_t gemv_smem(const GemvArgs& a, bool mfma, int esz, int cu0, int ncu) {
    const int ng = a.K >> a.lgG;
    int g0 = (cu0 * CHUNK_K) >> a.lgG, g1 = ((cu0 + ncu) * CHUNK_K + (1 << a.lgG) - 1) >> a.lgG;
    if ((ng * esz) % 16 || (g0 * esz) % 16 || ((g1 - g0) * esz) % 16) {
        g0 = 0;
        g1 = ng;
    }
    const size_t seg = size_t(g1 - g0) * esz;
    size_t s = ((size_t(a.rows) * ncu * CHUNK_K + 1023) & ~size_t(1023)) + ((a.TPW * 16 * seg + 1023) & ~size_t(1023));
    if (!a.red_alias) s += mfma ? size_t(a.TPW) * a.KS * 64 * 4 * 4 : size_t(a.TPW) * a.KS * 16 * a.rows * 4;
    s += 128 * 4 + 16 + 32;  // parameters, flag, zeros
    if (a.xp_x) s += size_t(4) * a.K;  // SRC_XP: the bf16 row and its norm weights
    s += size_t(a.TPW) * 16 * (g1 - g0) * gemv_table_bytes(a);  // per-weight decode tables
    return s;
}

size_t gemv_smem(const GemvArgs& a, bool mfma, int esz) { return gemv_smem(a, mfma, esz, 0, a.K / CHUNK_K); }

int esz_of(int sdt) { return sdt == MDX_DT_F32 ? 4 : (sdt == MDX_DT_F16 ? 2 : 1); }

// The kernel variants this thread's GEMV launches took since the last mdx_gemv_trace call (a diagnostic for
// tests: which source, decode form and product path a shape reaches).
constexpr int TRACE_MAX = 64;
thread_local int32_t g_trace[TRACE_MAX][7];
thread_local int g_trace_n = 0;

void trace_launch(bool mfma, int src, int sdt, const GemvArgs& a) {
    if (g_trace_n >= TRACE_MAX) return;
    int32_t* r = g_trace[g_trace_n++];
    r[0] = mfma;
    r[1] = src;
    r[2] = sdt;
    r[3] = a.rows;
    r[4] = a.TPW;
    r[5] = a.KS;
    r[6] = a.red_alias;
}

template <bool MFMA, int R, int SDT, int RING, int SRC>
int launch_gemv_h(const GemvArgs& a, int wgs, hipStream_t st) {
    trace_launch(MFMA, SRC, SDT, a);
    const size_t smem = gemv_smem(a, MFMA, esz_of(SDT));
    const void* fn = reinterpret_cast<const void*>(&gemv_kernel<MFMA, R, SDT, RING, SRC>);
    if (smem > 64 * 1024) allow_smem(fn, smem);
    const int threads = a.TPW * a.KS * WAVE;
    const int grid = wgs + (a.gf.on ? a.gf.nside : 0);
    hipLaunchKernelGGL((gemv_kernel<MFMA, R, SDT, RING, SRC>), dim3(unsigned(grid)), dim3(unsigned(threads)), smem, st, a);
    MDX_LAUNCHED();
    return MDX_OK;
}

constexpr int TB_RING = 4;  // weight ring depth of the table-only variants

template <bool MFMA, int R, int SDT, int RING, int TB>
int launch_gemv_tb(const GemvArgs& a, int wgs, hipStream_t st) {
    if (a.gf.on) {
        if constexpr (SDT == MDX_DT_F16) {  // (mdx_gdn_proj with a bf16 row: fp16 scales)
            if (a.xp_x) return launch_gemv_h<MFMA, R, SDT, TB_RING, SRC_XP + TB + SRC_GDN>(a, wgs, st);
        }
        return launch_gemv_h<MFMA, R, SDT, TB_RING, SRC_Q8 + TB + SRC_GDN>(a, wgs, st);
    }
    if constexpr (SDT == MDX_DT_F16) {  // (gemv_gn_fits: fp16 scales)
        if (a.gn_y) return launch_gemv_h<MFMA, R, SDT, TB_RING, SRC_GN + TB>(a, wgs, st);
    }
    if (a.hr) return launch_gemv_h<MFMA, R, SDT, TB_RING, SRC_HR + TB>(a, wgs, st);
    if (a.xp_x) return launch_gemv_h<MFMA, R, SDT, TB_RING, SRC_XP + TB>(a, wgs, st);
    return launch_gemv_h<MFMA, R, SDT, TB_RING, SRC_Q8 + TB>(a, wgs, st);
}

template <bool MFMA, int R, int SDT, int RING>
int launch_gemv_t(const GemvArgs& a, int wgs, hipStream_t st) {
    if constexpr (MFMA) {
        // per-weight decode tables in LDS: the table-only variants
        if (a.tbl == 1) return launch_gemv_tb<MFMA, R, SDT, RING, SRC_TBL>(a, wgs, st);
        if (a.tbl == 2) return launch_gemv_tb<MFMA, R, SDT, RING, SRC_TBL8>(a, wgs, st);
    }
    // the integral-only variant when the caller asserts integral scales that the integral form takes
    const bool io = a.assume_int && !a.cb && !a.force_exact && a.lgG >= (MFMA ? 7 : 5);
    if (io) {
        if (a.gf.on) {
            if constexpr (!MFMA && SDT == MDX_DT_F16) {
                if (a.xp_x) return launch_gemv_h<MFMA, R, SDT, RING, SRC_XP + SRC_INT_ONLY + SRC_GDN>(a, wgs, st);
            }
            return launch_gemv_h<MFMA, R, SDT, RING, SRC_Q8 + SRC_INT_ONLY + SRC_GDN>(a, wgs, st);
        }
        if constexpr (SDT == MDX_DT_F16) {
            if (a.gn_y) return launch_gemv_h<MFMA, R, SDT, RING, SRC_GN + SRC_INT_ONLY>(a, wgs, st);
        }
        if (a.hr) return launch_gemv_h<MFMA, R, SDT, RING, SRC_HR + SRC_INT_ONLY>(a, wgs, st);
        if (!MFMA && a.xp_x) return launch_gemv_h<MFMA, R, SDT, RING, SRC_XP + SRC_INT_ONLY>(a, wgs, st);
        return launch_gemv_h<MFMA, R, SDT, RING, SRC_Q8 + SRC_INT_ONLY>(a, wgs, st);
    }
    if (a.gf.on) {
        if constexpr (!MFMA && SDT == MDX_DT_F16) {
            if (a.xp_x) return launch_gemv_h<MFMA, R, SDT, RING, SRC_XP + SRC_GDN>(a, wgs, st);
        }
        return launch_gemv_h<MFMA, R, SDT, RING, SRC_Q8 + SRC_GDN>(a, wgs, st);
    }
    if constexpr (SDT == MDX_DT_F16) {
        if (a.gn_y) return launch_gemv_h<MFMA, R, SDT, RING, SRC_GN>(a, wgs, st);
    }
    if (a.hr) return launch_gemv_h<MFMA, R, SDT, RING, SRC_HR>(a, wgs, st);
    if (!MFMA && a.xp_x) return launch_gemv_h<MFMA, R, SDT, RING, SRC_XP>(a, wgs, st);
    return launch_gemv_h<MFMA, R, SDT, RING, SRC_Q8>(a, wgs, st);
}

template <int SDT, int RING>
int launch_gemv_s(const GemvArgs& a, bool mfma, int wgs, hipStream_t st) {
    if (mfma) return launch_gemv_t<true, 4, SDT, RING>(a, wgs, st);
    return launch_gemv_t<false, 1, SDT, RING>(a, wgs, st);
}

template <int RING>
int launch_gemv_d(const GemvArgs& a, int sdt, bool mfma, int wgs, hipStream_t st) {
    if (sdt == MDX_DT_F32) return launch_gemv_s<MDX_DT_F32, RING>(a, mfma, wgs, st);
    if (sdt == MDX_DT_F16) return launch_gemv_s<MDX_DT_F16, RING>(a, mfma, wgs, st);
    return launch_gemv_s<MDX_DT_FP8E4M3, RING>(a, mfma, wgs, st);
}

// Rows at which the MFMA path takes over from the VALU dot path (the VALU path handles one row).
constexpr int MFMA_MIN_ROWS = 2;

int ilog2(int64_t v) {
    int l = 0;
    while ((int64_t(1) << l) < v) ++l;
    return (int64_t(1) << l) == v ? l : -1;
}

int check_w4(const mdx_w4* w, const char* what) {
    MDX_CHECK(w && w->q && w->s_rel && w->s_channel, "%s: null weight pointer", what);
    MDX_CHECK(w->n > 0 && w->n % 16 == 0, "%s: N must be a positive multiple of 16 (got %lld)", what, (long long)w->n);
    MDX_CHECK(w->k > 0 && w->k % CHUNK_K == 0 && w->k <= 65536, "%s: K must be a multiple of 128 in 128..65536 (got %lld)",
              what, (long long)w->k);
    MDX_CHECK(w->group_size >= 16 && ilog2(w->group_size) >= 0 && w->k % w->group_size == 0,
              "%s: group_size must be a power of two >= 16 dividing K (got %lld)", what, (long long)w->group_size);
    MDX_CHECK(w->s_dtype == MDX_DT_F32 || w->s_dtype == MDX_DT_F16 || w->s_dtype == MDX_DT_FP8E4M3,
              "%s: s_rel dtype must be f32, f16 or fp8 e4m3", what);
    MDX_CHECK(w->layout == MDX_LAYOUT_ROW || w->layout == MDX_LAYOUT_TILE, "%s: unknown layout", what);
    MDX_CHECK(w->decode == MDX_DECODE_EXACT || w->decode == MDX_DECODE_AUTO || w->decode == MDX_DECODE_INTEGRAL,
              "%s: unknown decode mode", what);
    MDX_CHECK(aligned(w->q, 16), "%s: codes must be 16-byte aligned", what);
    MDX_CHECK(w->n * w->k / 2 < (int64_t(1) << 31), "%s: weight larger than 2 GiB", what);
    return MDX_OK;
}

// one GEMV launch over up to three matrices sharing K (or a gate/up pair)
// Validate a GEMV's operands and fill its arguments (geometry left to the caller); total = tiles.
int setup_gemv(const mdx_w4* const* ws, int nm, bool pair, const int8_t* xq, const float* xs, int rows, int epi,
               void* const* outs, const void* const* res, int out_dt, const uint16_t* lut, GemvArgs& a, int& total) {
    MDX_CHECK(aligned(xq, 16), "x must be 16-byte aligned");
    const mdx_w4& w0 = *ws[0];
    for (int i = 0; i < nm; ++i) {
        int rc = check_w4(ws[i], "weight");
        if (rc) return rc;
        MDX_CHECK(ws[i]->k == w0.k && ws[i]->group_size == w0.group_size && ws[i]->s_dtype == w0.s_dtype &&
                      ws[i]->layout == w0.layout && ws[i]->decode == w0.decode,
                  "fused matrices must share K, group size, scale dtype, layout and decode mode");
        MDX_CHECK(ws[i]->codebook == w0.codebook, "fused matrices must share one codebook");
        MDX_CHECK(aligned(ws[i]->s_rel, 16), "s_rel must be 16-byte aligned");
    }
    if (pair) MDX_CHECK(nm == 2 && ws[0]->n == ws[1]->n, "gate/up must have the same N");
    a = GemvArgs{};
    a.nm = nm;
    a.pair = pair ? 1 : 0;
    total = 0;
    for (int i = 0; i < 3; ++i) {
        const mdx_w4& w = *ws[i < nm ? i : 0];
        a.m[i] = MatArg{reinterpret_cast<const uint8_t*>(w.q), reinterpret_cast<const uint8_t*>(w.s_rel), w.s_channel,
                        int(w.n), int(w.n / 16)};
        if (i < nm) total += int(w.n / 16);
        a.out[i] = outs[i < nm ? i : 0];
        a.res[i] = res ? res[i < nm ? i : 0] : nullptr;
    }
    a.K = int(w0.k);
    a.lgG = ilog2(w0.group_size);
    a.layout = w0.layout;
    a.cb = w0.codebook;
    a.xq = xq;
    a.xs = xs;
    a.rows = rows;
    a.epi = epi;
    a.out_dt = out_dt;
    a.lut = lut;
    a.force_exact = w0.decode == MDX_DECODE_EXACT;
    a.pwo = 0;
    a.assume_int = 1;
    for (int i = 0; i < nm; ++i) a.assume_int = a.assume_int && ws[i]->decode == MDX_DECODE_INTEGRAL;
    return MDX_OK;
}

// The launch geometry: TPW tiles per work-group, KS K-slices per tile (at most 16 waves per
// work-group): the smallest split that puts >= 3072 waves on the chip (12 per CU), but no slice
// shorter than 4 chunks, measured best on MI355X for the 8-52 MB matrices of this model (longer
// streams per wave beat more, shorter waves: 4096 x 4096 takes 6.4 us at 8 slices against 7.6 at 12).
void gemv_geometry(int total, int K, bool pair, int rows, int& TPW, int& KS) {
    TPW = pair ? 2 : 1;
    // more than 8 rows: about one work-group per CU (up to six tiles each). Every work-group stages
    // all of its rows' K range, so wider work-groups stage less per CU: the 16-row MLP 46.3 -> 41.3 us
    // (gate/up pair 20.0 -> 15.4 us). At 8 rows the same geometry loses (MLP 30.8 -> 31.1 us, stack
    // 3.243 -> 3.272 ms). MDX_WIDE_ROWS moves the threshold (tuning sweeps).
    static const int wide_rows = [] {
        const char* e = getenv("MDX_WIDE_ROWS");
        return e ? atoi(e) : 9;
    }();
    if (rows >= wide_rows) {
        int t = std::min(6, total / 256);
        if (pair) t &= ~1;
        TPW = std::max(TPW, t);
    }
    const int NC = K / CHUNK_K;
    const int maxks = 16 / TPW;
    KS = 1;
    for (int d = 1; d <= maxks && 4 * d <= NC; ++d) {
        if (NC % d) continue;
        KS = d;
        if (int64_t(total) * d >= 3072) break;
    }
    // MDX_GEMV_TPW / MDX_GEMV_KS override the geometry (tuning sweeps); MDX_GEMV_PAIR_TPW / _KS only that of
    // gate/up pairs
    if (const char* env = pair ? getenv("MDX_GEMV_PAIR_TPW") : nullptr) {
        const int tpw = atoi(env);
        if (tpw >= 2 && tpw <= 6 && tpw % 2 == 0) TPW = tpw;
        KS = 1;
        for (int d = 1; d <= 16 / TPW && 4 * d <= NC; ++d) {
            if (NC % d) continue;
            KS = d;
            if (int64_t(total) * d >= 3072) break;
        }
    }
    if (const char* env = pair ? getenv("MDX_GEMV_PAIR_KS") : nullptr) {
        const int ks = atoi(env);
        if (ks >= 1 && ks * TPW <= 16 && NC % ks == 0) KS = ks;
    }
    if (const char* env = getenv("MDX_GEMV_TPW")) {
        const int tpw = atoi(env);
        if (tpw >= 1 && tpw <= 6 && (!pair || tpw % 2 == 0)) TPW = tpw;  // the parameter block holds 6 tiles
    }
    if (const char* env = getenv("MDX_GEMV_KS")) {
        const int ks = atoi(env);
        if (ks >= 1 && ks * TPW <= 16 && NC % ks == 0) KS = ks;
    }
    if (TPW * KS > 16) KS = 16 / TPW;
}

// Whether a one-matrix GEMV of `rows` rows over K quantises bf16 rows in its prologue (HR: at most
// 16 pieces of 8 per thread, at most 12 waves per work-group). Every work-group reads and quantises
// all of its rows, so this pays only for one or two rows: at 8 rows of 12288 the 256 work-groups
// of a down GEMV would read 50 MB of h between them and lose more than the prep launch costs.
bool gemv_hr_fits(const mdx_w4* w, int rows) {
    int TPW, KS;
    gemv_geometry(int(w->n / 16), int(w->k), false, rows, TPW, KS);
    return rows <= 2 && TPW * KS <= 12 && int64_t(rows) * (w->k / 8) <= int64_t(16) * TPW * KS * WAVE;
}

// Whether a GEMV of one row can run the row prep of its activation in its prologue (SRC_XP: K a
// multiple of 256 with at most XP_GPW 256-groups per wave).
bool gemv_xp_fits(const mdx_w4* const* ws, int nm, bool pair) {
    int total = 0;
    for (int i = 0; i < nm; ++i) total += int(ws[i]->n / 16);
    int TPW, KS;
    gemv_geometry(total, int(ws[0]->k), pair, 1, TPW, KS);
    return ws[0]->k % 256 == 0 && ws[0]->k / 256 <= int64_t(XP_GPW) * TPW * KS;
}

// Whether a one-matrix GEMV of `rows` rows takes the gated RMSNorm + quantisation of its activation in its
// prologue (SRC_GN: one or two rows, fp16 scales, K a multiple of 256, at most GN_PASSES head rows per
// lane). Every work-group reads both rows and their gate inputs (32 KB at K = 4096), which pays for one or
// two rows only.
bool gemv_gn_fits(const mdx_w4* w, int rows) {
    int TPW, KS;
    gemv_geometry(int(w->n / 16), int(w->k), false, rows, TPW, KS);
    return rows >= 1 && rows <= 2 && w->s_dtype == MDX_DT_F16 && w->k % 256 == 0 &&
           int64_t(rows) * (w->k / 128) <= int64_t(2) * GN_PASSES * TPW * KS;
}

// Extra activation sources and outputs of one launch (all optional).
struct GemvExtra {
    uint32_t* hmax_out = nullptr;      // EPI_SILU pair: the work-groups' |h| maxima
    const uint16_t* hr = nullptr;      // SRC_HR (gemv_hr_fits): bf16 rows with the maxima hmax[hmax_n]
    const uint32_t* hmax = nullptr;
    int hmax_n = 0;
    const uint16_t* xp_x = nullptr;    // SRC_XP (gemv_xp_fits): one bf16 row and its prep (no rotation)
    const uint16_t* xp_nw = nullptr;
    float xp_eps = 0.f;
    const GdnFold* gdn = nullptr;      // a Gated-DeltaNet projection (matrices qkv, z; bf16 outputs)
    const uint16_t* gn_y = nullptr;    // SRC_GN (gemv_gn_fits): raw rows, gate inputs, norm weights, eps, out
    const uint16_t* gn_z = nullptr;
    const uint16_t* gn_w = nullptr;
    float gn_eps = 0.f;
    uint16_t* gn_out = nullptr;
    int gn_gated = 0;
};

int run_gemv(const mdx_w4* const* ws, int nm, bool pair, const int8_t* xq, const float* xs, int rows, int epi,
             void* const* outs, const void* const* res, int out_dt, const uint16_t* lut, hipStream_t st,
             const GemvExtra& ex = GemvExtra{}) {
    MDX_CHECK(rows >= 1 && rows <= 16, "rows must be in 1..16 (got %d)", rows);
    MDX_CHECK(!ex.hr || (nm == 1 && !pair && ex.hmax && ex.hmax_n >= 4 && ex.hmax_n % 4 == 0 && aligned(ex.hmax, 16) &&
                         gemv_hr_fits(ws[0], rows)),
              "bf16-row GEMV geometry");
    MDX_CHECK(!ex.hmax_out || (pair && rows <= 16), "|h| maxima need a gate/up pair");
    MDX_CHECK(!ex.xp_x || (rows == 1 && gemv_xp_fits(ws, nm, pair)), "row-prep GEMV geometry");
    MDX_CHECK(!ex.gn_y || (nm == 1 && !pair && ex.gn_z && ex.gn_w && gemv_gn_fits(ws[0], rows)), "gated-norm GEMV geometry");
    // the activation rows live in LDS: above 128 KiB, run the rows in two halves
    if (rows > 8 && int64_t(rows) * ws[0]->k > 128 * 1024) {
        const int ra = 8, rb = rows - 8;
        int rc = run_gemv(ws, nm, pair, xq, xs, ra, epi, outs, res, out_dt, lut, st);
        if (rc) return rc;
        const int esz = out_dt == MDX_DT_F32 ? 4 : 2;
        void* o2[3];
        const void* r2[3];
        for (int i = 0; i < nm; ++i) {
            o2[i] = static_cast<uint8_t*>(outs[i]) + size_t(ra) * ws[pair ? 0 : i]->n * esz;
            r2[i] = res && res[i] ? static_cast<const uint8_t*>(res[i]) + size_t(ra) * ws[i]->n * esz : nullptr;
        }
        if (pair) o2[1] = o2[0];
        return run_gemv(ws, nm, pair, xq + size_t(ra) * ws[0]->k, xs + ra, rb, epi, o2, r2, out_dt, lut, st);
    }
    GemvArgs a;
    int total = 0;
    int rc = setup_gemv(ws, nm, pair, ex.hr || ex.xp_x || ex.gn_y ? nullptr : xq, xs, rows, epi, outs, res, out_dt, lut,
                        a, total);
    if (rc) return rc;
    bool mfma = rows >= MFMA_MIN_ROWS;
    gemv_geometry(total, a.K, pair, rows, a.TPW, a.KS);
    a.hmax_out = ex.hmax_out;
    a.hr = ex.hr;
    a.hmax = ex.hmax;
    a.hmax_n = ex.hmax_n;
    a.xp_x = ex.xp_x;
    a.xp_nw = ex.xp_nw;
    a.xp_eps = ex.xp_eps;
    a.gn_y = ex.gn_y;
    a.gn_z = ex.gn_z;
    a.gn_w = ex.gn_w;
    a.gn_eps = ex.gn_eps;
    a.gn_out = ex.gn_out;
    a.gn_gated = ex.gn_gated;
    const int wgs = (total + a.TPW - 1) / a.TPW;
    const int esz = esz_of(ws[0]->s_dtype);
    if (ex.gdn) {
        MDX_CHECK(nm == 2 && !pair && epi == EPI_STORE && out_dt == MDX_DT_BF16 && !res && rows <= ex.gdn->slots,
                  "Gated-DeltaNet projection: matrices qkv, z, bf16 outputs, no residual, rows <= slots");
        // the epilogue's stage and control words fit the activation region
        MDX_CHECK(((a.TPW * 16 * rows * 2 + 15) & ~15) + 4 * (2 + 3 * ex.gdn->slots) <= rows * a.K,
                  "Gated-DeltaNet projection stage");
        a.gf = *ex.gdn;
        a.gf.on = 1;
        a.gf.units = wgs;
        const int nw = a.TPW * a.KS;
        a.gf.nside = (rows * a.gf.HV + nw - 1) / nw;
    }
    MDX_CHECK(gemv_smem(a, mfma, esz) <= 160 * 1024, "activation of %d rows x K=%d exceeds LDS", rows, a.K);
    // per-weight decode tables in LDS when the scales are not asserted integral, a group spans a chunk
    // and the larger footprint still holds the grid's work-groups per CU (else fewer resident: at 8
    // rows the gate/up pair would drop from three work-groups per CU to two and lose more than the
    // tables save; there the lanes build their tables in the loop). Tables select the table-only
    // variants, which run on the MFMA kernel at every row count (at one row too: the products leave
    // the VALU to the decode).
    if (!a.assume_int && a.lgG >= 7) {
        const int per_cu = (wgs + 255) / 256;
        // 16-byte tables, with the split-K partials in the table region when that makes them fit (int8 rows,
        // a table region at least the partials' size); else (default codebook) 8-byte ones
        const size_t red_bytes = size_t(a.TPW) * a.KS * 64 * 4 * 4;
        const int ngr = (a.K >> a.lgG);
        const char* te = getenv("MDX_GEMV_TBL");  // MDX_GEMV_TBL=8: the 8-byte tier whenever it applies (tests)
        for (int tb = te && atoi(te) == 8 && !a.cb ? 2 : 1; tb <= 2; ++tb) {
            if (tb == 2 && a.cb) break;
            a.tbl = tb;
            if (int64_t(per_cu) * gemv_smem(a, true, esz) <= 160 * 1024) break;
            if (tb == 1 && !ex.hr && !ex.xp_x && !ex.gn_y && size_t(a.TPW) * 16 * ngr * 16 >= red_bytes) {
                a.red_alias = 1;
                if (int64_t(per_cu) * gemv_smem(a, true, esz) <= 160 * 1024) break;
                a.red_alias = 0;
            }
            a.tbl = 0;
        }
        if (a.tbl) mfma = true;
    }
    MDX_CHECK(!(mfma && a.xp_x) || a.tbl, "row-prep GEMV geometry (one row takes the VALU kernel or the tables)");
    // per-wave one-shots: one int8 row, caller-asserted integral scales with the default codebook,
    // G128, 16-byte runs of scales per slice and per row (MDX_GEMV_PWO=0 turns them off)
    const char* pe = getenv("MDX_GEMV_PWO");
    const int NCk = a.K / CHUNK_K;
    a.pwo = !mfma && rows == 1 && a.assume_int && !a.cb && a.lgG == 7 &&
            (NCk / a.KS) * esz % 16 == 0 && (a.K >> 7) * esz % 16 == 0 && aligned(xq, 16) && !(pe && atoi(pe) == 0);
    return launch_gemv_d<4>(a, ws[0]->s_dtype, mfma, wgs, st);
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

int prep_checks(int64_t rows, int64_t K, int32_t rot, const void* h, const void* x = nullptr, const void* q = nullptr,
                const void* nw = nullptr, const void* xn = nullptr) {
    MDX_CHECK(rows >= 0, "rows must be >= 0");
    MDX_CHECK(aligned(x, 8) && aligned(nw, 8) && aligned(xn, 8) && aligned(q, 4),
              "rows must be 8-byte aligned (int8 rows 4-byte aligned)");
    MDX_CHECK(K > 0 && K % 256 == 0 && K <= MAX_PREP_K, "K must be a multiple of 256 and <= 16384 (got %lld)",
              (long long)K);
    MDX_CHECK(rot == MDX_ROT_NONE || rot == MDX_ROT_H256 || (rot == MDX_ROT_MATRIX && h), "rotation");
    MDX_CHECK(rot != MDX_ROT_MATRIX || aligned(h, 8), "rotation matrix must be 8-byte aligned");
    MDX_CHECK(rows <= 65535, "rows must be <= 65535");
    return MDX_OK;
}

}  // namespace
}  // namespace mdx

using namespace mdx;

extern "C" int32_t mdx_gemv_trace(int32_t* out, int32_t max_records) {
    const int n = g_trace_n;
    for (int i = 0; i < n && i < max_records; ++i)
        for (int j = 0; j < 7; ++j) out[7 * i + j] = g_trace[i][j];
    g_trace_n = 0;
    return n;
}

extern "C" int mdx_w4a8_decode_linear(const int8_t* x, const float* x_scale, const mdx_w4* w, const void* residual,
                                      void* out, int32_t out_dtype, int64_t rows, void* stream) {
    MDX_CHECK(x && x_scale && out, "null pointer");
    MDX_CHECK(out_dtype == MDX_DT_F32 || out_dtype == MDX_DT_BF16, "out dtype must be f32 or bf16");
    const mdx_w4* ws[1] = {w};
    void* outs[1] = {out};
    const void* res[1] = {residual};
    return run_gemv(ws, 1, false, x, x_scale, int(rows), EPI_STORE, outs, res, out_dtype, nullptr,
                    static_cast<hipStream_t>(stream));
}

extern "C" int mdx_rot_quant(const uint16_t* x, const uint16_t* h, int32_t rot, int8_t* q, float* scale, int64_t rows,
                             int64_t K, void* stream) {
    MDX_CHECK(x && q && scale, "null pointer");
    int rc = prep_checks(rows, K, rot, h, x, q);
    if (rc) return rc;
    if (rows == 0) return MDX_OK;
    PrepArgs a{x, nullptr, 0.f, nullptr, h, rot, q, scale, int(K)};
    return launch_prep(a, rows, static_cast<hipStream_t>(stream));
}

extern "C" int mdx_rms_rot_quant(const uint16_t* x, const uint16_t* norm_w, float eps, uint16_t* xn_out,
                                 const uint16_t* h, int32_t rot, int8_t* q, float* scale, int64_t rows, int64_t K,
                                 void* stream) {
    MDX_CHECK(x && q && scale && norm_w, "null pointer");
    int rc = prep_checks(rows, K, rot, h, x, q, norm_w, xn_out);
    if (rc) return rc;
    if (rows == 0) return MDX_OK;
    PrepArgs a{x, norm_w, eps, xn_out, h, rot, q, scale, int(K)};
    return launch_prep(a, rows, static_cast<hipStream_t>(stream));
}

extern "C" int mdx_gate_rot_quant(const uint16_t* y, const uint16_t* gate, int64_t gate_row_stride, int64_t gate_head,
                                  int64_t gate_head_stride, int64_t gate_offset, const uint16_t* sig_lut,
                                  const uint16_t* h, int32_t rot, int8_t* q, float* scale, int64_t rows, int64_t K,
                                  void* stream) {
    MDX_CHECK(y && gate && sig_lut && q && scale, "null pointer");
    int rc = prep_checks(rows, K, rot, h, y, q);
    if (rc) return rc;
    MDX_CHECK(gate_head >= 8 && gate_head % 8 == 0 && K % gate_head == 0 && gate_head_stride % 8 == 0 &&
                  gate_offset % 8 == 0 && gate_row_stride % 8 == 0 && aligned(gate, 16),
              "gate rows: 16-byte aligned runs of whole heads");
    if (rows == 0) return MDX_OK;
    PrepArgs a{y, nullptr, 0.f, nullptr, h, rot, q, scale, int(K)};
    a.gate = gate;
    a.sig = sig_lut;
    a.g_row = gate_row_stride;
    a.g_head = int(gate_head);
    a.g_hstride = int(gate_head_stride);
    a.g_off = int(gate_offset);
    return launch_prep(a, rows, static_cast<hipStream_t>(stream));
}

extern "C" int mdx_gnorm_rot_quant(const uint16_t* y, const uint16_t* z, const uint16_t* gnorm_w, float eps,
                                   uint16_t* y_out, const uint16_t* h, int32_t rot, int8_t* q, float* scale, int64_t rows,
                                   int64_t K, void* stream) {
    MDX_CHECK(y && z && gnorm_w, "null pointer");
    MDX_CHECK((q && scale) || (!q && !scale && y_out && rot == MDX_ROT_NONE), "q and scale, or y_out only");
    int rc = prep_checks(rows, K, rot, h, y, q, nullptr, y_out);
    if (rc) return rc;
    MDX_CHECK(aligned(z, 8) && aligned(gnorm_w, 8), "8-byte aligned z / gnorm_w");
    if (rows == 0) return MDX_OK;
    PrepArgs a{y, nullptr, 0.f, y_out, h, rot, q, scale, int(K)};
    a.hw = gnorm_w;
    a.hz = z;
    a.heps = eps;
    return launch_prep(a, rows, static_cast<hipStream_t>(stream));
}

extern "C" int mdx_gnorm_linear(const uint16_t* y, const uint16_t* z, int32_t z_gated, const uint16_t* gnorm_w,
                                float eps, uint16_t* y_out, const mdx_w4* w, const uint16_t* residual, uint16_t* out,
                                int8_t* q, float* scale, int64_t rows, void* stream) {
    MDX_CHECK(y && z && gnorm_w && w && out, "null pointer");
    int rc = check_w4(w, "weight");
    if (rc) return rc;
    const int64_t K = w->k;
    MDX_CHECK(rows >= 1 && rows <= 16, "rows must be in 1..16");
    MDX_CHECK(K % 256 == 0 && aligned(y, 8) && aligned(z, 8) && aligned(gnorm_w, 8) && aligned(y_out, 8),
              "K % 256 == 0, 8-byte aligned rows");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    void* outs[1] = {out};
    const void* res[1] = {residual};
    const mdx_w4* ws[1] = {w};
    const bool overlap = y_out && y_out < y + rows * K && y < y_out + rows * K;
    if (!overlap && gemv_gn_fits(w, int(rows))) {  // one launch
        GemvExtra ex;
        ex.gn_y = y;
        ex.gn_z = z;
        ex.gn_w = gnorm_w;
        ex.gn_eps = eps;
        ex.gn_out = y_out;
        ex.gn_gated = z_gated != 0;
        return run_gemv(ws, 1, false, nullptr, nullptr, int(rows), EPI_STORE, outs, res, MDX_DT_BF16, nullptr, st, ex);
    }
    MDX_CHECK(q && scale && aligned(q, 16), "q / scale: the activation of this shape is quantised by its own launch");
    if ((rc = prep_checks(rows, K, MDX_ROT_NONE, nullptr, y, q, nullptr, y_out))) return rc;
    PrepArgs pa{y, nullptr, 0.f, y_out, nullptr, MDX_ROT_NONE, q, scale, int(K)};
    pa.hw = gnorm_w;
    pa.hz = z;
    pa.heps = eps;
    pa.hz_gated = z_gated != 0;
    if ((rc = launch_prep(pa, rows, st))) return rc;
    return run_gemv(ws, 1, false, q, scale, int(rows), EPI_STORE, outs, res, MDX_DT_BF16, nullptr, st);
}

extern "C" int mdx_rmsnorm(const uint16_t* x, const uint16_t* norm_w, float eps, uint16_t* out, int64_t rows, int64_t K,
                           void* stream) {
    MDX_CHECK(x && norm_w && out, "null pointer");
    MDX_CHECK(rows >= 0 && rows <= 65535 && K % 256 == 0 && K >= 256 && K <= MAX_PREP_K,
              "rows / K (K % 256 == 0, K <= %d)", MAX_PREP_K);
    MDX_CHECK(aligned(x, 16) && aligned(norm_w, 16) && aligned(out, 16), "16-byte aligned rows");
    if (rows == 0) return MDX_OK;
    PrepArgs a{x, norm_w, eps, out, nullptr, MDX_ROT_NONE, nullptr, nullptr, int(K)};
    return launch_prep(a, rows, static_cast<hipStream_t>(stream));
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* g, const uint16_t* u, const uint16_t* lut,
                                                       uint16_t* out, int64_t n) {
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += int64_t(gridDim.x) * 256)
        out[i] = f2bf(__fmul_rn(bf2f(lut[g[i]]), bf2f(u[i])));
}

extern "C" int mdx_silu_mul(const uint16_t* g, const uint16_t* u, const uint16_t* silu_lut, uint16_t* out, int64_t n,
                            void* stream) {
    MDX_CHECK(g && u && silu_lut && out && n >= 0, "null pointer / size");
    if (n == 0) return MDX_OK;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 1024);
    hipLaunchKernelGGL(silu_mul_kernel, dim3(unsigned(blocks)), dim3(256), 0, static_cast<hipStream_t>(stream), g, u,
                       silu_lut, out, n);
    MDX_LAUNCHED();
    return MDX_OK;
}

namespace mdx {
namespace {

// Workspace of mdx_mono_mlp (256-byte aligned pieces): a 4 KiB header whose word MLP_ERR is the error
// word (no launch of this library waits on another work-group, so it stays zero), then the gate/up
// work-groups' |h| maxima [16][N1 / 16] (fp32 bits, row-major), q1 [rows, K1] int8 | q2 [rows, N1]
// int8 | scales [64] f32 | h [rows, N1] bf16 | rotated h [rows, N1] bf16.
constexpr size_t MLP_HDR = 4096;
constexpr size_t MLP_ERR = 4;

struct MlpWs {
    uint32_t* hmax;  // [rows][N1 / 16] the gate/up work-groups' |h| maxima, row-major
    int8_t* q1;
    int8_t* q2;
    float* s;
    uint16_t* hb;
    uint16_t* hr;
    size_t bytes;
};

MlpWs mlp_ws(void* base, int64_t rows, int64_t K1, int64_t N1) {
    MlpWs w{};
    uint8_t* p = static_cast<uint8_t*>(base);
    size_t off = 0;
    auto take = [&](size_t bytes) {
        uint8_t* q = p ? p + off : nullptr;
        off += align256(bytes);
        return q;
    };
    take(MLP_HDR);
    w.hmax = reinterpret_cast<uint32_t*>(take(size_t(N1 / 16) * 16 * 4));
    w.q1 = reinterpret_cast<int8_t*>(take(size_t(rows) * K1));
    w.q2 = reinterpret_cast<int8_t*>(take(size_t(rows) * N1));
    w.s = reinterpret_cast<float*>(take(64 * 4));
    w.hb = reinterpret_cast<uint16_t*>(take(size_t(rows) * N1 * 2));
    w.hr = reinterpret_cast<uint16_t*>(take(size_t(rows) * N1 * 2));
    w.bytes = off;
    return w;
}

}  // namespace
}  // namespace mdx

extern "C" size_t mdx_mono_mlp_workspace(int64_t rows, int64_t K1, int64_t N1) {
    return mdx::mlp_ws(nullptr, rows, K1, N1).bytes;
}

extern "C" size_t mdx_mono_mlp_error_offset(void) { return 4 * mdx::MLP_ERR; }

extern "C" int mdx_mono_mlp(const uint16_t* xn, const uint16_t* norm_w, float eps, const uint16_t* h, int32_t rot,
                            const uint16_t* silu_lut, const mdx_w4* gate, const mdx_w4* up, const mdx_w4* down,
                            const uint16_t* residual, uint16_t* out, int64_t rows, void* workspace,
                            size_t workspace_bytes, void* stream) {
    MDX_CHECK(xn && silu_lut && gate && up && down && out && workspace, "null pointer");
    MDX_CHECK(rows >= 1 && rows <= 16, "rows must be in 1..16");
    const int64_t K1 = gate->k, N1 = gate->n;
    MDX_CHECK(up->n == N1 && up->k == K1 && down->k == N1 && down->n == K1, "gate/up [N1, K1], down [K1, N1] shapes");
    int rc = prep_checks(rows, K1, rot, h, xn, nullptr, norm_w);
    if (rc) return rc;
    if ((rc = prep_checks(rows, N1, rot, h))) return rc;
    MDX_CHECK(workspace_bytes >= mdx_mono_mlp_workspace(rows, K1, N1), "workspace too small");
    MDX_CHECK(aligned(workspace, 256), "workspace must be 256-byte aligned");
    MDX_CHECK(aligned(out, 4) && aligned(residual, 4), "out / residual must be 4-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    const MlpWs w = mlp_ws(workspace, rows, K1, N1);
    // Without a rotation, h needs no row prep launch: gate/up raises the rows' |h| slot maxima and
    // the down GEMV quantises h in its prologue (the same scale and codes as the row prep), when
    // its geometry holds the rows (MDX_MLP_HPREP=1 forces the prep launch).
    const char* hp = getenv("MDX_MLP_HPREP");
    const bool hr = rot == MDX_ROT_NONE && N1 % 64 == 0 && gemv_hr_fits(down, int(rows)) && !(hp && atoi(hp) != 0);
    const mdx_w4* gu[2] = {gate, up};
    // one row: the gate/up GEMV prepares x itself (no row prep launch); MDX_MLP_HPREP=1 keeps both
    // prep launches
    const char* xpe = getenv("MDX_MLP_XPREP");  // MDX_MLP_XPREP=1: the x prep launch at one row too (A/B)
    const bool xp = hr && rows == 1 && gemv_xp_fits(gu, 2, true) && aligned(xn, 16) &&
                    (!norm_w || aligned(norm_w, 16)) &&  // (the row and its weights are DMA'd in 16-byte pieces)
                    !(xpe && atoi(xpe) != 0);
    if (!xp) {
        PrepArgs pa{xn, norm_w, eps, nullptr, h, rot, w.q1, w.s, int(K1)};
        if ((rc = launch_prep(pa, rows, st))) return rc;
    }
    // gate/up, [prep of h], down
    void* o1[2] = {w.hb, w.hb};
    GemvExtra e1;
    if (hr) e1.hmax_out = w.hmax;
    if (xp) {
        e1.xp_x = xn;
        e1.xp_nw = norm_w;
        e1.xp_eps = eps;
    }
    if ((rc = run_gemv(gu, 2, true, w.q1, w.s, int(rows), EPI_SILU, o1, nullptr, MDX_DT_BF16, silu_lut, st, e1)))
        return rc;
    const mdx_w4* dn[1] = {down};
    void* o2[1] = {out};
    const void* r2[1] = {residual};
    if (hr) {
        GemvExtra e2;
        e2.hr = w.hb;
        e2.hmax = w.hmax;
        e2.hmax_n = int(N1 / 16);
        return run_gemv(dn, 1, false, nullptr, nullptr, int(rows), EPI_STORE, o2, r2, MDX_DT_BF16, nullptr, st, e2);
    }
    PrepArgs pb{w.hb, nullptr, 0.f, nullptr, h, rot, w.q2, w.s + 32, int(N1)};
    if ((rc = launch_prep(pb, rows, st))) return rc;
    return run_gemv(dn, 1, false, w.q2, w.s + 32, int(rows), EPI_STORE, o2, r2, MDX_DT_BF16, nullptr, st);
}

extern "C" int mdx_stream_gemv(const int8_t* x, const float* x_scale, const mdx_w4* const* mats, int32_t nmats,
                               int32_t gate_up, void* const* outs, const void* const* residuals, int32_t out_dtype,
                               const uint16_t* silu_lut, int64_t rows, void* stream) {
    MDX_CHECK(x && x_scale && mats && outs, "null pointer");
    MDX_CHECK(nmats >= 1 && nmats <= 3, "1..3 matrices");
    MDX_CHECK(out_dtype == MDX_DT_F32 || out_dtype == MDX_DT_BF16, "out dtype must be f32 or bf16");
    if (gate_up) MDX_CHECK(nmats == 2 && silu_lut && out_dtype == MDX_DT_BF16, "gate/up needs 2 matrices, bf16 out, a SiLU table");
    return run_gemv(mats, nmats, gate_up != 0, x, x_scale, int(rows), gate_up ? EPI_SILU : EPI_STORE, outs, residuals,
                    out_dtype, silu_lut, static_cast<hipStream_t>(stream));
}

extern "C" int mdx_gdn_proj(const int8_t* x, const float* x_scale, const mdx_w4* w_qkv, const mdx_w4* w_z, uint16_t* proj,
                            uint16_t* z, const uint16_t* xn, const uint16_t* wa, const uint16_t* wb,
                            const uint16_t* conv_w, uint16_t* conv_state, uint16_t* proj_buf, uint16_t* qkv_buf,
                            const int32_t* ctl, const float* dt_bias, const float* g_decay, float* gates,
                            uint16_t* z_gate, const uint16_t* x_row, const uint16_t* norm_w, float eps, int64_t rows,
                            int64_t HK, int64_t HV, int64_t slots, void* stream) {
    MDX_CHECK(((x && x_scale && xn) || (x_row && norm_w)) && w_qkv && w_z && proj && z && wa && wb && conv_w &&
                  conv_state && proj_buf && qkv_buf && ctl && dt_bias && g_decay && gates,
              "null pointer");
    MDX_CHECK(slots == 8 || slots == 16, "slots must be 8 or 16");
    MDX_CHECK(rows >= 1 && rows <= slots, "1 <= rows <= slots");
    MDX_CHECK(HK >= 1 && HV >= HK && HV % HK == 0 && HV % 2 == 0 && HV <= 128, "heads (HV even, <= 128)");
    MDX_CHECK(w_qkv->n == (2 * HK + HV) * GDN_DH && w_z->n == HV * GDN_DH, "qkv: N = (2 HK + HV) 128; z: N = HV 128");
    const int64_t K = w_qkv->k;
    MDX_CHECK(K >= 512 && K <= 4096 && K % 512 == 0 && aligned(xn, 16) && aligned(wa, 16) && aligned(wb, 16),
              "a / b input: K % 512 == 0, K <= 4096, 16-byte aligned rows");
    GdnFold f{};
    f.conv_w = conv_w;
    f.conv_state = conv_state;
    f.pb = proj_buf;
    f.qb = qkv_buf;
    f.ctl = ctl;
    f.xn = xn;
    f.wa = wa;
    f.wb = wb;
    f.dt_bias = dt_bias;
    f.g_decay = g_decay;
    f.gates = gates;
    f.zg = z_gate;
    f.HV = int(HV);
    f.slots = int(slots);
    GemvExtra ex;
    ex.gdn = &f;
    const mdx_w4* mats[2] = {w_qkv, w_z};
    void* outs[2] = {proj, z};
    if (x_row) {  // one bf16 row, its RMSNorm + quantisation in the launch
        MDX_CHECK(rows == 1 && w_qkv->s_dtype == MDX_DT_F16 && aligned(x_row, 16) && aligned(norm_w, 16) &&
                      gemv_xp_fits(mats, 2, false),
                  "a bf16 row: one row, fp16 scales, 16-byte aligned x_row / norm_w");
        ex.xp_x = x_row;
        ex.xp_nw = norm_w;
        ex.xp_eps = eps;
    }
    return run_gemv(mats, 2, false, x, x_scale, int(rows), EPI_STORE, outs, nullptr, MDX_DT_BF16, nullptr,
                    static_cast<hipStream_t>(stream), ex);
}
