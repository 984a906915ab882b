// W4A8 decode GEMV engine, row activation prep (norm / rotate / quantise) and the fused MLP.
//
// Reference semantics (comfy-mono-decode-xpu):
//   w4a8_decode_linear  csrc/w4a8_decode.sycl:4-11, 33-45, 139-166
//   rot_quant           csrc/act_prep.sycl:4-10, 70-91
//   mono_mlp            csrc/mono_mlp.sycl:109-167
//
// Scales are always the row-major [N, K/G] array (both layouts); a work-group stages its tiles'
// scale rows in LDS once. Weight stream. A wave owns one 16-column tile and a K slice. Its unit of work is a "chunk":
// 16 columns x 128 k = 1 KiB of codes, fetched with ONE 16-byte load per lane (lane l: column
// l % 16, quarter kq = l / 16 of the chunk, 32 consecutive k). In the tile-major layout the 64
// lanes' 16-byte pieces are adjacent, so every chunk is one contiguous 1 KiB burst; in the
// checkpoint (row-major) layout they are 16 pieces of 64 B. Lane l's dword j holds the codes of
// k = chunk + 32 kq + 8 j + [0, 8): low nibbles are the even k, high nibbles the odd k. All
// per-chunk address math is 32-bit pointer increments; group indices are shifts (G is a power
// of two).
//
// Activation. The int8 activation rows are staged in LDS with every 8-byte block de-interleaved
// ([x0 x2 x4 x6 | x1 x3 x5 x7]) so the low / high nibble words of a code dword line up with two
// activation words: no per-weight shuffles.
//
// Decode. Per-weight form: a 16-entry int8 table per (lane, scale) is built with the reference
// formula w8 = clamp(rint(cb[c] * s), +-127) (NaN -> 0), and codes are mapped through it with
// v_perm_b32 byte selects. Integral form, chosen per chunk under MDX_DECODE_AUTO when the
// codebook is c - 8 and every lane's scale of the chunk is an integer in [-15, 15] (a wave-uniform
// choice): then w8 = (c - 8) * s exactly, so sum_k x * w8 = s * (sum_k x * c - 8 sum_k x): the
// raw nibbles (0..15) feed the dot directly and 8 * sum_k x is precomputed per 32-k block of the
// activation. Both forms give the same int32 accumulator (mod 2^32) as the reference, so they
// can be mixed chunk by chunk.
//
// Products. Rows <= 2: v_dot4_i32_i8 on the VALU. Rows 3..16: v_mfma_i32_16x16x32_i8 with the
// activation rows as A (rows past the last are zero) and the decoded tile as B; lane l's dword j
// of codes is exactly its B fragment for the j-th MFMA of the chunk.
//
// Split-K partial sums of the waves of a work-group are int32 and are added through LDS:
// integer addition is associative, so every split gives the same bits.
#include <algorithm>
#include <stdio.h>
#include <stdlib.h>

#include "mdx_common.hpp"

namespace mdx {
namespace {

constexpr int WAVE = 64;
constexpr int CHUNK_K = 128;
constexpr int PREP_THREADS = 256;
constexpr int MAX_PREP_K = 16384;
constexpr int PREP_BLK = MAX_PREP_K / 8 / PREP_THREADS;  // 8-element blocks per thread at most

typedef int v4i __attribute__((ext_vector_type(4)));

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

// streamed-once weights: a non-temporal 16-byte load (does not displace reused data in L2)
__device__ __forceinline__ uint4 ldg_stream(const void* p) {
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// =================================================================================================
// Row prep: [RMSNorm] -> [rotation] -> absmax -> int8 quantisation. One work-group per row.
// Thread t owns the 8-element blocks b = t + 256 j (elements 8 b .. 8 b + 7), held in registers.
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
};

__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = __uint_as_float(w[i] << 16);
        f[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
    }
}

// Block sum of 256 per-thread partials in the canonical tree (p[t] + p[t + 128], + 64, ..., + 1)
__device__ float tree256(float p, float* red) {
    const int t = threadIdx.x;
    red[t] = p;
    __syncthreads();
    if (t < 128) red[t] = __fadd_rn(red[t], red[t + 128]);
    __syncthreads();
    float v = 0.f;
    if (t < 64) {
        v = __fadd_rn(red[t], red[t + 64]);
        for (int s = 32; s >= 1; s >>= 1) v = __fadd_rn(v, shfl_down(v, s));
        if (t == 0) red[300] = v;
    }
    __syncthreads();
    const float r = red[300];
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(PREP_THREADS) void prep_rows_kernel(PrepArgs a) {
    extern __shared__ float smem[];
    float* red = smem;                                   // [320]
    double* grp = reinterpret_cast<double*>(smem + 320);  // [4][256] fp64 butterflies
    float* xr = reinterpret_cast<float*>(grp + 4 * 256);  // [K] (rotation only)
    const int t = threadIdx.x;
    const int row = blockIdx.x, K = a.K, nb = K / 8;
    const uint16_t* x = a.x + int64_t(row) * K;
    float v[PREP_BLK][8];
    uint4 raw[PREP_BLK];
#pragma unroll
    for (int j = 0; j < PREP_BLK; ++j) {
        const int b = t + PREP_THREADS * j;
        if (b < nb) raw[j] = *reinterpret_cast<const uint4*>(x + 8 * b);
    }
#pragma unroll
    for (int j = 0; j < PREP_BLK; ++j) {
        const int b = t + PREP_THREADS * j;
        if (b < nb) unpack8(raw[j], v[j]);
    }
    if (a.gate) {
#pragma unroll
        for (int j = 0; j < PREP_BLK; ++j) {
            const int b = t + PREP_THREADS * j;
            if (b < nb) {
                const int i0 = 8 * b;
                const uint16_t* gp = a.gate + row * a.g_row + (i0 / a.g_head) * a.g_hstride + a.g_off + i0 % a.g_head;
                const uint4 gv = *reinterpret_cast<const uint4*>(gp);
                const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const uint16_t gb = uint16_t(gw[e >> 1] >> (16 * (e & 1)));
                    v[j][e] = bfround(__fmul_rn(v[j][e], bf2f(a.sig[gb])));
                }
            }
        }
    }
    if (a.nw) {
        // canonical RMSNorm: thread t's partial sums its own elements in increasing order
        float p = 0.f;
        bool first = true;
#pragma unroll
        for (int j = 0; j < PREP_BLK; ++j) {
            const int b = t + PREP_THREADS * j;
            if (b < nb)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float sq = __fmul_rn(v[j][e], v[j][e]);
                    p = first ? sq : __fadd_rn(p, sq);
                    first = false;
                }
        }
        const float ss = tree256(p, red);
        const float mean = __fdiv_rn(ss, float(K));
        const float r = __fdiv_rn(1.f, sqrt_rn(__fadd_rn(mean, a.eps)));
#pragma unroll
        for (int j = 0; j < PREP_BLK; ++j) {
            const int b = t + PREP_THREADS * j;
            if (b < nb) {
                float w[8];
                unpack8(*reinterpret_cast<const uint4*>(a.nw + 8 * b), w);
                uint32_t o[4];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[j][e] = bfround(__fmul_rn(__fmul_rn(v[j][e], r), w[e]));
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = uint32_t(f2bf(v[j][2 * e])) | (uint32_t(f2bf(v[j][2 * e + 1])) << 16);
                if (a.xn_out) *reinterpret_cast<uint4*>(a.xn_out + int64_t(row) * K + 8 * b) = make_uint4(o[0], o[1], o[2], o[3]);
            }
        }
    }
    if (!a.q) return;  // RMSNorm only (xn_out)
    if (a.rot != MDX_ROT_NONE) {
#pragma unroll
        for (int j = 0; j < PREP_BLK; ++j) {
            const int b = t + PREP_THREADS * j;
            if (b < nb)
#pragma unroll
                for (int e = 0; e < 8; ++e) xr[8 * b + e] = v[j][e];
        }
        __syncthreads();
        const int groups = K / 256;
        if (a.rot == MDX_ROT_H256) {
            // fp64 fast Walsh-Hadamard transform per 256-group: radix-4 stages along the base-4
            // digits (strides 1, 4, 16, 64), butterfly out_j = sum_k a_k H4[k][j] in a fixed order,
            // then * 1/16, rounded once to fp32 and once to bf16.
            const int wave = t / WAVE, lane = t % WAVE;
            for (int g0 = 0; g0 < groups; g0 += 4) {
                const int g = g0 + wave;
                double* bb = grp + wave * 256;
                if (g < groups)
                    for (int i = lane; i < 256; i += WAVE) bb[i] = double(xr[g * 256 + i]);
                __syncthreads();
                for (int st = 1; st < 256; st *= 4) {
                    if (g < groups) {
                        const int base = (lane / st) * (4 * st) + lane % st;
                        const double a0 = bb[base], a1 = bb[base + st], a2 = bb[base + 2 * st], a3 = bb[base + 3 * st];
                        bb[base] = __dsub_rn(__dadd_rn(__dadd_rn(a0, a1), a2), a3);
                        bb[base + st] = __dadd_rn(__dsub_rn(__dadd_rn(a0, a1), a2), a3);
                        bb[base + 2 * st] = __dadd_rn(__dadd_rn(__dsub_rn(a0, a1), a2), a3);
                        bb[base + 3 * st] = __dadd_rn(__dadd_rn(__dsub_rn(a1, a0), a2), a3);
                    }
                    __syncthreads();
                }
                if (g < groups)
                    for (int i = lane; i < 256; i += WAVE) xr[g * 256 + i] = bfround(float(__dmul_rn(bb[i], 0.0625)));
                __syncthreads();
            }
        } else {
            // generic bf16 matrix: fp64 sum over k in order of exact products, then fp32, then bf16
            for (int g = 0; g < groups; ++g) {
                double acc = 0.0;
                for (int k = 0; k < 256; ++k)
                    acc = __dadd_rn(acc, __dmul_rn(double(xr[g * 256 + k]), double(bf2f(a.h[k * 256 + t]))));
                __syncthreads();
                xr[g * 256 + t] = bfround(float(acc));
                __syncthreads();
            }
        }
#pragma unroll
        for (int j = 0; j < PREP_BLK; ++j) {
            const int b = t + PREP_THREADS * j;
            if (b < nb)
#pragma unroll
                for (int e = 0; e < 8; ++e) v[j][e] = xr[8 * b + e];
        }
    }
    // absmax (exact, order-free), scale, quantise
    float m = 0.f;
#pragma unroll
    for (int j = 0; j < PREP_BLK; ++j) {
        const int b = t + PREP_THREADS * j;
        if (b < nb)
#pragma unroll
            for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(v[j][e]));
    }
    m = wave_max(m);
    if (t % WAVE == 0) red[256 + t / WAVE] = m;
    __syncthreads();
    const float rm = fmaxf(fmaxf(red[256], red[257]), fmaxf(red[258], red[259]));
    const float s = fmaxf(__fdiv_rn(rm, 127.0f), 1e-30f);
    if (t == 0) a.scale[row] = s;
    uint16_t sb = f2bf(s);
    if ((sb & 0x7FFFu) == 0) sb = 0x0080u;
    const float sbf = bf2f(sb);
#pragma unroll
    for (int j = 0; j < PREP_BLK; ++j) {
        const int b = t + PREP_THREADS * j;
        if (b < nb) {
            uint32_t o[2] = {0, 0};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float d = bfround(__fdiv_rn(v[j][e], sbf));
                const int qv = int(fminf(fmaxf(rintf(d), -128.f), 127.f));
                o[e >> 2] |= (uint32_t(qv) & 0xFFu) << (8 * (e & 3));
            }
            *reinterpret_cast<uint2*>(a.q + int64_t(row) * K + 8 * b) = make_uint2(o[0], o[1]);
        }
    }
}

size_t prep_smem(int K, int rot) { return 320 * 4 + 4 * 256 * 8 + (rot != MDX_ROT_NONE ? size_t(K) * 4 : 0); }

int launch_prep(const PrepArgs& a, int64_t rows, hipStream_t st) {
    const size_t smem = prep_smem(a.K, a.rot);
    if (smem > 64 * 1024) allow_smem(reinterpret_cast<const void*>(&prep_rows_kernel), smem);
    hipLaunchKernelGGL(prep_rows_kernel, dim3(unsigned(rows)), dim3(PREP_THREADS), smem, st, a);
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
    int xglobal;          // MFMA only: activation too large for LDS, A fragments read from global
    int force_exact;      // MDX_DECODE_EXACT: never take the integral form
    int epi;
    void* out[3];
    const void* res[3];
    int out_dt;
    const uint16_t* lut;  // EPI_SILU
};

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

// four codes (one per byte, values 0..15) -> four int8 via the 16-byte table
__device__ __forceinline__ uint32_t lut4(const Lut& L, uint32_t c) {
    const uint32_t sel = c & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(L.w[1], L.w[0], sel);
    const uint32_t hi = __builtin_amdgcn_perm(L.w[3], L.w[2], sel);
    const uint32_t pick = ((c >> 1) & 0x04040404u) | 0x03020100u;
    return __builtin_amdgcn_perm(hi, lo, pick);
}

// per-weight decode of one chunk's four code dwords (two scales: dwords 0-1 and 2-3)
__device__ __forceinline__ void decode_exact(const uint32_t* wd, float s0, float s1, const float* cb, uint32_t* lo,
                                             uint32_t* hi) {
    const Lut L0 = make_lut(s0, cb);
    const Lut L1 = (__float_as_uint(s1) == __float_as_uint(s0)) ? L0 : make_lut(s1, cb);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const Lut& L = j < 2 ? L0 : L1;
        lo[j] = lut4(L, wd[j] & 0x0F0F0F0Fu);
        hi[j] = lut4(L, (wd[j] >> 4) & 0x0F0F0F0Fu);
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
__device__ __forceinline__ void store_out(const GemvArgs& a, int mi, int n, int r, int32_t acc, float xs, float sc) {
    const MatArg& m = a.m[mi];
    const float f = scaleback(acc, xs, sc);
    const int o = r * m.n + n;
    if (a.out_dt == MDX_DT_BF16) {
        uint16_t v = f2bf(f);
        if (a.res[mi]) v = f2bf(__fadd_rn(bf2f(reinterpret_cast<const uint16_t*>(a.res[mi])[o]), bf2f(v)));
        reinterpret_cast<uint16_t*>(a.out[mi])[o] = v;
    } else {
        float v = f;
        if (a.res[mi]) v = __fadd_rn(reinterpret_cast<const float*>(a.res[mi])[o], v);
        reinterpret_cast<float*>(a.out[mi])[o] = v;
    }
}

__device__ __forceinline__ void store_silu(const GemvArgs& a, int n, int r, int32_t ag, int32_t au, float xs, float scg,
                                           float scu) {
    const uint16_t g = f2bf(scaleback(ag, xs, scg));
    const uint16_t u = f2bf(scaleback(au, xs, scu));
    const float act = bf2f(a.lut[g]);
    reinterpret_cast<uint16_t*>(a.out[0])[r * a.m[0].n + n] = f2bf(__fmul_rn(act, bf2f(u)));
}

// red layout: [TPW][KS][16 columns][rows] (VALU) or [TPW][KS][64 lanes][4] (MFMA); sums the slices
template <bool MFMA>
__device__ __forceinline__ int32_t reduced(const GemvArgs& a, const int32_t* red, int ts, int r, int c) {
    uint32_t s = 0;
    for (int k = 0; k < a.KS; ++k) {
        if (MFMA) s += uint32_t(red[((ts * a.KS + k) * 64 + (r >> 2) * 16 + c) * 4 + (r & 3)]);
        else s += uint32_t(red[((ts * a.KS + k) * 16 + c) * a.rows + r]);
    }
    return int32_t(s);
}

template <bool MFMA>
__device__ void epilogue(const GemvArgs& a, const int32_t* red, const float* prml) {
    const int wg = blockIdx.x;
    const int per = 16 * a.rows;
    const float* xsl = prml + a.TPW * 16;
    if (a.epi == EPI_SILU) {
        for (int e = threadIdx.x; e < per; e += blockDim.x) {
            const int r = e >> 4, c = e & 15;
            const int n = wg * 16 + c;  // pair: work-group wg owns gate tile wg and up tile wg
            store_silu(a, n, r, reduced<MFMA>(a, red, 0, r, c), reduced<MFMA>(a, red, 1, r, c), xsl[r], prml[c],
                       prml[16 + c]);
        }
        return;
    }
    for (int e = threadIdx.x; e < a.TPW * per; e += blockDim.x) {
        const int ts = e / per, rem = e - ts * per, r = rem >> 4, c = rem & 15;
        int tile;
        const int mi = which_mat(a, wg * a.TPW + ts, tile);
        if (tile >= a.m[mi].tiles) continue;
        store_out(a, mi, tile * 16 + c, r, reduced<MFMA>(a, red, ts, r, c), xsl[r], prml[ts * 16 + c]);
    }
}

// -------------------------------------------------------------------------------------------------
// the kernel
// -------------------------------------------------------------------------------------------------
// natural-order code bytes of a code dword: [c0 c1 c2 c3], [c4 c5 c6 c7] from its low / high nibbles
__device__ __forceinline__ void nat_order(uint32_t lo, uint32_t hi, uint32_t& n0, uint32_t& n1) {
    n0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
    n1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
}

#define MDX_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// Copy `bytes` (a multiple of 16) from global to LDS with direct-to-LDS loads: one wave instruction
// moves 64 x 16 contiguous bytes, no registers involved. The caller waits and barriers.
__device__ __forceinline__ void dma_to_lds(const uint8_t* src, uint8_t* dst, int bytes) {
    const int lane = threadIdx.x % WAVE, nw = blockDim.x / WAVE, w = threadIdx.x / WAVE;
    for (int off = w * 1024; off < bytes; off += nw * 1024) {
        if (off + lane * 16 < bytes)
            __builtin_amdgcn_global_load_lds(src + off + lane * 16, MDX_LDS(dst + off), 16, 0, 0);
    }
}

template <bool MFMA, int R, int SDT, int RING>
__global__ __launch_bounds__(1024) void gemv_kernel(GemvArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int ESZ = SDT == MDX_DT_F32 ? 4 : (SDT == MDX_DT_F16 ? 2 : 1);
    const int K = a.K;
    const int ng = K >> a.lgG;
    const int per_tile = 16 * ng * ESZ;
    // LDS: activation rows (natural order) | scale blocks [TPW][16][ng] | reduction | parameters
    uint8_t* xl = lds;
    uint8_t* sl = xl + ((a.rows * K + 1023) & ~1023);
    int32_t* red = reinterpret_cast<int32_t*>(sl + ((a.TPW * per_tile + 1023) & ~1023));
    float* prml = reinterpret_cast<float*>(red + (MFMA ? a.TPW * a.KS * 64 * 4 : a.TPW * a.KS * 16 * a.rows));

    const int t = threadIdx.x;
    const int wave = t / WAVE, lane = t % WAVE;
    const int ts = wave / a.KS, slice = wave - ts * a.KS;
    int tile;
    const int mi = which_mat(a, blockIdx.x * a.TPW + ts, tile);
    const MatArg& M = a.m[mi];
    const bool live = tile < M.tiles;
    const int NC = K / CHUNK_K;
    const int c0 = live ? slice * NC / a.KS : 0, c1 = live ? (slice + 1) * NC / a.KS : 0;
    const int nch = c1 - c0;
    const int c = lane & 15, kq = lane >> 4;
    const int klane = 32 * kq;
    const int lgG = a.lgG;

    // weight ring first (registers): every slot issues one load; reads past the slice repeat its
    // last chunk so the wait counts are static
    const uint8_t* wp;
    int wstride;
    if (a.layout == MDX_LAYOUT_TILE) {
        wp = M.q + (tile * NC + c0) * 1024 + lane * 16;
        wstride = 1024;
    } else {
        wp = M.q + (tile * 16 + c) * (K / 2) + c0 * 64 + kq * 16;
        wstride = 64;
    }
    const int last = nch > 0 ? nch - 1 : 0;
    uint4 buf[RING];
#pragma unroll
    for (int p = 0; p < RING; ++p) buf[p] = ldg_stream(wp + (live ? min(p, last) : 0) * wstride);

    // then the one-shot operands straight into LDS: activation rows, the tiles' scale blocks
    dma_to_lds(reinterpret_cast<const uint8_t*>(a.xq), xl, a.rows * K);
    for (int tsi = 0; tsi < a.TPW; ++tsi) {
        int tl;
        const int mm = which_mat(a, blockIdx.x * a.TPW + tsi, tl);
        const uint8_t* sb = mm == 0 ? a.m[0].s : (mm == 1 ? a.m[1].s : a.m[2].s);
        const int tiles = mm == 0 ? a.m[0].tiles : (mm == 1 ? a.m[1].tiles : a.m[2].tiles);
        if (tl < tiles) dma_to_lds(sb + tl * per_tile, sl + tsi * per_tile, per_tile);
    }
    float prm = 0.f;
    if (t < a.TPW * 16) {
        int tl;
        const int mm = which_mat(a, blockIdx.x * a.TPW + t / 16, tl);
        const float* sc = mm == 0 ? a.m[0].sch : (mm == 1 ? a.m[1].sch : a.m[2].sch);
        const int tiles = mm == 0 ? a.m[0].tiles : (mm == 1 ? a.m[1].tiles : a.m[2].tiles);
        prm = sc[(tl < tiles ? tl : 0) * 16 + (t & 15)];
    } else if (t < a.TPW * 16 + a.rows) {
        prm = a.xs[t - a.TPW * 16];
    }
    float cb[16];
    bool cbdef = true;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        cb[i] = a.cb ? a.cb[i] : float(i - 8);
        cbdef = cbdef && cb[i] == float(i - 8);
    }
    const bool can_int = !a.force_exact && cbdef && (lgG >= (MFMA ? 7 : 5));
    if (t < a.TPW * 16 + a.rows) prml[t] = prm;
    __syncthreads();
    const uint8_t* scol = sl + (ts * 16 + c) * ng * ESZ;

    if (MFMA) {
        v4i accE = {0, 0, 0, 0};        // per-weight decoded chunks: one running MFMA sum
        int32_t tot[4] = {0, 0, 0, 0};  // integral chunks: sum of s * (chunk dot - 8 sum x)
        const bool xlive = (lane & 15) < a.rows;
        const uint8_t* xrow = xl + (xlive ? (lane & 15) : 0) * K + klane;
        for (int i0 = 0; i0 < nch; i0 += RING) {
#pragma unroll
            for (int p = 0; p < RING; ++p) {
                const int i = i0 + p;
                if (i < nch) {
                    const uint4 w = buf[p];
                    buf[p] = ldg_stream(wp + min(i + RING, last) * wstride);
                    const int ch = c0 + i;
                    const int k0 = ch * CHUNK_K + klane;
                    const float s0 = rd_scale<SDT>(scol + (k0 >> lgG) * ESZ);
                    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
                    const uint4* x4 = reinterpret_cast<const uint4*>(xrow + ch * CHUNK_K);
                    const uint4 xa = x4[0], xb = x4[1];
                    uint32_t xd[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
                    if (!xlive)
#pragma unroll
                        for (int j = 0; j < 8; ++j) xd[j] = 0;
                    const bool integ = can_int && __all(s0 == rintf(s0) && fabsf(s0) <= 15.f);
                    if (integ) {
                        v4i dacc = {0, 0, 0, 0};
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            uint32_t n0, n1;
                            nat_order(wd[j] & 0x0F0F0F0Fu, (wd[j] >> 4) & 0x0F0F0F0Fu, n0, n1);
                            dacc = __builtin_amdgcn_mfma_i32_16x16x32_i8(long(uint64_t(xd[2 * j]) | (uint64_t(xd[2 * j + 1]) << 32)),
                                                                         long(uint64_t(n0) | (uint64_t(n1) << 32)), dacc, 0, 0, 0);
                        }
                        // 8 * sum of the chunk's activation per row: own 32 bytes, then the 4 quarters
                        int xsum = 0;
#pragma unroll
                        for (int j = 0; j < 8; ++j) xsum = sdot4(int(xd[j]), 0x01010101, xsum);
                        xsum += shfl_xor(xsum, 16);
                        xsum += shfl_xor(xsum, 32);
                        const int sv = int(s0);
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int corr = 8 * __shfl(xsum, kq * 4 + r, 64);
                            tot[r] += __mul24(sv, dacc[r] - corr);
                        }
                    } else {
                        uint32_t lo[4], hi[4];
                        decode_exact(wd, s0, rd_scale<SDT>(scol + ((k0 + 16) >> lgG) * ESZ), cb, lo, hi);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            uint32_t n0, n1;
                            nat_order(lo[j], hi[j], n0, n1);
                            accE = __builtin_amdgcn_mfma_i32_16x16x32_i8(long(uint64_t(xd[2 * j]) | (uint64_t(xd[2 * j + 1]) << 32)),
                                                                         long(uint64_t(n0) | (uint64_t(n1) << 32)), accE, 0, 0, 0);
                        }
                    }
                }
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
                if (i < nch) {
                    const uint4 w = buf[p];
                    buf[p] = ldg_stream(wp + min(i + RING, last) * wstride);
                    const int ch = c0 + i;
                    const int k0 = ch * CHUNK_K + klane;
                    const float s0 = rd_scale<SDT>(scol + (k0 >> lgG) * ESZ);
                    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
                    uint32_t nat[8];
                    const bool integ = can_int && __all(s0 == rintf(s0) && fabsf(s0) <= 15.f);
                    if (integ) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) nat_order(wd[j] & 0x0F0F0F0Fu, (wd[j] >> 4) & 0x0F0F0F0Fu, nat[2 * j], nat[2 * j + 1]);
                    } else {
                        uint32_t lo[4], hi[4];
                        decode_exact(wd, s0, rd_scale<SDT>(scol + ((k0 + 16) >> lgG) * ESZ), cb, lo, hi);
#pragma unroll
                        for (int j = 0; j < 4; ++j) nat_order(lo[j], hi[j], nat[2 * j], nat[2 * j + 1]);
                    }
                    const int sv = integ ? int(s0) : 1;
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        if (r < a.rows) {
                            const uint4* x4 = reinterpret_cast<const uint4*>(xl + r * K + ch * CHUNK_K + klane);
                            const uint4 xa = x4[0], xb = x4[1];
                            const uint32_t xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
                            int d = 0, xsum = 0;
#pragma unroll
                            for (int j = 0; j < 8; ++j) d = sdot4(int(nat[j]), int(xv[j]), d);
                            if (integ) {
#pragma unroll
                                for (int j = 0; j < 8; ++j) xsum = sdot4(int(xv[j]), 0x01010101, xsum);
                            }
                            tot[r] += __mul24(sv, d - 8 * xsum);
                        }
                    }
                }
            }
        }
        // fold the four k quarters of each column (lanes c, c + 16, c + 32, c + 48)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            int v = tot[r];
            v += shfl_xor(v, 16);
            v += shfl_xor(v, 32);
            tot[r] = v;
        }
        if (lane < 16)
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (r < a.rows) red[((ts * a.KS + slice) * 16 + lane) * a.rows + r] = tot[r];
    }
    __syncthreads();
    epilogue<MFMA>(a, red, prml);
}

size_t gemv_smem(const GemvArgs& a, bool mfma, int esz) {
    const size_t per_tile = size_t(16) * (a.K >> a.lgG) * esz;
    size_t s = ((size_t(a.rows) * a.K + 1023) & ~size_t(1023)) + ((a.TPW * per_tile + 1023) & ~size_t(1023));
    s += mfma ? size_t(a.TPW) * a.KS * 64 * 4 * 4 : size_t(a.TPW) * a.KS * 16 * a.rows * 4;
    return s + 64 * 4;
}

int esz_of(int sdt) { return sdt == MDX_DT_F32 ? 4 : (sdt == MDX_DT_F16 ? 2 : 1); }

template <bool MFMA, int R, int SDT, int RING>
int launch_gemv_t(const GemvArgs& a, int wgs, hipStream_t st) {
    const size_t smem = gemv_smem(a, MFMA, esz_of(SDT));
    const void* fn = reinterpret_cast<const void*>(&gemv_kernel<MFMA, R, SDT, RING>);
    if (smem > 64 * 1024) allow_smem(fn, smem);
    const int threads = a.TPW * a.KS * WAVE;
    hipLaunchKernelGGL((gemv_kernel<MFMA, R, SDT, RING>), dim3(unsigned(wgs)), dim3(unsigned(threads)), smem, st, a);
    MDX_LAUNCHED();
    return MDX_OK;
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
    MDX_CHECK(w->decode == MDX_DECODE_EXACT || w->decode == MDX_DECODE_AUTO, "%s: unknown decode mode", what);
    MDX_CHECK(aligned(w->q, 16), "%s: codes must be 16-byte aligned", what);
    MDX_CHECK(w->n * w->k / 2 < (int64_t(1) << 31), "%s: weight larger than 2 GiB", what);
    return MDX_OK;
}

// one GEMV launch over up to three matrices sharing K (or a gate/up pair)
int run_gemv(const mdx_w4* const* ws, int nm, bool pair, const int8_t* xq, const float* xs, int rows, int epi,
             void* const* outs, const void* const* res, int out_dt, const uint16_t* lut, hipStream_t st) {
    MDX_CHECK(rows >= 1 && rows <= 16, "rows must be in 1..16 (got %d)", rows);
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
    MDX_CHECK(aligned(xq, 16), "x must be 16-byte aligned");
    const mdx_w4& w0 = *ws[0];
    for (int i = 0; i < nm; ++i) {
        int rc = check_w4(ws[i], "weight");
        if (rc) return rc;
        MDX_CHECK(ws[i]->k == w0.k && ws[i]->group_size == w0.group_size && ws[i]->s_dtype == w0.s_dtype &&
                      ws[i]->layout == w0.layout && ws[i]->decode == w0.decode,
                  "fused matrices must share K, group size, scale dtype, layout and decode mode");
        MDX_CHECK(ws[i]->codebook == w0.codebook, "fused matrices must share one codebook");
    }
    if (pair) MDX_CHECK(nm == 2 && ws[0]->n == ws[1]->n, "gate/up must have the same N");
    GemvArgs a{};
    a.nm = nm;
    a.pair = pair ? 1 : 0;
    int total = 0;
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
    const bool mfma = rows >= MFMA_MIN_ROWS;
    // geometry: TPW tiles per work-group, KS K-slices per tile (at most 16 waves per work-group):
    // the smallest split that puts >= 3072 waves on the chip (12 per CU), measured best on MI355X
    // for the 8-52 MB matrices of this model (longer streams per wave beat more, shorter waves)
    a.TPW = pair ? 2 : 1;
    const int NC = a.K / CHUNK_K;
    const int wgs = (total + a.TPW - 1) / a.TPW;
    const int maxks = 16 / a.TPW;
    a.KS = 1;
    for (int d = 1; d <= maxks && d <= NC; ++d) {
        if (NC % d) continue;
        a.KS = d;
        if (int64_t(total) * d >= 3072) break;
    }
    // MDX_GEMV_KS overrides the split (tuning sweeps)
    if (const char* env = getenv("MDX_GEMV_KS")) {
        const int ks = atoi(env);
        if (ks >= 1 && ks <= maxks && NC % ks == 0) a.KS = ks;
    }
    a.xglobal = 0;
    const int esz = esz_of(w0.s_dtype);
    MDX_CHECK((16 * (a.K >> a.lgG) * esz) % 16 == 0, "a tile's scale block must be a multiple of 16 bytes");
    for (int i = 0; i < nm; ++i) MDX_CHECK(aligned(ws[i]->s_rel, 16), "s_rel must be 16-byte aligned");
    MDX_CHECK(gemv_smem(a, mfma, esz) <= 160 * 1024, "activation of %d rows x K=%d exceeds LDS", rows, a.K);
    a.force_exact = w0.decode == MDX_DECODE_EXACT;
    return launch_gemv_d<4>(a, w0.s_dtype, mfma, wgs, st);
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

int prep_checks(int64_t rows, int64_t K, int32_t rot, const void* h) {
    MDX_CHECK(rows >= 0, "rows must be >= 0");
    MDX_CHECK(K > 0 && K % 256 == 0 && K <= MAX_PREP_K, "K must be a multiple of 256 and <= 16384 (got %lld)",
              (long long)K);
    MDX_CHECK(rot == MDX_ROT_NONE || rot == MDX_ROT_H256 || (rot == MDX_ROT_MATRIX && h), "rotation");
    return MDX_OK;
}

}  // namespace
}  // namespace mdx

using namespace mdx;

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
    int rc = prep_checks(rows, K, rot, h);
    if (rc) return rc;
    if (rows == 0) return MDX_OK;
    PrepArgs a{x, nullptr, 0.f, nullptr, h, rot, q, scale, int(K)};
    return launch_prep(a, rows, static_cast<hipStream_t>(stream));
}

extern "C" int mdx_rms_rot_quant(const uint16_t* x, const uint16_t* norm_w, float eps, uint16_t* xn_out,
                                 const uint16_t* h, int32_t rot, int8_t* q, float* scale, int64_t rows, int64_t K,
                                 void* stream) {
    MDX_CHECK(x && q && scale && norm_w, "null pointer");
    int rc = prep_checks(rows, K, rot, h);
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
    int rc = prep_checks(rows, K, rot, h);
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

extern "C" int mdx_rmsnorm(const uint16_t* x, const uint16_t* norm_w, float eps, uint16_t* out, int64_t rows, int64_t K,
                           void* stream) {
    MDX_CHECK(x && norm_w && out, "null pointer");
    MDX_CHECK(rows >= 0 && rows <= 65535 && K % 8 == 0 && K >= 8 && K <= 8 * PREP_THREADS * PREP_BLK,
              "rows / K (K % 8 == 0, K <= %d)", 8 * PREP_THREADS * PREP_BLK);
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

extern "C" size_t mdx_mono_mlp_workspace(int64_t rows, int64_t K1, int64_t N1) {
    return align256(size_t(rows) * K1) + align256(size_t(rows) * N1) + align256(64 * 4) + align256(size_t(rows) * N1 * 2);
}

extern "C" int mdx_mono_mlp(const uint16_t* xn, const uint16_t* norm_w, float eps, const uint16_t* h, int32_t rot,
                            const uint16_t* silu_lut, const mdx_w4* gate, const mdx_w4* up, const mdx_w4* down,
                            const uint16_t* residual, uint16_t* out, int64_t rows, void* workspace,
                            size_t workspace_bytes, void* stream) {
    MDX_CHECK(xn && silu_lut && gate && up && down && out && workspace, "null pointer");
    MDX_CHECK(rows >= 1 && rows <= 16, "rows must be in 1..16");
    const int64_t K1 = gate->k, N1 = gate->n;
    MDX_CHECK(up->n == N1 && up->k == K1 && down->k == N1, "gate/up [N1, K1], down [N2, N1] shapes");
    int rc = prep_checks(rows, K1, rot, h);
    if (rc) return rc;
    if ((rc = prep_checks(rows, N1, rot, h))) return rc;
    MDX_CHECK(workspace_bytes >= mdx_mono_mlp_workspace(rows, K1, N1), "workspace too small");
    MDX_CHECK(aligned(workspace, 256), "workspace must be 256-byte aligned");
    hipStream_t st = static_cast<hipStream_t>(stream);
    uint8_t* p = static_cast<uint8_t*>(workspace);
    int8_t* q1 = reinterpret_cast<int8_t*>(p);
    p += align256(size_t(rows) * K1);
    int8_t* q2 = reinterpret_cast<int8_t*>(p);
    p += align256(size_t(rows) * N1);
    float* s = reinterpret_cast<float*>(p);
    p += align256(64 * 4);
    uint16_t* hb = reinterpret_cast<uint16_t*>(p);
    PrepArgs pa{xn, norm_w, eps, nullptr, h, rot, q1, s, int(K1)};
    if ((rc = launch_prep(pa, rows, st))) return rc;
    const mdx_w4* gu[2] = {gate, up};
    void* o1[2] = {hb, hb};
    if ((rc = run_gemv(gu, 2, true, q1, s, int(rows), EPI_SILU, o1, nullptr, MDX_DT_BF16, silu_lut, st))) return rc;
    PrepArgs pb{hb, nullptr, 0.f, nullptr, h, rot, q2, s + 32, int(N1)};
    if ((rc = launch_prep(pb, rows, st))) return rc;
    const mdx_w4* dn[1] = {down};
    void* o2[1] = {out};
    const void* r2[1] = {residual};
    return run_gemv(dn, 1, false, q2, s + 32, int(rows), EPI_STORE, o2, r2, MDX_DT_BF16, nullptr, st);
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
