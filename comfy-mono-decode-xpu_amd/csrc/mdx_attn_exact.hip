// Exact tree-verify decode attention: the exactness fallback beside the fast flash-decoding kernel.
//
// Reference: the reference keeps a bit-identical port of its upstream library's decode attention as an A/B
// switch (csrc/attn_port.sycl:1-12, selected by MONO_DECODE_XPU_ATTN in comfy_mono_decode_xpu/layer.py:43,409)
// so that a run can be reproduced exactly when the fast kernel's reduction order is in question. That
// upstream kernel is third-party and not portable here; this kernel's results are instead fixed bit for
// bit by one canonical fp32 order, restated by the oracle (oracle/ref.py attention_exact), so any run can be
// reproduced on the CPU. Same operands and outputs as mdx_attn_decode.
//
// One wave per (head h, tree row s). The admitted tokens u = 0 .. n-1 are the cache prefix [0, L) in order,
// then the tree rows t < S whose bit is set in mask[s], ascending (none without a mask).
//   score[u] = fl(dot * scale), dot = ((q0 k0 + q1 k1) + q2 k2) + ..., every product and sum rounded (fp32)
//   m = max score;  e[u] = exp_c(score[u] - m)  (exp_c below: Cody-Waite reduction, degree-7 Taylor)
//   l: lane j sums e[u] over u = j, j + 64, ... in order, then a halving tree over the 64 lanes
//      (lane j adds lane j + 32, then + 16, ..., + 1)
//   o[d] = (((e0 v0[d]) + e1 v1[d]) + ...) over u in order;  out = bf16(o[d] / l), or 0 when n = 0.
// Every fp32 operation is a single IEEE operation (explicit _rn intrinsics, no contraction).
#include "mdx_common.hpp"

namespace mdx {
namespace {

constexpr int EX_MAXTOK = 16384;  // cache capacity + tree rows held in LDS (64 KiB of weights)

struct ExactArgs {
    const uint16_t* q;  // [1, H, S, D] strides qh, qs (dim stride 1)
    int64_t qh, qs;
    const uint16_t* key;    // [1, Hk, cap, D]
    const uint16_t* value;
    const int32_t* seqlen;
    const uint16_t* xk;  // [1, Hk, S, D] strides xh, xs
    int64_t xkh, xks;
    const uint16_t* xv;
    int64_t xvh, xvs;
    const int32_t* mask;  // [S] or null
    uint16_t* out;        // [1, S, H * D]
    int H, Hk, S, cap;
    float scale;
};

// e^x for x <= 0 in a fixed sequence of fp32 operations: n = rint(x log2 e), r = (x - n ln2_hi) - n ln2_lo
// (ln2_hi has 14 significant bits, so n ln2_hi is exact), p = the degree-7 Taylor polynomial of e^r by
// Horner's rule (coefficients fl32(1/k!)), e^x = p 2^n. Inputs below -80 (and NaN) give 0.
__device__ __forceinline__ float exp_c(float x) {
    if (!(x > -80.0f)) return 0.0f;
    const float n = __builtin_rintf(__fmul_rn(x, 0x1.715476p+0f));
    const float r = __fsub_rn(__fsub_rn(x, __fmul_rn(n, 0x1.62e4p-1f)), __fmul_rn(n, 0x1.7f7d1cp-20f));
    float p = 0x1.a01a02p-13f;
    p = __fadd_rn(__fmul_rn(p, r), 0x1.6c16c2p-10f);
    p = __fadd_rn(__fmul_rn(p, r), 0x1.111112p-7f);
    p = __fadd_rn(__fmul_rn(p, r), 0x1.555556p-5f);
    p = __fadd_rn(__fmul_rn(p, r), 0x1.555556p-3f);
    p = __fadd_rn(__fmul_rn(p, r), 0.5f);
    p = __fadd_rn(__fmul_rn(p, r), 1.0f);
    p = __fadd_rn(__fmul_rn(p, r), 1.0f);
    return __builtin_ldexpf(p, int(n));
}

template <int D>
__global__ __launch_bounds__(64) void attn_exact_kernel(ExactArgs a) {
    extern __shared__ float ew[];  // [n] scores, then weights
    __shared__ float qs[D];
    __shared__ int trow[16];
    const int lane = threadIdx.x;
    const int h = blockIdx.x / a.S, s = blockIdx.x % a.S;
    const int kh = h / (a.H / a.Hk);
    const int L = min(max(a.seqlen[0], 0), a.cap);
    const uint32_t m = a.mask ? uint32_t(a.mask[s]) & ((1u << a.S) - 1u) : 0u;
    int nt = 0;
    for (int t = 0; t < a.S; ++t)
        if ((m >> t) & 1u) {
            if (lane == 0) trow[nt] = t;
            ++nt;
        }
    const int n = L + nt;
    for (int d = lane; d < D; d += 64) qs[d] = bf2f(a.q[h * a.qh + s * a.qs + d]);
    __syncthreads();
    const uint16_t* kbase = a.key + int64_t(kh) * a.cap * D;
    const uint16_t* vbase = a.value + int64_t(kh) * a.cap * D;
    // scores, one token per lane at a time, the dot product in dimension order
    for (int u = lane; u < n; u += 64) {
        const uint16_t* kr = u < L ? kbase + int64_t(u) * D : a.xk + kh * a.xkh + trow[u - L] * a.xks;
        float acc = 0.0f;
        for (int d = 0; d < D; ++d) acc = __fadd_rn(acc, __fmul_rn(qs[d], bf2f(kr[d])));
        ew[u] = __fmul_rn(acc, a.scale);
    }
    __syncthreads();
    float mx = -__builtin_inff();
    for (int u = lane; u < n; u += 64) mx = fmaxf(mx, ew[u]);
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    float part = 0.0f;
    for (int u = lane; u < n; u += 64) {
        const float e = exp_c(__fsub_rn(ew[u], mx));
        ew[u] = e;
        part = __fadd_rn(part, e);
    }
    for (int o = 32; o >= 1; o >>= 1) {
        const float v = __shfl_down(part, o, 64);
        if (lane < o) part = __fadd_rn(part, v);
    }
    const float l = __shfl(part, 0, 64);
    __syncthreads();
    float o[D / 64];
#pragma unroll
    for (int i = 0; i < D / 64; ++i) o[i] = 0.0f;
    for (int u = 0; u < n; ++u) {
        const float w = ew[u];
        const uint16_t* vr = u < L ? vbase + int64_t(u) * D : a.xv + kh * a.xvh + trow[u - L] * a.xvs;
#pragma unroll
        for (int i = 0; i < D / 64; ++i) o[i] = __fadd_rn(o[i], __fmul_rn(w, bf2f(vr[lane + 64 * i])));
    }
    uint16_t* out = a.out + (int64_t(s) * a.H + h) * D;
#pragma unroll
    for (int i = 0; i < D / 64; ++i) out[lane + 64 * i] = n > 0 ? f2bf(__fdiv_rn(o[i], l)) : uint16_t(0);
}

}  // namespace
}  // namespace mdx

using namespace mdx;

extern "C" int mdx_attn_exact(const uint16_t* q, int64_t q_head_stride, int64_t q_row_stride, const uint16_t* key,
                              const uint16_t* value, const int32_t* seqlen, const uint16_t* xk, int64_t xk_head_stride,
                              int64_t xk_row_stride, const uint16_t* xv, int64_t xv_head_stride, int64_t xv_row_stride,
                              const int32_t* mask, uint16_t* out, int64_t H, int64_t Hk, int64_t S, int64_t D,
                              int64_t cap, float scale, void* stream) {
    MDX_CHECK(q && key && value && seqlen && xk && xv && out, "null pointer");
    MDX_CHECK(D == 64 || D == 128 || D == 256, "head_dim must be 64, 128 or 256");
    MDX_CHECK(S >= 1 && S <= 16 && Hk >= 1 && H >= Hk && H % Hk == 0 && H * S <= 65535, "1..16 rows, H % Hk == 0");
    MDX_CHECK(cap >= 1 && cap + S <= EX_MAXTOK, "cache capacity + rows must be <= 16384 (the weights sit in LDS)");
    ExactArgs a{q, q_head_stride, q_row_stride, key, value, seqlen, xk, xk_head_stride, xk_row_stride, xv, xv_head_stride,
                xv_row_stride, mask, out, int(H), int(Hk), int(S), int(cap), scale};
    const size_t lds = size_t(cap + S) * sizeof(float);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid(unsigned(H * S)), block(64);
    if (D == 64) {
        allow_smem(reinterpret_cast<const void*>(&attn_exact_kernel<64>), lds);
        hipLaunchKernelGGL(attn_exact_kernel<64>, grid, block, lds, st, a);
    } else if (D == 128) {
        allow_smem(reinterpret_cast<const void*>(&attn_exact_kernel<128>), lds);
        hipLaunchKernelGGL(attn_exact_kernel<128>, grid, block, lds, st, a);
    } else {
        allow_smem(reinterpret_cast<const void*>(&attn_exact_kernel<256>), lds);
        hipLaunchKernelGGL(attn_exact_kernel<256>, grid, block, lds, st, a);
    }
    MDX_LAUNCHED();
    return MDX_OK;
}
