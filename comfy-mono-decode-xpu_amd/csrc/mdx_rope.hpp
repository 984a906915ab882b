// Q/K RMSNorm + split-half RoPE pieces shared by the RoPE/KV kernel (mdx_rope_mtp.hip) and the tree-verify
// attention that runs the same prep in its own launch (mdx_attn.hip).
//
// Reference semantics (comfy-mono-decode-xpu): csrc/rope_kv.sycl:5-11,44-52 (each rotated output is
// bf16(t_j * f00 + t_{j+h} * f01), resp. bf16(t_{j+h} * f11 + t_j * f10), every product rounded, no FMA),
// :193-219 (the per-head norm bf16((x * scale) * w)).
#pragma once

#include "mdx_common.hpp"

namespace mdx {

__device__ __forceinline__ float rope_pair(float a, float fa, float b, float fb) {
    return __fadd_rn(__fmul_rn(a, fa), __fmul_rn(b, fb));
}

// One (row, head) of head_dim 128 by one wave, the RoPE/KV kernel's arithmetic for D = 128: lane l holds
// elements l and l + 64 (x0, x1, as floats of the bf16 inputs). With a norm (w0, w1: the lane's weights):
// the lane partial x0^2 + x1^2, the 64-lane halving tree, r = 1 / sqrt(sum / 128 + eps), x <- bf16((x r) w).
// Then RoPE over the first rd elements (rd = 32, 64 or 128; m: the rotation matrix [[f00, f01], [f10, f11]]
// of pair jj = l mod rd / 2, loaded by lanes l < min(rd, 64)): element d pairs with d ^ rd / 2. Every lane
// of the wave calls it (cross-lane sums and swaps); o0, o1 are the bf16 outputs of elements l, l + 64.
__device__ __forceinline__ void qk_rope128(float x0, float x1, bool norm, float w0, float w1, float eps, int rd,
                                           float4 m, int lane, uint16_t& o0, uint16_t& o1) {
    if (norm) {
        const float part = __fadd_rn(__fmul_rn(x0, x0), __fmul_rn(x1, x1));
        const float ss = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(tree_sum64(part))));
        const float r = __fdiv_rn(1.f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, 128.f), eps)));
        x0 = bfround(__fmul_rn(__fmul_rn(x0, r), w0));
        x1 = bfround(__fmul_rn(__fmul_rn(x1, r), w1));
    }
    const int half = rd / 2;
    // the partner of element l: element l + 64 of this lane (rd = 128), else lane l ^ half's element l ^ half,
    // by a lane swap (v_permlane32_swap / v_permlane16_swap: VALU, no LDS instruction; given v twice a swap
    // returns (own, partner) in the lanes without bit `half`, (partner, own) in the others)
    float p0 = x1;
    if (half != 64) {
        const uint32_t b = __float_as_uint(x0);
        const auto sw = half == 32 ? __builtin_amdgcn_permlane32_swap(b, b, false, false)
                                   : __builtin_amdgcn_permlane16_swap(b, b, false, false);
        p0 = __uint_as_float((lane & half) ? sw[0] : sw[1]);
    }
    float r0 = x0, r1 = x1;
    if (lane < rd) r0 = lane < half ? rope_pair(x0, m.x, p0, m.y) : rope_pair(x0, m.w, p0, m.z);
    if (rd == 128) r1 = rope_pair(x1, m.w, x0, m.z);
    o0 = f2bf(r0);
    o1 = f2bf(r1);
}

// qk_rope128 over NP (row, head)s at once (NP <= 64), the same arithmetic per row: the NP norm factors
// come from one division / square-root chain, lane i computing row i's, instead of one chain per row.
template <int NP>
__device__ __forceinline__ void qk_rope128_n(const float (&x0)[NP], const float (&x1)[NP], bool norm, float w0, float w1,
                                             float eps, int rd, const float4 (&m)[NP], int lane, uint16_t (&o0)[NP],
                                             uint16_t (&o1)[NP]) {
    static_assert(NP >= 1 && NP <= 64, "rows per call");
    float rs[NP];
    if (norm) {
        float ssv = 0.f;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const float part = __fadd_rn(__fmul_rn(x0[i], x0[i]), __fmul_rn(x1[i], x1[i]));
            const float ss = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(tree_sum64(part))));
            ssv = lane == i ? ss : ssv;
        }
        const float rv = __fdiv_rn(1.f, sqrt_rn(__fadd_rn(__fdiv_rn(ssv, 128.f), eps)));
#pragma unroll
        for (int i = 0; i < NP; ++i) rs[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rv), i));
    }
    const int half = rd / 2;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        float y0 = x0[i], y1 = x1[i];
        if (norm) {
            y0 = bfround(__fmul_rn(__fmul_rn(y0, rs[i]), w0));
            y1 = bfround(__fmul_rn(__fmul_rn(y1, rs[i]), w1));
        }
        float p0 = y1;
        if (half != 64) {
            const uint32_t b = __float_as_uint(y0);
            const auto sw = half == 32 ? __builtin_amdgcn_permlane32_swap(b, b, false, false)
                                       : __builtin_amdgcn_permlane16_swap(b, b, false, false);
            p0 = __uint_as_float((lane & half) ? sw[0] : sw[1]);
        }
        float r0 = y0, r1 = y1;
        if (lane < rd) r0 = lane < half ? rope_pair(y0, m[i].x, p0, m[i].y) : rope_pair(y0, m[i].w, p0, m[i].z);
        if (rd == 128) r1 = rope_pair(y1, m[i].w, y0, m[i].z);
        o0[i] = f2bf(r0);
        o1[i] = f2bf(r1);
    }
}

}  // namespace mdx
