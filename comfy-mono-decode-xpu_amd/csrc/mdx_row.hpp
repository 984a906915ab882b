// Row helpers shared by the row-prep and draft-row kernels (gfx950, wave64): bf16 quads in
// registers, the fp64 fast Walsh-Hadamard transform of a 256-group held 4 elements per lane, and the
// canonical RMSNorm factor of a row whose 256-groups are spread over the waves of a work-group.
#pragma once
#include "mdx_common.hpp"

namespace mdx {

__device__ __forceinline__ void unpack4(const uint2& v, float* f) {
    f[0] = __uint_as_float(v.x << 16);
    f[1] = __uint_as_float(v.x & 0xFFFF0000u);
    f[2] = __uint_as_float(v.y << 16);
    f[3] = __uint_as_float(v.y & 0xFFFF0000u);
}

__device__ __forceinline__ uint2 pack4(const float* f) {
    return make_uint2(uint32_t(f2bf(f[0])) | (uint32_t(f2bf(f[1])) << 16),
                      uint32_t(f2bf(f[2])) | (uint32_t(f2bf(f[3])) << 16));
}

// the value `v` of lane Q of this lane's quad (DPP quad_perm broadcast, both halves of the double)
template <int Q>
__device__ __forceinline__ double quad_lane(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = uint32_t(__builtin_amdgcn_mov_dpp(int(uint32_t(u)), Q * 0x55, 0xF, 0xF, false));
    const uint32_t hi = uint32_t(__builtin_amdgcn_mov_dpp(int(uint32_t(u >> 32)), Q * 0x55, 0xF, 0xF, false));
    return __builtin_bit_cast(double, uint64_t(lo) | (uint64_t(hi) << 32));
}

// output j of the radix-4 butterfly: the H4 row j applied to (a0, a1, a2, a3) left to right,
// ((a0 + a1) + a2) - a3, ((a0 + a1) - a2) + a3, ((a0 - a1) + a2) + a3, ((a1 - a0) + a2) + a3: row j has
// its one minus sign at position 3 - j (a - b and -b + a are the same IEEE operation)
__device__ __forceinline__ double h4_out(const double* a, int j) {
    double b[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) b[k] = (k == 3 - j) ? -a[k] : a[k];
    return __dadd_rn(__dadd_rn(__dadd_rn(b[0], b[1]), b[2]), b[3]);
}

// fp64 fast Walsh-Hadamard transform of one 256-group held 4 elements per lane (lane l: elements
// 4 l .. 4 l + 3): radix-4 stages along the base-4 digits of the element index (strides 1, 4, 16, 64).
// Digit 0 is the lane's own slot, digit 1 the lane within its quad, digits 2 and 3 the quad within
// the 16-lane row and the row; each lane computes its own output of every butterfly.
__device__ __forceinline__ void fwht256_lane(double* d, int lane) {
    double o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = h4_out(d, e);
    const int j1 = lane & 3, j2 = (lane >> 2) & 3, j3 = lane >> 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const double a[4] = {quad_lane<0>(o[e]), quad_lane<1>(o[e]), quad_lane<2>(o[e]), quad_lane<3>(o[e])};
        d[e] = h4_out(a, j1);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        double a[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) a[k] = __shfl(d[e], (lane & ~12) | (k << 2), 64);
        o[e] = h4_out(a, j2);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        double a[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) a[k] = __shfl(o[e], (lane & 15) | (k << 4), 64);
        d[e] = h4_out(a, j3);
    }
}

// The canonical RMSNorm factor r = 1 / sqrt(mean(x^2) + eps) of a row of K = 256 G elements held by a
// work-group: wave w owns groups w, w + W, ... (GPW per wave), lane l elements 4 l .. 4 l + 3 of each.
// Sum order: per group, the lane partial ((sq0 + sq1) + sq2) + sq3, the halving tree over the 64 lanes
// (l + 32, + 16, ..., + 1), then the group sums added in group order. gsum holds G <= 64 floats. Every
// thread of the work-group must call it (it contains a barrier); every thread gets r.
template <int GPW>
__device__ __forceinline__ float row_rms_factor(const float (&v)[GPW][4], int K, float eps, float* gsum) {
    const int W = blockDim.x / 64, w = threadIdx.x / 64, lane = threadIdx.x % 64, G = K / 256;
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) {
        float q = __fmul_rn(v[gi][0], v[gi][0]);
#pragma unroll
        for (int e = 1; e < 4; ++e) q = __fadd_rn(q, __fmul_rn(v[gi][e], v[gi][e]));
        q = tree_sum64(q);
        const int g = w + W * gi;
        if (lane == 0 && g < G) gsum[g] = q;
    }
    __syncthreads();
    const float gv = lane < G ? gsum[lane] : 0.f;
    float ss = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(gv)));
    for (int g = 1; g < G; ++g) ss = __fadd_rn(ss, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gv), g)));
    const float mean = __fdiv_rn(ss, float(K));
    return __fdiv_rn(1.f, sqrt_rn(__fadd_rn(mean, eps)));
}

// bf16(silu(z)) as the gated RMSNorm takes it: bf16(z / (1 + e^-z))
__device__ __forceinline__ float gnorm_gate(float z) { return bfround(__fdiv_rn(z, __fadd_rn(1.f, expf(-z)))); }

// The gated RMSNorm of two 128-element head rows held by one wave (lanes 0..31 the first, 32..63 the
// second; lane l holds elements 4 (l % 32) .. + 3 in v, their norm weights in hw and gate factors in gz =
// gnorm_gate(z)): v <- bf16(bf16(v hw rsq) * gz), rsq = 1 / sqrt(sum(v^2) / 128 + eps). Sum order: the
// lane partial ((sq0 + sq1) + sq2) + sq3, then a halving tree within each half (l + 16, + 8, ..., + 1),
// read back from lane 0 / 32. Every lane of the wave must call it.
__device__ __forceinline__ void gnorm_pair_g(float (&v)[4], const float (&hw)[4], const float (&gz)[4], float eps,
                                             int lane) {
    float q = __fmul_rn(v[0], v[0]);
#pragma unroll
    for (int e = 1; e < 4; ++e) q = __fadd_rn(q, __fmul_rn(v[e], v[e]));
    q = sum_x16(q);
    q = __fadd_rn(q, row_shl<8>(q));
    q = __fadd_rn(q, row_shl<4>(q));
    q = __fadd_rn(q, row_shl<2>(q));
    q = __fadd_rn(q, row_shl<1>(q));
    {
        const float q0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(q), 0));
        const float q32 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(q), 32));
        q = (lane & 32) ? q32 : q0;
    }
    const float rsq = __fdiv_rn(1.f, sqrt_rn(__fadd_rn(__fdiv_rn(q, 128.f), eps)));
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = bfround(__fmul_rn(bfround(__fmul_rn(__fmul_rn(v[e], hw[e]), rsq)), gz[e]));
}

// gnorm_pair_g from the gate inputs z
__device__ __forceinline__ void gnorm_pair(float (&v)[4], const float (&hw)[4], const float (&z)[4], float eps, int lane) {
    float gz[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) gz[e] = gnorm_gate(z[e]);
    gnorm_pair_g(v, hw, gz, eps, lane);
}

// The int8 row quantisation of the row prep: scale s = max(absmax / 127, 1e-30) (absmax: the row's
// maximum |v|, NaN ignored), codes rint(bf16(v * fl32(1 / sb))) clamped to [-128, 127], sb = bf16(s)
// (0x0080 when that rounds to zero). quant_rcp is 1 / sb.
__device__ __forceinline__ float quant_rcp(float s) {
    uint16_t sb = f2bf(s);
    if ((sb & 0x7FFFu) == 0) sb = 0x0080u;
    return __fdiv_rn(1.f, bf2f(sb));
}
__device__ __forceinline__ uint32_t quant4(const float (&v)[4], float rr) {
    uint32_t o = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float d = bfround(__fmul_rn(v[e], rr));
        const int qv = int(fminf(fmaxf(rintf(d), -128.f), 127.f));
        o |= (uint32_t(qv) & 0xFFu) << (8 * e);
    }
    return o;
}

}  // namespace mdx
