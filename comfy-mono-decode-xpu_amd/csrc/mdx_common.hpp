// Shared host/device helpers of libmdx (gfx950, wave64).
//
// Every floating-point step whose rounding is part of an operator's contract is written out
// here as an explicit IEEE single operation (no contraction): bf16 rounding is the software
// round-to-nearest-even of the top 16 bits, fp32 sums and products are separate
// __fadd_rn / __fmul_rn calls, so the CPU oracle can restate each result bit for bit.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "../../include/mdx.h"

namespace mdx {

// ---- error reporting (thread-local message, returned as a status code) ----------------------
void set_error(const char* fmt, ...);
#define MDX_CHECK(cond, ...)                 \
    do {                                     \
        if (!(cond)) {                       \
            ::mdx::set_error(__VA_ARGS__);   \
            return MDX_EINVAL;               \
        }                                    \
    } while (0)
#define MDX_HIP(call)                                                               \
    do {                                                                            \
        hipError_t e_ = (call);                                                     \
        if (e_ != hipSuccess) {                                                     \
            ::mdx::set_error("%s failed: %s", #call, hipGetErrorString(e_));        \
            return MDX_EHIP;                                                        \
        }                                                                           \
    } while (0)
#define MDX_LAUNCHED()                                                              \
    do {                                                                            \
        hipError_t e_ = hipGetLastError();                                          \
        if (e_ != hipSuccess) {                                                     \
            ::mdx::set_error("kernel launch failed: %s", hipGetErrorString(e_));    \
            return MDX_EHIP;                                                        \
        }                                                                           \
    } while (0)

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// ---- scalar conversions (device) ---------------------------------------------------------------
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// Round-to-nearest-even fp32 -> bf16 by the hardware conversion (v_cvt_pk_bf16_f32, two values per
// instruction): on gfx950 it gives the RNE result of the bit pattern for every non-NaN fp32 input,
// subnormals included (checked over all 2^32 patterns against the integer formulation
// u + 0x7FFF + ((u >> 16) & 1)), and a NaN for a NaN. f2bf makes every NaN the canonical quiet NaN
// 0x7FC0; bfround (the fp32 value of the bf16 rounding) keeps a NaN a NaN of unspecified payload,
// which no fp32 operation distinguishes.
__device__ __forceinline__ uint16_t f2bf(float f) {
    const uint16_t h = __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
    return f != f ? uint16_t(0x7FC0u) : h;
}

__device__ __forceinline__ float bfround(float f) { return bf2f(__builtin_bit_cast(uint16_t, static_cast<__bf16>(f))); }

// bfround of two values by one conversion instruction
typedef float mdx_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 mdx_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void bfround2(float& a, float& b) {
    const uint32_t u = __builtin_bit_cast(uint32_t, __builtin_convertvector(mdx_f32x2{a, b}, mdx_bf16x2));
    a = __uint_as_float(u << 16);
    b = __uint_as_float(u & 0xFFFF0000u);
}

__device__ __forceinline__ float fp16_to_f32(uint16_t h) {
    return float(__builtin_bit_cast(_Float16, h));
}

// OCP float8 e4m3fn (bias 7, no infinities, S.1111.111 = NaN) -> fp32, exact
__device__ __forceinline__ float fp8_to_f32(uint8_t b) {
    const uint32_t s = uint32_t(b >> 7) << 31, e = (b >> 3) & 15u, m = b & 7u;
    if (e == 15u && m == 7u) return __uint_as_float(s | 0x7FC00000u);
    if (e == 0u) {
        const float v = float(m) * 0.001953125f;  // m * 2^-9
        return s ? -v : v;
    }
    return __uint_as_float(s | ((e + 120u) << 23) | (m << 20));
}

__device__ __forceinline__ float load_scale(const void* s, int dtype, int64_t i) {
    if (dtype == MDX_DT_F32) return reinterpret_cast<const float*>(s)[i];
    if (dtype == MDX_DT_F16) return fp16_to_f32(reinterpret_cast<const uint16_t*>(s)[i]);
    return fp8_to_f32(reinterpret_cast<const uint8_t*>(s)[i]);
}

// correctly rounded fp32 square root (HIP's __fsqrt_rn maps to the approximate hardware sqrt unless
// the OCML rounded-operation mode is on; llvm.sqrt.f32 is lowered with the rounding correction)
__device__ __forceinline__ float sqrt_rn(float x) { return __builtin_sqrtf(x); }

// ---- wave64 helpers -----------------------------------------------------------------------------
__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

template <typename T>
__device__ __forceinline__ T shfl_down(T v, int d) { return __shfl_down(v, d, 64); }
template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int d) { return __shfl_xor(v, d, 64); }

// Cross-lane partners without the LDS crossbar (gfx950): v_permlane32_swap exchanges the wave's two
// halves, v_permlane16_swap rows 0 <-> 1 and 2 <-> 3, DPP row_ror:8 the halves of each row. Given v
// twice, a swap returns (own, partner) in the lower lanes and (partner, own) in the upper ones; a sum
// or maximum of the two is the same value either way (a + b and b + a are the same float), so each of
// these equals v op (the value of lane l ^ D) in every lane, bit for bit.
__device__ __forceinline__ float sum_x32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __fadd_rn(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_x16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __fadd_rn(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_x8(float v) {
    return __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false)));
}
__device__ __forceinline__ float max_x32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_x16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ int isum_x32(int v) {
    const auto r = __builtin_amdgcn_permlane32_swap(uint32_t(v), uint32_t(v), false, false);
    return int(r[0] + r[1]);
}
__device__ __forceinline__ int isum_x16(int v) {
    const auto r = __builtin_amdgcn_permlane16_swap(uint32_t(v), uint32_t(v), false, false);
    return int(r[0] + r[1]);
}

__device__ __forceinline__ float wave_max(float v) {
    for (int d = 32; d >= 1; d >>= 1) v = fmaxf(v, shfl_xor(v, d));
    return v;
}

// the value of lane l + D (D < 16) of lane l's row of 16 (DPP row_shl); lanes whose partner lies past
// the row read 0
template <int D>
__device__ __forceinline__ float row_shl(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + D, 0xF, 0xF, false));
}

// The halving-tree sum of the wave's 64 values in lane 0 (lane l adds lane l + s for s = 32, 16, ...,
// 1, each sum rounded): the strides below 16 by DPP, 32 and 16 by lane swaps. Only lane 0's result is
// the tree's.
__device__ __forceinline__ float tree_sum64(float q) {
    q = sum_x32(q);
    q = sum_x16(q);
    q = __fadd_rn(q, row_shl<8>(q));
    q = __fadd_rn(q, row_shl<4>(q));
    q = __fadd_rn(q, row_shl<2>(q));
    q = __fadd_rn(q, row_shl<1>(q));
    return q;
}

// The maximum of the wave's non-negative values, in every lane (lane 0's tree, broadcast).
__device__ __forceinline__ float wave_max_nn(float v) {
    v = max_x32(v);
    v = max_x16(v);
    v = fmaxf(v, row_shl<8>(v));
    v = fmaxf(v, row_shl<4>(v));
    v = fmaxf(v, row_shl<2>(v));
    v = fmaxf(v, row_shl<1>(v));
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

// fused_scaleback: (float(acc) * xs) * sc, each product rounded on its own
__device__ __forceinline__ float scaleback(int32_t acc, float xs, float sc) {
    float f = float(acc);
    f = __fmul_rn(f, xs);
    f = __fmul_rn(f, sc);
    return f;
}

}  // namespace mdx

namespace mdx {
// Raise a kernel's dynamic LDS limit above the 64 KiB default (gfx950 has 160 KiB per CU).
inline void allow_smem(const void* fn, size_t bytes) {
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes));
    (void)hipGetLastError();
}
}  // namespace mdx
