// torch XPU's top-k / argmax order as unique 64-bit ranks (gfx950): the radix key of the value in the
// high word, the complement of the element's position in the reference's gather sweep in the low
// word, so the k largest ranks in descending order are torch's result. Shared by the top-k kernels
// and the draft pick.
//
// Reference semantics (comfy-mono-decode-xpu): csrc/fast_topk.sycl:4-40 (bf16 radix key, argmax rank,
// gather order of 1024 threads x 4 loads of 8), csrc/fast_topk.sycl:145-157 (index back-mapping),
// csrc/topk_rows.sycl:7-11,33-43 (fp32 radix key, gather order of 1024 threads x 8 loads of 4).
#pragma once
#include "mdx_common.hpp"

namespace mdx {

enum Order : int {
    ORDER_BF16 = 0,    // torch XPU topk of one bf16 row: bf16 radix key, gather 1024 x 4 loads x 8
    ORDER_ARGMAX = 1,  // torch XPU argmax of a bf16 row: NaN first, -0 == +0, smallest index
    ORDER_F32 = 2,     // torch XPU topk of fp32 rows: fp32 radix key, gather 1024 x 8 loads x 4
};

// Position of element i in the gather order of a sweep of 1024 threads, each issuing `loads` vector
// loads of `width` elements per 32768-element iteration: (iteration, thread, load, lane).
template <int LOADS, int WIDTH>
__device__ __forceinline__ uint32_t gather_pos(uint32_t i) {
    const uint32_t it = i >> 15, off = i & 32767u;
    const uint32_t load = off / (1024u * WIDTH), thread = (off % (1024u * WIDTH)) / WIDTH, lane = off % WIDTH;
    return (it << 15) | (thread * (LOADS * WIDTH)) | (load * WIDTH) | lane;
}
template <int LOADS, int WIDTH>
__device__ __forceinline__ uint32_t gather_index(uint32_t g) {
    const uint32_t it = g >> 15, rem = g & 32767u;
    const uint32_t thread = rem / (LOADS * WIDTH), load = (rem / WIDTH) % LOADS, lane = rem % WIDTH;
    return (it << 15) | (load * 1024u * WIDTH) | (thread * WIDTH) | lane;
}

// radix keys: larger key = earlier in torch's descending order
__device__ __forceinline__ uint32_t key_bf16(uint16_t b) {
    if ((b & 0x7FFFu) > 0x7F80u) return 0xFFFFu;  // NaN on top
    return (b & 0x8000u) ? uint32_t(b ^ 0xFFFFu) : uint32_t(b | 0x8000u);
}
__device__ __forceinline__ uint32_t key_f32(uint32_t u) {  // +NaN on top, -NaN at the bottom
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ uint32_t key_argmax(uint16_t b) {
    if ((b & 0x7FFFu) > 0x7F80u) return 0xFFFFFFFFu;
    if ((b & 0x7FFFu) == 0) b = 0;  // -0 == +0
    return (b & 0x8000u) ? 0x7FFFu - (b & 0x7FFFu) : 0x8000u + b;
}

// the element's bits: bf16 (ORDER_BF16 / ORDER_ARGMAX), fp32 bits (ORDER_F32; a bf16 row widened).
// XF32 (fp32 rows) is a template parameter: a load chosen at run time would sit under a branch and be
// waited for at its join.
template <int ORD, bool XF32>
__device__ __forceinline__ uint32_t raw_of(const void* row, uint32_t i) {
    if (ORD == ORDER_F32 && XF32) return static_cast<const uint32_t*>(row)[i];
    return static_cast<const uint16_t*>(row)[i];
}

// the rank of element i from its loaded bits (raw_of)
template <int ORD, bool XF32 = false>
__device__ __forceinline__ uint64_t rank_raw(uint32_t u, uint32_t i) {
    if (ORD == ORDER_BF16) return (uint64_t(key_bf16(uint16_t(u))) << 32) | (0xFFFFFFFFu - gather_pos<4, 8>(i));
    if (ORD == ORDER_ARGMAX) return (uint64_t(key_argmax(uint16_t(u))) << 32) | (0xFFFFFFFFu - i);
    return (uint64_t(key_f32(XF32 ? u : u << 16)) << 32) | (0xFFFFFFFFu - gather_pos<8, 4>(i));
}

template <int ORD>
__device__ __forceinline__ uint32_t index_of(uint64_t r) {
    const uint32_t g = 0xFFFFFFFFu - uint32_t(r);
    if (ORD == ORDER_BF16) return gather_index<4, 8>(g);
    if (ORD == ORDER_ARGMAX) return g;
    return gather_index<8, 4>(g);
}

}  // namespace mdx
