// W8A8 linear for 1..16 rows: out[m, n] = bf16((float(acc[m, n]) * x_scale[m]) * w_scale[n]), acc the int32
// dot of the int8 activation row with the int8 weight row (exact: the products and their sums fit int32
// for K <= 65536). The int8 ConvRot lm_head: weights rotated by H256 per 256-column group and quantised
// per row, activations rotated the same way and quantised per row, so acc approximates x . W^T.
//
// Reference: the int8 head is read by omni_xpu_kernel's int8_linear_prequantized (0.2.0b3, a third-party
// library, called at comfy_mono_decode_xpu/draft_head.py:228 for the drafts; the verify's F.linear on the
// same int8 head, comfy_mono_decode_xpu/mtp_loop.py:221-225) and its exact logits are restated by the
// draft pick (csrc/draft_lmhead.sycl:217-220): (float(acc) * sx) * sw[n], two fp32 roundings, bf16 out.
//
// Every product is one v_mfma_i32_16x16x64_i8 (gfx950): A = 16 weight rows x 64 k, one 16-byte load per
// lane, so a wave instruction moves 1 KiB of the tile-major weight stream; B = 64 k of the activation
// rows as columns (rows >= `rows` are zero); D = 16 outputs x 16 rows, lane 16 g + c holding outputs
// 16 t + 4 g + i of row c. A lane's 16 weight bytes and 16 activation bytes cover the same 16 k, so the
// int32 sum pairs every weight with its activation whatever order the instruction adds them in. A wave
// owns a 16-row tile and a K slice; slices add their int32 partials in LDS (exact in any order).
//
// Tile-major weights: [N/16][K/64][64 lanes][16 B], lane 16 g + c holding row 16 t + c, k in
// [64 j + 16 g, 64 j + 16 g + 16) of block (t, j). Row-major [N, K] weights are read in place.
#include <algorithm>

#include "mdx_common.hpp"

namespace mdx {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int W8_RING = 4;

struct W8Args {
    const int8_t* x;       // [rows, K]
    const float* xs;       // [rows]
    const int8_t* w;
    const float* ws;       // [N]
    uint16_t* out;         // [rows, N]
    int N, K, rows, KS, TPW, tiles, layout;
};

__device__ __forceinline__ u32x4 ldnt16(const int8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

template <int RING>
__global__ __launch_bounds__(1024) void int8_linear_kernel(W8Args a) {
    extern __shared__ __align__(16) int32_t red8[];  // [TPW][KS][64][4]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ts = wave / a.KS, slice = wave % a.KS;
    const int tile = blockIdx.x * a.TPW + ts;
    const bool live = tile < a.tiles;
    const int NC = a.K / 64;
    const int c0 = live ? slice * NC / a.KS : 0, c1 = live ? (slice + 1) * NC / a.KS : 0;
    const int nch = c1 - c0, last = nch > 0 ? nch - 1 : 0;
    const int g = lane >> 4, c = lane & 15;
    const int8_t* wp;
    int wstride;
    if (a.layout == MDX_LAYOUT_TILE) {
        wp = a.w + (int64_t(live ? tile : 0) * NC + c0) * 1024 + lane * 16;
        wstride = 1024;
    } else {
        wp = a.w + int64_t((live ? tile : 0) * 16 + c) * a.K + c0 * 64 + 16 * g;
        wstride = 64;
    }
    // weights and the activation both travel in the ring (RING chunks ahead); whole ring rounds with no
    // conditions around the loads (a chunk past the slice re-reads the slice's last one and adds nothing)
    const bool xlive = c < a.rows;
    const int8_t* xp = a.x + int64_t(xlive ? c : 0) * a.K + c0 * 64 + 16 * g;
    u32x4 ring[RING], xring[RING];
#pragma unroll
    for (int p = 0; p < RING; ++p) {
        ring[p] = ldnt16(wp + int64_t(min(p, last)) * wstride);
        xring[p] = *reinterpret_cast<const u32x4*>(xp + min(p, last) * 64);
        __builtin_amdgcn_sched_barrier(0);
    }
    i32x4 acc = {0, 0, 0, 0};
    for (int i0 = 0; i0 < nch; i0 += RING) {
#pragma unroll
        for (int p = 0; p < RING; ++p) {
            // consume the slot, then refill it (the ring keeps its registers across iterations)
            const int i = i0 + p;
            u32x4 xv = xring[p];
            if (!xlive || i >= nch) xv = u32x4{0u, 0u, 0u, 0u};
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4, ring[p]), __builtin_bit_cast(i32x4, xv),
                                                        acc, 0, 0, 0);
            ring[p] = ldnt16(wp + int64_t(min(i + RING, last)) * wstride);
            xring[p] = *reinterpret_cast<const u32x4*>(xp + min(i + RING, last) * 64);
            __builtin_amdgcn_sched_barrier(0);  // both refills stay here, RING chunks ahead of their use
        }
    }
    if (a.KS > 1) {
        *reinterpret_cast<i32x4*>(red8 + ((ts * a.KS + slice) * 64 + lane) * 4) = acc;
        __syncthreads();
        if (slice != 0) return;
        for (int k = 1; k < a.KS; ++k) acc += *reinterpret_cast<const i32x4*>(red8 + ((ts * a.KS + k) * 64 + lane) * 4);
    }
    if (!live || c >= a.rows) return;
    const float xs = a.xs[c];
    const int n0 = tile * 16 + 4 * g;
    const f32x4 sw = *reinterpret_cast<const f32x4*>(a.ws + n0);
    uint16_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f2bf(scaleback(acc[i], xs, sw[i]));
    // four consecutive outputs of row c: one 8-byte store
    *reinterpret_cast<uint2*>(a.out + int64_t(c) * a.N + n0) =
        make_uint2(uint32_t(o[0]) | (uint32_t(o[1]) << 16), uint32_t(o[2]) | (uint32_t(o[3]) << 16));
}

}  // namespace
}  // namespace mdx

using namespace mdx;

extern "C" int mdx_int8_linear(const int8_t* x, const float* x_scale, const int8_t* w, const float* w_scale,
                               int32_t layout, uint16_t* out, int64_t rows, int64_t N, int64_t K, void* stream) {
    MDX_CHECK(x && x_scale && w && w_scale && out, "null pointer");
    MDX_CHECK(rows >= 1 && rows <= 16, "1 <= rows <= 16");
    MDX_CHECK(N >= 16 && N % 16 == 0 && N < (int64_t(1) << 31), "N % 16 == 0");
    MDX_CHECK(K >= 64 && K % 64 == 0 && K <= 65536, "K % 64 == 0, K <= 65536 (the int32 sum stays exact)");
    MDX_CHECK(layout == MDX_LAYOUT_ROW || layout == MDX_LAYOUT_TILE, "layout");
    MDX_CHECK(aligned(x, 16) && aligned(w, 16) && aligned(w_scale, 16) && aligned(out, 8),
              "16-byte aligned x / w / w_scale, 8-byte aligned out");
    const int tiles = int(N / 16), NC = int(K / 64);
    // split K until about 12 waves per CU are in flight (slices must divide the chunk count)
    int KS = 1;
    for (int d = 1; d <= 16; ++d)
        if (NC % d == 0) {
            KS = d;
            if (int64_t(tiles) * d >= 3072) break;
        }
    const int TPW = std::max(1, 4 / KS);
    W8Args a{x, x_scale, w, w_scale, out, int(N), int(K), int(rows), KS, TPW, tiles, layout};
    const int wgs = (tiles + TPW - 1) / TPW;
    const size_t lds = KS > 1 ? size_t(TPW) * KS * 64 * 4 * sizeof(int32_t) : 0;
    if (lds) allow_smem(reinterpret_cast<const void*>(&int8_linear_kernel<W8_RING>), lds);
    hipLaunchKernelGGL(int8_linear_kernel<W8_RING>, dim3(wgs), dim3(64 * TPW * KS), lds, static_cast<hipStream_t>(stream),
                       a);
    MDX_LAUNCHED();
    return MDX_OK;
}
