// bf16 decode linear for 1..16 rows: out[m, n] = bf16(sum_k x[m, k] * W[n, k]) with fp32 accumulation,
// optional bf16 residual (out = bf16(float(res) + float(bf16(acc)))). Serves the lm_head and the bf16
// projections of the MTP draft block.
//
// Reference: the lm_head is a library F.linear in the reference's loop (comfy_mono_decode_xpu/
// mtp_loop.py:221-225; draft_head.py:214-232 for the draft's head and block GEMMs); tolerance parity
// against float64 (bf16 outputs within 1e-2 relative).
//
// Every product is one v_mfma_f32_16x16x32_bf16: A = 16 weight rows x 32 k (one 16-byte load per
// lane: 1 KiB of the tile-major weight stream per wave instruction), B = the activation rows as
// columns (rows >= `rows` are zero), D = 16 outputs x 16 rows. A wave owns a 16-row tile of W and a
// K slice; slices of one tile (split-K when there are few tiles) add up in LDS in slice order.
// Weights stream through a register ring of RING loads per lane with clamped addresses (no branches
// in the loop, static wait counts).
//
// Tile-major weights: [N/16][K/32][64 lanes][8 bf16], lane 16 g + c holding row 16 t + c, k in
// [32 j + 8 g, 32 j + 8 g + 8) of block (t, j). Row-major [N, K] weights are read in place.
#include <stdlib.h>

#include <algorithm>

#include "mdx_common.hpp"

namespace mdx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int BF_RING = 4;
constexpr int BF_STREAM_RING = 8;  // bf16_stream_kernel (RING 4: 201 us, 16: 200 us against 197 us per lm_head launch)

struct Bf16Args {
    const uint16_t* x;     // [rows, K]
    const uint16_t* w;
    const uint16_t* res;   // [rows, N] or null
    uint16_t* out;         // [rows, N]
    int N, K, rows, KS, TPW, tiles, layout;
    int TW;                // bf16_stream_kernel: tiles per wave
};

__device__ __forceinline__ u32x4 ldnt(const uint16_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

template <int RING>
__global__ __launch_bounds__(1024) void bf16_linear_kernel(Bf16Args a) {
    extern __shared__ __align__(16) float red[];  // [TPW][KS][64][4]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ts = wave / a.KS, slice = wave % a.KS;
    const int tile = blockIdx.x * a.TPW + ts;
    const bool live = tile < a.tiles;
    const int NC = a.K / 32;
    const int c0 = live ? slice * NC / a.KS : 0, c1 = live ? (slice + 1) * NC / a.KS : 0;
    const int nch = c1 - c0, last = nch > 0 ? nch - 1 : 0;
    const int g = lane >> 4, c = lane & 15;
    const uint16_t* wp;
    int wstride;
    if (a.layout == MDX_LAYOUT_TILE) {
        wp = a.w + (int64_t(live ? tile : 0) * NC + c0) * 512 + lane * 8;
        wstride = 512;
    } else {
        wp = a.w + int64_t((live ? tile : 0) * 16 + c) * a.K + c0 * 32 + 8 * g;
        wstride = 32;
    }
    // weights and activation both travel in the ring (RING chunks ahead); whole ring rounds without
    // conditions around the loads (a chunk past the slice re-reads the last one and adds nothing)
    const bool xlive = c < a.rows;
    const uint16_t* xp = a.x + (xlive ? c : 0) * a.K + c0 * 32 + 8 * g;
    u32x4 ring[RING], xring[RING];
#pragma unroll
    for (int p = 0; p < RING; ++p) {
        // the same issue order as the loop's refills (static wait counts hold for every round)
        ring[p] = ldnt(wp + min(p, last) * wstride);
        xring[p] = *reinterpret_cast<const u32x4*>(xp + min(p, last) * 32);
        __builtin_amdgcn_sched_barrier(0);
    }
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int i0 = 0; i0 < nch; i0 += RING) {
#pragma unroll
        for (int p = 0; p < RING; ++p) {
            // consume the slot, then refill it (the old and new values never live at once, so the ring
            // keeps its registers across iterations instead of being copied at the loop end)
            const int i = i0 + p;
            u32x4 xv = xring[p];
            if (!xlive || i >= nch) xv = u32x4{0u, 0u, 0u, 0u};
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ring[p]), __builtin_bit_cast(bf16x8, xv),
                                                          acc, 0, 0, 0);
            ring[p] = ldnt(wp + min(i + RING, last) * wstride);
            xring[p] = *reinterpret_cast<const u32x4*>(xp + min(i + RING, last) * 32);
            __builtin_amdgcn_sched_barrier(0);  // both refills stay here, RING chunks ahead of their use
        }
    }
    // D: lane holds outputs n = 16 tile + 4 g + i of row c
    *reinterpret_cast<f32x4*>(red + ((ts * a.KS + slice) * 64 + lane) * 4) = acc;
    __syncthreads();
    if (slice != 0 || !live || c >= a.rows) return;
    // the slices' partials added in slice order; their reads four at a time (clamped, masked), so a
    // round trip to LDS serves four slices
    f32x4 s = acc;
    for (int k0 = 1; k0 < a.KS; k0 += 4) {
        f32x4 v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = *reinterpret_cast<const f32x4*>(red + ((ts * a.KS + min(k0 + j, a.KS - 1)) * 64 + lane) * 4);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (k0 + j < a.KS) s += v[j];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t o = int64_t(c) * a.N + tile * 16 + 4 * g + i;
        uint16_t v = f2bf(s[i]);
        if (a.res) v = f2bf(__fadd_rn(bf2f(a.res[o]), bf2f(v)));
        a.out[o] = v;
    }
}

// Many tiles (no split-K), tile-major weights: each wave streams TW consecutive tiles (TW x K / 32
// chunks of 1 KiB, contiguous in the tile-major layout) through one ring that runs on across the tile
// boundaries, and stores each tile's outputs from its accumulators as the tile completes (the same
// MFMA chain per tile as bf16_linear_kernel, so the same bits). About 2048-2560 waves in all: the whole
// grid is resident at once, instead of a last partial round of work-groups on a few CUs.
template <int RING>
__global__ __launch_bounds__(256) void bf16_stream_kernel(Bf16Args a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t0 = (blockIdx.x * (blockDim.x >> 6) + wave) * a.TW;
    const int nt = min(a.TW, a.tiles - t0);  // this wave's tiles
    if (nt <= 0) return;                     // (whole waves; the kernel has no barrier)
    const int NC = a.K / 32, total = nt * NC, last = total - 1;
    const int g = lane >> 4, c = lane & 15;
    const uint16_t* wp = a.w + int64_t(t0) * NC * 512 + lane * 8;
    const bool xlive = c < a.rows;
    const uint16_t* xp = a.x + (xlive ? c : 0) * a.K + 8 * g;
    u32x4 ring[RING], xring[RING];
    int rk = 0;  // the k chunk (within its tile) of the next refill
#pragma unroll
    for (int p = 0; p < RING; ++p) {
        ring[p] = ldnt(wp + min(p, last) * 512);
        xring[p] = *reinterpret_cast<const u32x4*>(xp + rk * 32);
        rk = rk + 1 == NC ? 0 : rk + 1;
        __builtin_amdgcn_sched_barrier(0);
    }
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    int ck = 0, tile = t0;  // chunks of the current tile consumed
    for (int i0 = 0; i0 < total; i0 += RING) {  // (NC % RING == 0: whole rounds end with the last tile)
#pragma unroll
        for (int p = 0; p < RING; ++p) {
            const int i = i0 + p;
            u32x4 xv = xring[p];
            if (!xlive) xv = u32x4{0u, 0u, 0u, 0u};
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ring[p]), __builtin_bit_cast(bf16x8, xv),
                                                          acc, 0, 0, 0);
            ring[p] = ldnt(wp + min(i + RING, last) * 512);
            xring[p] = *reinterpret_cast<const u32x4*>(xp + rk * 32);
            rk = rk + 1 == NC ? 0 : rk + 1;
            __builtin_amdgcn_sched_barrier(0);
            if (++ck == NC) {  // (uniform) the tile is complete: lane holds outputs 16 tile + 4 g + j of row c
                if (xlive) {
                    const int64_t o = int64_t(c) * a.N + tile * 16 + 4 * g;
                    uint16_t v[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        v[j] = f2bf(acc[j]);
                        if (a.res) v[j] = f2bf(__fadd_rn(bf2f(a.res[o + j]), bf2f(v[j])));
                    }
                    *reinterpret_cast<uint2*>(a.out + o) =
                        make_uint2(uint32_t(v[0]) | (uint32_t(v[1]) << 16), uint32_t(v[2]) | (uint32_t(v[3]) << 16));
                }
                acc = f32x4{0.f, 0.f, 0.f, 0.f};
                ck = 0;
                ++tile;
            }
        }
    }
}

}  // namespace
}  // namespace mdx

using namespace mdx;

extern "C" int mdx_bf16_linear(const uint16_t* x, const uint16_t* w, int32_t layout, const uint16_t* residual,
                               uint16_t* out, int64_t rows, int64_t N, int64_t K, void* stream) {
    MDX_CHECK(x && w && out, "null pointer");
    MDX_CHECK(rows >= 1 && rows <= 16, "1 <= rows <= 16");
    MDX_CHECK(N >= 16 && N % 16 == 0 && K >= 32 && K % 32 == 0 && N < (int64_t(1) << 31) && K <= 65536,
              "N % 16 == 0, K % 32 == 0");
    MDX_CHECK(layout == MDX_LAYOUT_ROW || layout == MDX_LAYOUT_TILE, "layout");
    MDX_CHECK(aligned(x, 16) && aligned(w, 16), "16-byte aligned x / w");
    const int tiles = int(N / 16), NC = int(K / 32);
    // split K until about 12 waves per CU are in flight (slices must divide the chunk count)
    int KS = 1;
    for (int d = 1; d <= 16; ++d)
        if (NC % d == 0) {
            KS = d;
            if (int64_t(tiles) * d >= 3072) break;
        }
    const int TPW = std::max(1, 4 / KS);
    Bf16Args a{x, w, residual, out, int(N), int(K), int(rows), KS, TPW, tiles, layout, 1};
    if (KS == 1 && layout == MDX_LAYOUT_TILE && NC % BF_STREAM_RING == 0 && aligned(out, 8) && !getenv("MDX_BF16_NOSTREAM")) {
        // the fewest tiles per wave that keep the whole grid resident (32 waves per CU): the lm_head's
        // 9496 tiles at two per wave, 197 us per 1.24 GB launch against 207 us for one tile per wave
        // (three per wave: 218 us)
        static const int resident = [] {
            int dev = 0, cus = 256;
            if (hipGetDevice(&dev) == hipSuccess) hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
            return 32 * std::max(cus, 1);
        }();
        a.TW = (tiles + resident - 1) / resident;
        const int waves = (tiles + a.TW - 1) / a.TW;
        hipLaunchKernelGGL(bf16_stream_kernel<BF_STREAM_RING>, dim3(unsigned((waves + 3) / 4)), dim3(256), 0,
                           static_cast<hipStream_t>(stream), a);
        MDX_LAUNCHED();
        return MDX_OK;
    }
    const int wgs = (tiles + TPW - 1) / TPW;
    const size_t lds = size_t(TPW) * KS * 64 * 4 * sizeof(float);
    allow_smem(reinterpret_cast<const void*>(&bf16_linear_kernel<BF_RING>), lds);
    hipLaunchKernelGGL(bf16_linear_kernel<BF_RING>, dim3(wgs), dim3(64 * TPW * KS), lds,
                       static_cast<hipStream_t>(stream), a);
    MDX_LAUNCHED();
    return MDX_OK;
}
