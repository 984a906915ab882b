// Row kernels of the MTP draft block (the fused draft-head ops of comfy_mono_decode_xpu/draft_head.py).
//
// Reference semantics (comfy-mono-decode-xpu, csrc/draft_fused.sycl):
//   draft_embed_norm_cat  :76-151  embedding row (int8 ConvRot: gather, scale, un-rotate; or a given bf16
//                                  row), then cat(RMSNorm_e(emb), RMSNorm_h(hidden))
//   draft_add_rmsnorm     :153-184 x = bf16(x + h) in place (no h: x unchanged), out = RMSNorm(x)
//   draft_sigmoid_mul     :186-203 out = bf16(a * bf16(sigmoid(gate))), gate = the second half of each
//                                  2 head_dim block of the q projection
//   draft_silu_mul        :205-218 out = bf16(bf16(silu(g)) * u) over the concatenated gate | up
//   draft_norm_rot_quant  :220-287 x = bf16(x + h) in place (optional), n = RMSNorm(x) (bf16), the
//                                  lm_head's ConvRot rotation xr = bf16(n_group . H256), scale =
//                                  max(amax(xr) / 127, 1e-30), q = clamp(rint(xr / bf16(scale)), -128, 127)
//
// The reference computes these in fp32 without a fixed reduction order (a draft only proposes tokens).
// Here every row op has one: the RMSNorm factor is the library's canonical one (row_rms_factor: lane
// partials, a 64-lane halving tree per 256-group, group sums in group order, IEEE divide and sqrt); the
// rotation is the exact fp64 FWHT of the row prep, rounded once to fp32 and once to bf16; sigmoid and
// SiLU are torch's own values of every bf16 input (lookup tables). So the CPU oracle restates every
// output bit for bit, and the reference's tolerance (1e-2 relative) bounds them against float64.
//
// Layout: one work-group per row, W = min(16, H / 256) waves; wave w owns the 256-groups w, w + W, ...;
// lane l holds elements 4 l .. 4 l + 3 of each of its groups in registers (GPW groups per wave).
#include <algorithm>

#include "mdx_common.hpp"
#include "mdx_row.hpp"

namespace mdx {
namespace {

constexpr int DR_MAXH = 16384;

enum DraftMode : int { DM_EMBED = 0, DM_ADDNORM = 1, DM_NRQ = 2 };

struct DraftArgs {
    int H;
    // DM_EMBED: the embedding row (gather: int8 q [V, H] * s[V] of token[row], clamped into [0, V); or a
    // given bf16 row emb[row]), the hidden row; out [rows, 2 H] = [RMSNorm_e(emb) | RMSNorm_h(hidden)]
    const int64_t* token;
    const int8_t* eq;
    const float* es;
    int64_t V;
    int unrot;
    const uint16_t* emb;
    const uint16_t* hidden;
    const uint16_t* we;
    const uint16_t* wh;
    float eps_e, eps_h;
    // DM_ADDNORM / DM_NRQ: x [rows, H] (x += h in place when h is given), norm weight w
    uint16_t* x;
    const uint16_t* h;
    const uint16_t* w;
    float eps;
    uint16_t* out;  // DM_EMBED: [rows, 2 H]; DM_ADDNORM: [rows, H]; DM_NRQ: xr [rows, H]
    int rot;        // DM_NRQ: MDX_ROT_NONE or MDX_ROT_H256
    int8_t* qx;     // DM_NRQ: int8 [rows, H] and scale [rows], or both null
    float* sx;
};

template <int GPW>
__device__ __forceinline__ void load_row(const uint16_t* p, int G, float (&v)[GPW][4], uint2 (&raw)[GPW]) {
    const int W = blockDim.x / 64, w = threadIdx.x / 64, lane = threadIdx.x % 64;
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) raw[gi] = *reinterpret_cast<const uint2*>(p + 256 * min(w + W * gi, G - 1) + 4 * lane);
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) unpack4(raw[gi], v[gi]);
}

template <int GPW>
__device__ __forceinline__ void store_row(uint16_t* p, int G, const float (&v)[GPW][4]) {
    const int W = blockDim.x / 64, w = threadIdx.x / 64, lane = threadIdx.x % 64;
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi)
        if (w + W * gi < G) *reinterpret_cast<uint2*>(p + 256 * (w + W * gi) + 4 * lane) = pack4(v[gi]);
}

// v <- bf16((v * r) * w) with the canonical factor r (every thread calls it)
template <int GPW>
__device__ __forceinline__ void rms_apply(float (&v)[GPW][4], const uint2 (&wraw)[GPW], int H, float eps, float* gsum) {
    const float r = row_rms_factor<GPW>(v, H, eps, gsum);
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) {
        float wv[4];
        unpack4(wraw[gi], wv);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[gi][e] = bfround(__fmul_rn(__fmul_rn(v[gi][e], r), wv[e]));
    }
}

template <int GPW>
__global__ __launch_bounds__(1024) void draft_row_kernel(DraftArgs a, int mode) {
    __shared__ float gsum[2][DR_MAXH / 256];
    __shared__ float wmax[16];
    const int W = blockDim.x / 64, w = threadIdx.x / 64, lane = threadIdx.x % 64;
    const int H = a.H, G = H / 256;
    const int64_t row = blockIdx.x;
    float v[GPW][4];
    uint2 raw[GPW], wraw[GPW];
    if (mode == DM_EMBED) {
        float hv[GPW][4];
        uint2 hraw[GPW], hwraw[GPW];
        if (a.eq) {
            int64_t t = a.token[row];
            t = t < 0 ? 0 : (t >= a.V ? a.V - 1 : t);
            const float sc = a.es[t];
            const int8_t* qr = a.eq + t * H + 4 * lane;
            uint32_t qw[GPW];
#pragma unroll
            for (int gi = 0; gi < GPW; ++gi) qw[gi] = *reinterpret_cast<const uint32_t*>(qr + 256 * min(w + W * gi, G - 1));
#pragma unroll
            for (int gi = 0; gi < GPW; ++gi)
#pragma unroll
                for (int e = 0; e < 4; ++e) v[gi][e] = __fmul_rn(float(int8_t(qw[gi] >> (8 * e))), sc);
            if (a.unrot) {
                // un-rotate: the group times H256, exact in fp64, then one rounding to fp32
#pragma unroll
                for (int gi = 0; gi < GPW; ++gi) {
                    double d[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) d[e] = double(v[gi][e]);
                    fwht256_lane(d, lane);
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[gi][e] = float(__dmul_rn(d[e], 0.0625));
                }
            }
#pragma unroll
            for (int gi = 0; gi < GPW; ++gi)
#pragma unroll
                for (int e = 0; e < 4; ++e) v[gi][e] = bfround(v[gi][e]);  // the embedding row is bf16
        } else if (a.token) {  // a bf16 table: the row at the token
            int64_t t = a.token[row];
            t = t < 0 ? 0 : (t >= a.V ? a.V - 1 : t);
            load_row<GPW>(a.emb + t * H, G, v, raw);
        } else {
            load_row<GPW>(a.emb + row * H, G, v, raw);
        }
        load_row<GPW>(a.hidden + row * H, G, hv, hraw);
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
            const int g = min(w + W * gi, G - 1);
            wraw[gi] = *reinterpret_cast<const uint2*>(a.we + 256 * g + 4 * lane);
            hwraw[gi] = *reinterpret_cast<const uint2*>(a.wh + 256 * g + 4 * lane);
        }
        rms_apply<GPW>(v, wraw, H, a.eps_e, gsum[0]);
        rms_apply<GPW>(hv, hwraw, H, a.eps_h, gsum[1]);
        store_row<GPW>(a.out + row * 2 * H, G, v);
        store_row<GPW>(a.out + row * 2 * H + H, G, hv);
        return;
    }
    // DM_ADDNORM / DM_NRQ: x (+ h, stored back), then the norm
    load_row<GPW>(a.x + row * H, G, v, raw);
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) wraw[gi] = *reinterpret_cast<const uint2*>(a.w + 256 * min(w + W * gi, G - 1) + 4 * lane);
    if (a.h) {
        float hv[GPW][4];
        uint2 hraw[GPW];
        load_row<GPW>(a.h + row * H, G, hv, hraw);
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi)
#pragma unroll
            for (int e = 0; e < 4; ++e) v[gi][e] = bfround(__fadd_rn(v[gi][e], hv[gi][e]));
        store_row<GPW>(a.x + row * H, G, v);  // every lane has read its elements of x above
    }
    rms_apply<GPW>(v, wraw, H, a.eps, gsum[0]);
    if (mode == DM_ADDNORM) {
        store_row<GPW>(a.out + row * H, G, v);
        return;
    }
    if (a.rot == MDX_ROT_H256) {
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
            double d[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) d[e] = double(v[gi][e]);
            fwht256_lane(d, lane);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[gi][e] = bfround(float(__dmul_rn(d[e], 0.0625)));
        }
    }
    store_row<GPW>(a.out + row * H, G, v);
    if (!a.qx) return;
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
    if (threadIdx.x == 0) a.sx[row] = s;
    const float div = bf2f(f2bf(s));  // the scale in the activation dtype (never 0: s >= 1e-30)
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) {
        const int g = w + W * gi;
        if (g < G) {
            uint32_t o = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int qv = int(fminf(fmaxf(rintf(__fdiv_rn(v[gi][e], div)), -128.f), 127.f));
                o |= (uint32_t(qv) & 0xFFu) << (8 * e);
            }
            *reinterpret_cast<uint32_t*>(a.qx + row * H + 256 * g + 4 * lane) = o;
        }
    }
}

int launch_draft_rows(const DraftArgs& a, int mode, int64_t rows, hipStream_t st) {
    const int G = a.H / 256, W = std::min(16, G), gpw = (G + W - 1) / W;
    const dim3 grid{unsigned(rows)}, block{unsigned(W * 64)};
    switch (gpw) {
        case 1: hipLaunchKernelGGL(draft_row_kernel<1>, grid, block, 0, st, a, mode); break;
        case 2: hipLaunchKernelGGL(draft_row_kernel<2>, grid, block, 0, st, a, mode); break;
        case 3: hipLaunchKernelGGL(draft_row_kernel<3>, grid, block, 0, st, a, mode); break;
        default: hipLaunchKernelGGL(draft_row_kernel<4>, grid, block, 0, st, a, mode); break;
    }
    MDX_LAUNCHED();
    return MDX_OK;
}

// out[r, i] = bf16(a[r, i] * sig[gate]), gate = qg[r * qg_row + (i / D) * 2 D + D + i % D]
__global__ __launch_bounds__(256) void draft_sigmoid_mul_kernel(const uint16_t* a, const uint16_t* qg, int64_t qg_row,
                                                                int64_t D, const uint16_t* sig, uint16_t* out,
                                                                int64_t rows, int64_t n) {
    const int64_t total = rows * n;
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += int64_t(gridDim.x) * 256) {
        const int64_t r = i / n, c = i % n;
        const uint16_t g = qg[r * qg_row + (c / D) * 2 * D + D + c % D];
        out[i] = f2bf(__fmul_rn(bf2f(a[i]), bf2f(sig[g])));
    }
}

// out[r, i] = bf16(silu[g] * u), g = gu[r * gu_row + i], u = gu[r * gu_row + n + i]
__global__ __launch_bounds__(256) void draft_silu_mul_kernel(const uint16_t* gu, int64_t gu_row, const uint16_t* silu,
                                                             uint16_t* out, int64_t rows, int64_t n) {
    const int64_t total = rows * n;
    for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += int64_t(gridDim.x) * 256) {
        const int64_t r = i / n, c = i % n;
        const uint16_t* p = gu + r * gu_row;
        out[i] = f2bf(__fmul_rn(bf2f(silu[p[c]]), bf2f(p[n + c])));
    }
}

int row_checks(int64_t rows, int64_t H) {
    MDX_CHECK(rows >= 0 && rows <= 65535, "rows (got %lld)", (long long)rows);
    MDX_CHECK(H >= 256 && H % 256 == 0 && H <= DR_MAXH, "hidden size: a multiple of 256, at most %d (got %lld)",
              DR_MAXH, (long long)H);
    return MDX_OK;
}

}  // namespace
}  // namespace mdx

using namespace mdx;

extern "C" int mdx_draft_embed_norm_cat(const int64_t* token, const int8_t* q, const float* s, int64_t V,
                                        int32_t unrotate, const uint16_t* emb, const uint16_t* hidden,
                                        const uint16_t* we, const uint16_t* wh, float eps_e, float eps_h,
                                        uint16_t* out, int64_t rows, int64_t H, void* stream) {
    if (int rc = row_checks(rows, H)) return rc;
    MDX_CHECK(hidden && we && wh && out, "null pointer");
    MDX_CHECK(q ? (token && s && V >= 1 && aligned(q, 4) && (H % 4) == 0) : (emb != nullptr && (!token || V >= 1)),
              "an int8 embedding table with token and scales, a bf16 table with token, or a bf16 embedding row");
    MDX_CHECK(aligned(hidden, 8) && aligned(we, 8) && aligned(wh, 8) && aligned(out, 8) && (!emb || aligned(emb, 8)),
              "8-byte aligned rows");
    if (rows == 0) return MDX_OK;
    DraftArgs a{};
    a.H = int(H);
    a.token = token;
    a.eq = q;
    a.es = s;
    a.V = V;
    a.unrot = unrotate;
    a.emb = q ? nullptr : emb;
    a.hidden = hidden;
    a.we = we;
    a.wh = wh;
    a.eps_e = eps_e;
    a.eps_h = eps_h;
    a.out = out;
    return launch_draft_rows(a, DM_EMBED, rows, static_cast<hipStream_t>(stream));
}

extern "C" int mdx_draft_add_rmsnorm(uint16_t* x, const uint16_t* h, const uint16_t* w, float eps, uint16_t* out,
                                     int64_t rows, int64_t H, void* stream) {
    if (int rc = row_checks(rows, H)) return rc;
    MDX_CHECK(x && w && out, "null pointer");
    MDX_CHECK(aligned(x, 8) && aligned(w, 8) && aligned(out, 8) && (!h || aligned(h, 8)), "8-byte aligned rows");
    if (rows == 0) return MDX_OK;
    DraftArgs a{};
    a.H = int(H);
    a.x = x;
    a.h = h;
    a.w = w;
    a.eps = eps;
    a.out = out;
    return launch_draft_rows(a, DM_ADDNORM, rows, static_cast<hipStream_t>(stream));
}

extern "C" int mdx_draft_norm_rot_quant(uint16_t* x, const uint16_t* h, const uint16_t* w, float eps, int32_t rot,
                                        uint16_t* xr, int8_t* qx, float* sx, int64_t rows, int64_t H, void* stream) {
    if (int rc = row_checks(rows, H)) return rc;
    MDX_CHECK(x && w && xr, "null pointer");
    MDX_CHECK((qx == nullptr) == (sx == nullptr), "qx and sx both given or both null");
    MDX_CHECK(rot == MDX_ROT_NONE || rot == MDX_ROT_H256, "rotation: none or H256");
    MDX_CHECK(aligned(x, 8) && aligned(w, 8) && aligned(xr, 8) && (!h || aligned(h, 8)) && (!qx || aligned(qx, 4)),
              "aligned rows");
    if (rows == 0) return MDX_OK;
    DraftArgs a{};
    a.H = int(H);
    a.x = x;
    a.h = h;
    a.w = w;
    a.eps = eps;
    a.out = xr;
    a.rot = rot;
    a.qx = qx;
    a.sx = sx;
    return launch_draft_rows(a, DM_NRQ, rows, static_cast<hipStream_t>(stream));
}

extern "C" int mdx_draft_sigmoid_mul(const uint16_t* a, const uint16_t* qg, int64_t qg_row_stride, int64_t head_dim,
                                     const uint16_t* sig_lut, uint16_t* out, int64_t rows, int64_t n, void* stream) {
    MDX_CHECK(a && qg && sig_lut && out, "null pointer");
    MDX_CHECK(rows >= 0 && n >= 0 && head_dim >= 1 && n % head_dim == 0 && qg_row_stride >= 2 * n,
              "a [rows, n], qg [rows, >= 2 n] with n a multiple of head_dim");
    if (rows == 0 || n == 0) return MDX_OK;
    const int64_t blocks = std::min<int64_t>((rows * n + 255) / 256, 1024);
    hipLaunchKernelGGL(draft_sigmoid_mul_kernel, dim3(unsigned(blocks)), dim3(256), 0, static_cast<hipStream_t>(stream), a,
                       qg, qg_row_stride, head_dim, sig_lut, out, rows, n);
    MDX_LAUNCHED();
    return MDX_OK;
}

extern "C" int mdx_draft_silu_mul(const uint16_t* gu, int64_t gu_row_stride, const uint16_t* silu_lut, uint16_t* out,
                                  int64_t rows, int64_t n, void* stream) {
    MDX_CHECK(gu && silu_lut && out, "null pointer");
    MDX_CHECK(rows >= 0 && n >= 0 && gu_row_stride >= 2 * n, "gu [rows, >= 2 n]");
    if (rows == 0 || n == 0) return MDX_OK;
    const int64_t blocks = std::min<int64_t>((rows * n + 255) / 256, 1024);
    hipLaunchKernelGGL(draft_silu_mul_kernel, dim3(unsigned(blocks)), dim3(256), 0, static_cast<hipStream_t>(stream), gu,
                       gu_row_stride, silu_lut, out, rows, n);
    MDX_LAUNCHED();
    return MDX_OK;
}
