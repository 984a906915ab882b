// Gated-DeltaNet step pieces shared by the standalone core (mdx_gdn.hip) and the projection GEMV that
// runs them in its own launch (mdx_gemv.hip): a row's gates, the tree ancestry of the causal conv, and the
// conv of one channel over this step's rows.
//
// Reference semantics (comfy-mono-decode-xpu): csrc/mono_gdn.sycl:313-374 (conv over tree ancestors and
// the shifted history, silu), :424-450 (a / b projections, decay and beta). Buffers as in mdx_gdn.hip:
// conv_state bf16 [C, 3]; pb, qb bf16 [2 parities][slots][C]; gates f32 [2][slots][HV][2]; ctl int32
// [2 + 3 slots] = pending, parity, accepted slots, parents, program.
#pragma once

#include "mdx_common.hpp"

namespace mdx {

constexpr int GDN_DH = 128, GDN_CW = 3, GDN_MAXS = 16;

// Whether a step's control words are usable: parity 0 / 1 and 0 <= pending <= slots.
__device__ __forceinline__ bool gdn_ctl_ok(int pending, int p, int slots) {
    return p >= 0 && p <= 1 && pending >= 0 && pending <= slots;
}

// Row ts's gates for value head h, computed by one wave: a = xn . wa[h] and b = xn . wb[h] (lane l sums its
// elements in order, the 8-element blocks l + 64 j, then a halving tree over the lanes; both rounded to
// bf16), then decay = exp(g_decay * softplus(a + dt_bias)) (softplus(x) = x above 20) and beta =
// bf16(sigmoid(b)). Lane 0's values are the results. K % 8 == 0, K <= 4096. The loads go out NB blocks
// at a time (8: all at once; fewer: fewer registers, the same sums).
template <int NB = 8>
__device__ __forceinline__ void gdn_gate_row(const uint16_t* xn_row, const uint16_t* wa_h, const uint16_t* wb_h, int K,
                                             float dt_bias, float g_decay, int lane, float& decay, float& beta) {
    static_assert(8 % NB == 0, "NB divides 8");
    float pa = 0.f, pb = 0.f;
#pragma unroll
    for (int i0 = 0; i0 < 8; i0 += NB) {
        uint4 xv[NB], av[NB], bv[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int b0 = lane + 64 * (i0 + j);
            const int bc = b0 < K / 8 ? b0 : 0;  // unconditional loads, masked below
            xv[j] = *reinterpret_cast<const uint4*>(xn_row + 8 * bc);
            av[j] = *reinterpret_cast<const uint4*>(wa_h + 8 * bc);
            bv[j] = *reinterpret_cast<const uint4*>(wb_h + 8 * bc);
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            if (lane + 64 * (i0 + j) >= K / 8) continue;
            const uint32_t xw[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
            const uint32_t aw[4] = {av[j].x, av[j].y, av[j].z, av[j].w};
            const uint32_t bw[4] = {bv[j].x, bv[j].y, bv[j].z, bv[j].w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int sh = (e & 1) ? 0 : 16;
                const uint32_t m = (e & 1) ? 0xFFFF0000u : 0xFFFFFFFFu;
                const float xe = __uint_as_float((xw[e >> 1] << sh) & m);
                pa = fmaf(xe, __uint_as_float((aw[e >> 1] << sh) & m), pa);
                pb = fmaf(xe, __uint_as_float((bw[e >> 1] << sh) & m), pb);
            }
        }
    }
    pa = tree_sum64(pa);
    pb = tree_sum64(pb);
    const float avv = __fadd_rn(bfround(pa), dt_bias);
    const float sp = avv > 20.f ? avv : log1pf(expf(avv));
    decay = expf(__fmul_rn(g_decay, sp));
    beta = bfround(__fdiv_rn(1.f, __fadd_rn(1.f, expf(-bfround(pb)))));
}

// The ancestry of tree row r (the same for every channel): byte d - 1 says where the conv tap at distance d
// reads, an earlier row of this step (0 .. R - 1) or history entry 16 + (CW - the number of taps so far that
// fell before this step).
__device__ __forceinline__ uint32_t gdn_ancestry(int r, int R, const int* parent) {
    int anc = r, miss = 0;
    uint32_t code = 0;
#pragma unroll
    for (int d = 1; d <= GDN_CW; ++d) {
        anc = anc >= 0 ? parent[anc] : -1;
        anc = anc >= R ? -1 : anc;  // a parent is an earlier row of this step
        miss += anc < 0;
        code |= uint32_t(anc >= 0 ? anc : 16 + GDN_CW - miss) << (8 * (d - 1));
    }
    return code;
}

// The causal conv (kernel 4) of channel c for this step, by one thread: the history shifted by the
// previous step's accepted rows (pending of them, slots acc[0..pending) of parity 1 - p) is written back
// to conv_state; each row ts < R gets y = bf16(fma chain of its taps) and out = bf16(y / (1 + e^-y)) in
// qb[p][ts][c], its projection in pb[p][ts][c]; rows R .. slots - 1 get zeros. proj_at(r): row r's bf16
// projection of the channel; anct[r]: gdn_ancestry of row r.
template <typename ProjAt>
__device__ __forceinline__ void gdn_conv_channel(int c, int64_t C, int R, int S, int pending, int p, const int* acc,
                                                 const uint32_t* anct, ProjAt proj_at, const uint16_t* conv_w,
                                                 uint16_t* conv_state, uint16_t* pb, uint16_t* qb) {
    constexpr int CW = GDN_CW;
    uint16_t old[CW], prevacc[CW];
#pragma unroll
    for (int r = 0; r < CW; ++r) {
        old[r] = conv_state[c * CW + r];
        const int j = pending + r - CW;
        int slot = acc[j < 0 ? 0 : j];
        slot = slot < 0 ? 0 : (slot >= S ? S - 1 : slot);
        prevacc[r] = pb[((1 - p) * S + slot) * C + c];
    }
    float w[CW + 1];
#pragma unroll
    for (int d = 0; d <= CW; ++d) w[d] = bf2f(conv_w[c * (CW + 1) + d]);
    uint16_t hist[CW];
#pragma unroll
    for (int r = 0; r < CW; ++r) {
        const int j = pending + r;
        hist[r] = j == 0 ? old[0] : (j == 1 ? old[1] : (j == 2 ? old[2] : prevacc[r]));
    }
#pragma unroll
    for (int r = 0; r < CW; ++r) conv_state[c * CW + r] = hist[r];
#pragma unroll
    for (int ts = 0; ts < GDN_MAXS; ++ts) {
        if (ts >= S) break;
        uint16_t out = 0, prv = 0;
        if (ts < R) {
            prv = proj_at(ts);
            const uint32_t code = anct[ts];
            float sum = fmaf(bf2f(prv), w[CW], 0.f);
#pragma unroll
            for (int d = 1; d <= CW; ++d) {
                const int src = (code >> (8 * (d - 1))) & 0xFF;
                const uint16_t hv = src == 16 ? hist[0] : (src == 17 ? hist[1] : hist[2]);
                const float v = src < 16 ? bf2f(proj_at(src)) : bf2f(hv);
                sum = fmaf(v, w[CW - d], sum);
            }
            const float y = bfround(sum);
            out = f2bf(__fdiv_rn(y, __fadd_rn(1.f, expf(-y))));
        }
        qb[(p * S + ts) * C + c] = out;
        pb[(p * S + ts) * C + c] = prv;
    }
}

// The same conv, one row per lane: row ts (< S) of channel c, the channel's rows on lanes of ONE wave.
// Every lane loads the channel's history and shifts it; the row-0 lane writes it back, an instruction
// after the wave's loads of it have returned (its data is the store's), so no lane reads the new state.
// Row ts < R: its ancestry (gdn_ancestry, three LDS reads), its taps and out as above; rows R .. S - 1
// store zeros. Bit-identical to gdn_conv_channel.
template <typename ProjAt>
__device__ __forceinline__ void gdn_conv_row(int c, int64_t C, int ts, int R, int S, int pending, int p,
                                             const int* acc, const int* parent, ProjAt proj_at,
                                             const uint16_t* conv_w, uint16_t* conv_state, uint16_t* pb,
                                             uint16_t* qb) {
    constexpr int CW = GDN_CW;
    uint16_t old[CW], prevacc[CW];
#pragma unroll
    for (int r = 0; r < CW; ++r) {
        old[r] = conv_state[c * CW + r];
        const int j = pending + r - CW;
        int slot = acc[j < 0 ? 0 : j];
        slot = slot < 0 ? 0 : (slot >= S ? S - 1 : slot);
        prevacc[r] = pb[((1 - p) * S + slot) * C + c];
    }
    float w[CW + 1];
#pragma unroll
    for (int d = 0; d <= CW; ++d) w[d] = bf2f(conv_w[c * (CW + 1) + d]);
    const bool live = ts < R;
    // the row's taps from LDS before the history arrives (clamped indices: no branches)
    const uint32_t code = gdn_ancestry(live ? ts : 0, R, parent);
    const uint16_t prv = live ? proj_at(ts) : uint16_t(0);
    uint16_t tap[CW];
#pragma unroll
    for (int d = 1; d <= CW; ++d) {
        const int src = (code >> (8 * (d - 1))) & 0xFF;
        tap[d - 1] = proj_at(src < 16 ? src : 0);
    }
    uint16_t hist[CW];
#pragma unroll
    for (int r = 0; r < CW; ++r) {
        const int j = pending + r;
        hist[r] = j == 0 ? old[0] : (j == 1 ? old[1] : (j == 2 ? old[2] : prevacc[r]));
    }
    if (ts == 0) {
#pragma unroll
        for (int r = 0; r < CW; ++r) conv_state[c * CW + r] = hist[r];
    }
    float sum = fmaf(bf2f(prv), w[CW], 0.f);
#pragma unroll
    for (int d = 1; d <= CW; ++d) {
        const int src = (code >> (8 * (d - 1))) & 0xFF;
        const uint16_t hv = src == 16 ? hist[0] : (src == 17 ? hist[1] : hist[2]);
        sum = fmaf(bf2f(src < 16 ? tap[d - 1] : hv), w[CW - d], sum);
    }
    const float y = bfround(sum);
    const uint16_t out = live ? f2bf(__fdiv_rn(y, __fadd_rn(1.f, expf(-y)))) : uint16_t(0);
    qb[(p * S + ts) * C + c] = out;
    pb[(p * S + ts) * C + c] = prv;
}

}  // namespace mdx
