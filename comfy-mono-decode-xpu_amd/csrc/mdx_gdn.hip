// Gated-DeltaNet decode core with deferred replay, for 1..16 tree-verify rows: the causal conv over
// tree ancestors, the gates, the q/k sums of squares, the delta-rule state update (replay of the
// previous step's accepted rows, then this step's verify program) and the gated RMSNorm.
//
// Reference semantics (comfy-mono-decode-xpu): csrc/mono_gdn.sycl:313-374 (conv), :424-450 (gates),
// :459-479 (sums), :398-571 (entries: replay of ctl's accepted slots from the previous parity, always
// committed; verify entries prog & 15 = slot, prog & 32 = commit; the persistent state keeps the replay
// only), :574-607 (gated RMSNorm). Tolerance parity against a float64 restatement (the reference's
// own arithmetic is Kitchen's fast-math build, not portable); the control walk (entry list, slots,
// ancestry, the buffers of the next step) is exact.
//
// Buffers (per layer): conv_state bf16 [C, 3]; pb, qb bf16 [2 parities][slots][C] (projections and
// conv outputs of each step, kept for the next step's replay); rec f32 [HV][128][128] (row-major
// [head][k row][v col]); gates f32 [2][slots][HV][2] (decay, beta); sums f32 [2][slots][HK][2]
// (q, k sum of squares); ctl int32 [2 + 3 slots] = pending, parity, accepted slots, parents, program.
// Channels of proj / qb: q [0, KD), k [KD, 2 KD), v [2 KD, 2 KD + HV 128), KD = HK 128.
//
// Launches: gdn_conv_kernel (one thread per channel: owns its conv history; the q / k work-groups also
// take their heads' sums of squares; extra work-groups, four per value head, compute the gates beside
// them), then gdn_head_kernel (eight work-groups of 256 per value head, 16 state columns each: thread
// (row group rg, column col) holds state rows 8 rg .. 8 rg + 7 of its column in registers; raw bf16
// outputs), then the gated RMSNorm per head in place (the row-prep kernel's head-norm mode, which the
// decode stack instead fuses into the output projection's activation prep: mdx_gdn_core_raw +
// mdx_gnorm_rot_quant).
#include <math.h>

#include "mdx_common.hpp"

namespace mdx {
namespace {

constexpr int DH = 128, CW = 3;
constexpr int MAXS = 16;

struct GdnArgs {
    const uint16_t* proj;   // [R, C]
    const uint16_t* xn;     // [R, K]: the normalised layer input (a = xn . wa[h], b = xn . wb[h])
    const uint16_t* wa;     // [HV, K]
    const uint16_t* wb;     // [HV, K]
    int K;
    const uint16_t* conv_w; // [C, 4]
    uint16_t* conv_state;   // [C, 3]
    uint16_t* pb;           // [2][slots][C]
    uint16_t* qb;           // [2][slots][C]
    const int32_t* ctl;
    const float* dt_bias;   // [HV]
    const float* g_decay;   // [HV]
    float* rec;             // [HV][128][128]
    float* gates;           // [2][slots][HV][2]
    float* sums;            // [2][slots][HK][2]
    float qscale;
    uint16_t* core;         // [R, HV * 128]
    int R, HK, HV, C, slots;
};


// This step's gates of head h: one wave per row computes a = xn . wa[h] and b = xn . wb[h] (lane l
// sums its elements in order, the 8-element blocks l + 64 j, then a halving tree over the lanes; both
// rounded to bf16), then decay = exp(g_decay * softplus(a + dt_bias)) and beta = bf16(sigmoid(b)) into
// gates[p][row][h]; rows R .. slots - 1 get zeros. The four work-groups of a head share its rows.
__device__ __forceinline__ void gate_row(const GdnArgs& a, int h, int ts, int lane, float& decay, float& beta) {
    const uint16_t* x = a.xn + int64_t(ts) * a.K;
    const uint16_t* wa = a.wa + int64_t(h) * a.K;
    const uint16_t* wb = a.wb + int64_t(h) * a.K;
    uint4 xv[8], av[8], bv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int b0 = lane + 64 * i;
        const int bc = b0 < a.K / 8 ? b0 : 0;  // unconditional loads, masked below
        xv[i] = *reinterpret_cast<const uint4*>(x + 8 * bc);
        av[i] = *reinterpret_cast<const uint4*>(wa + 8 * bc);
        bv[i] = *reinterpret_cast<const uint4*>(wb + 8 * bc);
    }
    float pa = 0.f, pb = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (lane + 64 * i >= a.K / 8) continue;
        const uint32_t xw[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
        const uint32_t aw[4] = {av[i].x, av[i].y, av[i].z, av[i].w};
        const uint32_t bw[4] = {bv[i].x, bv[i].y, bv[i].z, bv[i].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int sh = (e & 1) ? 0 : 16;
            const uint32_t m = (e & 1) ? 0xFFFF0000u : 0xFFFFFFFFu;
            const float xe = __uint_as_float((xw[e >> 1] << sh) & m);
            pa = fmaf(xe, __uint_as_float((aw[e >> 1] << sh) & m), pa);
            pb = fmaf(xe, __uint_as_float((bw[e >> 1] << sh) & m), pb);
        }
    }
    pa = tree_sum64(pa);  // (lane 0's values are the ones used)
    pb = tree_sum64(pb);
    const float avv = __fadd_rn(bfround(pa), a.dt_bias[h]);
    const float sp = avv > 20.f ? avv : log1pf(expf(avv));
    decay = expf(__fmul_rn(a.g_decay[h], sp));
    beta = bfround(__fdiv_rn(1.f, __fadd_rn(1.f, expf(-bfround(pb)))));
}

__device__ void gdn_gates_part(const GdnArgs& a, int h, int quarter) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int R = a.R, S = a.slots;
    // the control words are checked at the stores only, so that their load overlaps the others
    const int pending = a.ctl[0], p = a.ctl[1];
    const bool ok = p >= 0 && p <= 1 && pending >= 0 && pending <= S;
    for (int ts = quarter * 4 + wv; ts < S; ts += 16) {
        float decay = 0.f, beta = 0.f;
        if (ts < R) gate_row(a, h, ts, lane, decay, beta);
        if (lane == 0 && ok) {
            a.gates[((p * S + ts) * a.HV + h) * 2] = decay;
            a.gates[((p * S + ts) * a.HV + h) * 2 + 1] = beta;
        }
    }
}

// One thread per channel (it owns the channel's history); the work-group stages its 256 channels'
// projection rows in LDS, so the ancestors of a tree row are LDS reads by index. A work-group of q or
// k channels (two heads) also takes the sums of squares of its heads' conv outputs per row (lane l:
// elements l and l + 64, then a halving tree) into sums[p][row][kh][q / k]. The work-groups after
// the channels' compute this step's gates (four per value head).
__global__ __launch_bounds__(256) void gdn_conv_kernel(GdnArgs a) {
    __shared__ int sctl[2 + 3 * MAXS];
    __shared__ uint32_t anct[MAXS];
    __shared__ uint16_t prl[MAXS][256];
    __shared__ float sq[MAXS][256];
    const int t = threadIdx.x;
    const int nconv = (a.C + 255) / 256;
    if (int(blockIdx.x) >= nconv) {
        const int b = blockIdx.x - nconv;
        gdn_gates_part(a, b / 4, b % 4);
        return;
    }
    const int c = blockIdx.x * 256 + t;
    if (t < 2 + 3 * a.slots) sctl[t] = a.ctl[t];
    const int R = a.R;
    const int64_t C = a.C;
    const bool cl = c < a.C;
    // every load up front (clamped addresses, no branches): this step's projections of the channel,
    // its history, the previous step's accepted rows, its weights
    uint16_t pr[MAXS];
#pragma unroll
    for (int r = 0; r < MAXS; ++r) pr[r] = a.proj[(r < R ? r : R - 1) * C + (cl ? c : 0)];
#pragma unroll
    for (int r = 0; r < MAXS; ++r) prl[r][t] = pr[r];
    __syncthreads();
    const int S = a.slots, pending = sctl[0], p = sctl[1];
    if (!(p >= 0 && p <= 1 && pending >= 0 && pending <= S)) return;  // uniform
    const int* acc = sctl + 2;
    const int* parent = sctl + 2 + S;
    // the ancestry of row t (the same for every channel), walked once: byte d - 1 says where the tap
    // at distance d reads, an earlier row of this step (0 .. R - 1) or history entry 16 + (CW - the
    // number of taps so far that fell before this step)
    if (t < R) {
        int anc = t, miss = 0;
        uint32_t code = 0;
#pragma unroll
        for (int d = 1; d <= CW; ++d) {
            anc = anc >= 0 ? parent[anc] : -1;
            anc = anc >= R ? -1 : anc;  // a parent is an earlier row of this step
            miss += anc < 0;
            code |= uint32_t(anc >= 0 ? anc : 16 + CW - miss) << (8 * (d - 1));
        }
        anct[t] = code;
    }
    __syncthreads();
    if (!cl) return;  // (only a last, partial work-group of v channels, which takes no sums)
    uint16_t old[CW], prevacc[CW];
#pragma unroll
    for (int r = 0; r < CW; ++r) {
        old[r] = a.conv_state[c * CW + r];
        const int j = pending + r - CW;
        int slot = acc[j < 0 ? 0 : j];
        slot = slot < 0 ? 0 : (slot >= S ? S - 1 : slot);
        prevacc[r] = a.pb[((1 - p) * S + slot) * C + c];
    }
    float w[CW + 1];
#pragma unroll
    for (int d = 0; d <= CW; ++d) w[d] = bf2f(a.conv_w[c * (CW + 1) + d]);
    // the history shifted by the previous step's accepted rows
    uint16_t hist[CW];
#pragma unroll
    for (int r = 0; r < CW; ++r) {
        const int j = pending + r;
        hist[r] = j == 0 ? old[0] : (j == 1 ? old[1] : (j == 2 ? old[2] : prevacc[r]));
    }
#pragma unroll
    for (int r = 0; r < CW; ++r) a.conv_state[c * CW + r] = hist[r];
#pragma unroll
    for (int ts = 0; ts < MAXS; ++ts) {
        if (ts >= S) break;
        uint16_t out = 0;
        if (ts < R) {
            const uint32_t code = anct[ts];
            float sum = fmaf(bf2f(prl[ts][t]), w[CW], 0.f);
#pragma unroll
            for (int d = 1; d <= CW; ++d) {
                const int src = (code >> (8 * (d - 1))) & 0xFF;
                const uint16_t hv = src == 16 ? hist[0] : (src == 17 ? hist[1] : hist[2]);
                const float v = src < 16 ? bf2f(prl[src][t]) : bf2f(hv);
                sum = fmaf(v, w[CW - d], sum);
            }
            const float y = bfround(sum);
            out = f2bf(__fdiv_rn(y, __fadd_rn(1.f, expf(-y))));
        }
        a.qb[(p * S + ts) * C + c] = out;
        a.pb[(p * S + ts) * C + c] = ts < R ? prl[ts][t] : uint16_t(0);
        if (ts < R) sq[ts][t] = bf2f(out);
    }
    // q / k heads of this work-group: sums of squares per row (the v channels have none)
    const int KD = a.HK * DH;
    if (int(blockIdx.x) * 256 >= 2 * KD) return;
    __syncthreads();
    const int lane = t & 63, wv = t >> 6;
    if (wv & 1) return;  // wave 2 j owns head j of the work-group (its elements 0..63; 64..127 from wave 2 j + 1)
    const int c0 = blockIdx.x * 256 + 128 * (wv >> 1);
    const int which = c0 >= KD, kh = (c0 - which * KD) / DH;
    for (int ts = 0; ts < R; ++ts) {
        const float v0 = sq[ts][64 * wv + lane], v1 = sq[ts][64 * wv + 64 + lane];
        float part = fmaf(v1, v1, __fmul_rn(v0, v0));
        part = tree_sum64(part);
        if (lane == 0) a.sums[((p * S + ts) * a.HK + kh) * 2 + which] = part;
    }
}

// The delta rule of value head h over the columns [16 cs, 16 cs + 16) of its state (eight work-groups
// per head, one per CU: the columns are independent, and a thread's serial work per entry is 8 rows).
// Wave w owns columns 4 w .. 4 w + 3; lane l holds state rows 8 rg .. 8 rg + 7 (rg = l / 4) of column
// 4 w + l % 4 in registers, so a column's 16 row groups are 16 lanes of one wave: the k.S and q.S sums
// over the rows finish with four exchanges inside the wave and the waves run their entries without
// barriers. Outputs: the raw bf16 rows of the verify
// entries (the gated RMSNorm, which needs the whole head, is applied by whoever reads them); rows of
// this step that no verify entry writes are zeros.
constexpr int NSPLIT = 8, SC = DH / NSPLIT, HRG = 16, HRPG = DH / HRG, HT = HRG * SC, VPE = SC / 8;

// v + (the value of lane l + 4 of lane l's row of 16, cyclically): DPP row_ror:4
__device__ __forceinline__ float sum_r4(float v) {
    return __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xF, 0xF, false)));
}

__global__ __launch_bounds__(HT) void gdn_head_kernel(GdnArgs a) {
    __shared__ __align__(16) float kvec[2 * MAXS][DH], qvec[MAXS][DH];
    __shared__ float vvec[2 * MAXS][SC], rawc[MAXS][SC];
    __shared__ float egate[2 * MAXS][4];  // decay, beta, 1 / |k|, 1 / |q|
    __shared__ int ectl[2 + 3 * MAXS];
    const int t = threadIdx.x, lane = t % 64, h = blockIdx.x / NSPLIT, cs = blockIdx.x % NSPLIT;
    const int S = a.slots, R = a.R, HV = a.HV, HK = a.HK, KD = HK * DH;
    const int kh = h / (HV / HK);
    const int64_t C = a.C;
    // the state of this work-group's columns first (it does not depend on the control words)
    const int col = (t / 64) * 4 + (lane & 3), rg = lane >> 2;
    float st[HRPG];
    float* rs = a.rec + (int64_t(h) * DH + rg * HRPG) * DH + cs * SC + col;
#pragma unroll
    for (int r = 0; r < HRPG; ++r) st[r] = rs[r * DH];
    if (t < 2 + 3 * S) ectl[t] = a.ctl[t];
    __syncthreads();
    const int pending = ectl[0], p = ectl[1];
    if (!(p >= 0 && p <= 1 && pending >= 0 && pending <= S)) return;  // (uniform) invalid control words
    const int* acc = ectl + 2;
    const int* prog = ectl + 2 + 2 * S;
    // the entries: the leading valid accepted slots (replayed when all `pending` are valid), then the
    // leading program entries with a valid row (each wave ballots the same counts)
    const bool v0 = lane < pending && acc[lane < S ? lane : 0] >= 0 && acc[lane < S ? lane : 0] < S;
    const int E0 = __builtin_ctzll(~__ballot(v0));
    const bool replayed = E0 == pending;
    const int pl = prog[lane < S ? lane : 0];
    const bool v1 = replayed && lane < R && pl >= 0 && (pl & 15) < R;
    const int E1 = replayed ? __builtin_ctzll(~__ballot(v1)) : 0;
    const int E = E0 + E1;
    auto slot_of = [&](int e) { return e < E0 ? acc[e] : (prog[e - E0] & 15); };
    // raw inputs, every load issued before the first use: k (16 pieces of 8 per entry) and v (4 per
    // entry) of every entry, q (16 per entry) of the verify entries; the entries' gates and norms
    constexpr int KP = 2 * MAXS * 16 / HT, VP = 2 * MAXS * VPE;
    uint4 kraw[KP], qraw = make_uint4(0u, 0u, 0u, 0u), vraw = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int j = 0; j < KP; ++j) kraw[j] = make_uint4(0u, 0u, 0u, 0u);
    if (E > 0) {  // (uniform) indices clamped into [0, E): every slot read is a validated one
#pragma unroll
    for (int j = 0; j < KP; ++j) {
        const int i = min(t + HT * j, E * 16 - 1), e = i / 16;
        const int ts = slot_of(e), par = e < E0 ? 1 - p : p;
        kraw[j] = *reinterpret_cast<const uint4*>(a.qb + (par * S + ts) * C + KD + kh * DH + (i % 16) * 8);
    }
    {
        const int i = min(t, max(E1 * 16 - 1, 0)), e = E0 + i / 16;
        qraw = *reinterpret_cast<const uint4*>(a.qb + (p * S + slot_of(min(e, E - 1))) * C + kh * DH + (i % 16) * 8);
    }
    if (t < VP) {
        const int i = min(t, E * VPE - 1), e = i / VPE;
        const int ts = slot_of(e), par = e < E0 ? 1 - p : p;
        vraw = *reinterpret_cast<const uint4*>(a.qb + (par * S + ts) * C + 2 * KD + h * DH + cs * SC + (i % VPE) * 8);
    }
    }
    if (t < E) {
        const int e = t, ts = slot_of(e), par = e < E0 ? 1 - p : p;
        const float* sm = a.sums + ((par * S + ts) * HK + kh) * 2;
        const float* gt = a.gates + ((par * S + ts) * HV + h) * 2;
        const float sq = sm[0], sk = sm[1];
        egate[e][0] = gt[0];
        egate[e][1] = gt[1];
        egate[e][2] = __fdiv_rn(1.f, fmaxf(sqrt_rn(sk), 1e-12f));
        egate[e][3] = __fdiv_rn(1.f, fmaxf(sqrt_rn(sq), 1e-12f));
    }
    __syncthreads();
    // scaled into LDS: k * ki, (q * scale) * qi, v
#pragma unroll
    for (int j = 0; j < KP; ++j) {
        const int i = t + HT * j;
        if (i < E * 16) {
            const int e = i / 16, d0 = (i % 16) * 8;
            const float ki = egate[e][2];
            const uint32_t w[4] = {kraw[j].x, kraw[j].y, kraw[j].z, kraw[j].w};
#pragma unroll
            for (int q = 0; q < 8; ++q)
                kvec[e][d0 + q] = __fmul_rn(__uint_as_float((q & 1) ? (w[q >> 1] & 0xFFFF0000u) : (w[q >> 1] << 16)), ki);
        }
    }
    if (t < E1 * 16) {
        const int e = E0 + t / 16, d0 = (t % 16) * 8;
        const float qi = egate[e][3];
        const uint32_t w[4] = {qraw.x, qraw.y, qraw.z, qraw.w};
#pragma unroll
        for (int q = 0; q < 8; ++q)
            qvec[e - E0][d0 + q] =
                __fmul_rn(__fmul_rn(__uint_as_float((q & 1) ? (w[q >> 1] & 0xFFFF0000u) : (w[q >> 1] << 16)), a.qscale), qi);
    }
    if (t < E * VPE) {
        const int e = t / VPE, d0 = (t % VPE) * 8;
        const uint32_t w[4] = {vraw.x, vraw.y, vraw.z, vraw.w};
#pragma unroll
        for (int q = 0; q < 8; ++q)
            vvec[e][d0 + q] = __uint_as_float((q & 1) ? (w[q >> 1] & 0xFFFF0000u) : (w[q >> 1] << 16));
    }
    __syncthreads();
    for (int e = 0; e < E; ++e) {
        const bool verify = e >= E0;
        const bool commit = !verify || (prog[e - E0] & 32);
        const float decay = egate[e][0], beta = egate[e][1];
        float kr[HRPG], qr[HRPG];
        const float4* k4 = reinterpret_cast<const float4*>(kvec[e] + rg * HRPG);
#pragma unroll
        for (int j = 0; j < HRPG / 4; ++j) {
            const float4 v = k4[j];
            kr[4 * j] = v.x, kr[4 * j + 1] = v.y, kr[4 * j + 2] = v.z, kr[4 * j + 3] = v.w;
        }
        if (verify) {
            const float4* q4 = reinterpret_cast<const float4*>(qvec[e - E0] + rg * HRPG);
#pragma unroll
            for (int j = 0; j < HRPG / 4; ++j) {
                const float4 v = q4[j];
                qr[4 * j] = v.x, qr[4 * j + 1] = v.y, qr[4 * j + 2] = v.z, qr[4 * j + 3] = v.w;
            }
        }
        // k.S over the thread's 8 rows: four interleaved accumulators, then ((m0 + m1) + (m2 + m3));
        // then the column's 16 row groups (lanes of one residue mod 4): row_ror 8 and 4 inside each row
        // of 16 lanes, then the lane swaps across rows; each step adds values that already agree in
        // pairs, so every lane of the column ends with the same sum
        float m4[4] = {0.f, 0.f, 0.f, 0.f};
        if (commit) {
#pragma unroll
            for (int r = 0; r < HRPG; ++r) {
                st[r] = __fmul_rn(st[r], decay);
                m4[r & 3] = fmaf(st[r], kr[r], m4[r & 3]);
            }
        } else {
#pragma unroll
            for (int r = 0; r < HRPG; ++r) m4[r & 3] = fmaf(__fmul_rn(st[r], decay), kr[r], m4[r & 3]);
        }
        float kv = __fadd_rn(__fadd_rn(m4[0], m4[1]), __fadd_rn(m4[2], m4[3]));
        kv = sum_x32(sum_x16(sum_r4(sum_x8(kv))));
        const float delta = __fmul_rn(__fsub_rn(vvec[e][col], kv), beta);
        float r4[4] = {0.f, 0.f, 0.f, 0.f};
        if (commit) {
#pragma unroll
            for (int r = 0; r < HRPG; ++r) st[r] = fmaf(kr[r], delta, st[r]);
            if (verify)
#pragma unroll
                for (int r = 0; r < HRPG; ++r) r4[r & 3] = fmaf(st[r], qr[r], r4[r & 3]);
        } else {
#pragma unroll
            for (int r = 0; r < HRPG; ++r) r4[r & 3] = fmaf(fmaf(kr[r], delta, __fmul_rn(st[r], decay)), qr[r], r4[r & 3]);
        }
        if (verify) {
            float o = __fadd_rn(__fadd_rn(r4[0], r4[1]), __fadd_rn(r4[2], r4[3]));
            o = sum_x32(sum_x16(sum_r4(sum_x8(o))));
            if (rg == 0) rawc[slot_of(e)][col] = bfround(o);
        }
        if (e == E0 - 1 && replayed)
#pragma unroll
            for (int r = 0; r < HRPG; ++r) rs[r * DH] = st[r];
    }
    __syncthreads();
    unsigned written = 0;
    for (int e = E0; e < E; ++e) written |= 1u << slot_of(e);
    for (int i = t; i < R * SC; i += HT) {
        const int ts = i / SC, c = i % SC;
        a.core[ts * HV * DH + h * DH + cs * SC + c] = ((written >> ts) & 1) ? f2bf(rawc[ts][c]) : uint16_t(0);
    }
}

}  // namespace
}  // namespace mdx

using namespace mdx;

namespace {

int gdn_run(const uint16_t* proj, const uint16_t* xn, const uint16_t* wa, const uint16_t* wb, int64_t K,
            const uint16_t* conv_w, uint16_t* conv_state, uint16_t* proj_buf, uint16_t* qkv_buf, const int32_t* ctl,
            const float* dt_bias, const float* g_decay, float* rec_state, float* gates, float* sums, float qscale,
            uint16_t* core, int64_t rows, int64_t HK, int64_t HV, int64_t slots, hipStream_t st) {
    MDX_CHECK(proj && xn && wa && wb && conv_w && conv_state && proj_buf && qkv_buf && ctl && dt_bias && g_decay &&
                  rec_state && gates && sums && core,
              "null pointer");
    MDX_CHECK(slots == 8 || slots == 16, "slots must be 8 or 16");
    MDX_CHECK(rows >= 1 && rows <= slots, "1 <= rows <= slots");
    MDX_CHECK(HK >= 1 && HV >= HK && HV % HK == 0 && HV % 2 == 0 && HV <= 128, "heads (HV even, <= 128)");
    MDX_CHECK(K >= 512 && K <= 4096 && K % 512 == 0 && aligned(xn, 16) && aligned(wa, 16) && aligned(wb, 16),
              "a / b input: K % 512 == 0, K <= 4096, 16-byte aligned rows");
    GdnArgs a{};
    a.proj = proj;
    a.xn = xn;
    a.wa = wa;
    a.wb = wb;
    a.K = int(K);
    a.conv_w = conv_w;
    a.conv_state = conv_state;
    a.pb = proj_buf;
    a.qb = qkv_buf;
    a.ctl = ctl;
    a.dt_bias = dt_bias;
    a.g_decay = g_decay;
    a.rec = rec_state;
    a.gates = gates;
    a.sums = sums;
    a.qscale = qscale;
    a.core = core;
    a.R = int(rows);
    a.HK = int(HK);
    a.HV = int(HV);
    a.C = int(2 * HK * DH + HV * DH);
    a.slots = int(slots);
    hipLaunchKernelGGL(gdn_conv_kernel, dim3((a.C + 255) / 256 + 4 * a.HV), dim3(256), 0, st, a);
    MDX_LAUNCHED();
    hipLaunchKernelGGL(gdn_head_kernel, dim3(a.HV * NSPLIT), dim3(HT), 0, st, a);
    MDX_LAUNCHED();
    return MDX_OK;
}

}  // namespace

extern "C" int mdx_gdn_core_raw(const uint16_t* proj, const uint16_t* xn, const uint16_t* wa, const uint16_t* wb,
                                int64_t K, const uint16_t* conv_w, uint16_t* conv_state, uint16_t* proj_buf,
                                uint16_t* qkv_buf, const int32_t* ctl, const float* dt_bias, const float* g_decay,
                                float* rec_state, float* gates, float* sums, float qscale, uint16_t* core, int64_t rows,
                                int64_t HK, int64_t HV, int64_t slots, void* stream) {
    return gdn_run(proj, xn, wa, wb, K, conv_w, conv_state, proj_buf, qkv_buf, ctl, dt_bias, g_decay, rec_state, gates,
                   sums, qscale, core, rows, HK, HV, slots, static_cast<hipStream_t>(stream));
}

extern "C" int mdx_gdn_core(const uint16_t* proj, const uint16_t* z, const uint16_t* xn, const uint16_t* wa,
                            const uint16_t* wb, int64_t K, const uint16_t* conv_w,
                            uint16_t* conv_state, uint16_t* proj_buf, uint16_t* qkv_buf, const int32_t* ctl,
                            const float* dt_bias, const float* g_decay, float* rec_state, float* gates, float* sums,
                            const uint16_t* gnorm_w, float gnorm_eps, float qscale, uint16_t* core, int64_t rows,
                            int64_t HK, int64_t HV, int64_t slots, void* stream) {
    MDX_CHECK(z && gnorm_w, "null pointer");
    int rc = gdn_run(proj, xn, wa, wb, K, conv_w, conv_state, proj_buf, qkv_buf, ctl, dt_bias, g_decay, rec_state, gates,
                     sums, qscale, core, rows, HK, HV, slots, static_cast<hipStream_t>(stream));
    if (rc) return rc;
    // the gated RMSNorm of each head, in place
    return mdx_gnorm_rot_quant(core, z, gnorm_w, gnorm_eps, core, nullptr, MDX_ROT_NONE, nullptr, nullptr, rows,
                               HV * DH, stream);
}
