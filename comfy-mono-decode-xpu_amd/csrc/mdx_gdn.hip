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
// [head][k row][v col]); gates f32 [2][slots][HV][2] (decay, beta); ctl int32 [2 + 3 slots] = pending,
// parity, accepted slots, parents, program. The reference keeps the q / k sums of squares of each step
// in a buffer of its own for the next step's replay; here the delta-rule kernel takes them from the conv
// outputs it loads anyway (sums [2][slots][HK][2] stays in the argument list, neither read nor written).
// Channels of proj / qb: q [0, KD), k [KD, 2 KD), v [2 KD, 2 KD + HV 128), KD = HK 128.
//
// Launches: gdn_conv_kernel (one thread per channel: owns its conv history; extra work-groups, four per
// value head, compute the gates beside them), then gdn_head_kernel (eight work-groups of 256 per value
// head, 16 state columns each: thread (row group rg, column col) holds state rows 8 rg .. 8 rg + 7 of its
// column in registers; each entry's |k| and |q| from the pieces it loads: a thread's 8 squares in order,
// then a halving tree over the 16 threads of a head row; raw bf16 outputs), then the gated RMSNorm per head in place (the row-prep kernel's head-norm mode, which the
// decode stack instead fuses into the output projection's activation prep: mdx_gdn_core_raw +
// mdx_gnorm_rot_quant).
#include <math.h>

#include "mdx_common.hpp"
#include "mdx_gdn_ops.hpp"

namespace mdx {
namespace {

constexpr int DH = GDN_DH, CW = GDN_CW;
constexpr int MAXS = GDN_MAXS;

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


__device__ void gdn_gates_part(const GdnArgs& a, int h, int quarter) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int R = a.R, S = a.slots;
    // the control words are checked at the stores only, so that their load overlaps the others
    const int pending = a.ctl[0], p = a.ctl[1];
    const bool ok = gdn_ctl_ok(pending, p, S);
    for (int ts = quarter * 4 + wv; ts < S; ts += 16) {
        float decay = 0.f, beta = 0.f;
        if (ts < R)
            gdn_gate_row(a.xn + int64_t(ts) * a.K, a.wa + int64_t(h) * a.K, a.wb + int64_t(h) * a.K, a.K, a.dt_bias[h],
                         a.g_decay[h], lane, decay, beta);
        if (lane == 0 && ok) {
            a.gates[((p * S + ts) * a.HV + h) * 2] = decay;
            a.gates[((p * S + ts) * a.HV + h) * 2 + 1] = beta;
        }
    }
}

// One thread per channel (it owns the channel's history); the work-group stages its 256 channels'
// projection rows in LDS, so the ancestors of a tree row are LDS reads by index. The work-groups after
// the channels' compute this step's gates (four per value head).
__global__ __launch_bounds__(256) void gdn_conv_kernel(GdnArgs a) {
    __shared__ int sctl[2 + 3 * MAXS];
    __shared__ uint32_t anct[MAXS];
    __shared__ uint16_t prl[MAXS][256];
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
    const bool cl = c < a.C;
    // this step's projections of the channel, every load up front (clamped addresses, no branches)
    uint16_t pr[MAXS];
#pragma unroll
    for (int r = 0; r < MAXS; ++r) pr[r] = a.proj[(r < R ? r : R - 1) * int64_t(a.C) + (cl ? c : 0)];
#pragma unroll
    for (int r = 0; r < MAXS; ++r) prl[r][t] = pr[r];
    __syncthreads();
    const int S = a.slots, pending = sctl[0], p = sctl[1];
    if (!gdn_ctl_ok(pending, p, S)) return;  // uniform
    if (t < R) anct[t] = gdn_ancestry(t, R, sctl + 2 + S);
    __syncthreads();
    if (!cl) return;  // (only a last, partial work-group of v channels)
    gdn_conv_channel(c, a.C, R, S, pending, p, sctl + 2, anct, [&](int r) { return prl[r][t]; }, a.conv_w, a.conv_state,
                     a.pb, a.qb);
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

// the sum over the column's 16 row groups of a value each lane holds (every lane of the column gets it)
__device__ __forceinline__ float col_sum(float v) { return sum_x32(sum_x16(sum_r4(sum_x8(v)))); }

__global__ __launch_bounds__(HT) void gdn_head_kernel(GdnArgs a) {
    __shared__ __align__(16) float kvec[2 * MAXS][DH], qvec[MAXS][DH];
    __shared__ float vvec[2 * MAXS][SC], rawc[MAXS][SC];
    __shared__ float egate[2 * MAXS][4];  // decay, beta, 1 / |k|, 1 / |q|
    __shared__ float esum[2 * MAXS][2];   // sums of squares of q, k
    __shared__ int ectl[2 + 3 * MAXS];
    __shared__ float ekq[MAXS];           // k . q of the verify entries
    const int t = threadIdx.x, lane = t % 64, h = blockIdx.x / NSPLIT, cs = blockIdx.x % NSPLIT;
    const int S = a.slots, R = a.R, HV = a.HV, HK = a.HK, KD = HK * DH;
    const int kh = h / (HV / HK);
    const int64_t C = a.C;
    // the control words' load first, then the state of this work-group's columns (not needed before the
    // entry loops): the control words' wait (loads return in order) is not a wait for the state
    const int cw = t < 2 + 3 * S ? a.ctl[t] : 0;
    const int col = (t / 64) * 4 + (lane & 3), rg = lane >> 2;
    float st[HRPG];
    float* rs = a.rec + (int64_t(h) * DH + rg * HRPG) * DH + cs * SC + col;
#pragma unroll
    for (int r = 0; r < HRPG; ++r) st[r] = rs[r * DH];
    if (t < 2 + 3 * S) ectl[t] = cw;
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
    uint4 kraw[KP], qraw = make_uint4(0u, 0u, 0u, 0u), kqraw = make_uint4(0u, 0u, 0u, 0u), vraw = make_uint4(0u, 0u, 0u, 0u);
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
        const uint16_t* row = a.qb + (p * S + slot_of(min(e, E - 1))) * C + kh * DH + (i % 16) * 8;
        qraw = *reinterpret_cast<const uint4*>(row);
        kqraw = *reinterpret_cast<const uint4*>(row + KD);  // the same entry's k piece (for k . q)
    }
    if (t < VP) {
        const int i = min(t, E * VPE - 1), e = i / VPE;
        const int ts = slot_of(e), par = e < E0 ? 1 - p : p;
        vraw = *reinterpret_cast<const uint4*>(a.qb + (par * S + ts) * C + 2 * KD + h * DH + cs * SC + (i % VPE) * 8);
    }
    }
    if (t < E) {
        const int e = t, ts = slot_of(e), par = e < E0 ? 1 - p : p;
        const float* gt = a.gates + ((par * S + ts) * HV + h) * 2;
        egate[e][0] = gt[0];
        egate[e][1] = gt[1];
    }
    // the entries' sums of squares of k (every entry) and q (verify entries) from the loaded pieces: each
    // thread's 8 squares in order, then the 16 pieces of an entry (16 consecutive lanes) by a halving tree
    auto sq8 = [](const uint4 v) {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        float s_ = 0.f;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float f = __uint_as_float((q & 1) ? (w[q >> 1] & 0xFFFF0000u) : (w[q >> 1] << 16));
            s_ = fmaf(f, f, s_);
        }
        return s_;
    };
    auto sum16 = [](float v) {
#pragma unroll
        for (int d = 8; d >= 1; d >>= 1) v = __fadd_rn(v, __shfl_xor(v, d, 16));
        return v;
    };
#pragma unroll
    for (int j = 0; j < KP; ++j) {
        const int i = t + HT * j;
        const float ssum = sum16(sq8(kraw[j]));
        if (i < E * 16 && (i & 15) == 0) esum[i / 16][1] = ssum;
    }
    {
        // and the raw k . q of the verify entries (it does not depend on the state), the same way
        const uint32_t wq[4] = {qraw.x, qraw.y, qraw.z, qraw.w}, wk[4] = {kqraw.x, kqraw.y, kqraw.z, kqraw.w};
        float dkq = 0.f;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const uint32_t sh = (q & 1) ? 0u : 16u;
            dkq = fmaf(__uint_as_float((wk[q >> 1] << sh) & 0xFFFF0000u), __uint_as_float((wq[q >> 1] << sh) & 0xFFFF0000u), dkq);
        }
        const float ssum = sum16(sq8(qraw));
        dkq = sum16(dkq);
        if (t < E1 * 16 && (t & 15) == 0) esum[E0 + t / 16][0] = ssum, ekq[t / 16] = dkq;
    }
    __syncthreads();
    if (t < E) {
        const int e = t;
        const float ki = __fdiv_rn(1.f, fmaxf(sqrt_rn(esum[e][1]), 1e-12f));
        const float qi = __fdiv_rn(1.f, fmaxf(sqrt_rn(e >= E0 ? esum[e][0] : 0.f), 1e-12f));
        egate[e][2] = ki;
        egate[e][3] = qi;
        if (e >= E0) ekq[e - E0] = __fmul_rn(__fmul_rn(ekq[e - E0], ki), __fmul_rn(a.qscale, qi));  // normalised k . q
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
    // the step's output rows start as zeros: a row that no verify entry writes stays zero
    for (int i = t; i < R * SC; i += HT) rawc[i / SC][i % SC] = 0.f;
    if (t < E * VPE) {
        const int e = t / VPE, d0 = (t % VPE) * 8;
        const uint32_t w[4] = {vraw.x, vraw.y, vraw.z, vraw.w};
#pragma unroll
        for (int q = 0; q < 8; ++q)
            vvec[e][d0 + q] = __uint_as_float((q & 1) ? (w[q >> 1] & 0xFFFF0000u) : (w[q >> 1] << 16));
    }
    __syncthreads();
    // The entries in order, each one's operands loaded from LDS one entry ahead; the replayed entries
    // (always committed) first, then the verify entries. Entry e (decay d, beta b) on the running state S:
    // kv = k . (d S) = d (k . S), delta = b (v - kv); commit: S <- d S + k delta^T; verify: out =
    // (d S + k delta^T) . q = d (q . S) + delta (k . q). k . S over the thread's 8 rows in four interleaved
    // accumulators, then ((m0 + m1) + (m2 + m3)), then the column's 16 row groups (lanes of one residue
    // mod 4): row_ror 8 and 4 inside each row of 16 lanes, then the lane swaps across rows, so that every
    // lane of the column ends with the same sum; q . S the same way, beside it.
    const int E0c = replayed ? E0 : 0, Ec = replayed ? E : 0;
    auto load8 = [&](const float* src, float (&r8)[HRPG]) {
        const float4* p4 = reinterpret_cast<const float4*>(src + rg * HRPG);
        const float4 x0 = p4[0], x1 = p4[1];
        r8[0] = x0.x, r8[1] = x0.y, r8[2] = x0.z, r8[3] = x0.w, r8[4] = x1.x, r8[5] = x1.y, r8[6] = x1.z, r8[7] = x1.w;
    };
    auto dot_col = [&](const float (&r8)[HRPG]) {
        float m4[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) m4[r] = __fmul_rn(st[r], r8[r]);
#pragma unroll
        for (int r = 4; r < HRPG; ++r) m4[r & 3] = fmaf(st[r], r8[r], m4[r & 3]);
        return col_sum(__fadd_rn(__fadd_rn(m4[0], m4[1]), __fadd_rn(m4[2], m4[3])));
    };
    // two register sets per operand, alternating by entry (the loops unrolled by two: no copies of the
    // prefetched operands into the current ones)
    float kA[HRPG], kB[HRPG], qA[HRPG], qB[HRPG], vv = 0.f, decay = 0.f, beta = 0.f, kq = 0.f;
    int pr = 0;
    if (E0c > 0) {
        load8(kvec[0], kA);
        vv = vvec[0][col], decay = egate[0][0], beta = egate[0][1];
    }
    auto replay = [&](int e, const float (&kc)[HRPG], float (&kn)[HRPG]) {
        const int en = min(e + 1, E0c - 1);
        load8(kvec[en], kn);
        const float vn = vvec[en][col], dn = egate[en][0], bn = egate[en][1];
        const float delta = __fmul_rn(__fsub_rn(vv, __fmul_rn(decay, dot_col(kc))), beta);
#pragma unroll
        for (int r = 0; r < HRPG; ++r) st[r] = fmaf(kc[r], delta, __fmul_rn(st[r], decay));
        vv = vn, decay = dn, beta = bn;
    };
    for (int e = 0; e < E0c; e += 2) {
        replay(e, kA, kB);
        if (e + 1 < E0c) replay(e + 1, kB, kA);
    }
    if (E0c > 0)
#pragma unroll
        for (int r = 0; r < HRPG; ++r) rs[r * DH] = st[r];
    // verify entry E0 + j's output is held by row group j of its column (j < R <= 16) and written to LDS
    // after the loop (no LDS store on the serial path)
    float held = 0.f;
    if (Ec > E0c) {
        load8(kvec[E0c], kA);
        load8(qvec[0], qA);
        vv = vvec[E0c][col], decay = egate[E0c][0], beta = egate[E0c][1], kq = ekq[0], pr = prog[0];
    }
    auto verify = [&](int e, const float (&kc)[HRPG], const float (&qc)[HRPG], float (&kn)[HRPG], float (&qn)[HRPG]) {
        const int en = min(e + 1, Ec - 1);
        load8(kvec[en], kn);
        load8(qvec[en - E0c], qn);
        const float vn = vvec[en][col], dn = egate[en][0], bn = egate[en][1], kqn = ekq[en - E0c];
        const int prn = prog[en - E0c];
        const float ks = dot_col(kc), qs = dot_col(qc);
        const float delta = __fmul_rn(__fsub_rn(vv, __fmul_rn(decay, ks)), beta);
        const float o = fmaf(delta, kq, __fmul_rn(decay, qs));
        held = e - E0c == rg ? o : held;
        if (pr & 32)  // (uniform) committed
#pragma unroll
            for (int r = 0; r < HRPG; ++r) st[r] = fmaf(kc[r], delta, __fmul_rn(st[r], decay));
        vv = vn, decay = dn, beta = bn, kq = kqn, pr = prn;
    };
    for (int e = E0c; e < Ec; e += 2) {
        verify(e, kA, qA, kB, qB);
        if (e + 1 < Ec) verify(e + 1, kB, qB, kA, qA);
    }
    if (rg < Ec - E0c) rawc[prog[rg] & 15][col] = bfround(held);
    __syncthreads();
    for (int i = t; i < R * SC; i += HT) {
        const int ts = i / SC, c = i % SC;
        a.core[ts * HV * DH + h * DH + cs * SC + c] = f2bf(rawc[ts][c]);
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

extern "C" int mdx_gdn_delta(const uint16_t* qkv_buf, const int32_t* ctl, float* rec_state, const float* gates,
                             float qscale, uint16_t* core, int64_t rows, int64_t HK, int64_t HV, int64_t slots,
                             void* stream) {
    MDX_CHECK(qkv_buf && ctl && rec_state && gates && core, "null pointer");
    MDX_CHECK(slots == 8 || slots == 16, "slots must be 8 or 16");
    MDX_CHECK(rows >= 1 && rows <= slots, "1 <= rows <= slots");
    MDX_CHECK(HK >= 1 && HV >= HK && HV % HK == 0 && HV % 2 == 0 && HV <= 128, "heads (HV even, <= 128)");
    GdnArgs a{};
    a.qb = const_cast<uint16_t*>(qkv_buf);
    a.ctl = ctl;
    a.rec = rec_state;
    a.gates = const_cast<float*>(gates);
    a.qscale = qscale;
    a.core = core;
    a.R = int(rows);
    a.HK = int(HK);
    a.HV = int(HV);
    a.C = int(2 * HK * DH + HV * DH);
    a.slots = int(slots);
    hipLaunchKernelGGL(gdn_head_kernel, dim3(a.HV * NSPLIT), dim3(HT), 0, static_cast<hipStream_t>(stream), a);
    MDX_LAUNCHED();
    return MDX_OK;
}
