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
// take their heads' sums of squares; extra work-groups, four per value head, compute the a / b
// projections beside them), then gdn_head_kernel (one work-group of 512 per value head: thread
// (row group rg, column col) holds state rows 32 rg .. 32 rg + 31 of column col in registers).
#include <math.h>

#include "mdx_common.hpp"

namespace mdx {
namespace {

constexpr int DH = 128, CW = 3, RG = 4, RPG = DH / RG, GT = RG * DH;
constexpr int MAXS = 16;

struct GdnArgs {
    const uint16_t* proj;   // [R, C]
    const uint16_t* z;      // [R, HV * 128]
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
    const uint16_t* gnorm_w;// [128]
    float eps, qscale;
    uint16_t* core;         // [R, HV * 128]
    int R, HK, HV, C, slots;
};

__device__ __forceinline__ bool ctl_ok(const GdnArgs& a) {
    const int pending = a.ctl[0], p = a.ctl[1];
    return p >= 0 && p <= 1 && pending >= 0 && pending <= a.slots;
}

// a / b projections of this step's rows for head h: 2 R dot products of length K spread over the
// four work-groups of the head (one job per wave and pass); lane l sums its elements in order (the
// 8-element blocks l + 64 j), then a halving tree over the lanes. The bf16-rounded results go to
// gates[p][row][h][0 / 1]; the head kernel turns them into (decay, beta) in place.
__device__ void gdn_ab_part(const GdnArgs& a, int h, int quarter, int p) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int R = a.R, S = a.slots;
    for (int job = quarter * 4 + wv; job < 2 * R; job += 16) {
        const int kind = job / R, ts = job % R;
        const uint16_t* w = (kind == 0 ? a.wa : a.wb) + int64_t(h) * a.K;
        const uint16_t* x = a.xn + int64_t(ts) * a.K;
        uint4 xv[8], wvv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int b0 = lane + 64 * i;
            const int bc = b0 < a.K / 8 ? b0 : 0;  // unconditional loads, masked below
            xv[i] = *reinterpret_cast<const uint4*>(x + 8 * bc);
            wvv[i] = *reinterpret_cast<const uint4*>(w + 8 * bc);
        }
        float part = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (lane + 64 * i >= a.K / 8) continue;
            const uint32_t xw[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
            const uint32_t ww[4] = {wvv[i].x, wvv[i].y, wvv[i].z, wvv[i].w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float xe = __uint_as_float((e & 1) ? (xw[e >> 1] & 0xFFFF0000u) : (xw[e >> 1] << 16));
                const float we = __uint_as_float((e & 1) ? (ww[e >> 1] & 0xFFFF0000u) : (ww[e >> 1] << 16));
                part = fmaf(xe, we, part);
            }
        }
        for (int off = 32; off >= 1; off >>= 1) part = __fadd_rn(part, shfl_down(part, off));
        if (lane == 0) a.gates[((p * S + ts) * a.HV + h) * 2 + kind] = bfround(part);
    }
}

// One thread per channel (it owns the channel's history); the work-group stages its 256 channels'
// projection rows in LDS, so the ancestors of a tree row are LDS reads by index. A work-group of q or
// k channels (two heads) also takes the sums of squares of its heads' conv outputs per row (lane l:
// elements l and l + 64, then a halving tree) into sums[p][row][kh][q / k]. The work-groups after
// the channels' compute the a / b projections (four per value head).
__global__ __launch_bounds__(256) void gdn_conv_kernel(GdnArgs a) {
    __shared__ int sctl[2 + 3 * MAXS];
    __shared__ uint16_t prl[MAXS][256];
    __shared__ float sq[MAXS][256];
    const int t = threadIdx.x;
    const int nconv = (a.C + 255) / 256;
    if (int(blockIdx.x) >= nconv) {
        if (!ctl_ok(a)) return;
        const int b = blockIdx.x - nconv;
        gdn_ab_part(a, b / 4, b % 4, a.ctl[1]);
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
    if (!cl) return;  // (only a last, partial work-group of v channels, which takes no sums)
    const int* acc = sctl + 2;
    const int* parent = sctl + 2 + S;
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
    for (int ts = 0; ts < S; ++ts) {
        uint16_t out = 0;
        if (ts < R) {
            int anc = ts, miss = 0;
            float sum = 0.f;
#pragma unroll
            for (int d = 0; d <= CW; ++d) {
                if (d > 0) {
                    anc = anc >= 0 ? parent[anc] : -1;
                    anc = anc >= R ? -1 : anc;  // a parent is an earlier row of this step
                    miss += anc < 0;
                }
                const int hm = CW - miss;
                const uint16_t hv = hm == 0 ? hist[0] : (hm == 1 ? hist[1] : hist[2]);
                const float v = anc >= 0 ? bf2f(prl[anc][t]) : bf2f(hv);
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
        for (int off = 32; off >= 1; off >>= 1) part = __fadd_rn(part, shfl_down(part, off));
        if (lane == 0) a.sums[((p * S + ts) * a.HK + kh) * 2 + which] = part;
    }
}

__global__ __launch_bounds__(GT) void gdn_head_kernel(GdnArgs a) {
    __shared__ __align__(16) float kvec[2 * MAXS][DH], qvec[MAXS][DH], vvec[2 * MAXS][DH], rawb[MAXS][DH];
    __shared__ float mbuf[2][RG][DH], rbuf[2][RG][DH];
    __shared__ float egate[2 * MAXS][2], cgate[MAXS][2], csum[MAXS][2], rss[MAXS];
    __shared__ int ectl[2 + 3 * MAXS];
    if (!ctl_ok(a)) return;
    const int t = threadIdx.x, h = blockIdx.x;
    const int S = a.slots, R = a.R, HV = a.HV, HK = a.HK, KD = HK * DH;
    const int kh = h / (HV / HK);
    const int64_t C = a.C;
    if (t < 2 + 3 * S) ectl[t] = a.ctl[t];
    __syncthreads();
    const int pending = ectl[0], p = ectl[1];
    const int* acc = ectl + 2;
    const int* prog = ectl + 2 + 2 * S;
    int E0 = 0;
    while (E0 < pending && acc[E0] >= 0 && acc[E0] < S) ++E0;
    const bool replayed = E0 == pending;
    int E1 = 0;
    if (replayed)
        while (E1 < R && prog[E1] >= 0 && (prog[E1] & 15) < R) ++E1;
    const int E = E0 + E1;
    auto slot_of = [&](int e) { return e < E0 ? acc[e] : (prog[e - E0] & 15); };

    const int lane = t & 63, wv = t >> 6;
    // this step's gates from the a / b projections the conv launch left in gates[p] (then (decay, beta)
    // in their place, for this step's entries and the next step's replay); this step's q / k sums
    if (t < S) {
        float decay = 0.f, beta = 0.f;
        if (t < R) {
            const float av = __fadd_rn(a.gates[((p * S + t) * HV + h) * 2], a.dt_bias[h]);
            const float bv = a.gates[((p * S + t) * HV + h) * 2 + 1];
            const float sp = av > 20.f ? av : log1pf(expf(av));
            decay = expf(__fmul_rn(a.g_decay[h], sp));
            beta = bfround(__fdiv_rn(1.f, __fadd_rn(1.f, expf(-bv))));
        }
        cgate[t][0] = decay;
        cgate[t][1] = beta;
    } else if (t >= 64 && t < 64 + 2 * R) {
        const int which = (t - 64) / R, ts = (t - 64) % R;
        csum[ts][which] = a.sums[((p * S + ts) * HK + kh) * 2 + which];
    }
    __syncthreads();
    if (t < S) {
        a.gates[((p * S + t) * HV + h) * 2] = cgate[t][0];
        a.gates[((p * S + t) * HV + h) * 2 + 1] = cgate[t][1];
    }
    // the entries' inputs: k * ki, (q * scale) * qi, v, decay, beta
    if (t < E) {
        const int e = t, ts = slot_of(e);
        if (e < E0) {
            egate[e][0] = a.gates[(((1 - p) * S + ts) * HV + h) * 2];
            egate[e][1] = a.gates[(((1 - p) * S + ts) * HV + h) * 2 + 1];
        } else {
            egate[e][0] = cgate[ts][0];
            egate[e][1] = cgate[ts][1];
        }
    }
#pragma unroll 8
    for (int i = t; i < E * DH; i += GT) {
        const int e = i / DH, d = i % DH, ts = slot_of(e);
        const bool verify = e >= E0;
        const int par = verify ? p : 1 - p;
        const uint16_t* src = a.qb + (par * S + ts) * C;
        const float sk = verify ? csum[ts][1] : a.sums[((par * S + ts) * HK + kh) * 2 + 1];
        const float ki = __fdiv_rn(1.f, fmaxf(sqrt_rn(sk), 1e-12f));
        kvec[e][d] = __fmul_rn(bf2f(src[KD + kh * DH + d]), ki);
        vvec[e][d] = bf2f(src[2 * KD + h * DH + d]);
        if (verify) {
            const float qi = __fdiv_rn(1.f, fmaxf(sqrt_rn(csum[ts][0]), 1e-12f));
            qvec[e - E0][d] = __fmul_rn(__fmul_rn(bf2f(src[kh * DH + d]), a.qscale), qi);
        }
    }
    // the state: rows 32 rg + r of column col
    const int col = t % DH, rg = t / DH;
    float st[RPG];
    float* rs = a.rec + (int64_t(h) * DH + rg * RPG) * DH + col;
#pragma unroll
    for (int r = 0; r < RPG; ++r) st[r] = rs[r * DH];
    __syncthreads();
    for (int e = 0; e < E; ++e) {
        const bool verify = e >= E0;
        const bool commit = !verify || (prog[e - E0] & 32);
        const float decay = egate[e][0], beta = egate[e][1];
        // this entry's k^ (and q^) rows of the thread's row group, as 16-byte LDS broadcasts issued together
        float kr[RPG], qr[RPG];
        const float4* k4 = reinterpret_cast<const float4*>(kvec[e] + rg * RPG);
#pragma unroll
        for (int j = 0; j < RPG / 4; ++j) {
            const float4 v = k4[j];
            kr[4 * j] = v.x, kr[4 * j + 1] = v.y, kr[4 * j + 2] = v.z, kr[4 * j + 3] = v.w;
        }
        if (verify) {
            const float4* q4 = reinterpret_cast<const float4*>(qvec[e - E0] + rg * RPG);
#pragma unroll
            for (int j = 0; j < RPG / 4; ++j) {
                const float4 v = q4[j];
                qr[4 * j] = v.x, qr[4 * j + 1] = v.y, qr[4 * j + 2] = v.z, qr[4 * j + 3] = v.w;
            }
        }
        // kv partial over the 32 rows: four interleaved accumulators, then ((m0 + m1) + (m2 + m3))
        float m4[4] = {0.f, 0.f, 0.f, 0.f};
        if (commit) {
#pragma unroll
            for (int r = 0; r < RPG; ++r) {
                st[r] = __fmul_rn(st[r], decay);
                m4[r & 3] = fmaf(st[r], kr[r], m4[r & 3]);
            }
        } else {
#pragma unroll
            for (int r = 0; r < RPG; ++r) m4[r & 3] = fmaf(__fmul_rn(st[r], decay), kr[r], m4[r & 3]);
        }
        mbuf[e & 1][rg][col] = __fadd_rn(__fadd_rn(m4[0], m4[1]), __fadd_rn(m4[2], m4[3]));
        __syncthreads();  // the one barrier per entry (mbuf / rbuf alternate)
        const float kv = __fadd_rn(__fadd_rn(__fadd_rn(mbuf[e & 1][0][col], mbuf[e & 1][1][col]), mbuf[e & 1][2][col]),
                                   mbuf[e & 1][3][col]);
        const float delta = __fmul_rn(__fsub_rn(vvec[e][col], kv), beta);
        float r4[4] = {0.f, 0.f, 0.f, 0.f};
        if (commit) {
#pragma unroll
            for (int r = 0; r < RPG; ++r) st[r] = fmaf(kr[r], delta, st[r]);
            if (verify)
#pragma unroll
                for (int r = 0; r < RPG; ++r) r4[r & 3] = fmaf(st[r], qr[r], r4[r & 3]);
        } else {
#pragma unroll
            for (int r = 0; r < RPG; ++r) r4[r & 3] = fmaf(fmaf(kr[r], delta, __fmul_rn(st[r], decay)), qr[r], r4[r & 3]);
        }
        if (verify) rbuf[e & 1][rg][col] = __fadd_rn(__fadd_rn(r4[0], r4[1]), __fadd_rn(r4[2], r4[3]));
        if (e == E0 - 1 && replayed)
#pragma unroll
            for (int r = 0; r < RPG; ++r) rs[r * DH] = st[r];
        // the previous verify entry's output row (its partials are complete after this barrier)
        if (e > E0 && rg == 0) {
            const int pe = e - 1;
            rawb[slot_of(pe)][col] = bfround(__fadd_rn(__fadd_rn(__fadd_rn(rbuf[pe & 1][0][col], rbuf[pe & 1][1][col]),
                                                                 rbuf[pe & 1][2][col]), rbuf[pe & 1][3][col]));
        }
    }
    __syncthreads();
    if (E1 > 0 && rg == 0) {
        const int pe = E - 1;
        rawb[slot_of(pe)][col] = bfround(__fadd_rn(__fadd_rn(__fadd_rn(rbuf[pe & 1][0][col], rbuf[pe & 1][1][col]),
                                                             rbuf[pe & 1][2][col]), rbuf[pe & 1][3][col]));
    }
    unsigned written = 0;
    for (int e = E0; e < E; ++e) written |= 1u << slot_of(e);
    __syncthreads();
    // gated RMSNorm: one wave per row: lane l sums columns l and l + 64, then a halving tree
    for (int ts = wv; ts < R; ts += GT / 64) {
        if (!((written >> ts) & 1)) continue;
        const float x0 = rawb[ts][lane], x1 = rawb[ts][lane + 64];
        float s2 = __fadd_rn(__fmul_rn(x0, x0), __fmul_rn(x1, x1));
        for (int off = 32; off >= 1; off >>= 1) s2 = __fadd_rn(s2, shfl_down(s2, off));
        if (lane == 0) rss[ts] = s2;
    }
    __syncthreads();
    const float gw = bf2f(a.gnorm_w[col]);
    for (int ts = rg; ts < R; ts += RG) {
        uint16_t outv = 0;
        if ((written >> ts) & 1) {
            const float rsq = __fdiv_rn(1.f, sqrt_rn(__fadd_rn(__fdiv_rn(rss[ts], float(DH)), a.eps)));
            const float normed = bfround(__fmul_rn(__fmul_rn(rawb[ts][col], gw), rsq));
            const float zz = bf2f(a.z[ts * HV * DH + h * DH + col]);
            const float gz = bfround(__fdiv_rn(zz, __fadd_rn(1.f, expf(-zz))));
            outv = f2bf(__fmul_rn(normed, gz));
        }
        a.core[ts * HV * DH + h * DH + col] = outv;
    }
}

}  // namespace
}  // namespace mdx

using namespace mdx;

extern "C" int mdx_gdn_core(const uint16_t* proj, const uint16_t* z, const uint16_t* xn, const uint16_t* wa,
                            const uint16_t* wb, int64_t K, const uint16_t* conv_w,
                            uint16_t* conv_state, uint16_t* proj_buf, uint16_t* qkv_buf, const int32_t* ctl,
                            const float* dt_bias, const float* g_decay, float* rec_state, float* gates, float* sums,
                            const uint16_t* gnorm_w, float gnorm_eps, float qscale, uint16_t* core, int64_t rows,
                            int64_t HK, int64_t HV, int64_t slots, void* stream) {
    MDX_CHECK(proj && z && xn && wa && wb && conv_w && conv_state && proj_buf && qkv_buf && ctl && dt_bias && g_decay &&
                  rec_state && gates && sums && gnorm_w && core,
              "null pointer");
    MDX_CHECK(slots == 8 || slots == 16, "slots must be 8 or 16");
    MDX_CHECK(rows >= 1 && rows <= slots, "1 <= rows <= slots");
    MDX_CHECK(HK >= 1 && HV >= HK && HV % HK == 0 && HV <= 1024, "heads");
    MDX_CHECK(K >= 512 && K <= 4096 && K % 512 == 0 && aligned(xn, 16) && aligned(wa, 16) && aligned(wb, 16),
              "a / b input: K % 512 == 0, K <= 4096, 16-byte aligned rows");
    GdnArgs a{};
    a.proj = proj;
    a.z = z;
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
    a.gnorm_w = gnorm_w;
    a.eps = gnorm_eps;
    a.qscale = qscale;
    a.core = core;
    a.R = int(rows);
    a.HK = int(HK);
    a.HV = int(HV);
    a.C = int(2 * HK * DH + HV * DH);
    a.slots = int(slots);
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(gdn_conv_kernel, dim3((a.C + 255) / 256 + 4 * a.HV), dim3(256), 0, st, a);
    MDX_LAUNCHED();
    hipLaunchKernelGGL(gdn_head_kernel, dim3(a.HV), dim3(GT), 0, st, a);
    MDX_LAUNCHED();
    return MDX_OK;
}
