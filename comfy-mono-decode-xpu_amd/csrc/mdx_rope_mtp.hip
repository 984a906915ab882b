// Q/K RMSNorm + partial split-half RoPE + KV cache write, and the device-side MTP step bookkeeping.
//
// Reference semantics (comfy-mono-decode-xpu):
//   rope_kv          csrc/rope_kv.sycl:5-11, 44-52, 58-114
//   qk_norm_rope_kv  csrc/rope_kv.sycl:120-245 (the norm's reduction order is this library's own:
//                    per-lane partials in element order, then a halving tree over the 64 lanes)
//   mtp_prep_draft   csrc/mtp_loop.sycl:29-53
//   mtp_prep_verify  csrc/mtp_loop.sycl:55-84
//   mtp_accept       csrc/mtp_loop.sycl:86-196
//
// RoPE pair j < rd/2 with the row's rotation f = [[f00, f01], [f10, f11]]:
//   o[j]        = bf16((t[j] * f00) + (t[j + h] * f01))
//   o[j + h]    = bf16((t[j + h] * f11) + (t[j] * f10))
// each product rounded to fp32 on its own, the sum rounded once, then one bf16 rounding.
#include <algorithm>

#include "mdx_common.hpp"
#include "mdx_rope.hpp"

namespace mdx {
namespace {

constexpr int WAVE = 64;
constexpr int MAX_D = 256;

struct RopeArgs {
    const uint16_t* q;      // [S, Hq, D] rows of stride qs, heads of stride qh
    const uint16_t* k;      // [S, Hk, D]
    const uint16_t* v;      // [S, Hk, D]
    int64_t qs, qh, ks, kh, vs, vh;
    const uint16_t* wq;     // RMSNorm weights [D] (null: no norm)
    const uint16_t* wk;
    float epsq, epsk;
    const float* freqs;     // [S][rd/2][2][2], row stride fs (floats)
    int64_t fs;
    uint16_t* key;          // [Hk, cap, D]
    uint16_t* value;
    const int64_t* pos;     // [S]
    uint16_t* oq;           // [Hq, S, D]
    uint16_t* ok;           // [Hk, S, D]
    int S, Hq, Hk, D, rd, cap;
};

// one wave per (row s, head); heads: q (Hq), then k (Hk), then v (Hk)
__global__ __launch_bounds__(WAVE) void rope_kv_kernel(RopeArgs a) {
    __shared__ float xs[MAX_D];
    const int lane = threadIdx.x;
    const int H = a.Hq + 2 * a.Hk;
    const int s = blockIdx.x / H, h = blockIdx.x % H;
    const int D = a.D, per = D / WAVE;
    const int64_t p = a.pos[s];
    // a position outside the cache writes nothing (the callers bound their positions on the host;
    // this keeps a bad position from writing past the cache)
    const bool in_cache = p >= 0 && p < a.cap;
    if (h >= a.Hq + a.Hk) {  // v: cache write only
        const int hv = h - a.Hq - a.Hk;
        if (in_cache)
            for (int d = lane; d < D; d += WAVE)
                a.value[(int64_t(hv) * a.cap + p) * D + d] = a.v[s * a.vs + hv * a.vh + d];
        return;
    }
    const bool isq = h < a.Hq;
    const int hh = isq ? h : h - a.Hq;
    const uint16_t* src = isq ? a.q + s * a.qs + hh * a.qh : a.k + s * a.ks + hh * a.kh;
    const uint16_t* w = isq ? a.wq : a.wk;
    float x[MAX_D / WAVE];
#pragma unroll
    for (int j = 0; j < MAX_D / WAVE; ++j)
        if (j < per) x[j] = bf2f(src[lane + WAVE * j]);
    if (w) {
        // canonical order: lane partial over its elements d = lane + 64 j in order, halving tree
        float part = 0.f;
#pragma unroll
        for (int j = 0; j < MAX_D / WAVE; ++j)
            if (j < per) part = j == 0 ? __fmul_rn(x[0], x[0]) : __fadd_rn(part, __fmul_rn(x[j], x[j]));
        const float ss = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(tree_sum64(part))));
        const float r = __fdiv_rn(1.f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, float(D)), isq ? a.epsq : a.epsk)));
#pragma unroll
        for (int j = 0; j < MAX_D / WAVE; ++j)
            if (j < per) x[j] = bfround(__fmul_rn(__fmul_rn(x[j], r), bf2f(w[lane + WAVE * j])));
    }
#pragma unroll
    for (int j = 0; j < MAX_D / WAVE; ++j)
        if (j < per) xs[lane + WAVE * j] = x[j];
    __syncthreads();
    const int half = a.rd / 2;
    const float* f = a.freqs + s * a.fs;
    uint16_t* dst = isq ? a.oq + (int64_t(hh) * a.S + s) * D : a.ok + (int64_t(hh) * a.S + s) * D;
#pragma unroll
    for (int j = 0; j < MAX_D / WAVE; ++j) {
        if (j >= per) continue;
        const int d = lane + WAVE * j;
        float o = x[j];
        if (d < a.rd) {
            const int jj = d < half ? d : d - half;
            const float lo = xs[jj], hi = xs[jj + half];
            const float* m = f + jj * 4;  // [[f00, f01], [f10, f11]]
            o = d < half ? rope_pair(lo, m[0], hi, m[1]) : rope_pair(hi, m[3], lo, m[2]);
        }
        const uint16_t ob = f2bf(o);
        dst[d] = ob;
        if (!isq && in_cache) a.key[(int64_t(hh) * a.cap + p) * D + d] = ob;
    }
}

// ---- MTP loop bookkeeping -------------------------------------------------------------------
constexpr int RANKS = 7;

__global__ void mtp_prep_draft_kernel(const int64_t* st, int64_t k, const float* ftab, int64_t cap, int64_t n, float* freqs,
                                      int64_t* mpos, int np, int* mseq) {
    const int t = threadIdx.x;
    const int64_t p = st[0] + k, m = st[1] + k;
    const int64_t row = p < cap ? p : cap - 1;
    for (int64_t i = t; i < n; i += blockDim.x) freqs[i] = ftab[row * n + i];
    if (t < np) mpos[t] = m + t;
    if (t == 0) mseq[0] = int(m + 1);
}

__global__ void mtp_prep_verify_kernel(const int64_t* st, int64_t* apos, int np, int* aseq, int64_t* vpos,
                                       const int64_t* tree_pos, int rows, int* ctl, const int* tree_ctl, int slots,
                                       int parity, int64_t rope_offset) {
    const int t = threadIdx.x;
    const int64_t pos = st[0];
    if (t < np) apos[t] = pos + t;
    if (t == 0) aseq[0] = int(pos);
    if (t < rows) vpos[t] = tree_pos[t] + pos + rope_offset;
    if (t == 0) ctl[1] = parity;
    if (t < 2 * slots) ctl[2 + slots + t] = tree_ctl[t];
}

// The accept is two launches. accept_walk_kernel (one wave) walks the tree, writes the result record,
// the counters, ctl and the next token. accept_move_kernel (a grid) copies the chosen hidden row and
// performs the attention KV slot moves of an off-chain path: slot base + k <- slot base + path[k] for
// k ascending. path[k] >= k (a row never sits above its depth), so a move only reads a slot that no
// earlier move wrote; the one hazard is a later move overwriting a slot an earlier move still has to
// read, and a lane that owns one (table, head, d) element across all moves keeps that order without
// any barrier.
struct AcceptArgs {
    int64_t* st;
    const int64_t* toks;
    const int64_t* vtok;
    const int64_t* cand;  // [max(depth, 7)][7] or null
    const int* children;  // [slots][slots], -1 padded
    int rows, depth, slots;
    int64_t* nt;
    int* ctl;             // [2 + 3 slots]
    int64_t* result;      // [slots + 24]
};

__global__ __launch_bounds__(WAVE) void accept_walk_kernel(AcceptArgs a) {
    if (threadIdx.x != 0) return;
    const int S = a.slots;
    int path[16];
    int len = 1;
    path[0] = 0;
    for (bool grow = true; grow && len < a.rows;) {
        const int cur = path[len - 1];
        const int64_t want = a.toks[cur];
        grow = false;
        for (int j = 0; j < S; ++j) {
            const int c = a.children[cur * S + j];
            if (c < 0) break;
            if (a.vtok[c] == want) {
                path[len++] = c;
                grow = true;
                break;
            }
        }
    }
    const int row = path[len - 1];
    const bool on_chain = row == len - 1;
    const int kept = min(on_chain ? len : len - 1, a.depth);
    const int64_t pos = a.st[0];
    // record: [n, commit[slots], row, on_chain, nranks, ranks[7], pos, kept]; a 16-slot tree deeper
    // than 7 keeps the ranks of its first 7 chain nodes
    int64_t* r = a.result;
    r[0] = len;
    for (int i = 1; i <= S; ++i) r[i] = i < len ? a.vtok[path[i]] : (i == len ? a.toks[row] : -1);
    r[S + 1] = row;
    r[S + 2] = on_chain;
    int nr = 0;
    for (int i = 0; a.cand && i < len && path[i] < a.depth && nr < RANKS; ++i) {
        const int64_t* c = a.cand + path[i] * RANKS;
        int rank = 0;
        while (rank < RANKS && c[rank] != a.toks[path[i]]) ++rank;
        r[S + 4 + nr++] = rank;
    }
    r[S + 3] = nr;
    r[S + 4 + RANKS] = pos;
    r[S + 5 + RANKS] = kept;
    a.st[0] = pos + len;
    a.st[1] += kept;
    a.ctl[0] = len;
    for (int i = 0; i < S; ++i) a.ctl[2 + i] = i < len ? path[i] : i;
    a.nt[0] = a.toks[row];
}

struct MoveArgs {
    const int* ctl;          // ctl[0] = path length, ctl[2 + k] = path[k]
    const int64_t* result;   // row, on_chain and pos from the walk
    int slots;
    const uint16_t* x;       // [rows][hidden]
    uint16_t* hbuf;
    int64_t hidden;
    const int64_t* kv_ptrs;  // bf16 [kv_heads, cap, head_dim] per table entry
    int64_t nkv, kv_heads, cap, head_dim;
    int hid_blocks;
};

__global__ __launch_bounds__(256) void accept_move_kernel(MoveArgs a) {
    const int S = a.slots;
    if (int(blockIdx.x) < a.hid_blocks) {
        const int64_t row = a.result[S + 1];
        for (int64_t i = blockIdx.x * 256 + threadIdx.x; i < a.hidden; i += int64_t(a.hid_blocks) * 256)
            a.hbuf[i] = a.x[row * a.hidden + i];
        return;
    }
    if (a.result[S + 2]) return;  // on-chain: the slots already sit in order
    const int64_t e = int64_t(blockIdx.x - a.hid_blocks) * 256 + threadIdx.x;
    const int64_t per = a.kv_heads * a.head_dim;
    if (e >= a.nkv * per) return;
    const int64_t which = e / per, w = e % per, hh = w / a.head_dim, d = w % a.head_dim;
    uint16_t* p = reinterpret_cast<uint16_t*>(a.kv_ptrs[which]) + hh * a.cap * a.head_dim + d;
    const int len = a.ctl[0];
    const int64_t base = a.result[S + 4 + RANKS];
    for (int k = 1; k < len; ++k) {
        const int src = a.ctl[2 + k];
        if (src != k) p[((base + k) % a.cap) * a.head_dim] = p[((base + src) % a.cap) * a.head_dim];
    }
}

}  // namespace
}  // namespace mdx

using namespace mdx;

extern "C" int mdx_qk_norm_rope_kv(const uint16_t* q, int64_t q_row_stride, int64_t q_head_stride, const uint16_t* k,
                                   int64_t k_row_stride, int64_t k_head_stride, const uint16_t* v, int64_t v_row_stride,
                                   int64_t v_head_stride, const uint16_t* weight_q, const uint16_t* weight_k,
                                   float eps_q, float eps_k, const float* freqs, int64_t freqs_row_stride,
                                   uint16_t* key, uint16_t* value, const int64_t* position, uint16_t* q_out,
                                   uint16_t* k_out, int64_t S, int64_t Hq, int64_t Hk, int64_t D, int64_t cap,
                                   int64_t rd, void* stream) {
    MDX_CHECK(q && k && v && freqs && key && value && position && q_out && k_out, "null pointer");
    MDX_CHECK(S >= 1 && S <= 16, "1..16 rows (got %lld)", (long long)S);
    MDX_CHECK(Hq > 0 && Hk > 0 && Hq % Hk == 0, "heads");
    MDX_CHECK(D >= 64 && D <= MAX_D && D % 64 == 0, "head_dim must be 64, 128, 192 or 256");
    MDX_CHECK(rd >= 2 && rd <= D && rd % 2 == 0, "even rotary dimension in 2..head_dim");
    MDX_CHECK(cap >= 1, "cache capacity");
    MDX_CHECK((weight_q == nullptr) == (weight_k == nullptr), "norm weights: both or neither");
    RopeArgs a{q, k, v, q_row_stride, q_head_stride, k_row_stride, k_head_stride, v_row_stride, v_head_stride,
               weight_q, weight_k, eps_q, eps_k, freqs, freqs_row_stride, key, value, position, q_out, k_out,
               int(S), int(Hq), int(Hk), int(D), int(rd), int(cap)};
    hipLaunchKernelGGL(rope_kv_kernel, dim3(unsigned(S * (Hq + 2 * Hk))), dim3(WAVE), 0, static_cast<hipStream_t>(stream), a);
    MDX_LAUNCHED();
    return MDX_OK;
}

extern "C" int mdx_mtp_prep_draft(const int64_t* st, int64_t k, const float* ftab, int64_t ftab_rows, int64_t row_elems,
                                  float* freqs, int64_t* mpos, int64_t npos, int32_t* mseq, void* stream) {
    MDX_CHECK(st && ftab && freqs && mpos && mseq, "null pointer");
    MDX_CHECK(ftab_rows >= 1 && row_elems >= 1 && npos >= 0 && npos <= 256, "shapes");
    hipLaunchKernelGGL(mtp_prep_draft_kernel, dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream), st, k, ftab,
                       ftab_rows, row_elems, freqs, mpos, int(npos), mseq);
    MDX_LAUNCHED();
    return MDX_OK;
}

extern "C" int mdx_mtp_prep_verify(const int64_t* st, int64_t* apos, int64_t npos, int32_t* aseq, int64_t* vpos,
                                   const int64_t* tree_pos, int64_t rows, int32_t* ctl, const int32_t* tree_ctl,
                                   int64_t slots, int64_t parity, int64_t rope_offset, void* stream) {
    MDX_CHECK(st && apos && aseq && vpos && tree_pos && ctl && tree_ctl, "null pointer");
    MDX_CHECK(slots == 8 || slots == 16, "slots must be 8 or 16");
    MDX_CHECK(rows >= 1 && rows <= slots && npos >= 0 && npos <= 64, "rows / positions");
    hipLaunchKernelGGL(mtp_prep_verify_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), st, apos,
                       int(npos), aseq, vpos, tree_pos, int(rows), ctl, tree_ctl, int(slots), int(parity), rope_offset);
    MDX_LAUNCHED();
    return MDX_OK;
}

namespace mdx {
namespace {

// mtp_prep_verify's bookkeeping (work-group 0) and the verify rows' inputs: work-group r gathers row r's
// embedding (token nt[0] for the root row, which it also stores as vtok[0]; vtok[r] for the others) and
// its RoPE table row (position tree_pos[r] + st[0] + rope_offset, the vpos it also stores). Tokens and
// positions outside their tables are clamped into them.
__global__ __launch_bounds__(256) void prep_verify_rows_kernel(const int64_t* st, int64_t* apos, int np, int* aseq,
                                                               int64_t* vpos, const int64_t* tree_pos, int rows, int* ctl,
                                                               const int* tree_ctl, int slots, int parity,
                                                               int64_t rope_offset, const int64_t* nt, int64_t* vtok,
                                                               const uint16_t* embed, int64_t vocab, int hidden,
                                                               const float* ftab, int64_t frows, int fcols, uint16_t* x,
                                                               float* vfreqs) {
    const int t = threadIdx.x, r = blockIdx.x;
    const int64_t pos = st[0];
    if (r == 0) {
        if (t < np) apos[t] = pos + t;
        if (t == 0) aseq[0] = int(pos);
        if (t < rows) vpos[t] = tree_pos[t] + pos + rope_offset;
        if (t == 0) ctl[1] = parity;
        if (t < 2 * slots) ctl[2 + slots + t] = tree_ctl[t];
        if (t == 0) vtok[0] = nt[0];
    }
    int64_t tok = r == 0 ? nt[0] : vtok[r];
    tok = tok < 0 ? 0 : (tok >= vocab ? vocab - 1 : tok);
    int64_t fp = tree_pos[r] + pos + rope_offset;
    fp = fp < 0 ? 0 : (fp >= frows ? frows - 1 : fp);
    const uint4* src = reinterpret_cast<const uint4*>(embed + tok * hidden);
    uint4* dst = reinterpret_cast<uint4*>(x + int64_t(r) * hidden);
    for (int i = t; i < hidden / 8; i += 256) dst[i] = src[i];
    for (int i = t; i < fcols; i += 256) vfreqs[int64_t(r) * fcols + i] = ftab[fp * fcols + i];
}

}  // namespace
}  // namespace mdx

extern "C" int mdx_mtp_prep_verify_rows(const int64_t* st, int64_t* apos, int64_t npos, int32_t* aseq, int64_t* vpos,
                                        const int64_t* tree_pos, int64_t rows, int32_t* ctl, const int32_t* tree_ctl,
                                        int64_t slots, int64_t parity, int64_t rope_offset, const int64_t* nt,
                                        int64_t* vtok, const uint16_t* embed, int64_t vocab, int64_t hidden,
                                        const float* ftab, int64_t ftab_rows, int64_t ftab_cols, uint16_t* x,
                                        float* vfreqs, void* stream) {
    MDX_CHECK(st && apos && aseq && vpos && tree_pos && ctl && tree_ctl && nt && vtok && embed && ftab && x && vfreqs,
              "null pointer");
    MDX_CHECK(slots == 8 || slots == 16, "slots must be 8 or 16");
    MDX_CHECK(rows >= 1 && rows <= slots && npos >= 0 && npos <= 64, "rows / positions");
    MDX_CHECK(vocab >= 1 && hidden >= 8 && hidden % 8 == 0 && aligned(embed, 16) && aligned(x, 16) && ftab_rows >= 1 &&
                  ftab_cols >= 1,
              "embedding [vocab, hidden % 8 == 0] and RoPE table, 16-byte aligned rows");
    hipLaunchKernelGGL(mdx::prep_verify_rows_kernel, dim3(unsigned(rows)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       st, apos, int(npos), aseq, vpos, tree_pos, int(rows), ctl, tree_ctl, int(slots), int(parity),
                       rope_offset, nt, vtok, embed, vocab, int(hidden), ftab, ftab_rows, int(ftab_cols), x, vfreqs);
    MDX_LAUNCHED();
    return MDX_OK;
}

extern "C" int mdx_mtp_accept(int64_t* st, const int64_t* toks, const int64_t* vtok, const int64_t* cand,
                              const int32_t* children, int64_t rows, int64_t depth, int64_t slots, const uint16_t* x,
                              int64_t hidden, int64_t* nt, uint16_t* hbuf, int32_t* ctl, const int64_t* kv_ptrs,
                              int64_t nkv, int64_t kv_heads, int64_t kv_cap, int64_t head_dim, int64_t* result,
                              void* stream) {
    MDX_CHECK(st && toks && vtok && children && x && nt && hbuf && ctl && result, "null pointer");
    MDX_CHECK(slots == 8 || slots == 16, "slots must be 8 or 16");
    MDX_CHECK(rows >= 1 && rows <= slots && depth >= 0 && depth < rows, "rows / depth");
    MDX_CHECK(nkv == 0 || (kv_ptrs && kv_heads > 0 && kv_cap > slots && head_dim > 0),
              "kv pointer table (capacity must exceed the slot count)");
    MDX_CHECK(hidden > 0 && nkv >= 0 && nkv * kv_heads * head_dim < (int64_t(1) << 31), "sizes");
    hipStream_t s = static_cast<hipStream_t>(stream);
    AcceptArgs w{st, toks, vtok, cand, children, int(rows), int(depth), int(slots), nt, ctl, result};
    hipLaunchKernelGGL(accept_walk_kernel, dim3(1), dim3(WAVE), 0, s, w);
    MDX_LAUNCHED();
    const int hid_blocks = int(std::min<int64_t>((hidden + 255) / 256, 16));
    const int64_t mv_blocks = nkv ? (nkv * kv_heads * head_dim + 255) / 256 : 0;
    MoveArgs m{ctl, result, int(slots), x, hbuf, hidden, kv_ptrs, nkv, kv_heads, kv_cap, head_dim, hid_blocks};
    hipLaunchKernelGGL(accept_move_kernel, dim3(unsigned(hid_blocks + mv_blocks)), dim3(256), 0, s, m);
    MDX_LAUNCHED();
    return MDX_OK;
}
