/* libmdx: MI355X (gfx950) kernels of the W4A8 hybrid decode step, behind a plain C ABI.
 *
 * Every entry point enqueues its work on `stream` (a hipStream_t) and returns without a host
 * synchronisation. All pointers are device pointers unless stated otherwise. Argument contracts
 * are checked before anything is written; a violation returns MDX_EINVAL and sets the message
 * read by mdx_last_error(). The library never frees caller memory and is not re-entrant per
 * device: two threads must not enqueue on one device at the same time with shared workspaces.
 *
 * Each function names the reference operator it replaces (comfy-mono-decode-xpu, csrc/...).
 */
#ifndef MDX_H
#define MDX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define MDX_OK 0
#define MDX_EINVAL 1 /* argument contract violated; nothing was enqueued */
#define MDX_EHIP 2   /* HIP runtime error while enqueueing */

/* element types */
#define MDX_DT_F32 0
#define MDX_DT_F16 1
#define MDX_DT_FP8E4M3 2 /* OCP float8 e4m3fn */
#define MDX_DT_BF16 3

/* W4 weight layouts */
#define MDX_LAYOUT_ROW 0  /* codes [N, K/2]; s_rel [N, K/G] (the checkpoint layout) */
#define MDX_LAYOUT_TILE 1 /* codes [N/16][K/128][4][16][16 B]; s_rel [N, K/G] as in the row layout */

/* W4 decode contracts (both bit-exact w.r.t. w8 = isnan(r) ? 0 : clamp(r, -127, 127),
 * r = rint(codebook[code] * s_rel)) */
#define MDX_DECODE_EXACT 0 /* always the per-weight decode (any s_rel, any codebook) */
#define MDX_DECODE_AUTO 1  /* per 128-k chunk: where the codebook is code - 8 and the chunk's s_rel
                              is an integer in [-15, 15], w8 = (code - 8) * s_rel exactly and the dot
                              is factorised per group; elsewhere the per-weight decode. The int32
                              accumulator is the same either way (mod 2^32). */
#define MDX_DECODE_INTEGRAL 2 /* the caller asserts that the codebook is code - 8 (or NULL) and every
                                 s_rel is an integer in [-15, 15] (the GPTQ packer's integral output):
                                 the integral form throughout, without the per-launch check of the
                                 staged scales. Scales outside the assertion give wrong sums, never a
                                 fault. With group_size below 128 (MFMA rows) or 32, as AUTO. */

/* rotation applied by rot_quant-style prologues */
#define MDX_ROT_NONE 0    /* x_rot = x (the identity matrix) */
#define MDX_ROT_H256 1    /* x_rot = x_group . kron(H4, H4, H4, H4) / 16 (fast Walsh-Hadamard) */
#define MDX_ROT_MATRIX 2  /* x_rot = x_group . h for an arbitrary bf16 h [256, 256] */

/* A packed W4A8 linear: out[m, n] = scaleback(sum_k x[m, k] * w8[n, k]). */
typedef struct mdx_w4 {
    const void* q;           /* packed int4 codes (byte b: code of k = 2b low nibble, 2b + 1 high) */
    const void* s_rel;       /* relative group scales, dtype s_dtype */
    const float* s_channel;  /* [N] fp32 channel scales */
    const float* codebook;   /* [16] fp32, or NULL for code - 8 */
    int64_t n, k, group_size;
    int32_t s_dtype;         /* MDX_DT_F32, MDX_DT_F16 or MDX_DT_FP8E4M3 */
    int32_t layout;          /* MDX_LAYOUT_* */
    int32_t decode;          /* MDX_DECODE_* */
    int32_t reserved;
} mdx_w4;

/* The message of the last failed call on this thread ("" if none). */
const char* mdx_last_error(void);
/* ABI version of this library (bumped on any signature change). */
int mdx_version(void);

/* Small-M fused W4A8 decode linear.
 * Replaces: _C.w4a8_decode_linear, csrc/w4a8_decode.sycl:325-370 (bindings.cpp:72-75).
 *   out[m, n] = cast((float(acc[m, n]) * x_scale[m]) * s_channel[n]),  acc = sum_k x[m, k] * w8[n, k]
 *   mod 2^32; with `residual`: cast(float(residual) + float(cast(f))).
 * x: int8 [rows, K] contiguous, 16-byte aligned; x_scale f32 [rows]; out/residual [rows, N] of
 * out_dtype (MDX_DT_F32 or MDX_DT_BF16). 1 <= rows <= 16, K % 128 == 0, N % 16 == 0,
 * group_size % 16 == 0 and K % group_size == 0. */
int mdx_w4a8_decode_linear(const int8_t* x, const float* x_scale, const mdx_w4* w, const void* residual,
                           void* out, int32_t out_dtype, int64_t rows, void* stream);

/* ConvRot rotation + row-wise int8 quantisation.
 * Replaces: _C.rot_quant, csrc/act_prep.sycl:97-110 (kernel :30-94).
 *   xr = bf16(x_group . H) per 256-group (rot as MDX_ROT_*; h is read only for MDX_ROT_MATRIX),
 *   scale[r] = max(amax_r / 127, 1e-30), sb = bf16(scale) (0 -> 0x0080),
 *   q = int8(clamp(rint(float(bf16(xr / sb))), -128, 127)).
 * x bf16 [rows, K] contiguous, K % 256 == 0, K <= 16384; q int8 [rows, K]; scale f32 [rows]. */
int mdx_rot_quant(const uint16_t* x, const uint16_t* h, int32_t rot, int8_t* q, float* scale, int64_t rows,
                  int64_t K, void* stream);

/* Bytes of device workspace mdx_mono_mlp needs for `rows` rows, hidden K1, intermediate N1. */
size_t mdx_mono_mlp_workspace(int64_t rows, int64_t K1, int64_t N1);

/* Fused MLP block: down(silu(gate(q1)) * up(q1)) with q1 = rot_quant([RMSNorm](xn)).
 * Replaces: _C.mono_mlp, csrc/mono_mlp.sycl:34-180 (bindings.cpp:76-78); with norm_w != NULL also
 * the MLP.forward(x, norm) caller's norm (comfy_mono_decode_xpu/mono.py:187-190).
 *   [xn = bf16((x * r) * norm_w), r = 1 / sqrt(mean(x^2) + eps) in the library's fixed order]
 *   g, u = bf16 scaleback of the gate / up accumulators; h = bf16(float(silu_lut[g]) * float(u));
 *   q2, s2 = rot_quant(h); out = bf16((float(acc_down) * s2) * s_channel_down).
 * xn bf16 [rows, K1]; silu_lut bf16 [65536] (F.silu of every bf16 bit pattern); out bf16 [rows, N2].
 * gate/up: N1 x K1, down: N2 x N1; one codebook for all three; 1 <= rows <= 16. With residual (bf16
 * [rows, N2], may equal xn): out = bf16(float(residual) + float(bf16(down))) (layer_post's last phase,
 * csrc/mono_layer.sycl:303-313).
 * workspace: >= mdx_mono_mlp_workspace(rows, K1, N1) bytes, 256-byte aligned (the intermediates: the
 * gate/up work-groups' |h| maxima, q1, q2, row scales, h; zero-filling it once is recommended for the
 * diagnostic word of mdx_mono_mlp_error_offset, which no launch of this library sets). Calls that share a
 * workspace must be ordered (one stream). Four launches: row prep of x, gate/up, row prep of h, down;
 * without rotation at 1 row two (the row prep in the gate/up prologue, h quantised in the down
 * prologue), at 2 rows three. */
int mdx_mono_mlp(const uint16_t* xn, const uint16_t* norm_w, float eps, const uint16_t* h, int32_t rot,
                 const uint16_t* silu_lut, const mdx_w4* gate, const mdx_w4* up, const mdx_w4* down,
                 const uint16_t* residual, uint16_t* out, int64_t rows, void* workspace, size_t workspace_bytes,
                 void* stream);

/* Byte offset in the mdx_mono_mlp workspace of a diagnostic word reserved for in-kernel waits that give
 * up; no launch of this library waits on another work-group, so it stays as the caller left it (zero).
 * No counterpart in the reference. */
size_t mdx_mono_mlp_error_offset(void);

/* One launch of the stream GEMV engine over up to three W4 matrices sharing K (outputs per matrix),
 * or a gate/up pair with the SiLU-multiply epilogue into outs[0].
 * Replaces: the persistent stream engine of csrc/mono_common.hpp:143-316 as used by layer_pre's
 * projection phase (csrc/mono_layer.sycl:132-150) and the MLP phases (csrc/mono_mlp.sycl:114-167).
 * x int8 [rows, K] (16-byte aligned), x_scale f32 [rows]; outs[i] [rows, N_i] of out_dtype;
 * residuals (optional, may be NULL or hold NULLs) as in mdx_w4a8_decode_linear. */
int mdx_stream_gemv(const int8_t* x, const float* x_scale, const mdx_w4* const* mats, int32_t nmats, int32_t gate_up,
                    void* const* outs, const void* const* residuals, int32_t out_dtype, const uint16_t* silu_lut,
                    int64_t rows, void* stream);

/* RMSNorm + rotation + row quantisation of decode rows (xn_out optional).
 * Replaces: the row phase of layer_pre (csrc/mono_layer.sycl:126-130: rms_norm_row + rot_quant_row,
 * csrc/mono_common.hpp:452-505, 362-442). RMSNorm uses the library's fixed reduction order. */
int mdx_rms_rot_quant(const uint16_t* x, const uint16_t* norm_w, float eps, uint16_t* xn_out, const uint16_t* h,
                      int32_t rot, int8_t* q, float* scale, int64_t rows, int64_t K, void* stream);

/* Q/K RMSNorm (optional) + partial split-half RoPE + KV cache write, one launch.
 * Replaces: _C.rope_kv (csrc/rope_kv.sycl:58-114; weight_q = weight_k = NULL) and
 * _C.qk_norm_rope_kv (csrc/rope_kv.sycl:120-245; both weights given), bindings.cpp:84-90.
 *   [t = bf16((x * r) * w), r = 1 / sqrt(sum(x^2) / D + eps), per head, in the library's fixed order]
 *   pair j < rd/2, f = freqs[s, j] = [[f00, f01], [f10, f11]]:
 *   o[j] = bf16(t[j] * f00 + t[j + rd/2] * f01), o[j + rd/2] = bf16(t[j + rd/2] * f11 + t[j] * f10),
 *   each product rounded to fp32 on its own; lanes d >= rd pass through.
 * q/k/v bf16 rows s of stride *_row_stride and heads of stride *_head_stride (elements; the last dim
 * contiguous: a gated q is the first half of each [query, gate] head); freqs f32 [S, rd/2, 2, 2] with
 * row stride freqs_row_stride; key/value bf16 [Hk, cap, D]: rows position[s] are written with k
 * (rotated) and v; q_out [Hq, S, D], k_out [Hk, S, D]. 1 <= S <= 16, D in {64, 128, 192, 256}.
 * The caller owns in-range positions (0 <= position[s] < cap). */
int mdx_qk_norm_rope_kv(const uint16_t* q, int64_t q_row_stride, int64_t q_head_stride, const uint16_t* k,
                        int64_t k_row_stride, int64_t k_head_stride, const uint16_t* v, int64_t v_row_stride,
                        int64_t v_head_stride, const uint16_t* weight_q, const uint16_t* weight_k, float eps_q,
                        float eps_k, const float* freqs, int64_t freqs_row_stride, uint16_t* key, uint16_t* value,
                        const int64_t* position, uint16_t* q_out, uint16_t* k_out, int64_t S, int64_t Hq,
                        int64_t Hk, int64_t D, int64_t cap, int64_t rd, void* stream);

/* MTP draft k's rope row and MTP KV positions from the device loop state st (int64 [4]:
 * st[0] committed length, st[1] MTP KV length).
 * Replaces: _C.mtp_prep_draft, csrc/mtp_loop.sycl:29-53.
 *   p = st[0] + k; freqs = ftab[min(p, ftab_rows - 1)] (row_elems floats); mpos[i] = st[1] + k + i;
 *   mseq[0] = st[1] + k + 1. */
int mdx_mtp_prep_draft(const int64_t* st, int64_t k, const float* ftab, int64_t ftab_rows, int64_t row_elems,
                       float* freqs, int64_t* mpos, int64_t npos, int32_t* mseq, void* stream);

/* Verify-step positions and the deferred-delta ctl program.
 * Replaces: _C.mtp_prep_verify, csrc/mtp_loop.sycl:55-84.
 *   apos[i] = st[0] + i; aseq = st[0]; vpos[r] = tree_pos[r] + st[0] + rope_offset; ctl[1] = parity;
 *   ctl[2 + slots + i] = tree_ctl[i] for i < 2 slots (parents, programs). ctl int32 [2 + 3 slots]. */
int mdx_mtp_prep_verify(const int64_t* st, int64_t* apos, int64_t npos, int32_t* aseq, int64_t* vpos,
                        const int64_t* tree_pos, int64_t rows, int32_t* ctl, const int32_t* tree_ctl, int64_t slots,
                        int64_t parity, int64_t rope_offset, void* stream);

/* mdx_mtp_prep_verify plus the verify rows' inputs, one launch: vtok[0] = nt[0] (the root row's token);
 * x[r] = embed[vtok[r]] (bf16 [rows, hidden]) and vfreqs[r] = ftab[vpos[r]] (f32 [rows, ftab_cols]),
 * tokens and positions clamped into their tables. No counterpart in the reference, whose decode loop
 * gathers these with torch ops around mtp_prep_verify (comfy_mono_decode_xpu/mtp_loop.py:372-373): the
 * decode step's captured graph carries one launch instead of four. */
int mdx_mtp_prep_verify_rows(const int64_t* st, int64_t* apos, int64_t npos, int32_t* aseq, int64_t* vpos,
                             const int64_t* tree_pos, int64_t rows, int32_t* ctl, const int32_t* tree_ctl, int64_t slots,
                             int64_t parity, int64_t rope_offset, const int64_t* nt, int64_t* vtok,
                             const uint16_t* embed, int64_t vocab, int64_t hidden, const float* ftab,
                             int64_t ftab_rows, int64_t ftab_cols, uint16_t* x, float* vfreqs, void* stream);

/* The accept walk of one verify step, on the device.
 * Replaces: _C.mtp_accept, csrc/mtp_loop.sycl:86-196.
 *   path = [0]; extend by the first child c (children[cur][j], -1 terminated) with vtok[c] == toks[cur].
 *   result int64 [slots + 24] = [n, commit[slots], row, on_chain, nranks, ranks[7], pos, kept, ...];
 *   st[0] += n; st[1] += kept; ctl[0] = n; ctl[2 + i] = path[i] (i < n) else i; nt = toks[row];
 *   hbuf = x[row]; an off-chain path moves KV slot (pos + path[k]) % cap to (pos + k) % cap in every
 *   table of kv_ptrs (bf16 [kv_heads, cap, head_dim] each), k ascending.
 * cand: int64 [max(depth, 7)][7] draft candidates of the chain nodes for the rank record, or NULL.
 * slots in {8, 16}; kv_cap > slots. */
int mdx_mtp_accept(int64_t* st, const int64_t* toks, const int64_t* vtok, const int64_t* cand,
                   const int32_t* children, int64_t rows, int64_t depth, int64_t slots, const uint16_t* x,
                   int64_t hidden, int64_t* nt, uint16_t* hbuf, int32_t* ctl, const int64_t* kv_ptrs, int64_t nkv,
                   int64_t kv_heads, int64_t kv_cap, int64_t head_dim, int64_t* result, void* stream);

/* Bytes of device workspace the top-k entry points need for `rows` rows. The workspace must be zeroed
 * once when allocated; every launch leaves its counters at zero again. Launches that share one
 * workspace must be ordered (one stream). */
size_t mdx_topk_workspace(int64_t rows);

/* Exact top-k (k <= 8) of one bf16 row in torch's XPU topk order, or (argmax_order, k = 1) its argmax.
 * Replaces: _C.fast_topk, csrc/fast_topk.sycl:67-170 (bindings.cpp:91-92).
 *   topk rank: (bf16 radix key: NaN on top, -0 below +0; then earlier gather position of a sweep of
 *   1024 threads x 4 loads of 8 per 32768 elements); argmax rank: NaN first, -0 == +0, smallest index.
 * x bf16 [V], 32768 <= V < 2^31 (LDS bounds the practical V to a few million); values bf16 [k] = x[idx],
 * indices int64 [k], descending rank. */
int mdx_fast_topk(const uint16_t* x, int64_t V, int64_t k, int32_t argmax_order, uint16_t* values,
                  int64_t* indices, void* workspace, size_t workspace_bytes, void* stream);

/* fast_topk in topk order plus the argmax of the same row, one launch.
 * Replaces: _C.fast_pick, csrc/fast_topk.sycl:172-175. argmax: int64 [1]. */
int mdx_fast_pick(const uint16_t* x, int64_t V, int64_t k, uint16_t* values, int64_t* indices, int64_t* argmax,
                  void* workspace, size_t workspace_bytes, void* stream);

/* Exact top-k (k <= 64) of 1..16 rows in torch's XPU fp32 topk order (bf16 rows: of their fp32 values).
 * Replaces: _C.topk_rows, csrc/topk_rows.sycl:223-246.
 *   rank: (fp32 radix key, the sign-flipped bits: +NaN on top, -NaN at the bottom, -0 below +0; then
 *   earlier gather position of a sweep of 1024 threads x 8 loads of 4 per 32768 elements).
 * x [rows, n] of x_dtype (MDX_DT_F32 or MDX_DT_BF16), 4096 <= n < 2^31; values f32 [rows, k],
 * indices int64 [rows, k]. */
int mdx_topk_rows(const void* x, int32_t x_dtype, int64_t rows, int64_t n, int64_t k, float* values,
                  int64_t* indices, void* workspace, size_t workspace_bytes, void* stream);

/* mdx_topk_rows without a workspace argument: its partial lists and counters live in a file-scope
 * device array of the library (532,736 bytes per device, held until the process ends), so the call
 * allocates nothing (no hipMalloc, hipFree or allocating library routine; the first call on a device
 * takes the array's address and clears its counters with a fill kernel). rows <= 16 (larger counts are
 * rejected). Every call on a device shares that device's array: calls that overlap on one device (two
 * streams, two threads) race; calls on one stream are ordered and each leaves the counters at zero.
 * No counterpart in the reference: for callers that cannot allocate (code under HIP graph capture,
 * serving loops and harnesses that forbid allocation). */
int mdx_topk_rows_noalloc(const void* x, int32_t x_dtype, int64_t rows, int64_t n, int64_t k, float* values,
                          int64_t* indices, void* stream);

/* Gumbel-max sampling over each row's top k: out[r] = indices[r, j*], j* the first maximum over j of
 * values[r, j] * (1 / temperature) - log(-log(clamp(uniform[r, j], 1e-20, 1))), in fp32 (each
 * operation rounded as torch's elementwise kernels round it). values f32 / indices int64 / uniform f32
 * [rows, k] (topk_rows' outputs and torch.rand), out int64 [rows], k <= 64. No counterpart in the
 * reference's _C: the decode loop's sampling arithmetic over topk_rows (comfy_mono_decode_xpu/
 * sampling.py, upstream torch ops), fused into one launch. */
int mdx_topk_sample(const float* values, const int64_t* indices, const float* uniform, float temperature, int64_t rows,
                    int64_t k, int64_t* out, void* stream);

/* mdx_topk_sample with uniforms of its own: uniform[r, j] = (k + 0.5) 2^-23, k the top 23 bits of the
 * SplitMix64 output (Steele, Lea and Flood 2014) for the state seed + (n + 1) 0x9E3779B97F4A7C15,
 * n = counter[0] 1024 + 64 r + j (counter read on the device: the decode step's committed position, so
 * a captured graph draws fresh uniforms at every replay). rows <= 16. No counterpart in the reference
 * (torch's generator there); it keeps the generator's launches out of the decode step. */
int mdx_topk_sample_seeded(const float* values, const int64_t* indices, uint64_t seed, const int64_t* counter,
                           float temperature, int64_t rows, int64_t k, int64_t* out, void* stream);

/* Bytes of device workspace mdx_attn_decode needs for H query heads, Hk kv heads, S rows, head_dim D
 * and cache capacity cap. Zero it once when allocated: every launch leaves its counters at zero. */
size_t mdx_attn_workspace(int64_t H, int64_t Hk, int64_t S, int64_t D, int64_t cap, int64_t chunks_hint);

/* Decode attention of tree-verify rows (mask != NULL) or the MTP draft row (mask == NULL, S == 1).
 * Replaces: _C.attn_dpas, csrc/attn_dpas.sycl:269-342 (and the attn_core contract, layer.py:406-435).
 *   For query head h and row s (kv head kh = h / (H / Hk)): softmax over the scores
 *   q[h, s] . K[kh, t] / sqrt(D) of the cached tokens t in [0, L), L = clamp(seqlen[0], 0, cap), and of
 *   the tree rows t' with bit t' of mask[s] set (keys xk[kh, t'], values xv[kh, t']); out[s, h] =
 *   bf16(sum p V / sum p), or 0 if the row admits no token. P is rounded to bf16 for the P.V product;
 *   partial softmax states merge in fp32 (tolerance parity against a float64 reference).
 * q bf16 [H, S, D] (head / row strides in elements, rows contiguous); key/value bf16 [Hk, cap, D]
 * contiguous; xk/xv bf16 [Hk, S, D] (head / row strides as given, each); mask int32 [S]; out bf16
 * [S, H, D].
 * D in {64, 128, 256}; 1 <= S <= 16; (H / Hk) * S <= 64. seqlen is read on the device.
 * chunks_hint: 0 plans the context split (chunks of >= 128 tokens per wave); n > 0 splits the context
 * into at most n chunks per kv head of >= 32 tokens per wave (as the reference's chunks_hint steers
 * its split). */
int mdx_attn_decode(const uint16_t* q, int64_t q_head_stride, int64_t q_row_stride, const uint16_t* key,
                    const uint16_t* value, const int32_t* seqlen, const uint16_t* xk, int64_t xk_head_stride,
                    int64_t xk_row_stride, const uint16_t* xv, int64_t xv_head_stride, int64_t xv_row_stride,
                    const int32_t* mask, uint16_t* out, int64_t H,
                    int64_t Hk, int64_t S, int64_t D, int64_t cap, int64_t chunks_hint, void* workspace,
                    size_t workspace_bytes, void* stream);

/* Tree-verify attention with the Q/K RMSNorm + RoPE + KV write of mdx_qk_norm_rope_kv in the same launch
 * (no counterpart in the reference: it runs csrc/rope_kv.sycl:120-245 and csrc/attn_dpas.sycl:269-342 as
 * two calls, as mdx_qk_norm_rope_kv + mdx_attn_decode do). For callers that run both back to back on the
 * tree rows: one launch fewer per attention layer, every output bit-identical to that pair's.
 *   q, k, v, weight_q/_k, eps_q/_k, freqs, rd, key, value, position: as mdx_qk_norm_rope_kv (the tree
 *   rows' k / v are written to the cache at position[s]; those positions must lie at or past seqlen[0],
 *   outside the prefix the launch attends); k_out bf16 [Hk, S, D] receives the rows' k (the tree keys the
 *   launch attends), q_out bf16 [H, S, D] the rows' q (may be NULL); seqlen, mask, out, chunks_hint,
 *   workspace (mdx_attn_workspace bytes): as mdx_attn_decode.
 * D == 128, rd in {32, 64, 128}, mask != NULL, 16 < (H / Hk) * S <= 64 (fewer rows: the two calls). */
int mdx_attn_decode_rope(const uint16_t* q, int64_t q_row_stride, int64_t q_head_stride, const uint16_t* k,
                         int64_t k_row_stride, int64_t k_head_stride, const uint16_t* v, int64_t v_row_stride,
                         int64_t v_head_stride, const uint16_t* weight_q, const uint16_t* weight_k, float eps_q,
                         float eps_k, const float* freqs, int64_t freqs_row_stride, int64_t rd, uint16_t* key,
                         uint16_t* value, const int64_t* position, const int32_t* seqlen, const int32_t* mask,
                         uint16_t* k_out, uint16_t* q_out, uint16_t* out, int64_t H, int64_t Hk, int64_t S, int64_t D,
                         int64_t cap, int64_t chunks_hint, void* workspace, size_t workspace_bytes, void* stream);

/* bf16 decode linear for 1..16 rows: out = bf16(x . W^T) with fp32 accumulation (MFMA), optional
 * bf16 residual (out = bf16(float(residual) + float(bf16(acc)))).
 * Replaces: the lm_head F.linear of the device loop (comfy_mono_decode_xpu/mtp_loop.py:221-225) and the
 * bf16 GEMMs of the MTP draft block (comfy_mono_decode_xpu/draft_head.py:179-232).
 * x bf16 [rows, K] contiguous; W bf16 [N, K] row-major (MDX_LAYOUT_ROW) or tile-major (MDX_LAYOUT_TILE:
 * [N/16][K/32][64][8], lane 16 g + c holding row 16 t + c, k in [32 j + 8 g, + 8) of block (t, j));
 * out / residual bf16 [rows, N]. N % 16 == 0, K % 32 == 0. */
int mdx_bf16_linear(const uint16_t* x, const uint16_t* w, int32_t layout, const uint16_t* residual, uint16_t* out,
                    int64_t rows, int64_t N, int64_t K, void* stream);

/* W8A8 linear (the int8 ConvRot lm_head): out[m, n] = bf16((float(acc) * x_scale[m]) * w_scale[n]), acc the
 * exact int32 dot of the int8 row x[m] with the int8 weight row w[n] (two fp32 roundings, no FMA).
 * Replaces: omni_xpu_kernel int8_linear_prequantized(qx, sx, q, s, None, 2) (third-party, 0.2.0b3) as
 * called for the int8 head at comfy_mono_decode_xpu/draft_head.py:228 and by the verify's F.linear on that
 * head (comfy_mono_decode_xpu/mtp_loop.py:221-225); the logit formula is the draft pick's
 * (csrc/draft_lmhead.sycl:217-220).
 * x int8 [rows, K], x_scale f32 [rows], w int8 [N, K] row-major (MDX_LAYOUT_ROW) or tile-major
 * (MDX_LAYOUT_TILE: [N/16][K/64][64][16 B], lane 16 g + c holding row 16 t + c, k in [64 j + 16 g, + 16) of
 * block (t, j)), w_scale f32 [N], out bf16 [rows, N]. 1 <= rows <= 16, N % 16 == 0, K % 64 == 0,
 * K <= 65536. */
int mdx_int8_linear(const int8_t* x, const float* x_scale, const int8_t* w, const float* w_scale, int32_t layout,
                    uint16_t* out, int64_t rows, int64_t N, int64_t K, void* stream);

/* Gated-DeltaNet decode core of one layer with deferred replay, for 1..slots tree-verify rows.
 * Replaces: the GDN phases of _C.layer_gdn (csrc/mono_gdn.sycl:313-607) and _C.layer_gdn_core
 * (csrc/mono_gdn.sycl:702-704).
 *   conv: per channel, the history (conv_state) shifted by the previous step's accepted rows (their
 *   projections from proj_buf[1 - parity]), then for each row ts the k=4 causal conv over its tree
 *   ancestors (ctl parents; history past the root): y = bf16(sum of fma(v, w)), out = bf16(y / (1 + e^-y));
 *   gates: a = bf16(xn . wa[h]), b = bf16(xn . wb[h]) (fp32 dot in the library's fixed order),
 *   decay = exp(g_decay * softplus(a + dt_bias)), beta = bf16(sigmoid(b));
 *   entries: the previous step's accepted slots (replayed, committed; the persistent state keeps these)
 *   then this step's program (prog & 15 = slot, prog & 32 = commit): S *= decay, kv = k^ S,
 *   delta = (v - kv) beta, S += k^ delta, out = q^ S, with k^ = k / max(|k|, 1e-12),
 *   q^ = (q qscale) / max(|q|, 1e-12); gated RMSNorm: core = bf16(bf16((raw w) / sqrt(mean(raw^2) + eps))
 *   * bf16(silu(z))).
 * proj bf16 [rows, C] (C = 2 HK 128 + HV 128: q | k | v); z bf16 [rows, HV 128]; xn bf16 [rows, K] (the
 * normalised layer input), wa / wb bf16 [HV, K] (K % 512 == 0, K <= 4096); conv_w bf16 [C, 4]; conv_state bf16 [C, 3]; proj_buf, qkv_buf bf16 [2, slots, C]; ctl int32
 * [2 + 3 slots] = (pending, parity, accepted[slots], parents[slots], prog[slots]); rec_state f32
 * [HV, 128, 128]; gates f32 [2, slots, HV, 2]; sums f32 [2, slots, HK, 2] (the reference's buffer of
 * q / k sums of squares, neither read nor written: the norms are taken from qkv_buf); gnorm_w bf16 [128];
 * core bf16 [rows, HV 128] (rows without a verify entry are 0). slots in {8, 16}, HV even and <= 128. Tolerance
 * parity (float64 bound); the control walk is exact. */
int mdx_gdn_core(const uint16_t* proj, const uint16_t* z, const uint16_t* xn, const uint16_t* wa, const uint16_t* wb,
                 int64_t K, const uint16_t* conv_w,
                 uint16_t* conv_state, uint16_t* proj_buf, uint16_t* qkv_buf, const int32_t* ctl, const float* dt_bias,
                 const float* g_decay, float* rec_state, float* gates, float* sums, const uint16_t* gnorm_w,
                 float gnorm_eps, float qscale, uint16_t* core, int64_t rows, int64_t HK, int64_t HV, int64_t slots,
                 void* stream);

/* mdx_gdn_core without its last phase: core holds the raw bf16 outputs q^ S of the verify entries (the
 * gated RMSNorm left to mdx_gnorm_rot_quant, which the decode step fuses into the output projection's
 * activation prep). No counterpart of its own in the reference: the first phases of the same
 * layer_gdn (csrc/mono_gdn.sycl:313-571). */
int mdx_gdn_core_raw(const uint16_t* proj, const uint16_t* xn, const uint16_t* wa, const uint16_t* wb, int64_t K,
                     const uint16_t* conv_w, uint16_t* conv_state, uint16_t* proj_buf, uint16_t* qkv_buf,
                     const int32_t* ctl, const float* dt_bias, const float* g_decay, float* rec_state, float* gates,
                     float* sums, float qscale, uint16_t* core, int64_t rows, int64_t HK, int64_t HV, int64_t slots,
                     void* stream);

/* The Gated-DeltaNet input projections with the conv and the gates, in one launch: [proj | z] =
 * W4A8 GEMV of the int8 rows x / x_scale over {w_qkv, w_z} (as mdx_stream_gemv, bf16 outputs), with the
 * deferred causal conv of every qkv channel run by the tile that produced the channel (conv_state,
 * proj_buf, qkv_buf updated as mdx_gdn_core_raw's conv phase, bit for bit) and this step's gates (decay,
 * beta of rows < rows; zeros up to slots) computed by extra work-groups of the same launch from xn, wa,
 * wb, dt_bias, g_decay. Operands as in mdx_gdn_core; w_qkv->n = (2 HK + HV) 128, w_z->n = HV 128, K =
 * w_qkv->k. z_gate (optional, bf16 [rows, HV 128]) receives the gated RMSNorm's gate factors
 * bf16(z / (1 + e^-z)) of the z outputs, for mdx_gnorm_linear with z_gated. With x_row (one row, bf16
 * [K], 16-byte aligned; fp16 scales) the launch also runs the row prep of x_row (RMSNorm with norm_w, eps,
 * then the quantisation: mdx_rms_rot_quant with MDX_ROT_NONE, bit for bit) in its prologue, and x, x_scale
 * and xn are unused (may be NULL). Followed by mdx_gdn_delta. Replaces: the in_proj_qkv / in_proj_z GEMMs of
 * comfy_mono_decode_xpu/layer.py:593 with deltanet_conv_step_deferred and the a / b gates of
 * gated_delta_decode_deferred (comfy_mono_decode_xpu/layer.py:216-228; csrc/mono_gdn.sycl:313-374,
 * :424-450). */
int mdx_gdn_proj(const int8_t* x, const float* x_scale, const mdx_w4* w_qkv, const mdx_w4* w_z, uint16_t* proj,
                 uint16_t* z, const uint16_t* xn, const uint16_t* wa, const uint16_t* wb, const uint16_t* conv_w,
                 uint16_t* conv_state, uint16_t* proj_buf, uint16_t* qkv_buf, const int32_t* ctl,
                 const float* dt_bias, const float* g_decay, float* gates, uint16_t* z_gate, const uint16_t* x_row,
                 const uint16_t* norm_w, float eps, int64_t rows, int64_t HK, int64_t HV, int64_t slots,
                 void* stream);

/* The delta rule of a Gated-DeltaNet step after mdx_gdn_proj: the replay of the previous step's accepted
 * rows and this step's verify program over rec_state, from the conv outputs in qkv_buf and the gates in
 * gates; core receives the raw bf16 outputs q^ S (as mdx_gdn_core_raw). Replaces: the delta-rule phase of
 * gated_delta_decode_deferred (comfy_mono_decode_xpu/layer.py:224-228; csrc/mono_gdn.sycl:459-571). */
int mdx_gdn_delta(const uint16_t* qkv_buf, const int32_t* ctl, float* rec_state, const float* gates, float qscale,
                  uint16_t* core, int64_t rows, int64_t HK, int64_t HV, int64_t slots, void* stream);

/* Gated RMSNorm per 128-element head, then the rotation + row quantisation of mdx_rot_quant:
 * y' = bf16(bf16((y gnorm_w) / sqrt(mean_head(y^2) + eps)) * bf16(silu(z))). y_out (optional, may be y)
 * receives y'; with q = scale = NULL and rot = MDX_ROT_NONE only y' is written. y, z, y_out bf16
 * [rows, K], gnorm_w bf16 [128], K % 256 == 0. Replaces: the gated RMSNorm phase of _C.layer_gdn
 * (csrc/mono_gdn.sycl:574-607) together with the out_proj activation prep that follows it. */
int mdx_gnorm_rot_quant(const uint16_t* y, const uint16_t* z, const uint16_t* gnorm_w, float eps, uint16_t* y_out,
                        const uint16_t* h, int32_t rot, int8_t* q, float* scale, int64_t rows, int64_t K, void* stream);

/* The out_proj of a Gated-DeltaNet layer from its raw outputs: y' = the gated RMSNorm of y (z, gnorm_w, eps;
 * mdx_gnorm_rot_quant's arithmetic; with z_gated, z holds the gate factors bf16(z / (1 + e^-z)) instead, as
 * mdx_gdn_proj's z_gate), quantised per row without rotation, then out = W4A8 GEMV of w (with
 * residual as in mdx_w4a8_decode_linear; bf16). At one or two rows with fp16 scales, one launch: every
 * work-group of the GEMV normalises and quantises the rows in its prologue; otherwise two (the row prep into
 * q int8 [rows, K] / scale f32 [rows], then the GEMV), and q / scale must be given. y_out (optional)
 * receives y'; it may alias y only at the shapes that take two launches. y, z, y_out bf16 [rows, K];
 * gnorm_w bf16 [128]; K = w->k, K % 256 == 0. Replaces: the gated RMSNorm of gated_delta_decode_deferred
 * (csrc/mono_gdn.sycl:574-607) with layer_post's out_proj activation prep and out_proj
 * (csrc/mono_layer.sycl:157-318). */
int mdx_gnorm_linear(const uint16_t* y, const uint16_t* z, int32_t z_gated, const uint16_t* gnorm_w, float eps,
                     uint16_t* y_out, const mdx_w4* w, const uint16_t* residual, uint16_t* out, int8_t* q, float* scale,
                     int64_t rows, void* stream);

/* Sigmoid-gated rotation + row quantisation: y' = bf16(y * sig_lut[gate]), then rot_quant(y').
 * Replaces: the first phase of _C.layer_post (csrc/mono_layer.sycl:243-256: the gated attention output,
 * gate interleaved in q_proj's output as [head][query 256 | gate 256], or a separate [rows, K] gate).
 * Gate element of row r, column i: gate[r * gate_row_stride + (i / gate_head) * gate_head_stride +
 * gate_offset + i % gate_head] (interleaved: 8192, 256, 512, 256; separate: K, K, K, 0). */
int mdx_gate_rot_quant(const uint16_t* y, const uint16_t* gate, int64_t gate_row_stride, int64_t gate_head,
                       int64_t gate_head_stride, int64_t gate_offset, const uint16_t* sig_lut, const uint16_t* h,
                       int32_t rot, int8_t* q, float* scale, int64_t rows, int64_t K, void* stream);

/* RMSNorm of bf16 rows in the library's fixed order (out = bf16((x * r) * w), r = 1 / sqrt(mean(x^2) +
 * eps)). Serves the bf16 lm_head input of the decode loop (the final norm, comfy_mono_decode_xpu/
 * mtp_loop.py:221-225). x, out bf16 [rows, K], K % 256 == 0, K <= 16384, 16-byte aligned. */
int mdx_rmsnorm(const uint16_t* x, const uint16_t* norm_w, float eps, uint16_t* out, int64_t rows, int64_t K,
                void* stream);

/* out[i] = bf16(float(silu_lut[g[i]]) * float(u[i])) over n bf16 elements (the draft block's SwiGLU,
 * comfy_mono_decode_xpu/draft_head.py:214-226; the same rule as mono_mlp's gate/up epilogue). */
int mdx_silu_mul(const uint16_t* g, const uint16_t* u, const uint16_t* silu_lut, uint16_t* out, int64_t n,
                 void* stream);

/* ---- the fused draft-head row ops (comfy_mono_decode_xpu/draft_head.py:179-211) -------------------
 * One work-group per row, rows of hidden size H (H % 256 == 0, H <= 16384). RMSNorm is the library's
 * fixed order (as mdx_rmsnorm); rotations are the exact fp64 FWHT rounded once to fp32 and once to bf16;
 * sigmoid / SiLU come from bf16 lookup tables of torch's own values. The reference computes these in
 * fp32 without a fixed order (draft tokens are only proposals); its tolerance, 1e-2 relative, bounds
 * the difference. Rows of one call are independent: the reference's single-row ops are rows == 1. */

/* fc input of the MTP block: out[r] = [RMSNorm_e(e) | RMSNorm_h(hidden[r])] (bf16 [rows, 2 H]), with the
 * embedding row e = bf16(unrotate(q[t] * s[t])), t = token[r] clamped into [0, V) (int8 [V, H] table,
 * f32 scales [V]; unrotate: the group times H256, or none), or, with q == NULL, e = emb[t] from a bf16 table
 * [V, H] when token is given (t clamped likewise) and e = emb[r] (bf16 [rows, H]) when it is NULL.
 * Replaces: _C.draft_embed_norm_cat, csrc/draft_fused.sycl:76-151 (bindings.cpp:34-36). */
int mdx_draft_embed_norm_cat(const int64_t* token, const int8_t* q, const float* s, int64_t V, int32_t unrotate,
                             const uint16_t* emb, const uint16_t* hidden, const uint16_t* we, const uint16_t* wh,
                             float eps_e, float eps_h, uint16_t* out, int64_t rows, int64_t H, void* stream);

/* x = bf16(x + h) in place when h != NULL (else x is left alone), out = RMSNorm(x) (bf16 [rows, H]).
 * Replaces: _C.draft_add_rmsnorm, csrc/draft_fused.sycl:153-184 (bindings.cpp:37). */
int mdx_draft_add_rmsnorm(uint16_t* x, const uint16_t* h, const uint16_t* w, float eps, uint16_t* out, int64_t rows,
                          int64_t H, void* stream);

/* out[r, i] = bf16(a[r, i] * sig_lut[g]), g = qg[r * qg_row_stride + (i / head_dim) * 2 head_dim + head_dim +
 * i % head_dim] (the gate half of each head of the gated q projection). a, out bf16 [rows, n].
 * Replaces: _C.draft_sigmoid_mul, csrc/draft_fused.sycl:186-203 (bindings.cpp:38). */
int mdx_draft_sigmoid_mul(const uint16_t* a, const uint16_t* qg, int64_t qg_row_stride, int64_t head_dim,
                          const uint16_t* sig_lut, uint16_t* out, int64_t rows, int64_t n, void* stream);

/* out[r, i] = bf16(silu_lut[g] * u), g = gu[r * gu_row_stride + i], u = gu[r * gu_row_stride + n + i] (the
 * concatenated gate | up projection). Replaces: _C.draft_silu_mul, csrc/draft_fused.sycl:205-218
 * (bindings.cpp:39). */
int mdx_draft_silu_mul(const uint16_t* gu, int64_t gu_row_stride, const uint16_t* silu_lut, uint16_t* out,
                       int64_t rows, int64_t n, void* stream);

/* The draft's final norm and the lm_head's activation prep: x = bf16(x + h) in place (h optional),
 * xr = bf16(rotate(RMSNorm(x))) (rot MDX_ROT_H256 or MDX_ROT_NONE); with qx / sx: scale = max(amax(xr) /
 * 127, 1e-30) -> sx, qx = int8(clamp(rint(fl32(xr / bf16(scale))), -128, 127)).
 * Replaces: _C.draft_norm_rot_quant, csrc/draft_fused.sycl:220-287 (bindings.cpp:40-41). */
int mdx_draft_norm_rot_quant(uint16_t* x, const uint16_t* h, const uint16_t* w, float eps, int32_t rot, uint16_t* xr,
                             int8_t* qx, float* sx, int64_t rows, int64_t H, void* stream);

/* Bytes of device workspace the draft pick needs (zeroed once before its first use; every call leaves
 * its counter at zero again). */
size_t mdx_draft_pick_workspace(void);

/* Second stage of the two-stage draft lm_head: from approximate scores approx bf16 [N] of the whole
 * vocabulary, the exact logits of candidates -- bf16((float(acc) * x_scale) * w_scale[n]), acc the int32 dot
 * of the int8 row w[n] [K] with qx int8 [K] -- and of them the top-nout in torch topk's tie order and the
 * argmax (torch argmax rules). With w == NULL the scores are the logits. Candidates: the 32 best scores of
 * each of 32 contiguous segments. Writes top[:nout] and ranks_row[:nout] (each may be NULL), the draft
 * token (the argmax if argmax_first, else top[0]) to token[0] and vtok[children[0]], top[j] to
 * vtok[children[j]] (1 <= j < nchildren <= nout <= 8), and adds 1 to calls[0] (may be NULL).
 * 8192 <= N <= 262144; K % 64 == 0, K <= 16384.
 * Replaces: _C.draft_pick, csrc/draft_lmhead.sycl:82-291 (bindings.cpp:66-68, 86). */
int mdx_draft_pick(const uint16_t* approx, int64_t N, const int8_t* qx, const float* x_scale, const int8_t* w,
                   const float* w_scale, int64_t K, int64_t nout, int32_t argmax_first, int64_t* top, int64_t* ranks_row,
                   int64_t* token, int64_t* vtok, int64_t nvtok, const int64_t* children, int64_t nchildren,
                   int64_t* calls, void* workspace, size_t workspace_bytes, void* stream);

/* The draft pick of a bf16 lm_head: as mdx_draft_pick, the exact logits being those mdx_bf16_linear
 * gives for the row x bf16 [K] and the head w bf16 [N, K] (layout MDX_LAYOUT_TILE or _ROW), recomputed
 * for 16 candidates per segment with the same per-output MFMA chain and K split, so the result equals
 * mdx_bf16_linear + mdx_fast_topk whenever their top-nout lies within the candidates. top_values
 * (bf16 [nout], may be NULL) receives the top-nout logits. K % 32 == 0, K <= 4096. No counterpart in the
 * reference (whose draft head is int8); it serves the synthetic model's bf16 head. */
int mdx_draft_pick_bf16(const uint16_t* approx, const uint16_t* x, const uint16_t* w, int32_t layout, int64_t N, int64_t K,
                        int64_t nout, int32_t argmax_first, int64_t* top, uint16_t* top_values, int64_t* token,
                        int64_t* vtok, int64_t nvtok, const int64_t* children, int64_t nchildren, int64_t* calls,
                        void* workspace, size_t workspace_bytes, void* stream);

/* Exact tree-verify decode attention (the exactness fallback of mdx_attn_decode): the same operands and
 * output, computed in one canonical fp32 order (scores in dimension order, weights by a fixed exp
 * sequence, the normaliser by 64 ordered lane partials and a halving tree, o in token order; the oracle's
 * attention_exact restates it bit for bit). scale: the score scale (1/sqrt(D) in the callers).
 * Replaces: _C.attn_core (csrc/bindings.cpp:81, csrc/attn_port.sycl:355-365; called by
 * comfy_mono_decode_xpu/layer.py:428) in the role of the bit-identical attention port, csrc/attn_port.sycl:1-12
 * (selected by MONO_DECODE_XPU_ATTN, comfy_mono_decode_xpu/layer.py:43,409); not its arithmetic (its upstream
 * is third-party). The Python mirror exposes it as _C.attn_core and _C.attn_exact. D in {64, 128, 256},
 * 1..16 rows, cap + rows <= 16384. */
int mdx_attn_exact(const uint16_t* q, int64_t q_head_stride, int64_t q_row_stride, const uint16_t* key,
                   const uint16_t* value, const int32_t* seqlen, const uint16_t* xk, int64_t xk_head_stride,
                   int64_t xk_row_stride, const uint16_t* xv, int64_t xv_head_stride, int64_t xv_row_stride,
                   const int32_t* mask, uint16_t* out, int64_t H, int64_t Hk, int64_t S, int64_t D, int64_t cap,
                   float scale, void* stream);

/* Calibration: one streaming read of `bytes` (a multiple of 1024) from `src` with the W4A8 GEMV's load
 * pattern (1 KiB per wave instruction, four loads in flight per wave), over `work_groups` work-groups
 * of 256 threads; `sink` (4 bytes) is written only if the data hashes to a marker value. It has no
 * counterpart in the reference: it measures the read roof a single launch of a given size reaches,
 * beside the 8 TB/s spec figure. */
int mdx_stream_read(const void* src, int64_t bytes, int32_t work_groups, uint32_t* sink, void* stream);

/* Diagnostics: the GEMV kernel variants this thread launched since the previous call (at most 64 kept),
 * as records of seven int32: [MFMA kernel (0/1), source (0 int8 rows, 1 bf16 rows quantised in the
 * prologue, 2 one row prepared in the prologue; + 4 integral decode only, + 8 per-weight 16-byte tables
 * only, + 16 per-weight 8-byte tables only), scale dtype (MDX_DT_*), rows, tiles per work-group, K
 * slices, split-K partials kept in the table region (0/1)]. Up to max_records records are copied to out
 * (7 * max_records int32); returns how many launches were recorded, and
 * starts a new record. No counterpart in the reference: it lets tests name the decode path a shape takes. */
int32_t mdx_gemv_trace(int32_t* out, int32_t max_records);

/* Self-check of this library's fp32 -> bf16 rounding (the hardware conversion behind every bf16 result):
 * compares it with the integer round-to-nearest-even formulation (NaN -> 0x7FC0) over all 2^32 fp32 bit
 * patterns, adding the number of disagreements to *mismatches (caller zeroes it) and lowering *first
 * (caller sets 0xFFFFFFFF) to the smallest disagreeing pattern. No counterpart in the reference. */
int mdx_check_bf16_round(unsigned long long* mismatches, uint32_t* first, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* MDX_H */
