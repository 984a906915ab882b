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
 * gate/up: N1 x K1, down: N2 x N1; one codebook for all three; 1 <= rows <= 16.
 * workspace: >= mdx_mono_mlp_workspace(rows, K1, N1) bytes, 256-byte aligned. */
int mdx_mono_mlp(const uint16_t* xn, const uint16_t* norm_w, float eps, const uint16_t* h, int32_t rot,
                 const uint16_t* silu_lut, const mdx_w4* gate, const mdx_w4* up, const mdx_w4* down, uint16_t* out,
                 int64_t rows, void* workspace, size_t workspace_bytes, void* stream);

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

#ifdef __cplusplus
}
#endif
#endif /* MDX_H */
