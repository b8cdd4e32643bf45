/*
 * opengenie_amd — C ABI of the MI355X (gfx950) fused LTX-2.3 DiT block ops.
 *
 * One stateless entry point per fused op of plugyawn/opengenie
 * `ltx_serve/triton_ltx_ops.py` (cited per function as file:line of that
 * reference file). Conventions:
 *   - all pointers are device pointers the caller allocated; nothing here
 *     allocates, frees or synchronises;
 *   - strides are in elements; dtype arguments take the OGA_DT_* codes;
 *   - `stream` is a hipStream_t (NULL = the default stream); kernels are
 *     enqueued on it and the call returns without waiting;
 *   - the return value is 0 on success, a negative OGA_E* code for a bad
 *     argument (oga_last_error() then describes it), or a positive
 *     hipError_t from the launch.
 * Rounding: every op computes in float32 and rounds to bf16 (nearest even)
 * exactly where torch evaluating the reference's torch expression would hold
 * a bf16 result; an intermediate whose torch dtype is float32 is not rounded.
 */
#ifndef OPENGENIE_AMD_H
#define OPENGENIE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OGA_DT_BF16 = 0, OGA_DT_F32 = 1, OGA_DT_F16 = 2 };
enum { OGA_OK = 0, OGA_EINVAL = -1, OGA_EUNSUPPORTED = -2 };

/* Library identification and the last argument-error message (per thread). */
int oga_abi_version(void);
const char* oga_last_error(void);

/*
 * AdaZero from the Ada table: `fused_adazero_from_ada`
 * (triton_ltx_ops.py:40-91; Ada values :983-998; guard :1001-1018).
 * x, y: (batch*tokens, cols) bf16 contiguous, cols in {2048, 4096}.
 * table (P, cols): element (i, c) at table[i*tab_s0 + c*tab_s1].
 * timestep viewed (batch, tokens, P, cols) with strides ts_strides[4]
 * (a zero token stride is allowed: one timestep row shared by all tokens).
 * y = R(R?(R(rms_norm(x)) * R?(1 + scale)) + shift), with
 * shift/scale = R?(R?(table[i]) + ts[b, t, i]) as in the torch path.
 */
int oga_adazero_from_ada(const void* x, void* y, int64_t batch, int64_t tokens, int64_t cols,
                         const void* table, int table_dtype, int64_t tab_s0, int64_t tab_s1,
                         const void* timestep, int ts_dtype, const int64_t ts_strides[4],
                         int shift_index, int scale_index, float eps, void* stream);

/*
 * AdaZero from the Ada table straight into e4m3 codes: the composition of
 * `fused_adazero_from_ada` (triton_ltx_ops.py:40-91) and the input
 * quantizer of the FP8Linear that consumes its output (triton_ltx_ops.py:
 * 1691-1709 -> `fused_fp8_quantize_e4m3` :144-161). No single counterpart
 * in the reference; the codes equal quantizing oga_adazero_from_ada's bf16
 * output with oga_fp8_quantize_e4m3, and the bf16 rows never reach memory.
 * Arguments as oga_adazero_from_ada; q: (batch*tokens, cols) bytes;
 * input_scale: one float32 on the device (scale_zero_dim != 0 for a 0-dim
 * scale tensor, whose reciprocal and products round to bf16 as torch's).
 * Needs 16-byte table and timestep rows.
 */
int oga_adazero_from_ada_fp8(const void* x, void* q, int64_t batch, int64_t tokens, int64_t cols,
                             const void* table, int table_dtype, int64_t tab_s0, int64_t tab_s1,
                             const void* timestep, int ts_dtype, const int64_t ts_strides[4],
                             int shift_index, int scale_index, float eps, const float* input_scale,
                             int scale_zero_dim, void* stream);

/*
 * AdaZero with materialised scale/shift: `fused_adazero`
 * (triton_ltx_ops.py:8-37; guard :1626-1637).
 * x, y viewed (batch, tokens, cols); scale/shift are that shape after torch
 * broadcasting, given by strides (b, t, c) (zero for a broadcast axis).
 */
int oga_adazero(const void* x, void* y, int64_t batch, int64_t tokens, int64_t cols,
                const void* scale, int scale_dtype, const int64_t scale_strides[3],
                const void* shift, int shift_dtype, const int64_t shift_strides[3],
                float eps, void* stream);

/* `fused_adaln_affine_from_ada` (triton_ltx_ops.py:94-141):
 * y = R(R?(x * R?(1 + scale)) + shift). Same table/timestep convention. */
int oga_adaln_affine_from_ada(const void* x, void* y, int64_t batch, int64_t tokens, int64_t cols,
                              const void* table, int table_dtype, int64_t tab_s0, int64_t tab_s1,
                              const void* timestep, int ts_dtype, const int64_t ts_strides[4],
                              int shift_index, int scale_index, void* stream);

/* `fused_mul_from_ada` (triton_ltx_ops.py:695-739): y = R(x * gate). */
int oga_mul_from_ada(const void* x, void* y, int64_t batch, int64_t tokens, int64_t cols,
                     const void* table, int table_dtype, int64_t tab_s0, int64_t tab_s1,
                     const void* timestep, int ts_dtype, const int64_t ts_strides[4],
                     int gate_index, void* stream);

/* `fused_residual_gate_from_ada` (triton_ltx_ops.py:640-692) in the
 * production residual mode: out = R(x + R?(y * gate)). */
int oga_residual_gate_from_ada(const void* x, const void* y, void* out, int64_t batch, int64_t tokens,
                               int64_t cols, const void* table, int table_dtype, int64_t tab_s0,
                               int64_t tab_s1, const void* timestep, int ts_dtype,
                               const int64_t ts_strides[4], int gate_index, void* stream);

/* `fused_residual_gate_bias_from_ada` (triton_ltx_ops.py:204-262):
 * out = R(x + R?(R(y + R(bias)) * gate)). bias is (cols,) bf16 or f32. */
int oga_residual_gate_bias_from_ada(const void* x, const void* y, const void* bias, int bias_dtype,
                                    void* out, int64_t batch, int64_t tokens, int64_t cols,
                                    const void* table, int table_dtype, int64_t tab_s0, int64_t tab_s1,
                                    const void* timestep, int ts_dtype, const int64_t ts_strides[4],
                                    int gate_index, void* stream);

/*
 * A residual gate followed by the AdaZero pass that reads its output, in
 * one pass over the rows. No single counterpart in the reference: it is the
 * composition of `fused_residual_gate_bias_from_ada` (triton_ltx_ops.py
 * :204-262; bias NULL: `fused_residual_gate_from_ada`, :640-692) and
 * `fused_adazero_from_ada` (:40-91), optionally with the FP8Linear input
 * quantizer after it (`fused_fp8_quantize_e4m3`, :144-161), as the block
 * runs them back to back: the self-attention's residual (:3057-3064) then
 * the cross-attention's rms_norm + AdaLN (:2856-2862), and the
 * cross-attention's residual (:2881-2888) then the feed-forward's AdaZero
 * (:3226-3233).
 *   x_out = R(x + R?(R(y + R(bias)) * gate))  (bias NULL: R(x + R?(y * gate)))
 *   out   = AdaZero(x_out) with shift/scale rows shift_index/scale_index,
 *           bf16 rows, or with input_scale given the e4m3 codes of
 *           oga_adazero_from_ada_fp8 (scale_zero_dim as there).
 * Both outputs are bit-identical to the two (three) separate calls. Takes
 * cols 4096, a timestep row shared by all tokens (ts_strides[1] == 0), and
 * 16-byte table and timestep rows; bias, if given, (cols,) bf16 or f32,
 * 32-byte aligned. x_out may be x (in place); out must not overlap either.
 */
int oga_residual_gate_adazero_from_ada(const void* x, const void* y, const void* bias, int bias_dtype,
                                      void* x_out, void* out, int64_t batch, int64_t tokens, int64_t cols,
                                      const void* table, int table_dtype, int64_t tab_s0, int64_t tab_s1,
                                      const void* timestep, int ts_dtype, const int64_t ts_strides[4],
                                      int gate_index, int shift_index, int scale_index, float eps,
                                      const float* input_scale, int scale_zero_dim, void* stream);

/* `fused_residual_gate_bf16` (triton_ltx_ops.py:590-611):
 * out = R(x + R(y * gate)), gate bf16 broadcast to (batch, tokens, cols)
 * through strides (b, t, c). */
int oga_residual_gate_bf16(const void* x, const void* y, const void* gate, const int64_t gate_strides[3],
                           void* out, int64_t batch, int64_t tokens, int64_t cols, void* stream);

/* `fused_bias_add_bf16` (triton_ltx_ops.py:185-201): out = R(x + R(bias)),
 * x (rows, cols) bf16 contiguous, bias (cols,) bf16 or f32. */
int oga_bias_add_bf16(const void* x, const void* bias, int bias_dtype, void* out, int64_t rows,
                      int64_t cols, void* stream);

/* `fused_head_gate_mul_bf16` (triton_ltx_ops.py:614-637):
 * out[r, h*dim_head + d] = R(x[r, ...] * gates[r*g_s0 + h*g_s1]), bf16. */
int oga_head_gate_mul_bf16(const void* x, const void* gates, int64_t g_s0, int64_t g_s1, void* out,
                           int64_t rows, int64_t heads, int64_t dim_head, void* stream);

/*
 * `fused_fp8_quantize_e4m3` (triton_ltx_ops.py:144-161; torch path :146-148;
 * guard :1021-1022): q = e4m3fn(clamp(x * (1/scale), -448, 448)) for n
 * contiguous inputs of dtype x_dtype (OGA_DT_BF16 or OGA_DT_F16, the two the
 * reference's guard takes; x 16-byte aligned). scale is a device float32
 * with one element. scale_is_0dim selects torch's dtype rule for a 0-dim
 * scale tensor (the reciprocal taken to x's dtype before the multiply, the
 * product rounded to x's dtype) versus a (1,)-shaped one (float32 product).
 * q holds n e4m3fn codes.
 */
int oga_fp8_quantize_e4m3(const void* x, int x_dtype, const float* scale, int scale_is_0dim, void* q, int64_t n,
                          void* stream);

/* `fused_gelu_tanh_fp8_quantize_e4m3` (triton_ltx_ops.py:164-182; torch
 * path :165-169): the quantizer above applied to gelu_tanh(x) rounded to
 * x's dtype, with the GELU evaluated in float32 exactly as torch's GPU kernel
 * evaluates gelu(approximate='tanh') (the device tanhf), so the codes equal
 * torch's. The results for all 65536 inputs of x's dtype are a 128 KiB table
 * in a file-scope device array of the library, one per dtype and GPU, built
 * by the first call on that GPU (on the caller's stream; calls on other
 * streams wait for it through an event until it has completed) and only read
 * afterwards; the elements are quantized by looking them up in it. */
int oga_gelu_tanh_fp8_quantize_e4m3(const void* x, int x_dtype, const float* scale, int scale_is_0dim, void* q,
                                    int64_t n, void* stream);

/*
 * `fused_fp8_quantize_e4m3_per_head_4d` (triton_ltx_ops.py:265-317; torch
 * path :976-980; guard :1489-1499). x [B, N, H, D] contiguous, bf16 or fp16
 * (x_dtype), D in {64, 128}, H*D in {1024, 2048, 4096}. scale_out [B, H]
 * float32 = max(amax|x|, 1e-12) / 448; q [B, N, H, D] e4m3fn =
 * e4m3(clamp(x / scale, +-448)). `workspace` holds
 * oga_fp8_per_head_workspace_bytes(...) bytes of caller-owned device memory.
 */
int64_t oga_fp8_per_head_workspace_bytes(int64_t batch, int64_t tokens, int64_t heads, int64_t head_dim);
int oga_fp8_quantize_per_head(const void* x, int x_dtype, void* q, float* scale_out, void* workspace, int64_t batch,
                              int64_t tokens, int64_t heads, int64_t head_dim, void* stream);

/*
 * `fused_video_qk_rmsnorm_rope` (triton_ltx_ops.py:320-378; torch path
 * :958-973; guard :1502-1537). q, k, q_out, k_out: (batch*tokens, heads*128)
 * bf16 contiguous with heads*128 == cols in {2048, 4096}; weights (cols,)
 * bf16 or f32; cos/sin [batch or 1, heads, tokens, 64] with strides
 * cos_strides/sin_strides (last stride 1), bf16 or f32 (same dtype).
 * o = split-RoPE(R(x * inv * w)) with each torch op rounded per dtype.
 */
int oga_video_qk_rmsnorm_rope(const void* q, const void* k, const void* q_weight, const void* k_weight,
                              int weight_dtype, const void* cos, const void* sin, int cs_dtype,
                              const int64_t cos_strides[4], const int64_t sin_strides[4], void* q_out,
                              void* k_out, int64_t batch, int64_t tokens, int64_t cols, int64_t heads,
                              float eps, void* stream);

/* One-tensor form used by `fused_video_qk_rmsnorm_rope_separate`
 * (triton_ltx_ops.py:432-505), which launches it once for q and once for k. */
int oga_video_rmsnorm_rope(const void* x, const void* weight, int weight_dtype, const void* cos,
                           const void* sin, int cs_dtype, const int64_t cos_strides[4],
                           const int64_t sin_strides[4], void* out, int64_t batch, int64_t tokens,
                           int64_t cols, int64_t heads, float eps, void* stream);

/*
 * The attention module's q/k RMSNorm where no RoPE follows: the text
 * cross-attention's `attn_module.q_norm(q)`, `attn_module.k_norm(k)`
 * (triton_ltx_ops.py:1866-1867, the PytorchPreAttention path taken with
 * pe = None), i.e. torch.nn.functional.rms_norm over the last dimension.
 * x, out: (rows, cols) bf16 contiguous, cols in {2048, 4096}; weight (cols,)
 * bf16 or f32, or NULL for none. out = R(x * inv * w) (w = 1 without a
 * weight), inv = 1/sqrt(mean(x^2) + eps), rounded once.
 */
int oga_rmsnorm(const void* x, const void* weight, int weight_dtype, void* out, int64_t rows, int64_t cols,
                float eps, void* stream);

/* `fused_video_qk_bias_rmsnorm_rope` (triton_ltx_ops.py:508-587): q and k
 * first become R(q + R(q_bias)), R(k + R(k_bias)). */
int oga_video_qk_bias_rmsnorm_rope(const void* q, const void* k, const void* q_bias, const void* k_bias,
                                   int bias_dtype, const void* q_weight, const void* k_weight,
                                   int weight_dtype, const void* cos, const void* sin, int cs_dtype,
                                   const int64_t cos_strides[4], const int64_t sin_strides[4],
                                   void* q_out, void* k_out, int64_t batch, int64_t tokens, int64_t cols,
                                   int64_t heads, float eps, void* stream);

/* `fused_video_qkv_rmsnorm_rope_pack` (triton_ltx_ops.py:381-429): writes
 * qkv [batch, tokens, 3, heads, 128] = (rope(q), rope(k), v). */
int oga_video_qkv_rmsnorm_rope_pack(const void* q, const void* k, const void* v, const void* q_weight,
                                    const void* k_weight, int weight_dtype, const void* cos,
                                    const void* sin, int cs_dtype, const int64_t cos_strides[4],
                                    const int64_t sin_strides[4], void* qkv_out, int64_t batch,
                                    int64_t tokens, int64_t cols, int64_t heads, float eps, void* stream);

/*
 * FP8 linear: the patched `FP8Linear.forward` (triton_ltx_ops.py:1671-1718),
 * `fp8_linear_from_quantized_e4m3` (:742-759) and `fp8_linear_without_bias`
 * (:762-781). a [M, K] and w [N, K] are e4m3fn codes with row strides lda,
 * ldw (K-contiguous); scale_a, scale_b device float32 scalars.
 * out [M, N] bf16 (row stride ldo) = R(acc * (scale_a*scale_b)), then, if
 * bias (N,) is given, R(out + R(bias)) — the two roundings of `_scaled_mm`
 * followed by the separate bias add. K must be a multiple of 128; a, w rows
 * 16-byte aligned; out 16-byte aligned with ldo a multiple of 8.
 */
int oga_fp8_linear(const void* a, int64_t lda, const void* w, int64_t ldw, const float* scale_a,
                   const float* scale_b, const void* bias, int bias_dtype, void* out, int64_t ldo,
                   int64_t m, int64_t n, int64_t k, void* stream);

/*
 * The same FP8 linear (same reference interface) with a caller-owned device
 * workspace of oga_fp8_linear_workspace_bytes(m, n, k) bytes (16-byte
 * aligned). When the 256 x 256 output tiles do not fill a last round of the
 * CUs (e.g. M = 9216, N = 4096: 576 tiles on 256 CUs; or M = 256: 16 tiles),
 * the tiles of that round may be cut into K-chunks whose float32 partial
 * sums go to the workspace and are added in chunk order (deterministic);
 * the chunk count weighs the chunks' time against the partials' traffic,
 * and the size is 0 when no cut pays. A null or smaller workspace (and a
 * size of 0) runs oga_fp8_linear's schedule.
 */
int64_t oga_fp8_linear_workspace_bytes(int64_t m, int64_t n, int64_t k);

/*
 * Grouped FP8 linear: `groups` (1..4) linears of n_group output columns each
 * on one quantized input a [M, K], in one persistent launch — the exact
 * grouped Q/K/V (Q/K) projection of `fp8_qkv_from_grouped_mm` /
 * `fp8_qk_from_grouped_mm` (triton_ltx_ops.py:890-955: torch._scaled_grouped_mm
 * with one weight scale per linear, then + bias). w, scale_b, bias and out are
 * host arrays of `groups` device pointers: w[i] [n_group, K] e4m3 (row stride
 * ldw), scale_b[i] a float32 scalar, bias[i] (n_group,) bf16 16-byte aligned or
 * null, out[i] [M, n_group] bf16 (row stride ldo). out[i] = R(R(acc_i *
 * scale_a * scale_b[i]) + R(bias[i])) as oga_fp8_linear gives per group.
 * K >= 256 and a multiple of 128; n_group a multiple of 128, and of 256 when
 * groups > 1. Workspace: oga_fp8_linear_workspace_bytes(M, groups * n_group, K).
 */
int oga_fp8_linear_grouped_ws(const void* a, int64_t lda, const void* const* w, int64_t ldw, const float* scale_a,
                              const float* const* scale_b, const void* const* bias, int bias_dtype,
                              void* const* out, int64_t ldo, int64_t m, int64_t n_group, int64_t groups, int64_t k,
                              void* workspace, int64_t workspace_bytes, void* stream);
int oga_fp8_linear_ws(const void* a, int64_t lda, const void* w, int64_t ldw, const float* scale_a,
                      const float* scale_b, const void* bias, int bias_dtype, void* out, int64_t ldo,
                      int64_t m, int64_t n, int64_t k, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * The FP8 linear with its output dtype: out_dtype OGA_DT_BF16 (as
 * oga_fp8_linear_ws) or OGA_DT_F16, the patched FP8Linear.forward of an fp16
 * model (out_dtype = x.dtype, triton_ltx_ops.py:1697-1709):
 * out = R(R(acc * scale_a * scale_b) + R(bias)) with R rounding to fp16;
 * the bias of an fp16 output is passed as fp16 (bias_dtype OGA_DT_F16, the
 * reference's bias.to(out.dtype)). Other arguments as oga_fp8_linear_ws.
 */
int oga_fp8_linear_dt_ws(const void* a, int64_t lda, const void* w, int64_t ldw, const float* scale_a,
                         const float* scale_b, const void* bias, int bias_dtype, void* out, int out_dtype,
                         int64_t ldo, int64_t m, int64_t n, int64_t k, void* workspace, int64_t workspace_bytes,
                         void* stream);

/*
 * Dense non-causal attention: the video self-attention that the reference
 * runs through FlashAttention-3 flash_attn_func(q, k, v) on [B, N, H, D]
 * views (benchmarks/official_ltx23_benchmark.py:3294-3369).
 * q [B, Nq, H, D], k/v [B, Nk, H, D], o [B, Nq, H, D] bf16, D == 128; each
 * given by element strides (batch, token, head) with unit stride along D
 * (multiples of 8, 16-byte aligned bases). o = softmax(q k^T * scale) v with
 * float32 softmax and accumulation, P rounded to bf16 before the P.V product.
 * Up to 256 keys (the text cross-attention's prompt) each head's K and V stay
 * in LDS while a workgroup runs a range of its 32-query groups; the result
 * is bit for bit the streaming kernel's (the same key steps in the same
 * order).
 */
int oga_attention(const void* q, const int64_t q_strides[3], const void* k, const int64_t k_strides[3],
                  const void* v, const int64_t v_strides[3], void* o, const int64_t o_strides[3], int64_t batch,
                  int64_t nq, int64_t nk, int64_t heads, int64_t head_dim, float softmax_scale, void* stream);

/*
 * oga_attention with a caller-provided workspace of
 * oga_attention_workspace_bytes(batch, nq, nk, heads, head_dim) bytes
 * (16-byte aligned; 0 bytes and a null workspace run oga_attention). The
 * kernel runs one workgroup per 256-query block per CU at a time; the blocks
 * that would fill only part of a last round of the CUs (e.g. 1152 blocks on
 * 256 CUs at 9216 tokens x 32 heads) are cut into 2..8 parts over their keys,
 * whose float32 partial outputs, maxima and sums go to the workspace and are
 * merged by a second kernel on the same stream. Results agree with
 * oga_attention to float32 summation order. The size depends on the current
 * device's CU count; a smaller workspace is an error.
 * Same interface as oga_attention (benchmarks/official_ltx23_benchmark.py:3294-3369).
 */
int64_t oga_attention_workspace_bytes(int64_t batch, int64_t nq, int64_t nk, int64_t heads, int64_t head_dim);
int oga_attention_ws(const void* q, const int64_t q_strides[3], const void* k, const int64_t k_strides[3],
                     const void* v, const int64_t v_strides[3], void* o, const int64_t o_strides[3], int64_t batch,
                     int64_t nq, int64_t nk, int64_t heads, int64_t head_dim, float softmax_scale, void* workspace,
                     int64_t workspace_bytes, void* stream);

/*
 * oga_attention_ws whose output goes straight into the input quantizer of
 * the FP8 linear that reads it (the attention module's to_out,
 * triton_ltx_ops.py:1691-1709 / :762-781 after the attention call,
 * benchmarks/official_ltx23_benchmark.py:3294-3369): o8 receives
 * e4m3(clamp(R(o) * r, +-448)), one byte per element with o_strides, as
 * `fused_fp8_quantize_e4m3` (:144-161) writes for the bf16 o of
 * oga_attention_ws (r = 1/out_scale[0]; scale_zero_dim: a 0-dim scale, r and
 * the product rounded to bf16). No counterpart in the reference: the codes
 * are bit for bit those of the two calls, and the bf16 o is never written.
 * Same workspace as oga_attention_ws.
 */
int oga_attention_e4m3_out_ws(const void* q, const int64_t q_strides[3], const void* k, const int64_t k_strides[3],
                              const void* v, const int64_t v_strides[3], void* o8, const int64_t o_strides[3],
                              int64_t batch, int64_t nq, int64_t nk, int64_t heads, int64_t head_dim,
                              float softmax_scale, const float* out_scale, int scale_zero_dim, void* workspace,
                              int64_t workspace_bytes, void* stream);

/*
 * FP8 inputs of the attention (benchmarks/official_ltx23_benchmark.py
 * :3333-3340, descales from `fused_fp8_quantize_e4m3_per_head_4d`):
 * out[b, n, h, :] = R(e4m3(x8[b, n, h, :]) * descale[b, h]) as bf16;
 * x8/out contiguous [B, N, H, D], D a multiple of 16.
 */
int oga_fp8_dequant_per_head(const void* x8, const float* descale, void* out, int64_t batch, int64_t tokens,
                             int64_t heads, int64_t head_dim, void* stream);

/*
 * FP8 attention: FlashAttention-3's flash_attn_func on per-head e4m3 q, k, v
 * with float32 [B, H] descales, as the reference calls it for FP8 video
 * self-attention (official_ltx23_benchmark.py:3330-3340):
 *   O = softmax(q8 k8^T * qd kd * softmax_scale) v8 * vd,
 * both products on e4m3 MFMA, P rounded to e4m3 for the second (float32 row
 * sums). q8/k8/v8 [B, N, H, 128] e4m3 with element strides (b, n, h), each a
 * multiple of 16; o as for oga_attention. The workspace (256-byte aligned,
 * oga_attention_fp8_workspace_bytes) holds V rewritten d-major for the
 * second product, then float32 partials of a key-split last round of the CUs
 * when it is large enough.
 */
int64_t oga_attention_fp8_workspace_bytes(int64_t batch, int64_t nq, int64_t nk, int64_t heads, int64_t head_dim);
int oga_attention_fp8_ws(const void* q8, const int64_t q_strides[3], const void* k8, const int64_t k_strides[3],
                         const void* v8, const int64_t v_strides[3], const float* q_descale, const float* k_descale,
                         const float* v_descale, void* o, const int64_t o_strides[3], int64_t batch, int64_t nq,
                         int64_t nk, int64_t heads, int64_t head_dim, float softmax_scale, void* workspace,
                         int64_t workspace_bytes, void* stream);

/*
 * Conversion self-test: runs the device rounding primitives every kernel
 * uses on n float32 inputs: bf16_out[i] = bf16 bits of R(in[i]) and
 * e4m3_out[i] = e4m3fn(clamp(in[i], +-448)). No reference counterpart; it
 * lets a test pin the hardware conversions against the oracle bit by bit.
 */
int oga_selftest_convert(const float* in, uint16_t* bf16_out, uint8_t* e4m3_out, int64_t n, void* stream);

/*
 * Allocation-free variant of oga_fp8_quantize_per_head. No counterpart in
 * the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The amax partials live in a static device array of
 * oga_fp8_per_head_noalloc_max_bytes() bytes (1 MiB) that each GPU holds
 * until the process ends; a shape needing more (batch * ceil(tokens/16) *
 * heads * 4 bytes, e.g. up to 131072 tokens at 32 heads) is rejected with
 * OGA_EUNSUPPORTED. Nothing is allocated or freed. Calls on one GPU share
 * that array, so calls that overlap in time on one GPU race. Same results as
 * oga_fp8_quantize_per_head.
 */
int64_t oga_fp8_per_head_noalloc_max_bytes(void);
int oga_fp8_quantize_per_head_noalloc(const void* x, int x_dtype, void* q, float* scale_out, int64_t batch,
                                      int64_t tokens, int64_t heads, int64_t head_dim, void* stream);

/*
 * Schedule query of the token-row kernels: how many token rows of one batch
 * a single wave streams in sequence for an op of `kind` at this shape on the
 * current device (OGA_ROWS_ADAZERO: oga_adazero[_from_ada];
 * OGA_ROWS_ELEMENTWISE: the AdaLN affine, mul and residual-gate ops). 0 for
 * an unsupported shape. No reference counterpart; it lets a test show that
 * a shape reaches the multi-row code path of a kernel.
 */
enum { OGA_ROWS_ADAZERO = 0, OGA_ROWS_ELEMENTWISE = 1 };
int64_t oga_rows_per_wave(int kind, int64_t batch, int64_t tokens, int64_t cols);

#ifdef __cplusplus
}
#endif

#endif /* OPENGENIE_AMD_H */
