/*
 * claudemaxing_amd: C ABI of the MI355X (gfx950) QLoRA training-step kernel set.
 *
 * Every entry point
 *   - takes plain device pointers, element counts and strides, never torch types;
 *   - is stream-ordered on `stream` (a hipStream_t passed as void*, NULL = the null stream);
 *   - never allocates, never synchronises the host, holds no mutable global state (save the
 *     per-device address of cm_lmhead_ce_noalloc's scratch array, found once);
 *   - returns 0 on success, or a hipError_t value (hipErrorInvalidValue = 1 for bad arguments;
 *     launch failures are reported from hipGetLastError()). cm_error_string() names a code.
 *
 * Each declaration cites the reference (arturbaimuratov1-sys/claudemaxing, Triton) kernel and
 * host function whose behaviour it reproduces.
 */
#ifndef CLAUDEMAXING_AMD_H
#define CLAUDEMAXING_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CM_ABI_VERSION 9

/* Element types of tensor arguments. */
typedef enum {
  CM_F32 = 0,
  CM_F16 = 1,
  CM_BF16 = 2,
  CM_U8 = 3,
  CM_I32 = 4,
  CM_I64 = 5
} cm_dtype;

/* ABI version of the loaded library (CM_ABI_VERSION it was built with). */
int cm_abi_version(void);

/* Human-readable name of a return code of this library. Never NULL. */
const char* cm_error_string(int code);

/* ------------------------------------------------------------------------------------------ */
/* NF4 dequantization with the nested (double-quantized) absmax decoded in the same pass.
 * Replaces solution/nf4.py:26-46 (nf4_dequant_kernel) as launched by dequantize_nf4
 * (solution/nf4.py:64-82).
 *
 * Byte i of `packed` holds elements 2i (high nibble) and 2i+1 (low nibble). Element j belongs to
 * absmax block b = j / blocksize. With nested != 0 the block scale is
 *   s = code2[absmax_u8[b]] * absmax2[b / blocksize2] + offset[0]   (fp32 multiply, then add;
 *                                                                     never fused)
 * otherwise s = absmax_f32[b]. Output j = round_to_nearest_even(code[nibble_j] * s) in out_dtype
 * (CM_F16 or CM_F32, or CM_BF16). blocksize must be even and >= 32 (bitsandbytes' blocksizes),
 * blocksize2 >= 1. Bit-exact with the reference for every input.
 */
int cm_nf4_dequant(const uint8_t* packed, const void* absmax, int nested, const float* code,
                   const float* code2, const float* absmax2, const float* offset, void* out,
                   int out_dtype, int64_t n_bytes, int blocksize, int blocksize2, void* stream);

/* The adapters' weight gradients, up to 4 at once: job q computes sum over the T token rows of
 * outer(w_q[t], r_q[t]) in fp32, w_q [T, d_q] fp16 (row stride ldw_q, even; d_q a multiple of 8;
 * 4-byte aligned), r_q [T, rank] fp16 contiguous (16-byte aligned), into out_q: [rank, d_q] when
 * d_major_q = 0 (lora_A's gradient ga16^T xd16: w = xd16, r = ga16; out 4-byte aligned),
 * [d_q, rank] when 1 (lora_B's gradient g16^T a16: w = g16, r = a16; out 16-byte aligned).
 * Replaces the token-sum GEMMs of LoRABranch.backward (solution/lora.py:96-107). One launch;
 * the sums are formed in a fixed order (the same inputs give the same bits). The workspace
 * query returns 0 and `workspace` is not used (it may be null). rank must be 16. */
int64_t cm_lora_weight_grads_workspace_bytes(int64_t T, int max_d, int n_jobs);
int cm_lora_weight_grads(const void* const* w, const int64_t* ldw, const int* d,
                         const void* const* r, float* const* out, const int* d_major, int n_jobs,
                         int64_t T, int rank, void* workspace, int64_t ws_bytes, void* stream);

/* ------------------------------------------------------------------------------------------ */
/* fp16 products with an fp32 result, split along the contraction: C [M, N] fp32 =
 * A0 B0^T (+ A1 B1^T), A_q [M, K_q] and B_q [N, K_q] fp16 row-major (row strides lda_q, ldb_q,
 * multiples of 8; K_q multiples of 8; K1 = 0 for one pair). Replaces, in the training step, the
 * torch.mm / addmm calls of the MLP whose output is narrow next to their contraction: the down
 * projection's forward (F.linear of the dequantized weight, solution/nf4.py:102-130, the product
 * bitsandbytes' gemm_4bit falls back to) and the MLP input gradient dgate Wg + dup Wu (autograd
 * of the two projections, the reference's MLPInputRecompute backward). Work split into K-slices
 * whose fp32 partial tiles go to `workspace` (cm_gemm_f32_workspace_bytes bytes) and are added in
 * slice order: deterministic, sums in fp32 (their order differs from a library GEMM's). All
 * pointers 16-byte aligned, M * N a multiple of 4. */
int64_t cm_gemm_f32_workspace_bytes(int M, int N, int K0, int K1);
int cm_gemm_f32(const void* a0, int64_t lda0, const void* b0, int64_t ldb0, int K0,
                const void* a1, int64_t lda1, const void* b1, int64_t ldb1, int K1, int M, int N,
                float* out, void* workspace, int64_t ws_bytes, void* stream);
/* cm_gemm_f32 with a residual: out = residual + (the same sum), one more fp32 rounding, in the
 * slice-sum launch (residual [M, N] fp32 contiguous, 16-byte aligned, not overlapping out). No
 * counterpart in the reference: the end of transformers' Qwen2DecoderLayer.forward adds the
 * residual to the MLP's output in torch (`residual + hidden_states`). */
int cm_gemm_f32_add(const void* a0, int64_t lda0, const void* b0, int64_t ldb0, int K0,
                    const void* a1, int64_t lda1, const void* b1, int64_t ldb1, int K1, int M,
                    int N, const float* residual, float* out, void* workspace, int64_t ws_bytes,
                    void* stream);
/* cm_gemm_f32 with each B_q given k-major: element (n, k) of B_q at b_q[k * ldb_q + n] (ldb_q >=
 * N, a multiple of 8; N a multiple of 8), i.e. a weight W_q [K_q, N] as stored, so that
 * out = sum_q A_q W_q (the MLP input gradient dgate Wg + dup Wu on the weights expanded by
 * cm_nf4_dequant, without a transposed copy). The same bits as cm_gemm_f32 on the transposed
 * operands. Same workspace query. No counterpart in the reference (a layout of the operand). */
int cm_gemm_f32_kb(const void* a0, int64_t lda0, const void* b0, int64_t ldb0, int K0,
                   const void* a1, int64_t lda1, const void* b1, int64_t ldb1, int K1, int M,
                   int N, float* out, void* workspace, int64_t ws_bytes, void* stream);

/* The same expansion written transposed, fp16 only: out[c][r] = W[r][c] for the weight W
 * [rows, cols] (rows a multiple of 64, cols of 128; packed 4-byte, out 16-byte aligned), the values
 * bit-identical to cm_nf4_dequant's. No counterpart in the reference: the MLP backward of the
 * training step takes the gate/up weights this way, so that its input-gradient products
 * (dgate Wg, dup Wu) read both operands along the contraction. */
int cm_nf4_dequant_t(const uint8_t* packed, const void* absmax, int nested, const float* code,
                     const float* code2, const float* absmax2, const float* offset, void* out,
                     int64_t rows, int64_t cols, int blocksize, int blocksize2, void* stream);

/* ------------------------------------------------------------------------------------------ */
/* RMSNorm forward, one row per wavefront. Replaces solution/rmsnorm.py:28-47
 * (qwen_rmsnorm_fwd_kernel) as launched by RMSNorm.forward (solution/rmsnorm.py:147-192).
 *   rstd[r] = 1 / sqrt(sum_c x[r,c]^2 / n_cols + eps)            (fp32)
 *   normed = round_x(x * rstd);  out = round_out(normed * w)
 * x is row-major [n_rows, n_cols] with row stride x_row_stride (elements); out is contiguous.
 * With low16 != NULL (the SAVE_LOW path: fp32 x, frozen fp32 w), also writes
 *   low16[r,c] = fp16(normed * w) and small16[r * n_small + slot[c]] = fp16(normed) for slot[c] >= 0.
 * n_small = 0 says the weight has no tiny-|w| column: slot is then not read.
 */
int cm_rmsnorm_fwd(const void* x, int x_dtype, int64_t x_row_stride, const void* w, int w_dtype,
                   void* out, int out_dtype, float* rstd, void* low16, const int32_t* slot,
                   void* small16, int n_small, int64_t n_rows, int n_cols, float eps,
                   void* stream);

/* RMSNorm backward. Replaces solution/rmsnorm.py:51-91 (qwen_rmsnorm_bwd_kernel) as launched
 * by RMSNorm.backward (solution/rmsnorm.py:194-217).
 * saved_output == 0: `xs` holds x (x_dtype);  normed = x * rstd;  gn = round_x(dy * w).
 * saved_output != 0: `xs` holds the fp16 copy of the output (low16 of the forward); normed is
 *   small16[r, slot[c]] where slot[c] >= 0, else xs / w;  gn = dy * w (x is fp32: no rounding).
 *   dx[r,c] = round_x((gn - normed * sum_c(gn * normed) / n_cols) * rstd)
 * dw_partial (may be NULL) receives per-workgroup fp32 partial sums of dy * round_x(normed), one
 * row of n_cols per workgroup; the number of rows written is cm_rmsnorm_bwd_partials(n_rows).
 */
int cm_rmsnorm_bwd(const void* dy, int dy_dtype, const void* xs, int xs_dtype, const void* w,
                   int w_dtype, const float* rstd, void* dx, int dx_dtype, float* dw_partial,
                   const int32_t* slot, const void* small16, int n_small, int saved_output,
                   int64_t n_rows, int n_cols, void* stream);
/* Number of partial dw rows cm_rmsnorm_bwd writes for n_rows rows. */
int64_t cm_rmsnorm_bwd_partials(int64_t n_rows);

/* The residual add before a norm, fused into it. No counterpart in the reference: transformers'
 * Qwen2DecoderLayer.forward (modeling_qwen2.py) adds the residual in torch (`residual +
 * hidden_states`) and then calls the norm, which solution/rmsnorm.py:147-192 replaces.
 *   h = residual + x   (fp32, one rounding; residual contiguous fp32 [n_rows, n_cols]; x of any
 *                       float dtype with row stride x_row_stride), written to h
 *   then cm_rmsnorm_fwd of h (an fp32 input): out (fp32), rstd, and low16 / small16 as there.
 */
int cm_rmsnorm_add_fwd(const float* residual, const void* x, int x_dtype, int64_t x_row_stride,
                       const void* w, int w_dtype, float* h, float* out, float* rstd, void* low16,
                       const int32_t* slot, void* small16, int n_small, int64_t n_rows,
                       int n_cols, float eps, void* stream);

/* cm_rmsnorm_bwd for an fp32 x with the residual's gradient added and an fp16 copy written. No
 * counterpart in the reference: autograd adds the two gradients of the decoder layer's h (the
 * residual's and the norm's) in torch, and the projection before h casts that sum to fp16.
 *   dx = dres + (cm_rmsnorm_bwd's dx)   (fp32, one rounding; dres NULL: the norm's dx alone)
 *   dx16 = fp16(dx) when dx16 != NULL
 * dres, dx and dx16 are contiguous [n_rows, n_cols]; the other arguments as cm_rmsnorm_bwd's.
 */
int cm_rmsnorm_bwd_res(const void* dy, int dy_dtype, const void* xs, int xs_dtype, const void* w,
                       int w_dtype, const float* rstd, const float* dres, float* dx, void* dx16,
                       float* dw_partial, const int32_t* slot, const void* small16, int n_small,
                       int saved_output, int64_t n_rows, int n_cols, void* stream);

/* ------------------------------------------------------------------------------------------ */
/* Rotary position embedding, forward or backward (transposed rotation), on up to two tensors
 * (q and k) in one launch. Replaces solution/rope.py:17-43 (qwen_rope_kernel) as launched twice
 * by RoPE.forward / RoPE.backward (solution/rope.py:60-76, _rotate 46-57).
 * x_i is [B, H_i, T, D] with element strides (sb_i, sh_i, st_i, 1); cos/sin are [Bc, T, D] with
 * strides (cs_b, cs_t, 1); cs_b = 0 broadcasts one row of positions over the batch.
 * out_i is contiguous [B, H_i, T, D], or [B, T, H_i, D] (token-major) with bit 1 of flags. With
 * h = D/2 and bit 0 of flags selecting the backward rotation:
 *   forward:  o[:h] = x1*c1 - x2*s1;  o[h:] = x2*c2 + x1*s2
 *   backward: o[:h] = x1*c1 + x2*s2;  o[h:] = x2*c2 - x1*s1         (fp32 arithmetic)
 * Pass x1 = NULL (H1 = 0) to rotate one tensor. D must be even and <= 512. Each tensor has its
 * own input and output dtype; the two share one launch when the dtypes agree, and for fp32
 * cos/sin with fp32 x0/out0 and (x1, out1) = (fp16, fp32) or (fp32, fp16).
 */
int cm_rope(const void* x0, int x0_dtype, int64_t sb0, int64_t sh0, int64_t st0, int H0,
            void* out0, int out0_dtype, const void* x1, int x1_dtype, int64_t sb1, int64_t sh1,
            int64_t st1, int H1, void* out1, int out1_dtype, const void* cos, const void* sin,
            int cs_dtype, int64_t cs_b, int64_t cs_t, int B, int T, int D, int flags,
            void* stream);

/* ------------------------------------------------------------------------------------------ */
/* SwiGLU forward: out = round_out(round_g?(silu(g)) * u), silu(g) = g / (1 + 2^(-g*log2(e))).
 * Replaces solution/swiglu_recompute.py:36-48 (silu_mul_fwd_persistent) as launched by
 * SwiGLURecompute.forward (91-104) and MLPInputRecompute.forward (155-186).
 * round_silu != 0 rounds silu to g_dtype before the product. All tensors contiguous, n elements.
 */
int cm_swiglu_fwd(const void* gate, int g_dtype, const void* up, int u_dtype, void* out,
                  int out_dtype, int64_t n, int round_silu, void* stream);

/* SwiGLU backward with silu recomputed from gate. Replaces solution/swiglu_recompute.py:51-79
 * (silu_mul_bwd_recompute) as launched by SwiGLURecompute.backward (106-122) and
 * MLPInputRecompute.backward (188-215).
 *   sig = 1/(1 + 2^(-g*log2(e)));  d_up = round_u(dy * round_g?(g*sig));
 *   d_gate = round_g(round_g?(dy * u) * sig * (1 + g*(1 - sig)))
 * dgate may equal gate and dup may equal up (in place: every element is read before it is
 * written). want_dgate / want_dup select the outputs written.
 */
int cm_swiglu_bwd(const void* dy, int dy_dtype, const void* gate, int g_dtype, const void* up,
                  int u_dtype, void* dgate, void* dup, int64_t n, int want_dgate, int want_dup,
                  int round_silu, void* stream);

/* The two SwiGLU kernels above over rows: gate and up are [rows, cols] with rows ld_gu elements
 * apart (the two halves of one [rows, 2F] gate/up product, up = gate + F), out and dy rows
 * ld_out / ld_dy apart. The same values, element for element, as cm_swiglu_fwd / cm_swiglu_bwd
 * on contiguous copies. Replace the same reference kernels (solution/swiglu_recompute.py:36-48,
 * 51-79) where the MLP multiplies both projections in one product
 * (MLPInputRecompute.forward / backward, swiglu_recompute.py:155-215). cols and every ld a
 * multiple of 8, ld >= cols, all pointers 16-byte aligned; dgate / dup may equal gate / up.
 */
int cm_swiglu_fwd_rows(const void* gate, int g_dtype, const void* up, int u_dtype,
                       int64_t ld_gu, void* out, int out_dtype, int64_t ld_out, int64_t rows,
                       int64_t cols, int round_silu, void* stream);
int cm_swiglu_bwd_rows(const void* dy, int dy_dtype, int64_t ld_dy, const void* gate,
                       int g_dtype, const void* up, int u_dtype, int64_t ld_gu, void* dgate,
                       void* dup, int64_t rows, int64_t cols, int want_dgate, int want_dup,
                       int round_silu, void* stream);

/* ------------------------------------------------------------------------------------------ */
/* LoRA dropout mask pack. Replaces solution/lora.py:30-42 (lora_dropout_pack_kernel) as
 * launched by _pack (lora.py:60-66).
 *   xd[i] = fp16(keep[i] ? x[i] * scale : 0);  bits[i/8] bit (i%8) = keep[i] != 0
 * keep is a bool/uint8 array of n elements; n must be a multiple of 8. Bit-exact.
 */
int cm_lora_pack(const void* x, int x_dtype, const uint8_t* keep, void* xd16, uint8_t* bits,
                 int64_t n, float scale, void* stream);

/* LoRA dropout mask unpack. Replaces solution/lora.py:45-57 (lora_dropout_unpack_kernel) as
 * launched by _unpack (lora.py:69-75).
 *   keep = bits[i/8] >> (i%8) & 1;  xd[i] = fp16(keep ? x16[i]*scale : 0);
 *   dx[i] = round_dx(keep ? g16[i]*scale : 0)
 * n must be a multiple of 8. Bit-exact.
 */
int cm_lora_unpack(const void* x16, const uint8_t* bits, const void* g16, void* xd16, void* dx,
                   int dx_dtype, int64_t n, float scale, void* stream);

/* ------------------------------------------------------------------------------------------ */
/* Cross-entropy statistics of full logits, one row per workgroup (the fallback when logits
 * exist anyway). Replaces solution/lm_head_loss.py:54-96 (lm_head_xent_rows_kernel) as launched
 * by _rows / head_metrics_from_logits (lm_head_loss.py:168-172, 285-297).
 *   loss[r] = label ? lse - z[t] : 0;  entropy[r] = lse - sum(e^z z)/sum(e^z);
 *   correct[r] = label && first_argmax == t.  With write_grad, the row is overwritten by
 *   round((softmax - onehot) * grad_scale) (zero for unlabelled rows).
 * logits [n_rows, n_cols] (f16/bf16/f32) with row stride `row_stride`; target int64 [n_rows]
 * with -100 = ignored.
 */
int cm_xent_rows(void* logits, int logits_dtype, int64_t row_stride, const int64_t* target,
                 float* loss, float* entropy, int32_t* correct, int64_t n_rows, int64_t n_cols,
                 int write_grad, float grad_scale, void* stream);

/* ------------------------------------------------------------------------------------------ */
/* Fused LM head + cross-entropy with per-row loss, entropy, accuracy and the hidden-state
 * gradient. The full [n_rows, V] logits are never stored: per vocabulary chunk one fp16 buffer of
 * n_rows x chunk values lives in the workspace. Replaces the chunk loop of _FusedHeadLoss.forward
 * (solution/lm_head_loss.py:192-245: torch.mm + lm_head_vocab_chunk_kernel (108-160) + torch.mm
 * per vocabulary chunk, label fix-up 230-236).
 *   z[r,v] = fp16(sum_k hidden[r,k] * W[v,k])          (fp32 accumulation, rounded to fp16)
 *   lse_r = log sum_v e^{z[r,v]};  loss[r] = label ? lse_r - z[r,t_r] : 0;
 *   entropy[r] = lse_r - sum_v softmax(z)_v z_v;  correct[r] = label && first_argmax_v z == t_r
 *   grad (if not NULL) [n_rows, H] fp32 = grad_scale * sum_v (softmax_v - [v == t_r]) W[v,:]
 *     (zero rows for unlabelled targets)
 * hidden fp16 [n_rows, H] (row stride ld_h), W fp16 [V, H] (row stride ld_w), target int64.
 * Both contractions read W as stored (the gradient pass through transposing LDS reads), so no
 * transposed copy of the weight exists. H, ld_h, ld_w must be multiples of 8 and the bases
 * 16-byte aligned.
 * The vocabulary is walked in chunks of chunk_cols columns (rounded up to a multiple of 256, at
 * most 262144; 0 = the library's default, which keeps the chunk buffer at 128 MiB or less); the
 * result does not depend on the chunk size beyond fp32 rounding.
 * workspace: device memory of cm_lmhead_ce_workspace_bytes(n_rows, V, H, chunk_cols) bytes,
 * 256-B aligned.
 */
int cm_lmhead_ce(const void* hidden, int64_t ld_h, const void* weight, int64_t ld_w,
                 const int64_t* target, int64_t n_rows, int64_t vocab, int hidden_size,
                 int64_t chunk_cols, float* loss, float* entropy, int32_t* correct, float* grad,
                 float grad_scale, void* workspace, int64_t workspace_bytes, void* stream);
/* Workspace bytes cm_lmhead_ce needs for these sizes (chunk_cols as passed to cm_lmhead_ce). */
int64_t cm_lmhead_ce_workspace_bytes(int64_t n_rows, int64_t vocab, int hidden_size,
                                     int64_t chunk_cols);
/* The plan cm_lmhead_ce runs with a gradient at these sizes: *chunk = the vocabulary chunk's
 * columns (the last chunk takes the rest), *n_split = the gradient contraction's K-slices.
 * A query only (no launch, no device access); no counterpart in the reference, whose chunk is
 * its own rule (lm_head_loss.py:209-211). */
int cm_lmhead_ce_plan(int64_t n_rows, int64_t vocab, int hidden_size, int64_t chunk_cols,
                      int64_t* chunk, int* n_split);

/* cm_lmhead_ce without a workspace argument: it allocates nothing (no hipMalloc / hipFree or
 * allocating library call, on any call). No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation). The arguments and results are cm_lmhead_ce's.
 *
 * Its scratch is a file-scope device array of CM_LMHEAD_NOALLOC_SCRATCH_BYTES, one per GPU,
 * held by that GPU until the process ends; its device address is looked up once per device on
 * the first call with that device current, so call it with the stream's device current. The
 * gradient pass splits its contraction into K-slices (one fp32 [n_rows, H] accumulator each);
 * the scratch holds the vocabulary chunk's buffers and the slices' accumulators, and the entry
 * point picks the (slices, chunk) pair it estimates fastest among those that fit: chunk_cols
 * when given, with the most slices (up to cm_lmhead_ce's count) that fit beside it; else, over
 * the slice counts, the chunks (multiples of 256 columns) from the largest that fits down to
 * half of it. Where it runs cm_lmhead_ce's slice count and chunk, the results are bit-identical to
 * cm_lmhead_ce's; with fewer slices only the fp32 summation order of the gradient differs
 * (within the same tolerances). Sizes whose smallest layout (or the given chunk's) does not fit
 * return CM_ERROR_SCRATCH_TOO_SMALL before anything is launched. Every call on one GPU uses that GPU's
 * one array: calls that overlap on one GPU (other streams, other threads) race; nothing in the
 * array needs to start at any value, so stream-ordered calls need nothing between them.
 */
#define CM_LMHEAD_NOALLOC_SCRATCH_BYTES (64LL << 20)
#define CM_ERROR_SCRATCH_TOO_SMALL 20001
int cm_lmhead_ce_noalloc(const void* hidden, int64_t ld_h, const void* weight, int64_t ld_w,
                         const int64_t* target, int64_t n_rows, int64_t vocab,
                         int hidden_size, int64_t chunk_cols, float* loss,
                         float* entropy, int32_t* correct, float* grad, float grad_scale,
                         void* stream);
/* The plan cm_lmhead_ce_noalloc runs at these sizes (want_grad: a gradient is asked for): the
 * chunk's columns and the K-slices, as cm_lmhead_ce_plan; CM_ERROR_SCRATCH_TOO_SMALL when
 * nothing fits. A query only. */
int cm_lmhead_ce_noalloc_plan(int64_t n_rows, int64_t vocab, int hidden_size, int64_t chunk_cols,
                              int want_grad, int64_t* chunk, int* n_split);

/* ------------------------------------------------------------------------------------------ */
/* Causal grouped-query attention over a packed batch of variable-length rows, forward. Replaces,
 * for the packed batch of the fused training forward (solution/lm_head_loss.py:300-363, whose
 * mask 332-336 is block-diagonal over the rows and causal inside each), the attention the
 * reference computes with that dense mask through grouped SDPA (solution/attention.py:332-373,
 * installed last by apply(), solution/__init__.py:25-34). No mask is read: query t of a row
 * attends keys 0..t of the same row.
 *   out[t, h, :] = sum_j softmax_j(scale * q[h,t] . k[h/(H/G), j]) v[h/(H/G), j]
 * q [H][N][D] with element strides (sq_h, sq_t, 1); k, v [G][N][D] likewise; f32 or f16 inputs
 * are rounded to fp16 (as fp16 autocast rounds them); fp16 MFMA products, fp32 accumulation and
 * softmax. out fp16 [N][H][D] contiguous. lse2 f32 [H][n_pad] receives the log2-domain
 * log-sum-exp of scale * q.k of every padded position (the backward's input).
 * rows_image: DEVICE memory (16-byte aligned) holding cm_attn_rows_bytes() bytes that
 * cm_attn_rows_image wrote for the batch's row bounds (its token count must be n_tokens = N),
 * copied there by the caller. n_pad: the padded positions the launch is sized for, a multiple of
 * 64 (at most 64 x 65535) at least the image's padded count (cm_attn_padded_tokens of its bounds):
 * blocks past the image's own count do nothing, so one launch (or one captured graph) sized for a
 * capacity serves every row structure of N tokens that fits it, the image being rewritten in
 * between. Kernels
 * check the image against n_tokens and n_pad, and write nothing for rows inconsistent with them.
 * head_dim must be 128, H a multiple of G. Bases 16-byte aligned (out 8), strides multiples of 8
 * (f16) or 4 (f32) elements, workspace 256-byte aligned, cm_attn_workspace_bytes(n_pad, H, G,
 * head_dim, 0) bytes.
 */
int cm_attn_fwd(const void* q, int q_dtype, int64_t sq_h, int64_t sq_t, const void* k,
                int k_dtype, int64_t sk_h, int64_t sk_t, const void* v, int v_dtype,
                int64_t sv_h, int64_t sv_t, const void* rows_image, int64_t n_tokens,
                int64_t n_pad, int H, int G, int head_dim, float scale, void* out, float* lse2,
                void* workspace, int64_t workspace_bytes, void* stream);

/* Backward of cm_attn_fwd (the same q, k, v, rows image, n_tokens, n_pad and scale; out and lse2
 * as it wrote them;
 * dout fp16 [N][H][D] contiguous). Writes dq [H][N][D] (dq_dtype), dk and dv [G][N][D]
 * (dkv_dtype), contiguous; f32 or f16; with grads_token_major != 0 they are [N][H][D] and
 * [N][G][D] instead (the layout of the projections the gradients flow back into). dk and dv
 * sum the contributions of the H/G query heads of
 * each group in a fixed order (no atomics: the same bits on every run). Workspace:
 * cm_attn_workspace_bytes(n_pad, H, G, head_dim, 1) bytes, 256-byte aligned.
 */
int cm_attn_bwd(const void* q, int q_dtype, int64_t sq_h, int64_t sq_t, const void* k,
                int k_dtype, int64_t sk_h, int64_t sk_t, const void* v, int v_dtype,
                int64_t sv_h, int64_t sv_t, const void* out, const void* dout, const float* lse2,
                const void* rows_image, int64_t n_tokens, int64_t n_pad, int H, int G,
                int head_dim, float scale, void* dq, int dq_dtype, void* dk, void* dv,
                int dkv_dtype, int grads_token_major, void* workspace, int64_t workspace_bytes,
                void* stream);

/* Padded token count of a packed batch: sum over rows of round_up(length, 64); -1 for invalid
 * bounds (not monotone, bounds[0] != 0, n_rows outside 1..128). */
int64_t cm_attn_padded_tokens(const int64_t* bounds, int n_rows);

/* The row bounds as the attention kernels read them: bounds (HOST array of n_rows + 1 row ends,
 * 0 = bounds[0] <= ... <= bounds[n_rows] = N, n_rows <= 128) written as an image of
 * cm_attn_rows_bytes() bytes to the HOST buffer `image`, for the caller to copy to device memory.
 * Returns the padded token count (cm_attn_padded_tokens), or -1 for invalid bounds. No counterpart
 * in the reference, whose mask carries the rows (lm_head_loss.py:332-336). */
int64_t cm_attn_rows_bytes(void);
int64_t cm_attn_rows_image(const int64_t* bounds, int n_rows, void* image);

/* Workspace bytes of cm_attn_fwd / cm_attn_fwd_rope (backward = 0) or cm_attn_bwd /
 * cm_attn_bwd_rope (backward = 1); -1 if the sizes are unsupported. */
int64_t cm_attn_workspace_bytes(int64_t n_pad, int H, int G, int head_dim, int backward);

/* cm_attn_fwd / cm_attn_bwd with the rotary embedding fused in: q and k are the projections
 * before the rotation (transformers' apply_rotary_pos_emb, which solution/rope.py:60-82 replaces,
 * is then not called), rotated on their way into the kernels' fp16 copies of q and k, and the
 * backward returns the gradients of the unrotated q and k (the transposed rotation applied to the
 * gradients of the rotated ones in the launch that sums dK and dV). With h = D / 2 and c, s the
 * token's cos / sin rows:
 *   rotate:     o[d] = x[d] c[d] - x[d+h] s[d],   o[d+h] = x[d+h] c[d+h] + x[d] s[d+h]
 *   transposed: o[d] = g[d] c[d] + g[d+h] s[d+h], o[d+h] = g[d+h] c[d+h] - g[d] s[d]
 * in fp32 with each product rounded before the sum (the bits of cm_rope followed by the unfused
 * entry). cos, sin: fp32 [N][head_dim] of the packed tokens, row stride cs_t (a multiple of 4,
 * at least head_dim), 16-byte aligned. The backward writes dK and dV in their own dtypes
 * (dk_dtype, dv_dtype). No counterpart in the reference, which launches its RoPE kernel apart. */
int cm_attn_fwd_rope(const void* q, int q_dtype, int64_t sq_h, int64_t sq_t, const void* k,
                     int k_dtype, int64_t sk_h, int64_t sk_t, const void* v, int v_dtype,
                     int64_t sv_h, int64_t sv_t, const float* cos, const float* sin, int64_t cs_t,
                     const void* rows_image, int64_t n_tokens, int64_t n_pad, int H, int G,
                     int head_dim, float scale, void* out, float* lse2, void* workspace,
                     int64_t workspace_bytes, void* stream);
int cm_attn_bwd_rope(const void* q, int q_dtype, int64_t sq_h, int64_t sq_t, const void* k,
                     int k_dtype, int64_t sk_h, int64_t sk_t, const void* v, int v_dtype,
                     int64_t sv_h, int64_t sv_t, const float* cos, const float* sin, int64_t cs_t,
                     const void* out, const void* dout, const float* lse2,
                     const void* rows_image, int64_t n_tokens, int64_t n_pad, int H, int G,
                     int head_dim, float scale, void* dq, int dq_dtype, void* dk, int dk_dtype,
                     void* dv, int dv_dtype, int grads_token_major, void* workspace,
                     int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------------ */
/* A rank-16 LoRA adapter on a frozen base projection, fused per token row: forward. Replaces,
 * for one adapter of the training step, LoRABranch.forward (solution/lora.py:78-94: the pack
 * kernel 30-42, the fp16 casts of the adapter weights, lora_B(lora_A(xd)) as two GEMMs, the
 * scaling) and the widening add onto the base output done by its caller (the patched peft
 * forward, lora.py:136-186). Row t of T, K inputs, N outputs, R = rank = 16:
 *   xd = fp16(keep ? x * scale_p : 0)    (bits: the mask LSB-first, T*K/8 bytes)
 *   a16[t][r] = fp16(sum_k xd[k] * fp16(weight_a[r][k]))
 *   out[t][n] = fp32(base16[t][n]) + fp32(fp16(fp16(sum_r a16[t][r] * fp16(weight_b[n][r]))
 *                                          * scaling))
 * x fp32 [T, K], keep bool/uint8 [T, K] (8-byte aligned), weight_a fp32 [R, K], weight_b fp32
 * [N, R], base16 fp16 [T, N] (the base projection's output), out fp32 [T, N], a16 fp16 [T, R].
 * K and N multiples of 8 and <= 2048; x, weight_a, weight_b, out 16-byte aligned, base16 and
 * a16 8-byte aligned. The rank-16 products run on the matrix cores (fp16 operands, fp32
 * accumulation, like the GEMMs they replace; the order of the sums differs from theirs).
 */
int cm_lora_fused_fwd(const float* x, const uint8_t* keep, const float* weight_a,
                      const float* weight_b, const void* base16, float* out, uint8_t* bits,
                      void* a16, int64_t T, int K, int N, int rank, float scale_p,
                      float scaling, void* stream);

/* Backward, part 1 (LoRABranch.backward, solution/lora.py:96-107, up to lora_A's output):
 *   gbase16 = fp16(grad)                    (the gradient of the base projection's output)
 *   g16 = fp16(gbase16 * scaling)           (the gradient of lora_B's output)
 *   ga16[t][r] = fp16(sum_n g16[t][n] * fp16(weight_b[n][r]))
 * grad fp32 [T, N]; outputs fp16 [T, N], [T, N], [T, R]. N a multiple of 8 and <= 2048; grad
 * 16-byte aligned, gbase16 and g16 8-byte aligned.
 */
int cm_lora_fused_bwd1(const float* grad, const float* weight_b, void* gbase16, void* g16,
                       void* ga16, int64_t T, int N, int rank, float scaling, void* stream);

/* The two calls above for up to 4 adapters on the same input x (and of one rank, dropout
 * scale and scaling) in one launch each: adapter i's operands are element i of the arrays, its
 * output width N[i]. The same values as one call per adapter; the adapters' row tiles run side
 * by side. Replaces the per-adapter launches of solution/lora.py:78-186 for the q and v adapters
 * of an attention block (LoRABranch there runs once per adapter layer).
 */
int cm_lora_fused_fwd_multi(const float* x, int64_t T, int K, int rank, float scale_p,
                            float scaling, int n_jobs, const uint8_t* const* keep,
                            const float* const* weight_a, const float* const* weight_b,
                            const void* const* base16, float* const* out, uint8_t* const* bits,
                            void* const* a16, const int* N, void* stream);
int cm_lora_fused_bwd1_multi(int64_t T, int rank, float scaling, int n_jobs,
                             const float* const* grad, const float* const* weight_b,
                             void* const* gbase16, void* const* g16, void* const* ga16,
                             const int* N, void* stream);

/* Backward, part 2, after the caller's base input gradient dxb16 = gbase16 @ W (fp16 [T, K]):
 *   gxd = fp16(sum_r ga16[t][r] * fp16(weight_a[r][k]))
 *   dx[t][k] = fp32(dxb16[t][k]) + (keep ? gxd * scale_p : 0)     (dx may be NULL: then
 *                                                                   dxb16 is not read)
 *   with dxb16 NULL and dx given: dx[t][k] += (keep ? gxd * scale_p : 0)   (a second adapter on
 *                                                                   the same input)
 *   xd16[t][k] = fp16(keep ? x16[t][k] * scale_p : 0)   (lora_A's input rebuilt, the unpack
 *                                                         kernel solution/lora.py:45-57)
 * keep = the bits of the forward. K a multiple of 8 and <= 2048; ga16, weight_a and dx 16-byte
 * aligned, dxb16, x16 and xd16 8-byte aligned. The 16 rank products are summed in rank order.
 */
int cm_lora_fused_bwd2(const void* dxb16, const void* ga16, const float* weight_a,
                       const void* x16, const uint8_t* bits, float* dx, void* xd16, int64_t T,
                       int K, int rank, float scale_p, void* stream);

/* ------------------------------------------------------------------------------------------ */
/* NF4 weights expanded inside an fp16 matrix-core GEMM (the fp16 weight is never written to
 * memory). Replaces, per frozen 4-bit linear of the training step, the pair "dequantize_nf4
 * (solution/nf4.py:64-82, kernel 26-46) -> fp16 GEMM" that the reference's patched bitsandbytes
 * matmul runs (solution/nf4.py:102-130: forward F.linear(x, W) and the input gradient
 * grad @ W) and the MLP recompute's two 4-bit matmuls (solution/swiglu_recompute.py:165-166,
 * 198-199).
 *
 * One weight: bitsandbytes' NF4 storage of W [rows, cols] (row-major, element j = flat index),
 * the same fields cm_nf4_dequant takes. Every element is expanded exactly as cm_nf4_dequant
 * expands it to fp16. Requirements: packed 16-byte aligned; rows and cols multiples of 64;
 * blocksize a power of two >= 32; every weight of one call has the same cols and nested flag.
 */
typedef struct cm_nf4_weight {
  const uint8_t* packed;   /* [rows * cols / 2] */
  const void* absmax;      /* uint8 [blocks] (nested) or fp32 [blocks] */
  int nested;
  const float* code;       /* [16] */
  const float* code2;      /* [256] (nested) */
  const float* absmax2;    /* (nested) */
  const float* offset;     /* [1] (nested) */
  int blocksize;
  int blocksize2;
  int64_t rows;            /* out_features */
  int64_t cols;            /* in_features */
  const float* scale_map;  /* NULL, or the weight's fp32 block scales from cm_nf4_scale_map */
} cm_nf4_weight;

/* The block scales of one NF4 weight decoded to fp32 (nested: code2[absmax_u8[b]] *
 * absmax2[b / blocksize2] + offset, multiply then add; else absmax_f32[b]), stored transposed:
 * smap[c * rows + r] = the scale of the block holding element (r, c * blocksize), for
 * c < cols / blocksize. cols must be a multiple of blocksize; smap holds rows * cols / blocksize
 * floats, 16-byte aligned. A frozen weight's map is computed once; with it in cm_nf4_weight the
 * fused GEMMs read one scale per block instead of decoding the nested absmax in their loops.
 * No counterpart in the reference (its dequant kernel decodes the nested absmax per call,
 * solution/nf4.py:35-38). */
int cm_nf4_scale_map(const cm_nf4_weight* w, float* smap, void* stream);

/* Forward, for n_w (1..3) weights sharing the input:
 *   out_i[t][n] = round(sum_k x[t][k] * fp16(W_i[n][k]) + bias_i[n])     (fp32 sums)
 * x fp16 [m, cols] with row stride ldx (a multiple of 8, 16-byte aligned); bias NULL or an
 * array of n_w fp16 pointers (entries may be NULL); out_i [m, rows_i] with row stride ldo[i] (a
 * multiple of 4). out_dtype CM_F16 (round = to fp16) or CM_F32 (round = to fp16, then widened:
 * the fp16 linear followed by .to(float32)).
 * workspace: device memory of cm_nf4_linear_workspace_bytes(m, w, n_w, 0) bytes (16-byte
 * aligned) for the fp32 partial sums of a split contraction; NULL (or fewer bytes) runs the
 * contraction unsplit: the same results, on fewer workgroups.
 */
int cm_nf4_linear_fwd(const void* x, int64_t ldx, int64_t m, const cm_nf4_weight* w, int n_w,
                      const void* const* bias, void* const* out, const int64_t* ldo,
                      int out_dtype, void* workspace, int64_t workspace_bytes, void* stream);

/* Input gradient, summed over n_w (1..3) weights:
 *   dx[t][k] = round(sum_i sum_n g_i[t][n] * fp16(W_i[n][k]))             (fp32 sums)
 * g_i fp16 [m, rows_i] with row stride ldg[i] (a multiple of 8, 16-byte aligned); dx [m, cols]
 * with row stride lddx (a multiple of 4), dx_dtype CM_F16 or CM_F32 (rounded to fp16, then
 * widened). With two weights this is the MLP's dgate Wg + dup Wu rounded once. workspace as for
 * cm_nf4_linear_fwd (backward = 1).
 */
int cm_nf4_linear_bwd(const void* const* g, const int64_t* ldg, int64_t m,
                      const cm_nf4_weight* w, int n_w, void* dx, int64_t lddx, int dx_dtype,
                      void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes of cm_nf4_linear_fwd (backward = 0) or cm_nf4_linear_bwd (backward = 1) for
 * these sizes (0: the call does not split its contraction), -1 for invalid weights. */
int64_t cm_nf4_linear_workspace_bytes(int64_t m, const cm_nf4_weight* w, int n_w, int backward);

/* Several NF4 weights expanded by one launch: out[i] receives weight w[i] as cm_nf4_dequant
 * writes it (the same values, element for element), [rows, cols] in out_dtype (fp32, fp16 or
 * bf16). Replaces the reference's per-weight nf4_dequant_kernel launches
 * (solution/nf4.py:26-46, launched per weight by dequantize_nf4, nf4.py:64-82) where a decoder
 * layer expands its o, gate, up and down weights together. At most 8 weights; one launch when
 * every weight takes the vector path (4-byte aligned packed bytes in whole 4-byte units,
 * 16-byte aligned outputs) and all share one nestedness, else one cm_nf4_dequant per weight.
 * The fused GEMMs' scale_map is not read.
 */
int cm_nf4_dequant_group(const cm_nf4_weight* w, int n_w, void* const* out, int out_dtype,
                         void* stream);

/* ---- On-box peak probes (measurement only; no counterpart in the reference) ----------------
 * The roofline denominators as this board attains them, which bench.py reports beside the
 * published 8 TB/s and 2.5 PFLOP/s. Neither is part of the training step. */

/* Streams `bytes` (a multiple of 16, 16-byte aligned) from src: read only when dst is NULL
 * (sink: 4 bytes of device memory the kernel may write), else copied to dst (nontemporal
 * stores). One pass of 256-lane workgroups, each over per_lane (1, 4 or 16) x 4 KiB, with 16-byte
 * loads, nontemporal when nt_loads is non-zero. */
int cm_probe_hbm(const void* src, void* dst, int64_t bytes, int per_lane, int nt_loads,
                 uint32_t* sink, void* stream);

/* fp16 matrix-core rate: 2048 workgroups of 4 wavefronts, each issuing iters x 2 x chains
 * v_mfma_f32_32x32x16_f16 on `chains` (2, 4 or 8) independent accumulators, operands taken from
 * `operands` (512 x 8 fp16 = 8 KiB, 16-byte aligned; use non-zero data). sink: 4 bytes of
 * device memory. */
int cm_probe_mfma_f16(const void* operands, int iters, int chains, float* sink, void* stream);
/* Matrix-core FLOPs of one cm_probe_mfma_f16 call (0 for invalid arguments). */
int64_t cm_probe_mfma_f16_flops(int iters, int chains);

/* Launch floor: `blocks` workgroups of `threads` (a multiple of 64, at most 1024) threads that
 * do nothing; a kernel trace gives the device time a launch of that grid costs. */
int cm_probe_launch(int blocks, int threads, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CLAUDEMAXING_AMD_H */
