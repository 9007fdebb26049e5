/*
 * ferrite_hip.h — C ABI of the MI355X (gfx950) kernels behind ferrite.kernels.
 *
 * Every entry point takes device pointers, sizes and attributes as plain C types,
 * enqueues its kernels on `stream` (a hipStream_t passed as void*, NULL = the
 * default stream), never synchronises, never allocates, and returns 0 on
 * success. A non-zero return is one of the FERRITE_ERR_* codes; the message
 * for the calling thread's last failure is ferrite_hip_last_error(). Work runs
 * on the stream's device: per-device state (the CU count that shapes a grid, a
 * kernel's LDS limit, the no-alloc scratch array) is looked up for that device,
 * whichever device is current on the calling thread, and set up once per
 * device. Entry points are reentrant and may be called from several threads.
 *
 * All tensors are dense and row-major (last dimension contiguous). Outputs are
 * preallocated by the caller, exactly as XLA preallocates the out_shape buffers
 * of the reference's pallas_call custom calls. Inputs are read-only.
 *
 * Each function replaces one Pallas kernel of the reference (paths relative to
 * the reference repository, src/ferrite/kernels/):
 *
 *   ferrite_hip_attn_fwd      flash_attention.py:91-175  (_fwd_kernel + _flash_forward,
 *                                                          custom call "ferrite_flash_attention_fwd")
 *   ferrite_hip_attn_bwd_delta flash_attention.py:328-329 (delta = rowsum(f32 dO * f32 O),
 *                                                          an XLA fusion in the reference)
 *   ferrite_hip_attn_bwd_dkv  flash_attention.py:197-221, :253-279 ("ferrite_flash_attention_bwd_dkv")
 *   ferrite_hip_attn_bwd_dq   flash_attention.py:224-243, :281-306 ("ferrite_flash_attention_bwd_dq")
 *   ferrite_hip_attn_bwd_dq_delta  the same dQ with delta (flash_attention.py:328-329)
 *                                  computed inside it and written out for dK/dV
 *   ferrite_hip_attn_fwd_ex, _bwd_dkv_ex, _bwd_dq_ex, _bwd_dq_delta_ex  the same with a
 *                                  workspace, in which long-context grids split their
 *                                  longest tiles between two workgroups
 *   ferrite_hip_attn_fwd_qkv / _bwd_qkv  the causal forward and backward read and
 *                                  written in the model's token-major layouts, with the
 *                                  head transposes of model/gpt.py:137-138 folded in
 *   ferrite_hip_add_rmsnorm   rmsnorm.py:52-56, :77-110  ("ferrite_add_rmsnorm")
 *   ferrite_hip_rmsnorm       rmsnorm.py:46-49, :77-110  ("ferrite_rmsnorm")
 *   ferrite_hip_rmsnorm_bwd   rmsnorm.py:159-166, :128-131, :148-153 (the custom_vjp backward of
 *                                                          _norm/_add_norm, XLA fusions in the reference)
 *   ferrite_hip_matmul        matmul.py:27-38, :52-86    ("ferrite_matmul")
 *   ferrite_hip_matmul_ex     matmul.py:99-104 (the VJP's products, transposed operands read in place)
 *   ferrite_hip_matmul_gelu   model/gpt.py:141 (the MLP's matmul and jax.nn.gelu, an XLA fusion
 *                                               after the matmul custom call in the reference)
 *   ferrite_hip_adamw         ../model/train.py:59-74    (adamw_update, XLA fusions in the reference)
 *   ferrite_hip_cross_entropy_fwd/_bwd ../model/gpt.py:147-152 (loss_fn and its autodiff, XLA in the reference)
 *   ferrite_hip_heads_split/_merge ../model/gpt.py:137-138 (the head transposes, XLA copies in the reference)
 *   ferrite_hip_decode_attention ../serving/engine.py:89-104 (_cache_attention + _write_cache, XLA in the
 *                                                          reference, whose README.md:283-285 names this kernel next)
 *
 * The one layout change against the reference: the softmax statistics
 * (logsumexp `lse` and `delta`) are compact f32 [B, H, S] arrays instead of the
 * reference's lane-replicated [B, H, S, 128] (flash_attention.py:156-160, :329).
 */
#ifndef FERRITE_HIP_H
#define FERRITE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types. */
#define FERRITE_F32 0
#define FERRITE_BF16 1

/* Epilogue modes of ferrite_hip_matmul_gelu. */
#define FERRITE_GELU 1      /* out = gelu(x @ y), aux <- x @ y */
#define FERRITE_GELU_GRAD 2 /* out = (x @ y) * gelu'(aux) */

/* Return codes. */
#define FERRITE_OK 0
#define FERRITE_ERR_INVALID_ARGUMENT 1 /* shape / dtype / attribute not supported */
#define FERRITE_ERR_LAUNCH 2           /* hipLaunchKernel or hipGetLastError failed */

/* Message describing the calling thread's most recent failure ("" if none). */
const char* ferrite_hip_last_error(void);

/* Library version string, e.g. "ferrite_hip 0.1.0 gfx950". */
const char* ferrite_hip_version(void);

/*
 * Fused residual-add + RMSNorm (rmsnorm.py:52-56):
 *   h = f32(x) + f32(residual);  store h rounded to x's dtype
 *   y = h * rsqrt(sum(h*h)/dim + eps) * f32(weight); store y in x's dtype
 * y uses the unrounded f32 h. x, residual, h, y: [rows, dim] of x_dtype;
 * weight: [dim] of w_dtype. rows >= 0, dim >= 1.
 */
int ferrite_hip_add_rmsnorm(const void* x, const void* residual, const void* weight, void* h, void* y,
                            int64_t rows, int64_t dim, int x_dtype, int w_dtype, float eps, void* stream);

/* Plain RMSNorm (rmsnorm.py:46-49): y = x * rsqrt(mean(x^2) + eps) * weight. */
int ferrite_hip_rmsnorm(const void* x, const void* weight, void* y, int64_t rows, int64_t dim, int x_dtype,
                        int w_dtype, float eps, void* stream);

/*
 * RMSNorm backward (rmsnorm.py:159-166), with the fused add's direct term
 * (rmsnorm.py:148-153):
 *   inv = rsqrt(mean(h^2) + eps);  xhat = h * inv;  dxhat = dy * weight
 *   dh  = inv * (dxhat - xhat * mean(dxhat * xhat)) + dh_direct
 *   dweight = sum over rows of dy * xhat
 * h, dy, dh_direct: [rows, dim] of x_dtype (dh_direct may be NULL: no direct
 * term); weight, dweight: [dim] of w_dtype; dh: [rows, dim] of dh_dtype (x_dtype,
 * or FERRITE_F32). Statistics and sums are f32; dweight is summed in a fixed
 * order (deterministic). `workspace` is device memory of
 * ferrite_hip_rmsnorm_bwd_workspace(rows, dim) bytes owned by the caller.
 */
int64_t ferrite_hip_rmsnorm_bwd_workspace(int64_t rows, int64_t dim);
int ferrite_hip_rmsnorm_bwd(const void* h, const void* weight, const void* dy, const void* dh_direct, void* dh,
                            void* dweight, void* workspace, int64_t rows, int64_t dim, int x_dtype, int w_dtype,
                            int dh_dtype, float eps, void* stream);

/*
 * ferrite_hip_rmsnorm_bwd without a workspace argument, for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving/training
 * loops, harnesses that forbid hipMalloc. No counterpart in the reference (XLA
 * owns its scratch there). Same arguments minus `workspace`, same kernels and
 * bitwise the same results. Its scratch (the partial dweight rows) is a fixed
 * FERRITE_RMSNORM_BWD_SCRATCH_BYTES device array inside the library, one per
 * GPU, held until the process ends; the call itself allocates nothing. A shape
 * needing more scratch fails with FERRITE_ERR_INVALID_ARGUMENT (the fast path
 * needs min(512, ceil(rows / 16)) * dim * 4 bytes, so any rows with dim <= 4096;
 * unaligned or other dims also need 4 * rows more). Every call on one GPU uses
 * that GPU's one array: calls that overlap in time on the same GPU (two streams,
 * two threads) race and give wrong dweight. Nothing in the array needs to
 * start at zero.
 */
#define FERRITE_RMSNORM_BWD_SCRATCH_BYTES (8u << 20)
int ferrite_hip_rmsnorm_bwd_noalloc(const void* h, const void* weight, const void* dy, const void* dh_direct,
                                    void* dh, void* dweight, int64_t rows, int64_t dim, int x_dtype, int w_dtype,
                                    int dh_dtype, float eps, void* stream);

/*
 * a_out <- a and b_out <- b, `bytes` each, with 16-byte non-temporal loads and
 * stores: add+RMSNorm's access pattern (two streams in, two out) without its
 * arithmetic. No counterpart in the reference; it measures the HBM ceiling for
 * HBM-bound kernels of that shape (bench.py reports it beside add+RMSNorm).
 * bytes % 16 == 0; all pointers 16-byte aligned; the buffers must not overlap.
 */
int ferrite_hip_stream_copy2(const void* a, const void* b, void* a_out, void* b_out, int64_t bytes, void* stream);

/*
 * The two one-direction halves of that ceiling, with no counterpart in the
 * reference either. ferrite_hip_stream_read loads every byte of `a` once
 * (16-byte non-temporal loads) and folds the words with XOR, leaving one 32-bit
 * word per workgroup in sink[0 .. blocks); ferrite_hip_stream_fill stores
 * `value` in every 32-bit word of `out` (16-byte non-temporal stores).
 * `blocks` is the number of 256-thread workgroups of the persistent grid
 * (0: 512, two per CU; at most 65536); sink holds at least that many words
 * (512 when blocks is 0). bytes % 16 == 0; a and out 16-byte aligned, sink
 * 4-byte aligned.
 */
int ferrite_hip_stream_read(const void* a, int64_t bytes, void* sink, int blocks, void* stream);
int ferrite_hip_stream_fill(void* out, int64_t bytes, uint32_t value, int blocks, void* stream);

/*
 * The matrix-pipe counterpart of those ceilings, with no counterpart in the
 * reference: `blocks` workgroups of `waves` (4 or 8: one or two per SIMD) each
 * issue `iters` x 8 v_mfma_f32_32x32x16_bf16 (32768 FLOPs each) over eight
 * independent accumulators of register operands, with no memory traffic.
 * bench.py times it as the bf16 MFMA rate this part sustains. Each wave writes
 * one float to sink[blocks * waves]. 1 <= blocks <= 65536, 1 <= iters <= 2^24.
 */
int ferrite_hip_mfma_ceiling(float* sink, int blocks, int waves, int iters, void* stream);

/*
 * out[M, N] = x[M, K] @ y[K, N] with f32 accumulation (matmul.py:27-38, :52-86).
 * in_dtype FERRITE_BF16 uses bf16 MFMA; FERRITE_F32 uses fp32 MFMA (true fp32
 * products, the reference's Precision.HIGHEST, _compat.py:17-25). Ragged shapes
 * need no padding from the caller: out-of-range elements read as zero, which is
 * what the reference's zero padding contributes. out_dtype may differ from
 * in_dtype. M, N, K >= 1.
 */
int ferrite_hip_matmul(const void* x, const void* y, void* out, int64_t m, int64_t n, int64_t k, int in_dtype,
                       int out_dtype, void* stream);

/*
 * The matmul with operands that may be given transposed, and an optional
 * K split (matmul.py:99-104, the VJP's products: dx = g @ y^T and dy = x^T @ g
 * without materialised transposes). out[M, N] = op(x) @ op(y):
 *   x_t == 0: x is [M, K];  x_t != 0: x holds x^T, stored [K, M]
 *   y_t == 0: y is [K, N];  y_t != 0: y holds y^T, stored [N, K]
 * Transposed operands need bf16, K % 64 == 0, N % 8 == 0 (M % 8 == 0 when x_t)
 * and 16-byte aligned pointers; otherwise the call fails with
 * FERRITE_ERR_INVALID_ARGUMENT. With a workspace of at least
 * ferrite_hip_matmul_workspace(m, n, k, in_dtype) bytes (0 = the shape does not
 * split), a problem with few output tiles (bf16; f32 with very few, after its split
 * inside each workgroup) splits K across workgroups and sums the f32 partials in a
 * fixed order (deterministic); with NULL it does not split across workgroups.
 */
int64_t ferrite_hip_matmul_workspace(int64_t m, int64_t n, int64_t k, int in_dtype);
int ferrite_hip_matmul_ex(const void* x, const void* y, void* out, int64_t m, int64_t n, int64_t k, int x_t, int y_t,
                          int in_dtype, int out_dtype, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * The MLP's up-projection and its GELU in one pass (model/gpt.py:141:
 * jax.nn.gelu(x @ w1, approximate=True), the tanh form), and the matching
 * gradient pass. bf16 operands and outputs; x_t / y_t, the workspace and the K
 * split as in ferrite_hip_matmul_ex. aux and out are distinct [M, N] bf16 buffers.
 *   mode FERRITE_GELU:      aux <- bf16(op(x) @ op(y))  (the pre-activation u)
 *                           out <- bf16(gelu(aux))
 *   mode FERRITE_GELU_GRAD: aux holds u;
 *                           out <- bf16(bf16(op(x) @ op(y)) * gelu'(u))
 * gelu and gelu' are taken in f32 from the bf16-rounded values, as an elementwise
 * pass after the product computes them. Shapes the DMA-fed kernel takes apply
 * them in its store (or in the K split's reduction); others run the product and
 * then an elementwise pass.
 */
int ferrite_hip_matmul_gelu(const void* x, const void* y, void* out, void* aux, int64_t m, int64_t n, int64_t k,
                            int x_t, int y_t, int mode, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Decode attention over a static KV cache (../serving/engine.py:89-104).
 * q, k_new, v_new: [B, H, D]; k_cache, v_cache: [B, H, max_len, D], all of
 * `dtype`; pos: device int32 [B]. Writes k_new/v_new into the caches at row
 * pos[b], then out[b, h] = softmax_j(scale * q . k_j) . v_j over j = 0..pos[b]
 * (f32 statistics). A pos outside [0, max_len) writes nothing and gives NaN.
 * D in {64, 128, 256}; all pointers 16-byte aligned. Where the keys are split
 * over workgroups (chunks of a power of two from 256 keys up, as few as keep
 * the grid within 512 workgroups), `workspace` (device memory of
 * ferrite_hip_decode_attention_workspace(b, h, max_len, d) bytes; 0 when a
 * head's keys fit one chunk) holds the f32 partials.
 */
int64_t ferrite_hip_decode_attention_workspace(int64_t b, int64_t h, int64_t max_len, int64_t d);
int ferrite_hip_decode_attention(const void* q, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                                 const int32_t* pos, void* out, int64_t b, int64_t h, int64_t max_len, int64_t d,
                                 int dtype, float scale, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Head layout changes. heads_split: tokens [B, S, groups, H, D] -> groups
 * tensors heads[g] of [B, H, S, D]; heads_merge is the inverse. `heads` is a
 * host array of `groups` (1..4) device pointers; all tensors dense, of `dtype`.
 */
int ferrite_hip_heads_split(const void* tokens, void* const* heads, int64_t b, int64_t s, int64_t groups, int64_t h,
                            int64_t d, int dtype, void* stream);
int ferrite_hip_heads_merge(void* const* heads, void* tokens, int64_t b, int64_t s, int64_t groups, int64_t h,
                            int64_t d, int dtype, void* stream);

/*
 * Softmax cross-entropy of f32 logits [n, v] against int64 targets [n]
 * (../model/gpt.py:147-152): lse[i] = logsumexp_j logits[i, j] and
 * loss[i] = lse[i] - logits[i, targets[i]] (NaN for a target outside [0, v)),
 * both f32 [n]. The mean over rows is the caller's.
 */
int ferrite_hip_cross_entropy_fwd(const float* logits, const int64_t* targets, float* loss, float* lse, int64_t n,
                                  int64_t v, void* stream);

/*
 * Gradient of scale * sum_i loss[i] w.r.t. the logits, times the device scalar
 * *dloss: grad[i, j] = (exp(logits[i, j] - lse[i]) - [j == targets[i]]) * (*dloss) * scale,
 * written as grad_dtype [n, v]. lse from ferrite_hip_cross_entropy_fwd.
 */
int ferrite_hip_cross_entropy_bwd(const float* logits, const int64_t* targets, const float* lse, const float* dloss,
                                  float scale, void* grad, int64_t n, int64_t v, int grad_dtype, void* stream);

/*
 * One AdamW step over n_tensors parameter tensors (../model/train.py:59-74):
 *   gnorm = sqrt(sum over all tensors of sum(g^2))   (f32, fixed summation order)
 *   g *= min(1, max_grad_norm / (gnorm + 1e-6))
 *   m = beta1*m + (1-beta1)*g;  v = beta2*v + (1-beta2)*g*g
 *   p -= lr * ((m/bc1) / (sqrt(v/bc2) + eps) + (decay[i] ? weight_decay : 0) * p)
 * with bc = 1 - beta^step. If step_scalars (device f32[3]) is not NULL, lr, bc1
 * and bc2 are read from it at run time instead ({lr, 1 - beta1^step,
 * 1 - beta2^step}; `lr` and `step` are then ignored), so a captured graph can
 * replay the call with each step's values. params[i] (param_dtype) and exp_avg[i], exp_avg_sq[i]
 * (f32) are updated in place; grads[i] (grad_dtype) are read. The pointer, numel
 * and decay arrays are host memory; the tensors are device memory. grad_norm
 * (device f32 scalar, may be NULL) receives the pre-clip gnorm. `workspace` is
 * device memory of ferrite_hip_adamw_workspace(n_tensors) bytes. No host
 * synchronisation: the clip scale stays on the device.
 */
int64_t ferrite_hip_adamw_workspace(int64_t n_tensors);
int ferrite_hip_adamw(int64_t n_tensors, void* const* params, const void* const* grads, float* const* exp_avg,
                      float* const* exp_avg_sq, const int64_t* numel, const int32_t* decay, int param_dtype,
                      int grad_dtype, float lr, float beta1, float beta2, float eps, float weight_decay,
                      float max_grad_norm, int64_t step, const float* step_scalars, float* grad_norm,
                      void* workspace, void* stream);

/*
 * Flash attention forward (flash_attention.py:91-175).
 * q: [B, H, Sq, D]; k, v: [B, H, Sk, D]; o: [B, H, Sq, D], all of `dtype`.
 * lse: f32 [B, H, Sq] = logsumexp_j(scale * q_i . k_j) over the visible keys.
 * causal != 0 masks key j > query i and requires Sq == Sk. Supported head dims
 * (those the reference's _validate accepts, flash_attention.py:341-343): any
 * D <= 128 (zero-padded inside the kernel to 64 or 128) and any multiple of 128
 * (D > 256, and f32 or unaligned operands at D = 256, run slab-wise: 128 output
 * columns per workgroup, the scores recomputed per slab). The same holds for
 * the backward entry points below on
 * [B, H, S, D] tensors; the packed-QKV entry points (ferrite_hip_attn_fwd_qkv,
 * ferrite_hip_attn_bwd_qkv) are the exception and take head_dim 64 or 128 only.
 * Sq, Sk >= 1; Sq and Sk need not be multiples of any tile size.
 */
int ferrite_hip_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int64_t b, int64_t h,
                         int64_t sq, int64_t sk, int64_t d, int dtype, int causal, float scale, void* stream);

/*
 * ferrite_hip_attn_fwd with a workspace (the same kernels and arguments, plus
 * `workspace` of `workspace_bytes` device bytes, 256-byte aligned). Where
 * ferrite_hip_attn_fwd_workspace returns a size above 0 and the workspace holds
 * it (bf16 causal self-attention with head dim <= 64, S a multiple of 128 with
 * an even number of 128-row tiles, B H S / 128 <= 2 x CUs: the long-context
 * shapes whose grid is resident all at once, such as 1 x 8 x 8192 x 64), the
 * longest query tiles' key sweeps are split between the two workgroups of a
 * CU and their partial softmax states merged in a fixed order: lse agrees
 * with the unsplit kernel to f32 rounding, O to the bf16 rounding of the
 * probabilities (each share rounds p against its own running max), and a
 * rerun gives the same bits. Otherwise (NULL workspace, too small, other
 * shapes) it is
 * ferrite_hip_attn_fwd. The workspace must be zero-filled before its first
 * use; a call leaves it ready for the next one (per-pair counts stay even).
 * Calls sharing one workspace must not overlap in time. The reference's
 * pallas_call has no scratch (flash_attention.py:146-174); XLA FFI would hand
 * this buffer over as the handler's scratch allocation.
 */
int64_t ferrite_hip_attn_fwd_workspace(int64_t b, int64_t h, int64_t sq, int64_t sk, int64_t d, int dtype,
                                       int causal);
int ferrite_hip_attn_fwd_ex(const void* q, const void* k, const void* v, void* o, float* lse, int64_t b, int64_t h,
                            int64_t sq, int64_t sk, int64_t d, int dtype, int causal, float scale, void* workspace,
                            int64_t workspace_bytes, void* stream);

/* delta[B, H, S] = sum_d f32(dO) * f32(O) (flash_attention.py:328). */
int ferrite_hip_attn_bwd_delta(const void* o, const void* dout, float* delta, int64_t b, int64_t h, int64_t s,
                               int64_t d, int dtype, void* stream);

/*
 * dK, dV of flash attention (flash_attention.py:197-221). Inputs q, k, v, dout of
 * `dtype`, lse and delta f32 [B, H, Sq] from ferrite_hip_attn_fwd and
 * ferrite_hip_attn_bwd_delta. dk, dv: [B, H, Sk, D] of `dtype`.
 */
int ferrite_hip_attn_bwd_dkv(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                             const float* delta, void* dk, void* dv, int64_t b, int64_t h, int64_t sq, int64_t sk,
                             int64_t d, int dtype, int causal, float scale, void* stream);

/* dQ of flash attention (flash_attention.py:224-243). dq: [B, H, Sq, D] of `dtype`. */
int ferrite_hip_attn_bwd_dq(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                            const float* delta, void* dq, int64_t b, int64_t h, int64_t sq, int64_t sk, int64_t d,
                            int dtype, int causal, float scale, void* stream);

/*
 * dQ of flash attention that also produces delta (flash_attention.py:224-243 with
 * :328-329 folded in): delta[B, H, Sq] = sum_d f32(dO) * f32(O) is computed from o
 * inside the dQ kernel, used there and written to `delta` (an output here), so the
 * dK/dV call that reads it comes after this one and no separate delta pass runs.
 * bf16 with head dims up to 128 run the fused kernel; other inputs run
 * ferrite_hip_attn_bwd_delta and then ferrite_hip_attn_bwd_dq, with the same result.
 */
int ferrite_hip_attn_bwd_dq_delta(const void* q, const void* k, const void* v, const void* o, const void* dout,
                                  const float* lse, float* delta, void* dq, int64_t b, int64_t h, int64_t sq,
                                  int64_t sk, int64_t d, int dtype, int causal, float scale, void* stream);

/*
 * ferrite_hip_attn_bwd_dkv, _bwd_dq and _bwd_dq_delta with a workspace (the same
 * kernels and arguments, plus `workspace` of `workspace_bytes` device bytes,
 * 256-byte aligned; flash_attention.py:246-307 runs the reference's two backward
 * kernels with no scratch). Where ferrite_hip_attn_bwd_workspace returns a size
 * above 0 and the workspace holds it (the long-context shapes of
 * ferrite_hip_attn_fwd_ex: bf16 causal self-attention, head dim <= 64, S a
 * multiple of 128 with an even number of 128-row tiles, B H S / 128 <= 2 x CUs),
 * each kernel splits its longest causal sweeps between the two workgroups of a
 * CU: the dK/dV of a long key block, or the dQ of a long query tile, is summed
 * from two partial sums (the same bits in either order, and on a rerun); it
 * agrees with the unsplit kernel to the f32 rounding of the summation order.
 * Otherwise (NULL workspace, too small, other shapes) each is the call without
 * _ex. One workspace serves both backward kernels of a step, one after the
 * other on a stream. It must be zero-filled before its first use; a call leaves
 * it ready for the next one (per-pair counts stay even). Calls sharing one
 * workspace must not overlap in time.
 */
int64_t ferrite_hip_attn_bwd_workspace(int64_t b, int64_t h, int64_t sq, int64_t sk, int64_t d, int dtype,
                                       int causal);
int ferrite_hip_attn_bwd_dkv_ex(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                                const float* delta, void* dk, void* dv, int64_t b, int64_t h, int64_t sq, int64_t sk,
                                int64_t d, int dtype, int causal, float scale, void* workspace, int64_t workspace_bytes,
                                void* stream);
int ferrite_hip_attn_bwd_dq_ex(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                               const float* delta, void* dq, int64_t b, int64_t h, int64_t sq, int64_t sk, int64_t d,
                               int dtype, int causal, float scale, void* workspace, int64_t workspace_bytes,
                               void* stream);
int ferrite_hip_attn_bwd_dq_delta_ex(const void* q, const void* k, const void* v, const void* o, const void* dout,
                                     const float* lse, float* delta, void* dq, int64_t b, int64_t h, int64_t sq,
                                     int64_t sk, int64_t d, int dtype, int causal, float scale, void* workspace,
                                     int64_t workspace_bytes, void* stream);

/*
 * Causal flash attention on the model's token-major layouts (model/gpt.py:136-138:
 * the fused projection reshaped to [B, S, 3, H, D], heads transposed in and out
 * around flash_attention). qkv: bf16 [B, S, 3, H, D] (q, k, v of head h at
 * [.., 0, h, :], [.., 1, h, :], [.., 2, h, :]); o: bf16 [B, S, H, D]; lse: f32
 * [B, H, S]. The kernels read the heads and write O in place, so no transposed
 * copies exist. Needs D of 64 or 128, S % 64 == 0 and 16-byte aligned tensors;
 * the numbers are bitwise those of ferrite_hip_attn_fwd on transposed copies.
 */
int ferrite_hip_attn_fwd_qkv(const void* qkv, void* o, float* lse, int64_t b, int64_t s, int64_t h, int64_t d,
                             float scale, void* stream);

/*
 * Its backward: dout bf16 [B, S, H, D]; delta f32 [B, H, S] is an output (computed
 * inside dQ, then read by dK/dV); dqkv bf16 [B, S, 3, H, D] receives dQ, dK, dV in
 * the projection's layout. Bitwise ferrite_hip_attn_bwd_dq_delta + _dkv on copies.
 */
int ferrite_hip_attn_bwd_qkv(const void* qkv, const void* o, const void* dout, const float* lse, float* delta,
                             void* dqkv, int64_t b, int64_t s, int64_t h, int64_t d, float scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FERRITE_HIP_H */
