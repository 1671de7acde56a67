/*
 * mi_kernels.h — C ABI of the MI355X (gfx950) fused non-GEMM layer kernels.
 *
 * Every compute entry point replaces one free function of the reference's
 * C++ kernel interface, FINAL_CLEAN_CODE/include/kernels.h (cited per
 * function as kernels.h:line), with the same argument meaning, the same
 * overwrite-versus-accumulate contract and the same aliasing rules.  The
 * differences are the ones a C ABI needs:
 *
 *  - C linkage and an "mi_" prefix (the C++ names with the reference's exact
 *    signatures live in kernels.h of this directory and forward here);
 *  - an explicit stream (a hipStream_t passed as void*; NULL = the legacy
 *    default stream);
 *  - an int status instead of exit(): 0 on success, a hipError_t value for
 *    a runtime failure, or one of the MI_ERR_* codes below; mi_last_error()
 *    returns the message of the most recent failure on the calling thread.
 *
 * All pointers are device pointers owned by the caller, fp32 row-major
 * contiguous (ids int32).  Calls are asynchronous on `stream` and perform no
 * host synchronisation.  The column reductions (dgamma/dbeta/dbias) and the
 * embedding gradients are deterministic (no float atomics), so repeated calls
 * on identical inputs give identical bits.  The column reductions are
 * two-pass and use a library-owned device workspace; it is allocated on first
 * use (or by mi_workspace_reserve) and may not grow while the stream is being
 * captured into a graph.  Growth never frees or synchronises: the buffer it
 * replaces stays allocated (queued kernels, a launch on another thread or an
 * instantiated graph may still use it) until mi_workspace_release().
 * Workspaces are kept per device and per slot.  Calls on an explicit stream
 * or on the null stream share the device's slot: they must not run
 * concurrently on different streams of the same device (one stream
 * serialises them).  Calls on the per-thread default stream
 * (hipStreamPerThread, which the include/kernels.h entry points use, as the
 * reference's `--default-stream per-thread` build does) use a slot of the
 * calling thread's own, so host threads may issue them concurrently.  A
 * thread's slot is kept after the thread exits, until mi_workspace_release().
 */
#ifndef MI_KERNELS_H
#define MI_KERNELS_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI_OK 0
#define MI_ERR_INVALID_ARG (-1)    /* bad size, NULL pointer, unsupported shape */
#define MI_ERR_CAPTURE_ALLOC (-2)  /* workspace growth needed during capture */

/* ----- runtime helpers (so a ctypes driver needs no other library) ------ */

const char* mi_last_error(void);
const char* mi_version(void);
int mi_device_count(int* count);
int mi_set_device(int device);
int mi_malloc(void** ptr, size_t bytes);
int mi_free(void* ptr);
int mi_memcpy_h2d(void* dst, const void* src, size_t bytes);
int mi_memcpy_d2h(void* dst, const void* src, size_t bytes);
int mi_memset_zero(void* ptr, size_t bytes, void* stream);
int mi_stream_sync(void* stream);
int mi_device_sync(void);
/* Grow the shared workspace slot of the current device (the one calls on
 * explicit streams and the null stream use) to >= bytes now (call before
 * graph capture).  mi_workspace_bytes() reports its current size. */
int mi_workspace_reserve(size_t bytes);
size_t mi_workspace_bytes(void);
/* The same for the slot that calls on `stream` from the calling thread use:
 * the thread's own slot for hipStreamPerThread, else the shared slot.  For a
 * caller that captures the per-thread stream into a graph.  Refused with
 * MI_ERR_CAPTURE_ALLOC while `stream` is capturing. */
int mi_workspace_reserve_stream(size_t bytes, void* stream);
size_t mi_workspace_bytes_stream(void* stream);
/* Synchronise the current device, then free its workspace buffers (every
 * slot's current buffer and every one a growth retired).  Only for a caller
 * who will not replay a graph captured with workspace-using calls; the next
 * call that needs a workspace allocates a new one. */
int mi_workspace_release(void);
/* Workspace an entry point needs for the given shape (bytes).  The token
 * embedding backward needs none: mi_embedding_backward_workspace returns 0. */
size_t mi_layernorm_backward_workspace(int rows, int cols);
size_t mi_bias_backward_workspace(int rows, int cols);
size_t mi_embedding_backward_workspace(int batch_seq);

/* ----- LayerNorm --------------------------------------------------------- */

/* y = (x - mean) * inv_std * gamma + beta per row, biased variance,
 * inv_std = 1/sqrt(var + eps).  Replaces layernorm_forward (kernels.h:53-54,
 * FINAL_CLEAN_CODE/src/kernels/layernorm.cu:60-66). */
int mi_layernorm_forward(const float* x, const float* gamma, const float* beta,
                         float* out, int rows, int cols, float eps, void* stream);

/* As mi_layernorm_forward and also writes mean[rows], inv_std[rows].
 * Replaces layernorm_forward_save (kernels.h:56-58, layernorm.cu:111-119). */
int mi_layernorm_forward_save(const float* x, const float* gamma, const float* beta,
                              float* out, float* mean, float* inv_std,
                              int rows, int cols, float eps, void* stream);

/* residual_out = a + b; out = LN(residual_out) with saved stats.  Replaces
 * residual_layernorm_forward_save (kernels.h:60-64, layernorm.cu:173-183). */
int mi_residual_layernorm_forward_save(const float* a, const float* b,
                                       const float* gamma, const float* beta,
                                       float* residual_out, float* out,
                                       float* mean, float* inv_std,
                                       int rows, int cols, float eps, void* stream);

/* grad_x = dx (overwrite); dgamma += sum_r g*xhat; dbeta += sum_r g.
 * Replaces layernorm_backward (kernels.h:66-70, layernorm.cu:273-289). */
int mi_layernorm_backward(const float* grad_out, const float* x,
                          const float* mean, const float* inv_std, const float* gamma,
                          float* grad_x, float* dgamma, float* dbeta,
                          int rows, int cols, void* stream);

/* grad_residual += dx; dgamma, dbeta accumulate.  Replaces
 * layernorm_backward_residual (kernels.h:72-76, layernorm.cu:291-308). */
int mi_layernorm_backward_residual(const float* grad_out, const float* x,
                                   const float* mean, const float* inv_std,
                                   const float* gamma, float* grad_residual,
                                   float* dgamma, float* dbeta,
                                   int rows, int cols, void* stream);

/* Allocation-free variant of mi_layernorm_backward (same arguments, same
 * results bit for bit: it runs the same kernels).  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Its partial rows live in a static device array of
 * MI_LN_BWD_NOALLOC_MAX_BYTES per device instead of the library workspace;
 * the call makes no hipMalloc / hipFree.  The array is part of the
 * library's code object, so every process that loads the library holds it
 * (16 MiB + 256 B) on each device where the library's code is loaded, until
 * the process ends, whether or not this entry point is ever called.
 * A shape whose partial rows need more (mi_layernorm_backward_workspace
 * reports the need) is rejected with MI_ERR_INVALID_ARG.  Every call on a
 * device shares that device's array: calls that overlap on one device (two
 * streams, or two threads) race and must be serialised by the caller. */
#define MI_LN_BWD_NOALLOC_MAX_BYTES ((size_t)16 * 1024 * 1024 + 256)
int mi_layernorm_backward_noalloc(const float* grad_out, const float* x,
                                  const float* mean, const float* inv_std,
                                  const float* gamma, float* grad_x,
                                  float* dgamma, float* dbeta,
                                  int rows, int cols, void* stream);

/* ----- residual / bias / ReLU ------------------------------------------- */

/* out = a + b over n elements; out may alias a or b.  Replaces residual_add
 * (kernels.h:88, FINAL_CLEAN_CODE/src/kernels/activations.cu:70-82). */
int mi_residual_add(const float* a, const float* b, float* out, long long n, void* stream);

/* out = (residual + x) + bias[c].  Replaces residual_add_with_bias
 * (kernels.h:90-92, activations.cu:119-137). */
int mi_residual_add_with_bias(const float* residual, const float* x, const float* bias,
                              float* out, int rows, int cols, void* stream);

/* out[r, c] += bias[c] in place.  Replaces bias_add (kernels.h:104,
 * activations.cu:146-151). */
int mi_bias_add(float* out, const float* bias, int rows, int cols, void* stream);

/* out = max(in, 0).  Replaces relu_forward (kernels.h:78,
 * activations.cu:10-14). */
int mi_relu_forward(const float* in, float* out, long long n, void* stream);

/* grad_in = in > 0 ? grad_out : 0.  Replaces relu_backward (kernels.h:79,
 * activations.cu:38-50). */
int mi_relu_backward(const float* in, const float* grad_out, float* grad_in,
                     long long n, void* stream);

/* out = max(in + bias[c], 0).  Replaces bias_relu_forward (kernels.h:106-107,
 * activations.cu:181-197). */
int mi_bias_relu_forward(const float* in, const float* bias, float* out,
                         int rows, int cols, void* stream);

/* grad_in = mask > 0 ? grad_out : 0; dbias += column sums of grad_in
 * (deterministic).  Replaces relu_backward_with_bias_backward
 * (kernels.h:81-83, activations.cu:274-283). */
int mi_relu_backward_with_bias_backward(const float* mask, const float* grad_out,
                                        float* grad_in, float* dbias,
                                        int rows, int cols, void* stream);

/* dbias += column sums of grad (deterministic).  Replaces bias_backward
 * (kernels.h:111, activations.cu:234-240). */
int mi_bias_backward(const float* grad, float* dbias, int rows, int cols, void* stream);

/* ----- bias + tanh-GELU (new operators in the slots of bias_relu_forward
 * and relu_backward_with_bias_backward; the reference has no GELU) ------- */

/* out = gelu_tanh(in + bias[c]). */
int mi_bias_gelu_forward(const float* in, const float* bias, float* out,
                         int rows, int cols, void* stream);

/* u = in + bias[c] (recomputed); grad_in = grad_out * gelu_tanh'(u);
 * dbias += column sums of grad_in (deterministic). */
int mi_gelu_backward_with_bias_backward(const float* in, const float* bias,
                                        const float* grad_out, float* grad_in,
                                        float* dbias, int rows, int cols, void* stream);

/* ----- embedding --------------------------------------------------------- */

/* out[i, :] = table[tokens[i], :].  vocab > 0 bounds the ids: an id outside
 * [0, vocab) yields a zero row instead of a read out of bounds; vocab <= 0
 * trusts the ids as the reference does.  Replaces embedding_forward
 * (kernels.h:131-132, FINAL_CLEAN_CODE/src/kernels/embedding.cu:13-20). */
int mi_embedding_forward(const float* table, const int* tokens, float* out,
                         int batch_seq, int dim, int vocab, void* stream);

/* grad_table[tokens[i], :] += grad_out[i, :], each table row accumulated in
 * increasing i (deterministic, same order as the CPU loop); one kernel, no
 * workspace.  vocab > 0 skips ids outside [0, vocab); vocab <= 0 trusts the
 * ids (negative ids are skipped).  Replaces embedding_backward
 * (kernels.h:133-134, embedding.cu:33-40). */
int mi_embedding_backward(const float* grad_out, const int* tokens, float* grad_table,
                          int batch_seq, int dim, int vocab, void* stream);

/* embeddings[b, t, :] += pos_table[t, :] in place.  Replaces
 * pos_embedding_forward (kernels.h:135-136, embedding.cu:52-59). */
int mi_pos_embedding_forward(const float* pos_table, float* embeddings,
                             int batch, int seq, int dim, void* stream);

/* grad_pos[t, :] += sum over b (in increasing b) of grad_out[b, t, :].
 * Replaces pos_embedding_backward (kernels.h:137-138, embedding.cu:72-79). */
int mi_pos_embedding_backward(const float* grad_out, float* grad_pos_table,
                              int batch, int seq, int dim, void* stream);

/* Fused token + position gather: out[b, t, :] = table[id, :] + pos[t, :].
 * Bit-identical to mi_embedding_forward followed by mi_pos_embedding_forward
 * (one fp32 add per element), in one pass.  The reference issues the two
 * calls back to back (FINAL_CLEAN_CODE/src/model/transformer.cu:345-346). */
int mi_embedding_pos_forward(const float* table, const float* pos_table,
                             const int* tokens, float* out,
                             int batch, int seq, int dim, int vocab, void* stream);

/* Fused token + position backward: mi_embedding_backward(grad_out, tokens,
 * grad_table, batch * seq, dim, vocab) and mi_pos_embedding_backward(grad_out,
 * grad_pos_table, batch, seq, dim) in one launch, bit-identical to the two
 * calls (same accumulation orders).  The reference issues the two calls back
 * to back (FINAL_CLEAN_CODE/src/model/transformer.cu:581-584). */
int mi_embedding_pos_backward(const float* grad_out, const int* tokens,
                              float* grad_table, float* grad_pos_table,
                              int batch, int seq, int dim, int vocab, void* stream);

/* ----- softmax and cross-entropy ----------------------------------------- */

/* out[r, :] = exp(x[r, :] - max) / sum, per row.  Replaces softmax_forward
 * (kernels.h:122, FINAL_CLEAN_CODE/src/kernels/activations.cu:394-435). */
int mi_softmax_forward(const float* x, float* out, int rows, int cols, void* stream);

/* Softmax cross-entropy with the reference kernel's arithmetic
 * (activations.cu:438-477): p = e * (1 / (sum + 1e-9)),
 * loss[b] = -log(p[target] + 1e-9), grad = p - onehot(target).  Waits for
 * the stream, copies the per-row losses back and stores their mean, summed
 * in row order on the host, in *loss.  A target outside [0, vocab) gives a
 * NaN loss and leaves that row's gradient at p.  Replaces
 * cross_entropy_forward (kernels.h:124-125, activations.cu:479-499), which
 * returns the loss; uses the library workspace for the per-row losses. */
int mi_cross_entropy_forward(const float* logits, const int* targets, float* grad,
                             int batch, int vocab, float* loss, void* stream);

/* As above with grad scaled by 1 / batch, per-row losses in losses[batch]
 * and their mean written to the device scalar *loss_out, summed in a fixed
 * order (no host sync, no memset, no atomics; graph-capturable).  Replaces
 * cross_entropy_forward_v2 (kernels.h:127-129, activations.cu:517-532). */
int mi_cross_entropy_forward_v2(const float* logits, const int* targets, float* grad,
                                float* losses, float* loss_out, int batch, int vocab,
                                void* stream);

/* Workspace bytes mi_cross_entropy_forward needs for `batch` rows. */
size_t mi_cross_entropy_workspace(int batch);

/* ----- optimizer step over the flat parameter buffer ---------------------- */

/* buf[i] *= scale.  Replaces scale_buffer (kernels.h:113,
 * FINAL_CLEAN_CODE/src/kernels/activations.cu:349-358). */
int mi_scale_buffer(float* buf, float scale, long long n, void* stream);

/* *d_result += sum of buf[i]^2, with a deterministic two-pass sum (per-block
 * partials in the library workspace, then a fixed-order total) instead of
 * the reference's per-block float atomicAdd.  Replaces buffer_norm_sq_acc
 * (kernels.h:118, activations.cu:360-381). */
int mi_buffer_norm_sq_acc(const float* buf, long long n, float* d_result, void* stream);

/* *d_clip_scale = sqrt(*d_norm_sq) > max_norm ? max_norm / sqrt(*d_norm_sq)
 * : 1.  Replaces compute_clip_scale (kernels.h:120, activations.cu:383-392). */
int mi_compute_clip_scale(const float* d_norm_sq, float* d_clip_scale, float max_norm,
                          void* stream);

/* One clipped Adam step, the arithmetic of adam_clipped_kernel
 * (FINAL_CLEAN_CODE/src/model/transformer.cu:598-617) evaluated as written:
 * g = grad * grad_scale * (*d_clip_scale); m = beta1 m + (1 - beta1) g;
 * v = beta2 v + (1 - beta2) g g; param -= lr (m / bc1) / (sqrt(v / bc2) + eps). */
int mi_adam_clipped(float* param, const float* grad, float* m, float* v,
                    const float* d_clip_scale, float lr, float beta1, float beta2, float eps,
                    float bc1, float bc2, float grad_scale, long long n, void* stream);

/* TransformerModel::update_adam (transformer.cu:619-636) in one call: bias
 * corrections 1 - beta^step on the host, the gradient norm² into *d_norm_sq
 * (overwritten, no memset), the clip scale for max norm 1 / grad_scale (1
 * when grad_scale <= 0) into *d_clip_scale, then the Adam step.  Three
 * kernels, graph-capturable; step >= 1. */
int mi_adam_update(float* param, const float* grad, float* m, float* v, long long n, float lr,
                   float beta1, float beta2, float eps, int step, float grad_scale,
                   float* d_norm_sq, float* d_clip_scale, void* stream);

/* Workspace bytes mi_buffer_norm_sq_acc / mi_adam_update need for n floats. */
size_t mi_norm_sq_workspace(long long n);

/* ----- 16-bit activation storage ----------------------------------------- */
/* Half buffers hold IEEE binary16 values, bf16 buffers the upper 16 bits of
 * fp32; both are passed as void* (2 bytes per element).  Conversions round
 * to nearest even. */

/* out16[i] = half(in[i]).  Replaces float_to_half_buffer (kernels.h:115,
 * FINAL_CLEAN_CODE/src/kernels/activations.cu:325-329,337-341). */
int mi_float_to_half(const float* in, void* out16, long long n, void* stream);

/* out[i] = float(in16[i]).  Replaces half_to_float_buffer (kernels.h:116,
 * activations.cu:331-335,343-347). */
int mi_half_to_float(const void* in16, float* out, long long n, void* stream);

/* bf16 counterparts (no reference counterpart: the bf16 storage variant of
 * the same path). */
int mi_float_to_bf16(const float* in, void* out16, long long n, void* stream);
int mi_bf16_to_float(const void* in16, float* out, long long n, void* stream);

/* out16 = half(max(in + bias, 0)).  Replaces bias_relu_forward_to_half
 * (kernels.h:108-109, activations.cu:199-217). */
int mi_bias_relu_forward_to_half(const float* in, const float* bias, void* out16, int rows,
                                 int cols, void* stream);

/* out16 = half / bf16 (gelu(in + bias)): the bias+GELU forward with 16-bit
 * activation storage (no reference counterpart; takes the slot of
 * bias_relu_forward_to_half for the GELU path). */
int mi_bias_gelu_forward_to_half(const float* in, const float* bias, void* out16, int rows,
                                 int cols, void* stream);
int mi_bias_gelu_forward_to_bf16(const float* in, const float* bias, void* out16, int rows,
                                 int cols, void* stream);

/* grad_in = float(mask16) > 0 ? grad_out : 0; dbias += column sums
 * (deterministic).  Replaces relu_backward_with_bias_backward_half_mask
 * (kernels.h:84-86, activations.cu:285-323). */
int mi_relu_backward_with_bias_backward_half_mask(const void* mask16, const float* grad_out,
                                                  float* grad_in, float* dbias, int rows,
                                                  int cols, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MI_KERNELS_H */
