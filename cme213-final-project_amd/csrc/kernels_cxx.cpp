// The reference-signature C++ entry points (include/kernels.h): each one
// forwards to its mi_* C entry point on hipStreamPerThread and exits on
// failure like the reference's CUDA_CHECK_LAST
// (FINAL_CLEAN_CODE/include/common.h:20-30).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#include "kernels.h"

namespace {

void* per_thread_stream() { return reinterpret_cast<void*>(hipStreamPerThread); }

void check(int rc, const char* file, int line) {
    if (rc != MI_OK) {
        std::fprintf(stderr, "HIP error at %s:%d — %s\n", file, line, mi_last_error());
        std::exit(EXIT_FAILURE);
    }
}

}  // namespace

#define MI_CHECK(call) check((call), __FILE__, __LINE__)

void layernorm_forward(const float* x, const float* gamma, const float* beta, float* out,
                       int rows, int cols, float eps) {
    MI_CHECK(mi_layernorm_forward(x, gamma, beta, out, rows, cols, eps, per_thread_stream()));
}

void layernorm_forward_save(const float* x, const float* gamma, const float* beta, float* out,
                            float* mean, float* inv_std, int rows, int cols, float eps) {
    MI_CHECK(mi_layernorm_forward_save(x, gamma, beta, out, mean, inv_std, rows, cols, eps,
                                       per_thread_stream()));
}

void residual_layernorm_forward_save(const float* a, const float* b, const float* gamma,
                                     const float* beta, float* residual_out, float* out,
                                     float* mean, float* inv_std, int rows, int cols, float eps) {
    MI_CHECK(mi_residual_layernorm_forward_save(a, b, gamma, beta, residual_out, out, mean,
                                                inv_std, rows, cols, eps, per_thread_stream()));
}

void layernorm_backward(const float* grad_out, const float* x, const float* mean,
                        const float* inv_std, const float* gamma, float* grad_x, float* dgamma,
                        float* dbeta, int rows, int cols) {
    MI_CHECK(mi_layernorm_backward(grad_out, x, mean, inv_std, gamma, grad_x, dgamma, dbeta, rows,
                                   cols, per_thread_stream()));
}

void layernorm_backward_residual(const float* grad_out, const float* x, const float* mean,
                                 const float* inv_std, const float* gamma, float* grad_residual,
                                 float* dgamma, float* dbeta, int rows, int cols) {
    MI_CHECK(mi_layernorm_backward_residual(grad_out, x, mean, inv_std, gamma, grad_residual,
                                            dgamma, dbeta, rows, cols, per_thread_stream()));
}

void relu_forward(const float* in, float* out, int n) {
    MI_CHECK(mi_relu_forward(in, out, n, per_thread_stream()));
}

void relu_backward(const float* in, const float* grad_out, float* grad_in, int n) {
    MI_CHECK(mi_relu_backward(in, grad_out, grad_in, n, per_thread_stream()));
}

void relu_backward_with_bias_backward(const float* mask, const float* grad_out, float* grad_in,
                                      float* dbias, int rows, int cols) {
    MI_CHECK(mi_relu_backward_with_bias_backward(mask, grad_out, grad_in, dbias, rows, cols,
                                                 per_thread_stream()));
}

void residual_add(const float* a, const float* b, float* out, int n) {
    MI_CHECK(mi_residual_add(a, b, out, n, per_thread_stream()));
}

void residual_add_with_bias(const float* residual, const float* x, const float* bias, float* out,
                            int rows, int cols) {
    MI_CHECK(mi_residual_add_with_bias(residual, x, bias, out, rows, cols, per_thread_stream()));
}

void bias_add(float* out, const float* bias, int rows, int cols) {
    MI_CHECK(mi_bias_add(out, bias, rows, cols, per_thread_stream()));
}

void bias_relu_forward(const float* in, const float* bias, float* out, int rows, int cols) {
    MI_CHECK(mi_bias_relu_forward(in, bias, out, rows, cols, per_thread_stream()));
}

void bias_backward(const float* grad, float* dbias, int rows, int cols) {
    MI_CHECK(mi_bias_backward(grad, dbias, rows, cols, per_thread_stream()));
}

void bias_gelu_forward(const float* in, const float* bias, float* out, int rows, int cols) {
    MI_CHECK(mi_bias_gelu_forward(in, bias, out, rows, cols, per_thread_stream()));
}

void gelu_backward_with_bias_backward(const float* in, const float* bias, const float* grad_out,
                                      float* grad_in, float* dbias, int rows, int cols) {
    MI_CHECK(mi_gelu_backward_with_bias_backward(in, bias, grad_out, grad_in, dbias, rows, cols,
                                                 per_thread_stream()));
}

void embedding_forward(const float* table, const int* tokens, float* out, int batch_seq,
                       int dim) {
    MI_CHECK(mi_embedding_forward(table, tokens, out, batch_seq, dim, 0, per_thread_stream()));
}

void embedding_backward(const float* grad_out, const int* tokens, float* grad_table,
                        int batch_seq, int dim) {
    MI_CHECK(mi_embedding_backward(grad_out, tokens, grad_table, batch_seq, dim, 0,
                                   per_thread_stream()));
}

void pos_embedding_forward(const float* pos_table, float* embeddings, int batch, int seq,
                           int dim) {
    MI_CHECK(mi_pos_embedding_forward(pos_table, embeddings, batch, seq, dim,
                                      per_thread_stream()));
}

void pos_embedding_backward(const float* grad_out, float* grad_pos_table, int batch, int seq,
                            int dim) {
    MI_CHECK(mi_pos_embedding_backward(grad_out, grad_pos_table, batch, seq, dim,
                                       per_thread_stream()));
}

void softmax_forward(const float* x, float* out, int rows, int cols) {
    MI_CHECK(mi_softmax_forward(x, out, rows, cols, per_thread_stream()));
}

float cross_entropy_forward(const float* logits, const int* targets, float* grad, int batch,
                            int vocab) {
    float loss = 0.0f;
    MI_CHECK(mi_cross_entropy_forward(logits, targets, grad, batch, vocab, &loss,
                                      per_thread_stream()));
    return loss;
}

void cross_entropy_forward_v2(const float* logits, const int* targets, float* grad,
                              float* d_losses, float* d_loss_out, int batch, int vocab) {
    MI_CHECK(mi_cross_entropy_forward_v2(logits, targets, grad, d_losses, d_loss_out, batch, vocab,
                                         per_thread_stream()));
}

void scale_buffer(float* buf, float scale, int n) {
    MI_CHECK(mi_scale_buffer(buf, scale, n, per_thread_stream()));
}

void buffer_norm_sq_acc(const float* buf, int n, float* d_result) {
    MI_CHECK(mi_buffer_norm_sq_acc(buf, n, d_result, per_thread_stream()));
}

void compute_clip_scale(const float* d_norm_sq, float* d_clip_scale, float max_norm) {
    MI_CHECK(mi_compute_clip_scale(d_norm_sq, d_clip_scale, max_norm, per_thread_stream()));
}

void relu_backward_with_bias_backward_half_mask(const __half* mask, const float* grad_out,
                                                float* grad_in, float* dbias, int rows,
                                                int cols) {
    MI_CHECK(mi_relu_backward_with_bias_backward_half_mask(mask, grad_out, grad_in, dbias, rows,
                                                           cols, per_thread_stream()));
}

void bias_relu_forward_to_half(const float* in, const float* bias, __half* out, int rows,
                               int cols) {
    MI_CHECK(mi_bias_relu_forward_to_half(in, bias, out, rows, cols, per_thread_stream()));
}

void float_to_half_buffer(const float* in, __half* out, int n) {
    MI_CHECK(mi_float_to_half(in, out, n, per_thread_stream()));
}

void half_to_float_buffer(const __half* in, float* out, int n) {
    MI_CHECK(mi_half_to_float(in, out, n, per_thread_stream()));
}
