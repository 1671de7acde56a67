// extern "C" entry points onto the reference's own CPU routines.
//
// TEST INFRASTRUCTURE ONLY (the checker of the checker).  The reference's
// CPU routines sit inside CUDA test programs whose other code needs the CUDA
// runtime, so the files cannot be compiled whole here.  build_ref.sh copies
// the exact line ranges holding the host routines (no edits, no stand-in
// headers) into a temporary directory, compiles this file against them with
// g++, writes only oracle/_ref/libref_cpu.so and deletes the excerpts.
// Nothing of the reference's source is kept in the repository.
//
//   ln_cpu.inc       FC/tests/test_layernorm.cu:8-24        layernorm_cpu
//   emb_cpu.inc      NC/tests/test_embedding.cu:16-41       embedding_forward_cpu,
//                                                           embedding_backward_cpu,
//                                                           pos_embedding_cpu
//   fill_pattern.inc FC/tests/test_fusion_benchmark.cu:8-12 fill_pattern
//   ln_f64.inc       FC/tests/test_model_reference.cu:49-68 layernorm (double)
//   softmax_ce.inc   NC/tests/test_softmax_ce.cu:26-75      softmax_cpu,
//                                                           cross_entropy_cpu
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <vector>

#include "ln_cpu.inc"
#include "emb_cpu.inc"
#include "fill_pattern.inc"
#include "ln_f64.inc"
#include "softmax_ce.inc"

extern "C" {

void ref_layernorm_cpu(const float* x, const float* gamma, const float* beta,
                       float* out, int rows, int cols, float eps) {
    layernorm_cpu(x, gamma, beta, out, rows, cols, eps);
}

void ref_layernorm_f64(const double* x, const double* gamma, const double* beta,
                       double* out, int rows, int cols, double eps) {
    std::vector<double> xv(x, x + (size_t)rows * cols), ov;
    layernorm(xv, gamma, beta, ov, rows, cols, eps);
    std::copy(ov.begin(), ov.end(), out);
}

void ref_embedding_forward_cpu(const float* table, const int* tokens, float* out,
                               int batch_seq, int dim) {
    embedding_forward_cpu(table, tokens, out, batch_seq, dim);
}

void ref_embedding_backward_cpu(const float* grad_out, const int* tokens,
                                float* grad_table, int batch_seq, int dim,
                                int vocab_size) {
    embedding_backward_cpu(grad_out, tokens, grad_table, batch_seq, dim, vocab_size);
}

void ref_pos_embedding_cpu(const float* pos_table, float* embeddings, int batch,
                           int seq, int dim) {
    pos_embedding_cpu(pos_table, embeddings, batch, seq, dim);
}

void ref_fill_pattern(float* v, int n, float scale, float shift) {
    std::vector<float> tmp((size_t)n);
    fill_pattern(tmp, scale, shift);
    std::copy(tmp.begin(), tmp.end(), v);
}

void ref_softmax_cpu(const float* x, float* out, int rows, int cols) {
    softmax_cpu(x, out, rows, cols);
}

float ref_cross_entropy_cpu(const float* logits, const int* targets, float* grad, int batch,
                            int vocab) {
    return cross_entropy_cpu(logits, targets, grad, batch, vocab);
}

}  // extern "C"
