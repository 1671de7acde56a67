/*
 * CPU oracle for the fused non-GEMM layer path (LayerNorm, residual adds,
 * bias + ReLU / tanh-GELU, token + position embedding).
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker, never the product:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load liboracle.so.  The HIP library never links or calls it.
 *
 * Every float routine restates the reference's host/CPU code statement for
 * statement (same float type, same sequential summation order, same
 * evaluation order of each expression).  Where the reference has no CPU
 * twin, the routine follows the reference GPU kernel's arithmetic with the
 * reductions done sequentially (cited per function).  Paths below are
 * relative to the reference root:
 *   FC/ = FINAL_CLEAN_CODE/, NC/ = NEW_code/.
 *
 * Double-precision variants (suffix _f64) give the error budget the tests
 * log next to the float comparison.
 *
 * Built with gcc -O2 -ffp-contract=off (no FMA contraction, SSE2 float
 * arithmetic), so each expression rounds exactly as written.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

/* Number of host threads the row-parallel loops use (1 = the reference's
 * single-threaded CPU path).  Results do not depend on it: rows are
 * independent and every column sum stays sequential over rows. */
void orc_set_threads(int n) { g_threads = n < 1 ? 1 : n; }
int orc_get_threads(void) { return g_threads; }

/* ------------------------------------------------------------------ */
/* Test-input generators used by the reference's own tests.            */
/* ------------------------------------------------------------------ */

/* srand(seed) as in FC/tests/test_layernorm.cu:35 and
 * NC/tests/test_embedding.cu:57. */
void orc_srand(unsigned seed) { srand(seed); }

/* v = (float)rand()/RAND_MAX - 0.5f, FC/tests/test_layernorm.cu:36 and
 * NC/tests/test_embedding.cu:58,107,149. Continues the current sequence. */
void orc_fill_rand_unit(float* v, long n) {
    for (long i = 0; i < n; ++i) v[i] = (float)rand() / RAND_MAX - 0.5f;
}

/* t = rand() % vocab, NC/tests/test_embedding.cu:59. */
void orc_fill_rand_tokens(int* t, long n, int vocab) {
    for (long i = 0; i < n; ++i) t[i] = rand() % vocab;
}

/* fill_pattern, FC/tests/test_fusion_benchmark.cu:8-12. */
void orc_fill_pattern(float* v, long n, float scale, float shift) {
    for (long i = 0; i < n; ++i)
        v[i] = scale * sinf(0.013f * (float)i) +
               0.5f * scale * cosf(0.021f * (float)(i + 7)) + shift;
}

/* ------------------------------------------------------------------ */
/* LayerNorm                                                           */
/* ------------------------------------------------------------------ */

/* LN forward, FC/tests/test_layernorm.cu:8-24 (layernorm_cpu): sequential
 * float sums, biased variance, inv_std = 1.0f / sqrtf(var + eps).  When
 * mean / inv_std are non-NULL the row statistics are also saved, as
 * layernorm_save_kernel does (FC/src/kernels/layernorm.cu:102-105). */
void orc_layernorm_forward(const float* x, const float* gamma, const float* beta,
                           float* out, float* save_mean, float* save_inv_std,
                           int rows, int cols, float eps) {
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (long)r * cols;
        float* yr = out + (long)r * cols;
        float mean = 0.0f;
        for (int c = 0; c < cols; ++c) mean += xr[c];
        mean /= cols;
        float var = 0.0f;
        for (int c = 0; c < cols; ++c) {
            float d = xr[c] - mean;
            var += d * d;
        }
        var /= cols;
        float inv_std = 1.0f / sqrtf(var + eps);
        for (int c = 0; c < cols; ++c)
            yr[c] = (xr[c] - mean) * inv_std * gamma[c] + beta[c];
        if (save_mean) save_mean[r] = mean;
        if (save_inv_std) save_inv_std[r] = inv_std;
    }
}

/* Double LN forward, FC/tests/test_model_reference.cu:49-68. Inputs are
 * the float tensors widened to double. */
void orc_layernorm_forward_f64(const float* x, const float* gamma, const float* beta,
                               double* out, double* save_mean, double* save_inv_std,
                               int rows, int cols, double eps) {
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (long)r * cols;
        double mean = 0.0;
        for (int c = 0; c < cols; ++c) mean += xr[c];
        mean /= cols;
        double var = 0.0;
        for (int c = 0; c < cols; ++c) {
            double d = xr[c] - mean;
            var += d * d;
        }
        double inv_std = 1.0 / sqrt(var / cols + eps);
        for (int c = 0; c < cols; ++c)
            out[(long)r * cols + c] = (xr[c] - mean) * inv_std * gamma[c] + beta[c];
        if (save_mean) save_mean[r] = mean;
        if (save_inv_std) save_inv_std[r] = inv_std;
    }
}

/* Residual + LN forward: r = a + b (written), then LN(r) with saved stats.
 * Semantics of residual_layernorm_save_kernel
 * (FC/src/kernels/layernorm.cu:121-171); FC/tests/test_fusion_benchmark.cu
 * :162-165 pins it as residual_add followed by layernorm_forward_save. */
void orc_residual_layernorm_forward(const float* a, const float* b,
                                    const float* gamma, const float* beta,
                                    float* residual_out, float* out,
                                    float* save_mean, float* save_inv_std,
                                    int rows, int cols, float eps) {
    long n = (long)rows * cols;
    for (long i = 0; i < n; ++i) residual_out[i] = a[i] + b[i];
    orc_layernorm_forward(residual_out, gamma, beta, out, save_mean, save_inv_std,
                          rows, cols, eps);
}

/* LN backward.  The reference has no CPU LN backward; this follows the
 * arithmetic of layernorm_backward_dx_kernel (FC/src/kernels/layernorm.cu
 * :207-234) with the two row sums done sequentially in float, and of
 * layernorm_backward_dweight_kernel (:253-267) with each column summed
 * sequentially over rows and then added into dgamma / dbeta.
 * add_to_grad = 0: grad_x = dx (layernorm_backward, :273-289);
 * add_to_grad = 1: grad_x += dx (layernorm_backward_residual, :291-308).
 * dgamma and dbeta always accumulate (+=), as in the reference. */
void orc_layernorm_backward(const float* grad_out, const float* x,
                            const float* mean, const float* inv_std,
                            const float* gamma, float* grad_x,
                            float* dgamma, float* dbeta,
                            int rows, int cols, int add_to_grad) {
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
    for (int r = 0; r < rows; ++r) {
        const float* go = grad_out + (long)r * cols;
        const float* xi = x + (long)r * cols;
        float* gx = grad_x + (long)r * cols;
        float mu = mean[r];
        float is = inv_std[r];
        float sum_dxhat = 0.0f;
        float sum_dxhat_xhat = 0.0f;
        for (int i = 0; i < cols; ++i) {
            float x_hat = (xi[i] - mu) * is;
            float dx_hat = go[i] * gamma[i];
            sum_dxhat += dx_hat;
            sum_dxhat_xhat += dx_hat * x_hat;
        }
        float mean_dxhat = sum_dxhat / cols;
        float mean_dxhat_xhat = sum_dxhat_xhat / cols;
        for (int i = 0; i < cols; ++i) {
            float x_hat = (xi[i] - mu) * is;
            float dx_hat = go[i] * gamma[i];
            float dx = is * (dx_hat - mean_dxhat - x_hat * mean_dxhat_xhat);
            if (add_to_grad)
                gx[i] += dx;
            else
                gx[i] = dx;
        }
    }
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
    for (int c = 0; c < cols; ++c) {
        float dg = 0.0f;
        float db = 0.0f;
        for (int r = 0; r < rows; ++r) {
            float go = grad_out[(long)r * cols + c];
            float x_hat = (x[(long)r * cols + c] - mean[r]) * inv_std[r];
            dg += go * x_hat;
            db += go;
        }
        dgamma[c] += dg;
        dbeta[c] += db;
    }
}

/* Double LN backward from first principles: statistics recomputed in double
 * from x (as orc_layernorm_forward_f64), dx by the same closed form,
 * column sums in double.  Outputs are overwritten (no accumulation). */
void orc_layernorm_backward_f64(const float* grad_out, const float* x,
                                const float* gamma, double eps,
                                double* grad_x, double* dgamma, double* dbeta,
                                int rows, int cols) {
    double* mu = (double*)malloc(sizeof(double) * (rows > 0 ? rows : 1));
    double* rs = (double*)malloc(sizeof(double) * (rows > 0 ? rows : 1));
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
    for (int r = 0; r < rows; ++r) {
        const float* xi = x + (long)r * cols;
        const float* go = grad_out + (long)r * cols;
        double m = 0.0;
        for (int c = 0; c < cols; ++c) m += xi[c];
        m /= cols;
        double v = 0.0;
        for (int c = 0; c < cols; ++c) {
            double d = xi[c] - m;
            v += d * d;
        }
        double is = 1.0 / sqrt(v / cols + eps);
        mu[r] = m;
        rs[r] = is;
        double s1 = 0.0, s2 = 0.0;
        for (int c = 0; c < cols; ++c) {
            double xh = (xi[c] - m) * is;
            double dh = (double)go[c] * gamma[c];
            s1 += dh;
            s2 += dh * xh;
        }
        s1 /= cols;
        s2 /= cols;
        for (int c = 0; c < cols; ++c) {
            double xh = (xi[c] - m) * is;
            double dh = (double)go[c] * gamma[c];
            grad_x[(long)r * cols + c] = is * (dh - s1 - xh * s2);
        }
    }
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
    for (int c = 0; c < cols; ++c) {
        double dg = 0.0, db = 0.0;
        for (int r = 0; r < rows; ++r) {
            double go = grad_out[(long)r * cols + c];
            double xh = (x[(long)r * cols + c] - mu[r]) * rs[r];
            dg += go * xh;
            db += go;
        }
        dgamma[c] = dg;
        dbeta[c] = db;
    }
    free(mu);
    free(rs);
}

/* ------------------------------------------------------------------ */
/* Residual / bias / ReLU                                              */
/* ------------------------------------------------------------------ */

/* out = a + b, FC/src/kernels/activations.cu:52-56 (one IEEE add).
 * In-place (out == a) is allowed, as test_fusion_benchmark.cu:234 uses. */
void orc_residual_add(const float* a, const float* b, float* out, long n) {
    for (long i = 0; i < n; ++i) out[i] = a[i] + b[i];
}

/* out = (residual + x) + bias[c], order of FC/src/kernels/activations.cu
 * :99-102 and :116 (double form: test_model_reference.cu:175-180). */
void orc_residual_add_with_bias(const float* residual, const float* x,
                                const float* bias, float* out, int rows, int cols) {
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) {
            long i = (long)r * cols + c;
            out[i] = residual[i] + x[i] + bias[c];
        }
}

/* out += bias[c] in place, FC/src/kernels/activations.cu:139-144. */
void orc_bias_add(float* out, const float* bias, int rows, int cols) {
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) out[(long)r * cols + c] += bias[c];
}

/* FC/src/kernels/activations.cu:5-8. */
void orc_relu_forward(const float* in, float* out, long n) {
    for (long i = 0; i < n; ++i) out[i] = (in[i] > 0.0f) ? in[i] : 0.0f;
}

/* FC/src/kernels/activations.cu:16-20. */
void orc_relu_backward(const float* in, const float* grad_out, float* grad_in, long n) {
    for (long i = 0; i < n; ++i) grad_in[i] = (in[i] > 0.0f) ? grad_out[i] : 0.0f;
}

/* v = in + bias[c]; out = v > 0 ? v : 0, FC/src/kernels/activations.cu
 * :153-161 (CPU twin in double: test_model_reference.cu:167-172). */
void orc_bias_relu_forward(const float* in, const float* bias, float* out,
                           int rows, int cols) {
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) {
            long i = (long)r * cols + c;
            float v = in[i] + bias[c];
            out[i] = (v > 0.0f) ? v : 0.0f;
        }
}

/* dbias[c] += sum_r grad[r, c], sequential over rows.  Semantics of
 * bias_backward_kernel (FC/src/kernels/activations.cu:221-232), which the
 * reference sums with float atomics in an unspecified order. */
void orc_bias_backward(const float* grad, float* dbias, int rows, int cols) {
    for (int c = 0; c < cols; ++c) {
        float s = 0.0f;
        for (int r = 0; r < rows; ++r) s += grad[(long)r * cols + c];
        dbias[c] += s;
    }
}

/* gin = mask > 0 ? g : 0 (written); dbias[c] += sum_r gin.  Semantics of
 * fused_relu_backward_bias_backward_kernel (FC/src/kernels/activations.cu
 * :247-272), column sums sequential over rows. */
void orc_relu_backward_with_bias_backward(const float* mask, const float* grad_out,
                                          float* grad_in, float* dbias,
                                          int rows, int cols) {
    for (int c = 0; c < cols; ++c) {
        float s = 0.0f;
        for (int r = 0; r < rows; ++r) {
            long i = (long)r * cols + c;
            float g = (mask[i] > 0.0f) ? grad_out[i] : 0.0f;
            grad_in[i] = g;
            s += g;
        }
        dbias[c] += s;
    }
}

/* ------------------------------------------------------------------ */
/* bias + tanh-approximation GELU (no reference twin: the reference uses
 * bias + ReLU, FC/src/kernels/activations.cu:181-197 / :274-283, and this
 * pair takes those slots).  Formula: Hendrycks & Gimpel 2016,
 *   gelu(u) = 0.5 u (1 + tanh(sqrt(2/pi) (u + 0.044715 u^3))),
 *   gelu'(u) = 0.5 (1 + t) + 0.5 u (1 - t^2) sqrt(2/pi) (1 + 3*0.044715 u^2),
 * t = tanh(...).  u = in + bias[c] is recomputed in the backward.        */
/* ------------------------------------------------------------------ */

#define GELU_K0 0.7978845608028654f /* sqrt(2/pi) */
#define GELU_K1 0.044715f

void orc_bias_gelu_forward(const float* in, const float* bias, float* out,
                           int rows, int cols) {
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) {
            long i = (long)r * cols + c;
            float u = in[i] + bias[c];
            float z = GELU_K0 * (u + GELU_K1 * u * u * u);
            out[i] = 0.5f * u * (1.0f + tanhf(z));
        }
}

/* gin = g * gelu'(u) (written); dbias[c] += sum_r gin, sequential over rows. */
void orc_gelu_backward_with_bias_backward(const float* in, const float* bias,
                                          const float* grad_out, float* grad_in,
                                          float* dbias, int rows, int cols) {
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) {
            long i = (long)r * cols + c;
            float u = in[i] + bias[c];
            float z = GELU_K0 * (u + GELU_K1 * u * u * u);
            float t = tanhf(z);
            float d = 0.5f * (1.0f + t) +
                      0.5f * u * (1.0f - t * t) * GELU_K0 * (1.0f + 3.0f * GELU_K1 * u * u);
            grad_in[i] = grad_out[i] * d;
        }
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
    for (int c = 0; c < cols; ++c) {
        float s = 0.0f;
        for (int r = 0; r < rows; ++r) s += grad_in[(long)r * cols + c];
        dbias[c] += s;
    }
}

void orc_bias_gelu_forward_f64(const float* in, const float* bias, double* out,
                               int rows, int cols) {
    const double k0 = 0.79788456080286535587989211986876; /* sqrt(2/pi) */
    const double k1 = 0.044715;
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) {
            long i = (long)r * cols + c;
            double u = (double)in[i] + (double)bias[c];
            /* 0.5 u (1 + tanh z) written as u / (1 + e^{-2z}): the same
             * function without the cancellation of 1 + tanh z, which in
             * double loses every digit below u = -7 (true values 1e-16
             * down to the underflow limit). */
            out[i] = u / (1.0 + exp(-2.0 * k0 * (u + k1 * u * u * u)));
        }
}

/* Double backward; u is the float sum in + bias (the value the float paths
 * see), widened.  dbias is overwritten with the double column sum. */
void orc_gelu_backward_with_bias_backward_f64(const float* in, const float* bias,
                                              const float* grad_out, double* grad_in,
                                              double* dbias, int rows, int cols) {
    const double k0 = 0.79788456080286535587989211986876;
    const double k1 = 0.044715;
    for (int c = 0; c < cols; ++c) dbias[c] = 0.0;
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c) {
            long i = (long)r * cols + c;
            double u = (double)(in[i] + bias[c]);
            double t = tanh(k0 * (u + k1 * u * u * u));
            double d = 0.5 * (1.0 + t) + 0.5 * u * (1.0 - t * t) * k0 * (1.0 + 3.0 * k1 * u * u);
            double gi = (double)grad_out[i] * d;
            grad_in[i] = gi;
            dbias[c] += gi;
        }
}

/* ------------------------------------------------------------------ */
/* Embedding                                                           */
/* ------------------------------------------------------------------ */

/* out[i, :] = table[tokens[i], :], NC/tests/test_embedding.cu:16-21. */
void orc_embedding_forward(const float* table, const int* tokens, float* out,
                           int batch_seq, int dim) {
    for (int i = 0; i < batch_seq; ++i)
        for (int j = 0; j < dim; ++j)
            out[(long)i * dim + j] = table[(long)tokens[i] * dim + j];
}

/* grad_table[tokens[i], :] += grad_out[i, :] in increasing i,
 * NC/tests/test_embedding.cu:23-32.  The reference CPU routine zero-fills
 * the table first (:26); here the caller zeroes, matching the += contract
 * of the reference kernel (FC/src/kernels/embedding.cu:22-31). */
void orc_embedding_backward(const float* grad_out, const int* tokens,
                            float* grad_table, int batch_seq, int dim) {
    for (int i = 0; i < batch_seq; ++i) {
        int tok = tokens[i];
        for (int j = 0; j < dim; ++j)
            grad_table[(long)tok * dim + j] += grad_out[(long)i * dim + j];
    }
}

/* embeddings[b, s, :] += pos_table[s, :], NC/tests/test_embedding.cu:34-41. */
void orc_pos_embedding_forward(const float* pos_table, float* embeddings,
                               int batch, int seq, int dim) {
    for (int b = 0; b < batch; ++b)
        for (int s = 0; s < seq; ++s)
            for (int d = 0; d < dim; ++d)
                embeddings[((long)b * seq + s) * dim + d] += pos_table[(long)s * dim + d];
}

/* grad_pos[s, :] += grad_out[b, s, :] for b = 0..batch-1 in order.  No CPU
 * twin in the reference; semantics of pos_embedding_backward_kernel
 * (FC/src/kernels/embedding.cu:61-70) with the batch loop sequential. */
void orc_pos_embedding_backward(const float* grad_out, float* grad_pos_table,
                                int batch, int seq, int dim) {
    for (int b = 0; b < batch; ++b)
        for (int s = 0; s < seq; ++s)
            for (int d = 0; d < dim; ++d)
                grad_pos_table[(long)s * dim + d] += grad_out[((long)b * seq + s) * dim + d];
}

/* ----- softmax and cross-entropy ----------------------------------------- */

/* Row softmax, NC/tests/test_softmax_ce.cu:26-44: max from the first
 * element, out = expf(x - max), sequential sum, out /= sum. */
void orc_softmax_forward(const float* x, float* out, int rows, int cols) {
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
    for (int r = 0; r < rows; ++r) {
        const float* row_in = x + (long)r * cols;
        float* row_out = out + (long)r * cols;
        float max_val = row_in[0];
        for (int c = 1; c < cols; ++c) max_val = fmaxf(max_val, row_in[c]);
        float sum = 0.0f;
        for (int c = 0; c < cols; ++c) {
            row_out[c] = expf(row_in[c] - max_val);
            sum += row_out[c];
        }
        for (int c = 0; c < cols; ++c) row_out[c] /= sum;
    }
}

/* Cross-entropy as the reference's CPU test states it,
 * NC/tests/test_softmax_ce.cu:46-75: log-sum-exp loss, grad = softmax -
 * onehot (unscaled); returns the mean loss (sequential float sum / batch). */
float orc_cross_entropy_cpu(const float* logits, const int* targets, float* grad,
                            int batch, int vocab) {
    float total_loss = 0.0f;
    for (int i = 0; i < batch; ++i) {
        int target = targets[i];
        const float* l = logits + (long)i * vocab;
        float max_logit = l[0];
        for (int j = 1; j < vocab; ++j) max_logit = fmaxf(max_logit, l[j]);
        float sum_exp = 0.0f;
        for (int j = 0; j < vocab; ++j) sum_exp += expf(l[j] - max_logit);
        float log_sum_exp = logf(sum_exp) + max_logit;
        float loss = log_sum_exp - l[target];
        total_loss += loss;
        for (int j = 0; j < vocab; ++j) {
            float softmax_j = expf(l[j] - max_logit) / sum_exp;
            grad[(long)i * vocab + j] = softmax_j;
            if (j == target) grad[(long)i * vocab + j] -= 1.0f;
        }
    }
    return total_loss / batch;
}

/* Cross-entropy with the arithmetic of the reference's GPU kernel
 * (FC/src/kernels/activations.cu:438-477) and its row reductions done
 * sequentially: e = expf(l - max) with max starting at -FLT_MAX,
 * p = e * (1 / (sum + 1e-9)), loss = -logf(p[t] + 1e-9), grad[t] = p[t] - 1,
 * then every grad element times scale.  A target outside [0, vocab) gives a
 * NaN loss and no onehot term (the library's defined behaviour; the
 * reference reads out of bounds). */
void orc_cross_entropy_rows(const float* logits, const int* targets, float* grad,
                            float* losses, int batch, int vocab, float scale) {
#pragma omp parallel for schedule(static) num_threads(g_threads) if (g_threads > 1)
    for (int b = 0; b < batch; ++b) {
        const float* row = logits + (long)b * vocab;
        float* g = grad + (long)b * vocab;
        float row_max = -3.402823466e+38f;
        for (int i = 0; i < vocab; ++i) row_max = fmaxf(row_max, row[i]);
        float sum = 0.0f;
        for (int i = 0; i < vocab; ++i) {
            float e = expf(row[i] - row_max);
            g[i] = e;
            sum += e;
        }
        float inv_sum = 1.0f / (sum + 1e-9f);
        for (int i = 0; i < vocab; ++i) g[i] *= inv_sum;
        int tgt = targets[b];
        if (tgt >= 0 && tgt < vocab) {
            losses[b] = -logf(g[tgt] + 1e-9f);
            g[tgt] -= 1.0f;
        } else {
            losses[b] = nanf("");
        }
        for (int i = 0; i < vocab; ++i) g[i] *= scale;
    }
}

/* Mean of per-row losses summed in row order, as the host loop of
 * cross_entropy_forward (FC/src/kernels/activations.cu:494-497). */
float orc_loss_mean(const float* losses, int n) {
    float total = 0.0f;
    for (int i = 0; i < n; ++i) total += losses[i];
    return total / n;
}

/* Double-precision cross-entropy from first principles (log-sum-exp):
 * loss = log(sum exp(l - max)) + max - l[t], grad = softmax - onehot. */
void orc_cross_entropy_f64(const float* logits, const int* targets, double* grad,
                           double* losses, int batch, int vocab) {
    for (int b = 0; b < batch; ++b) {
        const float* row = logits + (long)b * vocab;
        double m = row[0];
        for (int i = 1; i < vocab; ++i) m = row[i] > m ? row[i] : m;
        double s = 0.0;
        for (int i = 0; i < vocab; ++i) s += exp((double)row[i] - m);
        int t = targets[b];
        losses[b] = log(s) + m - (double)row[t];
        for (int i = 0; i < vocab; ++i) {
            double p = exp((double)row[i] - m) / s;
            grad[(long)b * vocab + i] = p - (i == t ? 1.0 : 0.0);
        }
    }
}

/* Double-precision softmax. */
void orc_softmax_forward_f64(const float* x, double* out, int rows, int cols) {
    for (int r = 0; r < rows; ++r) {
        const float* row = x + (long)r * cols;
        double m = row[0];
        for (int c = 1; c < cols; ++c) m = row[c] > m ? row[c] : m;
        double s = 0.0;
        for (int c = 0; c < cols; ++c) s += exp((double)row[c] - m);
        for (int c = 0; c < cols; ++c) out[(long)r * cols + c] = exp((double)row[c] - m) / s;
    }
}

/* ----- optimizer step ------------------------------------------------------ */

/* buf[i] *= scale, FC/src/kernels/activations.cu:349-352. */
void orc_scale_buffer(float* buf, float scale, long n) {
    for (long i = 0; i < n; ++i) buf[i] *= scale;
}

/* Sum of squares in double.  The reference accumulates float block sums
 * with atomicAdd (activations.cu:360-375), which has no fixed order; the
 * tests hold float results to a relative bound against this value. */
double orc_sumsq_f64(const float* buf, long n) {
    double s = 0.0;
    for (long i = 0; i < n; ++i) s += (double)buf[i] * (double)buf[i];
    return s;
}

/* Clip scale, FC/src/kernels/activations.cu:383-387. */
float orc_clip_scale(float norm_sq, float max_norm) {
    float norm = sqrtf(norm_sq);
    return (norm > max_norm) ? (max_norm / norm) : 1.0f;
}

/* One clipped Adam step, FC/src/model/transformer.cu:598-617 statement for
 * statement (clip scale passed by value instead of through a device
 * pointer). */
void orc_adam_clipped(float* param, const float* grad, float* m, float* v, float clip,
                      float lr, float beta1, float beta2, float eps, float bc1, float bc2,
                      float grad_scale, long n) {
    for (long i = 0; i < n; ++i) {
        float g = grad[i] * grad_scale * clip;
        float mi = beta1 * m[i] + (1.0f - beta1) * g;
        float vi = beta2 * v[i] + (1.0f - beta2) * g * g;
        m[i] = mi;
        v[i] = vi;
        float m_hat = mi / bc1;
        float v_hat = vi / bc2;
        param[i] -= lr * m_hat / (sqrtf(v_hat) + eps);
    }
}

/* Host bias corrections of TransformerModel::update_adam
 * (FC/src/model/transformer.cu:621-622): 1 - powf(beta, step). */
void orc_adam_bias_corrections(float beta1, float beta2, int step, float* bc1, float* bc2) {
    *bc1 = 1.0f - powf(beta1, (float)step);
    *bc2 = 1.0f - powf(beta2, (float)step);
}

/* ----- 16-bit storage ------------------------------------------------------ */

/* float -> IEEE binary16, round to nearest even (overflow to inf, NaN kept
 * quiet), from the format definitions; the conversion __float2half_rn of
 * FC/src/kernels/activations.cu:206,328 performs. */
uint16_t orc_f2h_one(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520: inf */
    if (a < 0x38800000u) {                                   /* below 2^-14 */
        if (a < 0x33000000u) return (uint16_t)sign;           /* <= 2^-25: zero */
        uint32_t e = a >> 23;
        uint32_t m = (a & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e;                            /* 14..24 */
        uint32_t r = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((((a >> 23) - 127u + 15u)) << 10) | ((a & 0x7fffffu) >> 13);
    uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
}

float orc_h2f_one(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, x;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-8f; /* m * 2^-24, exact */
        memcpy(&x, &v, 4);
        x |= sign;
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e - 15u + 127u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* float -> bf16: upper 16 bits, round to nearest even; NaN kept quiet. */
uint16_t orc_f2bf_one(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

float orc_bf2f_one(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void orc_float_to_half(const float* in, uint16_t* out, long n) {
    for (long i = 0; i < n; ++i) out[i] = orc_f2h_one(in[i]);
}
void orc_half_to_float(const uint16_t* in, float* out, long n) {
    for (long i = 0; i < n; ++i) out[i] = orc_h2f_one(in[i]);
}
void orc_float_to_bf16(const float* in, uint16_t* out, long n) {
    for (long i = 0; i < n; ++i) out[i] = orc_f2bf_one(in[i]);
}
void orc_bf16_to_float(const uint16_t* in, float* out, long n) {
    for (long i = 0; i < n; ++i) out[i] = orc_bf2f_one(in[i]);
}

/* bias_relu_to_half_kernel, FC/src/kernels/activations.cu:199-207. */
void orc_bias_relu_forward_to_half(const float* in, const float* bias, uint16_t* out,
                                   int rows, int cols) {
    for (long idx = 0; idx < (long)rows * cols; ++idx) {
        float val = in[idx] + bias[idx % cols];
        val = (val > 0.0f) ? val : 0.0f;
        out[idx] = orc_f2h_one(val);
    }
}

/* fused_relu_backward_bias_backward_half_mask_kernel
 * (FC/src/kernels/activations.cu:285-311) with the column sums sequential:
 * grad_in = half2float(mask) > 0 ? grad_out : 0; dbias += column sums. */
void orc_relu_backward_with_bias_backward_half_mask(const uint16_t* mask,
                                                    const float* grad_out, float* grad_in,
                                                    float* dbias, int rows, int cols) {
    for (int c = 0; c < cols; ++c) {
        float sum = 0.0f;
        for (int r = 0; r < rows; ++r) {
            long idx = (long)r * cols + c;
            float g = (orc_h2f_one(mask[idx]) > 0.0f) ? grad_out[idx] : 0.0f;
            grad_in[idx] = g;
            sum += g;
        }
        dbias[c] += sum;
    }
}
