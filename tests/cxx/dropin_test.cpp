// Runs the reference's own test scenarios through the drop-in C++ interface
// (include/kernels.h: the reference's signatures, default per-thread stream,
// exit-on-error), checking results against the CPU oracle (liboracle.so).
//
//   FC/tests/test_layernorm.cu:26-56      LN forward, srand(42) inputs
//   FC/tests/test_fusion_benchmark.cu      fused vs unfused pairs: bias+ReLU,
//                                          residual+LN forward, LN backward +
//                                          residual (the reference accepts
//                                          1e-6..1e-4; here they must agree
//                                          bit for bit), plus the new
//                                          bias+GELU pair
//   NC/tests/test_embedding.cu:43-182      embedding fwd / bwd / pos fwd,
//                                          srand(42) inputs
//   NC/tests/test_softmax_ce.cu:77-178     softmax [256,512] and cross-entropy
//                                          [128,4096], srand(42) inputs, the
//                                          reference's own bounds
// Exit status 0 = all checks passed.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "kernels.h"

extern "C" {
void orc_srand(unsigned seed);
void orc_fill_rand_unit(float* v, long n);
void orc_fill_rand_tokens(int* t, long n, int vocab);
void orc_fill_pattern(float* v, long n, float scale, float shift);
void orc_layernorm_forward(const float* x, const float* gamma, const float* beta, float* out,
                           float* mean, float* inv_std, int rows, int cols, float eps);
void orc_embedding_forward(const float* table, const int* tokens, float* out, int bt, int dim);
void orc_embedding_backward(const float* g, const int* tokens, float* gt, int bt, int dim);
void orc_pos_embedding_forward(const float* pos, float* emb, int batch, int seq, int dim);
void orc_softmax_forward(const float* x, float* out, int rows, int cols);
float orc_cross_entropy_cpu(const float* logits, const int* targets, float* grad, int batch,
                            int vocab);
}

static int g_fail = 0;

#define HIPCHECK(x)                                                              \
    do {                                                                         \
        hipError_t e_ = (x);                                                     \
        if (e_ != hipSuccess) {                                                  \
            std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), \
                         __FILE__, __LINE__);                                    \
            std::exit(2);                                                        \
        }                                                                        \
    } while (0)

template <class T>
struct Dev {
    T* p = nullptr;
    size_t n = 0;
    explicit Dev(size_t count) : n(count) { HIPCHECK(hipMalloc(&p, count * sizeof(T) + 16)); }
    Dev(const std::vector<T>& h) : Dev(h.size()) { put(h); }
    ~Dev() { (void)hipFree(p); }
    void put(const std::vector<T>& h) {
        HIPCHECK(hipMemcpy(p, h.data(), n * sizeof(T), hipMemcpyHostToDevice));
    }
    std::vector<T> get() const {
        HIPCHECK(hipStreamSynchronize(hipStreamPerThread));
        std::vector<T> h(n);
        HIPCHECK(hipMemcpy(h.data(), p, n * sizeof(T), hipMemcpyDeviceToHost));
        return h;
    }
    void zero() { HIPCHECK(hipMemset(p, 0, n * sizeof(T))); }
};

static float max_abs_diff(const std::vector<float>& a, const std::vector<float>& b) {
    float d = 0.0f;
    for (size_t i = 0; i < a.size(); ++i) d = std::fmax(d, std::fabs(a[i] - b[i]));
    return d;
}

static void check(bool ok, const char* what, double value) {
    std::printf("  %-48s %.3e %s\n", what, value, ok ? "PASS" : "FAIL");
    if (!ok) ++g_fail;
}

static bool same_bits(const std::vector<float>& a, const std::vector<float>& b) {
    return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * 4) == 0;
}

static std::vector<float> pattern(size_t n, float scale, float shift = 0.0f) {
    std::vector<float> v(n);
    orc_fill_pattern(v.data(), static_cast<long>(n), scale, shift);
    return v;
}

static void test_layernorm() {
    std::printf("layernorm_forward (FC/tests/test_layernorm.cu)\n");
    const int rows = 2048, cols = 128;
    std::vector<float> hx(rows * cols), hg(cols, 1.0f), hb(cols, 0.0f), ref(rows * cols);
    orc_srand(42);
    orc_fill_rand_unit(hx.data(), rows * cols);
    orc_layernorm_forward(hx.data(), hg.data(), hb.data(), ref.data(), nullptr, nullptr, rows,
                          cols, 1e-5f);
    Dev<float> x(hx), g(hg), b(hb), out(rows * cols);
    layernorm_forward(x.p, g.p, b.p, out.p, rows, cols);  // default eps, as the reference calls it
    const float err = max_abs_diff(out.get(), ref);
    check(err < 1e-5f, "max abs error vs CPU (reference bound 1e-3)", err);
}

static void test_fusion_pairs() {
    std::printf("fused vs unfused (FC/tests/test_fusion_benchmark.cu)\n");
    {  // bias + ReLU: bias_add then relu_forward vs bias_relu_forward
        const int rows = 2048, cols = 512, n = rows * cols;
        auto hin = pattern(n, 0.1f), hbias = pattern(cols, 0.001f);
        Dev<float> work(hin), fused_in(hin), bias(hbias), unfused(n), fused(n);
        bias_add(work.p, bias.p, rows, cols);
        relu_forward(work.p, unfused.p, n);
        bias_relu_forward(fused_in.p, bias.p, fused.p, rows, cols);
        check(same_bits(unfused.get(), fused.get()), "bias+ReLU fused == unfused (bits)",
              max_abs_diff(unfused.get(), fused.get()));
    }
    {  // residual + LN forward
        const int rows = 2048, cols = 128, n = rows * cols;
        auto ha = pattern(n, 0.1f), hb = pattern(n, 0.08f);
        auto hgam = pattern(cols, 0.03f, 1.0f), hbet = pattern(cols, 0.02f);
        Dev<float> a(ha), b(hb), gam(hgam), bet(hbet);
        Dev<float> ru(n), ou(n), mu(rows), iu(rows), rf(n), of(n), mf(rows), jf(rows);
        residual_add(a.p, b.p, ru.p, n);
        layernorm_forward_save(ru.p, gam.p, bet.p, ou.p, mu.p, iu.p, rows, cols);
        residual_layernorm_forward_save(a.p, b.p, gam.p, bet.p, rf.p, of.p, mf.p, jf.p, rows, cols);
        check(same_bits(ru.get(), rf.get()) && same_bits(ou.get(), of.get()) &&
                  same_bits(mu.get(), mf.get()) && same_bits(iu.get(), jf.get()),
              "residual+LN fwd fused == unfused (bits)", max_abs_diff(ou.get(), of.get()));
        std::vector<float> ref(n), hr(n);
        for (int i = 0; i < n; ++i) hr[i] = ha[i] + hb[i];
        orc_layernorm_forward(hr.data(), hgam.data(), hbet.data(), ref.data(), nullptr, nullptr,
                              rows, cols, 1e-5f);
        const float err = max_abs_diff(of.get(), ref);
        check(err < 1e-5f, "residual+LN fwd vs CPU", err);
    }
    {  // LN backward + residual accumulate vs LN backward then residual_add
        const int rows = 2048, cols = 128, n = rows * cols;
        auto hx = pattern(n, 0.1f), hgr = pattern(n, 0.05f), hres = pattern(n, 0.02f);
        auto hgam = pattern(cols, 0.03f, 1.0f), hbet = pattern(cols, 0.01f);
        Dev<float> x(hx), grad(hgr), gam(hgam), bet(hbet), out(n), mean(rows), inv(rows), dx(n);
        Dev<float> res_u(hres), res_f(hres), dgu(cols), dbu(cols), dgf(cols), dbf(cols);
        dgu.zero(); dbu.zero(); dgf.zero(); dbf.zero();
        layernorm_forward_save(x.p, gam.p, bet.p, out.p, mean.p, inv.p, rows, cols);
        layernorm_backward(grad.p, x.p, mean.p, inv.p, gam.p, dx.p, dgu.p, dbu.p, rows, cols);
        residual_add(res_u.p, dx.p, res_u.p, n);  // in place, as the reference test does
        layernorm_backward_residual(grad.p, x.p, mean.p, inv.p, gam.p, res_f.p, dgf.p, dbf.p,
                                    rows, cols);
        // The accumulated dx is row-local and identical; dgamma/dbeta are
        // column sums whose (fixed) order follows each form's workgroup
        // shape (the residual form runs 16-wave workgroups where the plain
        // one runs 8), so they are held to the reference's criterion
        // (FC/tests/test_fusion_benchmark.cu:276).
        check(same_bits(res_u.get(), res_f.get()), "LN bwd+residual fused == unfused dx (bits)",
              max_abs_diff(res_u.get(), res_f.get()));
        const float dg_err = max_abs_diff(dgu.get(), dgf.get());
        const float db_err = max_abs_diff(dbu.get(), dbf.get());
        check(dg_err < 1e-4f, "LN bwd+residual dgamma (reference bound 1e-4)", dg_err);
        check(db_err < 1e-4f, "LN bwd+residual dbeta (reference bound 1e-4)", db_err);
    }
    {  // bias + GELU: bias_add then GELU of the sum vs bias_gelu_forward; bwd repeatable
        const int rows = 512, cols = 3072, n = rows * cols;
        auto hin = pattern(n, 1.5f), hbias = pattern(cols, 0.02f), hgo = pattern(n, 1.0f);
        Dev<float> in(hin), work(hin), bias(hbias), zero_bias(std::vector<float>(cols, 0.0f));
        Dev<float> y1(n), y2(n), go(hgo), gin1(n), gin2(n), db1(cols), db2(cols);
        bias_gelu_forward(in.p, bias.p, y1.p, rows, cols);
        bias_add(work.p, bias.p, rows, cols);
        bias_gelu_forward(work.p, zero_bias.p, y2.p, rows, cols);
        check(same_bits(y1.get(), y2.get()), "bias+GELU fused == bias_add then GELU (bits)",
              max_abs_diff(y1.get(), y2.get()));
        db1.zero(); db2.zero();
        gelu_backward_with_bias_backward(in.p, bias.p, go.p, gin1.p, db1.p, rows, cols);
        gelu_backward_with_bias_backward(in.p, bias.p, go.p, gin2.p, db2.p, rows, cols);
        check(same_bits(gin1.get(), gin2.get()) && same_bits(db1.get(), db2.get()),
              "GELU bwd + dbias repeatable (bits)", 0.0);
    }
}

static void test_embedding() {
    std::printf("embedding (NC/tests/test_embedding.cu)\n");
    const int V = 512, D = 128, B = 16, T = 32, BT = B * T;
    std::vector<float> table(V * D), gout(BT * D), pos(T * D);
    std::vector<int> tokens(BT);
    orc_srand(42);
    orc_fill_rand_unit(table.data(), V * D);
    orc_fill_rand_tokens(tokens.data(), BT, V);
    orc_fill_rand_unit(gout.data(), BT * D);
    orc_fill_rand_unit(pos.data(), T * D);
    std::vector<float> ref_out(BT * D), ref_gt(V * D, 0.0f);
    orc_embedding_forward(table.data(), tokens.data(), ref_out.data(), BT, D);
    orc_embedding_backward(gout.data(), tokens.data(), ref_gt.data(), BT, D);
    std::vector<float> ref_emb = ref_out;
    orc_pos_embedding_forward(pos.data(), ref_emb.data(), B, T, D);

    Dev<float> dt(table), dg(gout), dp(pos), out(BT * D), gt(V * D);
    Dev<int> tok(tokens);
    embedding_forward(dt.p, tok.p, out.p, BT, D);
    check(same_bits(out.get(), ref_out), "embedding_forward == CPU (bits)", 0.0);
    gt.zero();
    embedding_backward(dg.p, tok.p, gt.p, BT, D);
    check(same_bits(gt.get(), ref_gt), "embedding_backward == CPU (bits)",
          max_abs_diff(gt.get(), ref_gt));
    pos_embedding_forward(dp.p, out.p, B, T, D);
    check(same_bits(out.get(), ref_emb), "pos_embedding_forward == CPU (bits)", 0.0);
}

static void test_softmax_ce() {
    std::printf("softmax / cross-entropy (NC/tests/test_softmax_ce.cu)\n");
    {
        const int rows = 256, cols = 512, n = rows * cols;
        std::vector<float> hx(n), ref(n);
        orc_srand(42);
        orc_fill_rand_unit(hx.data(), n);
        orc_softmax_forward(hx.data(), ref.data(), rows, cols);
        Dev<float> x(hx), out(n);
        softmax_forward(x.p, out.p, rows, cols);
        const float err = max_abs_diff(out.get(), ref);
        check(err < 1e-5f, "softmax max abs error (reference bound 1e-5)", err);
    }
    {
        const int batch = 128, vocab = 4096, n = batch * vocab;
        std::vector<float> hl(n), gref(n);
        std::vector<int> ht(batch);
        orc_srand(42);
        orc_fill_rand_unit(hl.data(), n);
        orc_fill_rand_tokens(ht.data(), batch, vocab);
        const float loss_ref = orc_cross_entropy_cpu(hl.data(), ht.data(), gref.data(), batch, vocab);
        Dev<float> l(hl), g(n), losses(batch), loss_out(1);
        Dev<int> t(ht);
        const float loss = cross_entropy_forward(l.p, t.p, g.p, batch, vocab);
        const float grad_err = max_abs_diff(g.get(), gref);
        const float loss_err = std::fabs(loss_ref - loss) / (std::fabs(loss_ref) + 1e-8f);
        check(grad_err < 1e-4f, "cross-entropy grad error (reference bound 1e-4)", grad_err);
        check(loss_err < 1e-2f, "cross-entropy loss rel error (reference bound 1e-2)", loss_err);
        // v2: grad scaled by 1/batch, the mean loss left on the device
        cross_entropy_forward_v2(l.p, t.p, g.p, losses.p, loss_out.p, batch, vocab);
        const float loss2 = loss_out.get()[0];
        const std::vector<float> g2 = g.get();
        float g2_err = 0.0f;
        for (int i = 0; i < n; ++i) g2_err = std::fmax(g2_err, std::fabs(g2[i] * batch - gref[i]));
        const float loss2_err = std::fabs(loss_ref - loss2) / (std::fabs(loss_ref) + 1e-8f);
        check(g2_err < 1e-4f && loss2_err < 1e-2f, "cross-entropy v2 (device loss, grad/batch)",
              loss2_err);
    }
}

int main() {
    test_layernorm();
    test_fusion_pairs();
    test_embedding();
    test_softmax_ce();
    std::printf("%s (%d failure%s)\n", g_fail ? "FAILED" : "PASSED", g_fail, g_fail == 1 ? "" : "s");
    return g_fail ? 1 : 0;
}
