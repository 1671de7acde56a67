// The reference's own kernel timing loops, at its shapes, through the
// drop-in C++ interface (include/kernels.h):
//   * FINAL_CLEAN_CODE/tests/test_fusion_benchmark.cu: bias+ReLU 2048x512,
//     residual+LayerNorm forward and LayerNorm backward + residual 2048x128,
//     fused and unfused (10 warm-up calls, then `iters` calls on the same
//     buffers between two events), and the LayerNorm forward of
//     correctness_matrix (2048x128); inputs: the fusion harness's sin/cos
//     fill pattern;
//   * FINAL_CLEAN_CODE/tests/benchmark_all.cu:124-163, the LayerNorm
//     bandwidth grid (six shapes, 10 warm-up calls, 200 timed);
//   * FINAL_CLEAN_CODE/tests/deep_profile.cu:121-173, LayerNorm forward at
//     2048x{128,256,512} (20 warm-up calls, 500 timed);
//   the last two with their srand(42), rand()/RAND_MAX - 0.5 inputs,
//   gamma = 1, beta = 0.
// Calls launch on the per-thread default stream, as the reference's do; the
// events are recorded there.  Prints one JSON object: per case, microseconds
// per call and the number of timed calls.  Run by bench.py --workload
// refshapes.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <string>
#include <utility>
#include <vector>

#include "kernels.h"

namespace {

#define CK(x)                                                                         \
    do {                                                                              \
        hipError_t e_ = (x);                                                          \
        if (e_ != hipSuccess) {                                                       \
            std::fprintf(stderr, "HIP error at %s:%d — %s\n", __FILE__, __LINE__,     \
                         hipGetErrorString(e_));                                      \
            std::exit(EXIT_FAILURE);                                                  \
        }                                                                             \
    } while (0)

std::vector<float> pattern(int n, float scale, float shift = 0.0f) {
    std::vector<float> v(n);
    for (int i = 0; i < n; ++i)
        v[i] = scale * sinf(0.013f * static_cast<float>(i)) +
               0.5f * scale * cosf(0.021f * static_cast<float>(i + 7)) + shift;
    return v;
}

float* dev(const std::vector<float>& h) {
    float* p = nullptr;
    CK(hipMalloc(&p, h.size() * sizeof(float)));
    CK(hipMemcpy(p, h.data(), h.size() * sizeof(float), hipMemcpyHostToDevice));
    return p;
}

float* dev_zero(int n) {
    float* p = nullptr;
    CK(hipMalloc(&p, static_cast<size_t>(n) * sizeof(float)));
    CK(hipMemset(p, 0, static_cast<size_t>(n) * sizeof(float)));
    return p;
}

// The reference harnesses' input generator (glibc rand() after srand(seed)).
std::vector<float> rand_unit(int n, unsigned seed = 42) {
    std::vector<float> v(n);
    std::srand(seed);
    for (auto& x : v) x = static_cast<float>(std::rand()) / static_cast<float>(RAND_MAX) - 0.5f;
    return v;
}

struct Timed {
    double us;
    int calls;
};

Timed time_us(const std::function<void()>& call, int iters, int warmup = 10) {
    hipStream_t st = hipStreamPerThread;
    for (int i = 0; i < warmup; ++i) call();
    CK(hipDeviceSynchronize());
    hipEvent_t a, b;
    CK(hipEventCreate(&a));
    CK(hipEventCreate(&b));
    CK(hipEventRecord(a, st));
    for (int i = 0; i < iters; ++i) call();
    CK(hipEventRecord(b, st));
    CK(hipEventSynchronize(b));
    float ms = 0.0f;
    CK(hipEventElapsedTime(&ms, a, b));
    CK(hipEventDestroy(a));
    CK(hipEventDestroy(b));
    return {1e3 * ms / iters, iters};
}

}  // namespace

int main(int argc, char** argv) {
    const int scale = argc > 1 ? std::atoi(argv[1]) : 1;  // iteration multiplier
    const int R = 2048, C = 128, n = R * C;
    float* x = dev(pattern(n, 0.1f));
    float* a = dev(pattern(n, 0.1f));
    float* b = dev(pattern(n, 0.08f));
    float* grad = dev(pattern(n, 0.05f));
    float* gamma = dev(pattern(C, 0.03f, 1.0f));
    float* beta = dev(pattern(C, 0.02f));
    float* res = dev_zero(n);
    float* out = dev_zero(n);
    float* mean = dev_zero(R);
    float* inv = dev_zero(R);
    float* dx = dev_zero(n);
    float* gres = dev(pattern(n, 0.02f));
    float* dg = dev_zero(C);
    float* db = dev_zero(C);
    layernorm_forward_save(x, gamma, beta, out, mean, inv, R, C);

    const int Rb = 2048, Cb = 512, nb = Rb * Cb;
    float* work = dev(pattern(nb, 0.1f));
    float* bias = dev(pattern(Cb, 0.001f));
    float* bout = dev_zero(nb);
    CK(hipDeviceSynchronize());

    std::vector<std::pair<std::string, Timed>> r;
    r.emplace_back("ln_fwd", time_us([&] { layernorm_forward(x, gamma, beta, out, R, C); },
                                     300 * scale));
    r.emplace_back("residual_ln_unfused", time_us([&] {
                       residual_add(a, b, res, n);
                       layernorm_forward_save(res, gamma, beta, out, mean, inv, R, C);
                   }, 300 * scale));
    r.emplace_back("residual_ln_fused", time_us([&] {
                       residual_layernorm_forward_save(a, b, gamma, beta, res, out, mean, inv, R,
                                                       C);
                   }, 300 * scale));
    r.emplace_back("ln_bwd_residual_unfused", time_us([&] {
                       layernorm_backward(grad, x, mean, inv, gamma, dx, dg, db, R, C);
                       residual_add(gres, dx, gres, n);
                   }, 200 * scale));
    r.emplace_back("ln_bwd_residual_fused", time_us([&] {
                       layernorm_backward_residual(grad, x, mean, inv, gamma, gres, dg, db, R, C);
                   }, 200 * scale));
    r.emplace_back("bias_relu_unfused", time_us([&] {
                       bias_add(work, bias, Rb, Cb);
                       relu_forward(work, bout, nb);
                   }, 200 * scale));
    r.emplace_back("bias_relu_fused",
                   time_us([&] { bias_relu_forward(work, bias, bout, Rb, Cb); }, 200 * scale));

    // LayerNorm forward grids of benchmark_all.cu (10 + 200 calls) and
    // deep_profile.cu (20 + 500 calls), gamma = 1, beta = 0.
    struct Grid {
        const char* tag;
        int rows, cols, warmup, iters;
    };
    const Grid grids[] = {{"ln_grid", 1024, 64, 10, 200},   {"ln_grid", 1024, 128, 10, 200},
                          {"ln_grid", 2048, 128, 10, 200},  {"ln_grid", 4096, 128, 10, 200},
                          {"ln_grid", 2048, 256, 10, 200},  {"ln_grid", 2048, 512, 10, 200},
                          {"ln_deep", 2048, 128, 20, 500},  {"ln_deep", 2048, 256, 20, 500},
                          {"ln_deep", 2048, 512, 20, 500}};
    for (const Grid& gd : grids) {
        const int gn = gd.rows * gd.cols;
        float* gx = dev(rand_unit(gn));
        float* gg = dev(std::vector<float>(gd.cols, 1.0f));
        float* gb = dev(std::vector<float>(gd.cols, 0.0f));
        float* gy = dev_zero(gn);
        CK(hipDeviceSynchronize());
        const std::string name = std::string(gd.tag) + "_" + std::to_string(gd.rows) + "x" +
                                 std::to_string(gd.cols);
        r.emplace_back(name, time_us([&] { layernorm_forward(gx, gg, gb, gy, gd.rows, gd.cols); },
                                     gd.iters * scale, gd.warmup));
        CK(hipDeviceSynchronize());
        CK(hipFree(gx));
        CK(hipFree(gg));
        CK(hipFree(gb));
        CK(hipFree(gy));
    }

    std::printf("{");
    for (size_t i = 0; i < r.size(); ++i)
        std::printf("%s\"%s\": {\"us\": %.4f, \"calls\": %d}", i ? ", " : "",
                    r[i].first.c_str(), r[i].second.us, r[i].second.calls);
    std::printf("}\n");
    return 0;
}
