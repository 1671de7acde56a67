// Floors that a LayerNorm / bias+GELU step cannot beat on this GPU, measured
// with plain kernels in the step's own launch structure, beside the library's
// own steps in the same process (bench.py --workload floor).
//
//   empty_chain   K dependent launches of an empty kernel of G workgroups
//                 (256 threads) per step, K = 1, 2, 3, G = 48, 256, 2048,
//                 16384: the fixed cost of a dependent launch;
//   config0_floor BASELINE config 0's bytes in its three dependent launches,
//                 as plain streaming kernels: a copy of [4096, 768] (the
//                 LayerNorm forward's 25.2 MB), an a + b -> c of [4096, 768]
//                 (the backward's 37.7 MB) and an empty 48-workgroup launch
//                 (the dgamma/dbeta finalize);
//   config0_step  the library's config-0 step (layernorm_forward_save +
//                 layernorm_backward through include/kernels.h);
//   headline_floor the headline step's bytes in its six launches, in its
//                 order: copy [8192, 768], copy [8192, 3072], a + b -> c
//                 [8192, 768], empty 48, a + b -> c [8192, 3072], empty 96;
//   headline_step the library's headline step (LayerNorm forward + backward
//                 on [8192, 768], bias+GELU forward + backward on
//                 [8192, 3072]);
//   block12_floor BASELINE config 3's bytes in its launch structure, 12 layers
//                 with their own buffers: per layer two 2-in-2-out adds (the
//                 residual LayerNorm forwards), a copy (bias+GELU forward),
//                 then in reverse an a + b -> c with an empty 96-workgroup
//                 launch (GELU backward + dbias finalize) and two in-place
//                 c += a + b with empty 48-workgroup launches (the residual
//                 LayerNorm backwards + finalizes);
//   block12_step  the library's config-3 step on the same buffers.
// Each *_floor / *_step case also reports *_host: the host's time to issue
// one step (the launches only), against which the GPU time shows whether a
// step is bound by the host's launch rate.
//
// Every case rotates buffer sets so that at least 1 GB of other data passes
// between two uses of a tensor (more than the 256 MB last-level cache), as
// bench.py does; the streaming kernels use 16-byte non-temporal accesses in a
// 16384 x 256 grid-stride loop (the fastest plain copy form measured here).
// Times are HIP events around `iters` steps after 20 warm-up steps, on the
// per-thread default stream.  Prints one JSON object.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <utility>
#include <vector>

#include "kernels.h"

namespace {

#define CK(x)                                                                     \
    do {                                                                          \
        hipError_t e_ = (x);                                                      \
        if (e_ != hipSuccess) {                                                   \
            std::fprintf(stderr, "HIP error at %s:%d: %s\n", __FILE__, __LINE__,  \
                         hipGetErrorString(e_));                                  \
            std::exit(EXIT_FAILURE);                                              \
        }                                                                         \
    } while (0)

constexpr int kThreads = 256;
constexpr int kStreamBlocks = 16384;
typedef float f4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void empty_kernel() {}

__global__ __launch_bounds__(kThreads) void copy_kernel(const f4* __restrict__ a,
                                                        f4* __restrict__ c, long long n) {
    const long long step = static_cast<long long>(gridDim.x) * kThreads;
    for (long long i = blockIdx.x * kThreads + threadIdx.x; i < n; i += step)
        __builtin_nontemporal_store(__builtin_nontemporal_load(a + i), c + i);
}

__global__ __launch_bounds__(kThreads) void add_kernel(const f4* __restrict__ a,
                                                       const f4* __restrict__ b,
                                                       f4* __restrict__ c, long long n) {
    const long long step = static_cast<long long>(gridDim.x) * kThreads;
    for (long long i = blockIdx.x * kThreads + threadIdx.x; i < n; i += step)
        __builtin_nontemporal_store(__builtin_nontemporal_load(a + i) +
                                        __builtin_nontemporal_load(b + i),
                                    c + i);
}

// r = a + b and y = a - b: the residual LayerNorm forward's two reads and two writes.
__global__ __launch_bounds__(kThreads) void add2_kernel(const f4* __restrict__ a,
                                                        const f4* __restrict__ b,
                                                        f4* __restrict__ r, f4* __restrict__ y,
                                                        long long n) {
    const long long step = static_cast<long long>(gridDim.x) * kThreads;
    for (long long i = blockIdx.x * kThreads + threadIdx.x; i < n; i += step) {
        const f4 x = __builtin_nontemporal_load(a + i);
        const f4 z = __builtin_nontemporal_load(b + i);
        __builtin_nontemporal_store(x + z, r + i);
        __builtin_nontemporal_store(x - z, y + i);
    }
}

// c += a + b: the residual LayerNorm backward's three reads and one write.
__global__ __launch_bounds__(kThreads) void add3_kernel(const f4* __restrict__ a,
                                                        const f4* __restrict__ b,
                                                        f4* __restrict__ c, long long n) {
    const long long step = static_cast<long long>(gridDim.x) * kThreads;
    for (long long i = blockIdx.x * kThreads + threadIdx.x; i < n; i += step)
        __builtin_nontemporal_store(__builtin_nontemporal_load(c + i) +
                                        (__builtin_nontemporal_load(a + i) +
                                         __builtin_nontemporal_load(b + i)),
                                    c + i);
}

hipStream_t st() { return hipStreamPerThread; }

void empty(int blocks) {
    hipLaunchKernelGGL(empty_kernel, dim3(blocks), dim3(kThreads), 0, st());
}

void copy(const float* a, float* c, long long n) {
    hipLaunchKernelGGL(copy_kernel, dim3(kStreamBlocks), dim3(kThreads), 0, st(),
                       reinterpret_cast<const f4*>(a), reinterpret_cast<f4*>(c), n / 4);
}

void add(const float* a, const float* b, float* c, long long n) {
    hipLaunchKernelGGL(add_kernel, dim3(kStreamBlocks), dim3(kThreads), 0, st(),
                       reinterpret_cast<const f4*>(a), reinterpret_cast<const f4*>(b),
                       reinterpret_cast<f4*>(c), n / 4);
}

void add2(const float* a, const float* b, float* r, float* y, long long n) {
    hipLaunchKernelGGL(add2_kernel, dim3(kStreamBlocks), dim3(kThreads), 0, st(),
                       reinterpret_cast<const f4*>(a), reinterpret_cast<const f4*>(b),
                       reinterpret_cast<f4*>(r), reinterpret_cast<f4*>(y), n / 4);
}

void add3(const float* a, const float* b, float* c, long long n) {
    hipLaunchKernelGGL(add3_kernel, dim3(kStreamBlocks), dim3(kThreads), 0, st(),
                       reinterpret_cast<const f4*>(a), reinterpret_cast<const f4*>(b),
                       reinterpret_cast<f4*>(c), n / 4);
}

float* buf(size_t n, float v) {
    float* p = nullptr;
    CK(hipMalloc(&p, n * sizeof(float)));
    unsigned bits = 0;
    std::memcpy(&bits, &v, sizeof(bits));
    CK(hipMemsetD32(reinterpret_cast<hipDeviceptr_t>(p), bits, n));
    return p;
}

// Host time to issue one step, microseconds (set by time_steps).
double g_host_us = 0.0;

// Microseconds per step over `iters` steps after 20 warm-up steps (GPU time
// between two events); g_host_us receives the host's issue time per step
// over the same loop.  A step whose host time reaches its GPU time is bound
// by the host's launch rate, not by the GPU.
double time_steps(const std::function<void(int)>& step, int iters) {
    for (int k = 0; k < 20; ++k) step(k);
    CK(hipDeviceSynchronize());
    hipEvent_t a, b;
    CK(hipEventCreate(&a));
    CK(hipEventCreate(&b));
    CK(hipEventRecord(a, st()));
    const auto t0 = std::chrono::steady_clock::now();
    for (int k = 0; k < iters; ++k) step(20 + k);
    const auto t1 = std::chrono::steady_clock::now();
    CK(hipEventRecord(b, st()));
    CK(hipEventSynchronize(b));
    float ms = 0.0f;
    CK(hipEventElapsedTime(&ms, a, b));
    CK(hipGetLastError());
    CK(hipEventDestroy(a));
    CK(hipEventDestroy(b));
    g_host_us = std::chrono::duration<double, std::micro>(t1 - t0).count() / iters;
    return 1e3 * ms / iters;
}

// One buffer set of a LayerNorm (+ optional bias+GELU) step: inputs of the
// forward and the backward, outputs, statistics.
struct Set {
    float *x, *y, *mean, *rstd, *dy, *dx;  // LayerNorm [R, C]
    float *h, *o, *dh, *gin;               // bias+GELU [R, F] (F = 0: none)
};

std::vector<Set> make_sets(int n, int R, int C, int F, const float* gamma, const float* beta) {
    std::vector<Set> s(n);
    for (Set& e : s) {
        const size_t rc = size_t(R) * C, rf = size_t(R) * F;
        e.x = buf(rc, 0.5f);
        e.y = buf(rc, 0.0f);
        e.dy = buf(rc, 0.25f);
        e.dx = buf(rc, 0.0f);
        e.mean = buf(R, 0.0f);
        e.rstd = buf(R, 0.0f);
        e.h = F ? buf(rf, 0.1f) : nullptr;
        e.o = F ? buf(rf, 0.0f) : nullptr;
        e.dh = F ? buf(rf, 0.3f) : nullptr;
        e.gin = F ? buf(rf, 0.0f) : nullptr;
        layernorm_forward_save(e.x, gamma, beta, e.y, e.mean, e.rstd, R, C);
    }
    CK(hipDeviceSynchronize());
    return s;
}

void free_sets(std::vector<Set>& s) {
    CK(hipDeviceSynchronize());
    for (Set& e : s)
        for (float* p : {e.x, e.y, e.dy, e.dx, e.mean, e.rstd, e.h, e.o, e.dh, e.gin})
            if (p) CK(hipFree(p));
    s.clear();
}

int sets_for(size_t set_bytes) {
    const size_t want = (size_t(1) << 30) / set_bytes + 2;
    return static_cast<int>(want < 4 ? 4 : (want > 64 ? 64 : want));
}

}  // namespace

int main(int argc, char** argv) {
    const int scale = argc > 1 ? std::atoi(argv[1]) : 1;
    std::vector<std::pair<std::string, double>> out;
    // time a case and record its GPU and host-issue times per step
    auto rec = [&](const std::string& name, const std::function<void(int)>& step, int iters) {
        out.emplace_back(name, time_steps(step, iters));
        out.emplace_back(name + "_host", g_host_us);
    };

    for (int blocks : {48, 256, 2048, 16384})
        for (int k = 1; k <= 3; ++k)
            out.emplace_back("empty_chain_" + std::to_string(k) + "x" + std::to_string(blocks),
                             time_steps([&](int) {
                                 for (int j = 0; j < k; ++j) empty(blocks);
                             }, 2000 * scale));

    const int C = 768;
    float* gamma = buf(4096, 1.0f);
    float* beta = buf(4096, 0.0f);

    // Config 0: [4096, 768].
    {
        const int R = 4096;
        const long long n = 1ll * R * C;
        std::vector<Set> s = make_sets(sets_for(6 * n * 4), R, C, 0, gamma, beta);
        const int ns = static_cast<int>(s.size());
        float* dg = buf(C, 0.0f);
        float* db = buf(C, 0.0f);
        rec("config0_floor", [&](int k) {
                             const Set& f = s[k % ns];
                             const Set& b = s[(k + ns - 1) % ns];
                             copy(f.x, f.y, n);
                             add(b.dy, b.x, b.dx, n);
                             empty(48);
                         }, 400 * scale);
        rec("config0_step", [&](int k) {
                             const Set& f = s[k % ns];
                             const Set& b = s[(k + ns - 1) % ns];
                             layernorm_forward_save(f.x, gamma, beta, f.y, f.mean, f.rstd, R, C);
                             layernorm_backward(b.dy, b.x, b.mean, b.rstd, gamma, b.dx, dg, db, R,
                                                C);
                         }, 400 * scale);
        free_sets(s);
        CK(hipFree(dg));
        CK(hipFree(db));
    }

    // Headline: [8192, 768] and [8192, 3072].
    {
        const int R = 8192, F = 3072;
        const long long n = 1ll * R * C, nf = 1ll * R * F;
        float* bias = buf(F, 0.01f);
        std::vector<Set> s = make_sets(sets_for((6 * n + 4 * nf) * 4), R, C, F, gamma, beta);
        const int ns = static_cast<int>(s.size());
        float* dg = buf(C, 0.0f);
        float* db = buf(C, 0.0f);
        float* dbias = buf(F, 0.0f);
        rec("headline_floor", [&](int k) {
                             const Set& f = s[k % ns];
                             const Set& b = s[(k + ns - 1) % ns];
                             copy(f.x, f.y, n);
                             copy(f.h, f.o, nf);
                             add(b.dy, b.x, b.dx, n);
                             empty(48);
                             add(b.h, b.dh, b.gin, nf);
                             empty(96);
                         }, 200 * scale);
        rec("headline_step", [&](int k) {
                             const Set& f = s[k % ns];
                             const Set& b = s[(k + ns - 1) % ns];
                             layernorm_forward_save(f.x, gamma, beta, f.y, f.mean, f.rstd, R, C);
                             bias_gelu_forward(f.h, bias, f.o, R, F);
                             layernorm_backward(b.dy, b.x, b.mean, b.rstd, gamma, b.dx, dg, db, R,
                                                C);
                             gelu_backward_with_bias_backward(b.h, bias, b.dh, b.gin, dbias, R,
                                                              F);
                         }, 200 * scale);
        free_sets(s);
        CK(hipFree(dg));
        CK(hipFree(db));
        CK(hipFree(dbias));
        CK(hipFree(bias));
    }
    // Config 3: GPT-2-small non-GEMM block x12, [8192, 768] / [8192, 3072], each layer
    // with its own inputs and outputs (as bench.py's block12 workload), one residual-
    // stream gradient shared by all layers.
    {
        const int R = 8192, F = 3072, L = 12;
        const long long n = 1ll * R * C, nf = 1ll * R * F;
        struct Layer {
            float *a, *m, *h, *gy1, *gy2, *gh;                    // inputs
            float *r1, *r2, *y1, *y2, *m1, *s1, *m2, *s2, *o, *gin;  // outputs
        };
        std::vector<Layer> ly(L);
        for (Layer& e : ly) {
            e.a = buf(n, 0.5f); e.m = buf(n, 0.25f); e.h = buf(nf, 0.1f);
            e.gy1 = buf(n, 0.3f); e.gy2 = buf(n, 0.2f); e.gh = buf(nf, 0.4f);
            e.r1 = buf(n, 0.0f); e.r2 = buf(n, 0.0f); e.y1 = buf(n, 0.0f); e.y2 = buf(n, 0.0f);
            e.m1 = buf(R, 0.0f); e.s1 = buf(R, 1.0f); e.m2 = buf(R, 0.0f); e.s2 = buf(R, 1.0f);
            e.o = buf(nf, 0.0f); e.gin = buf(nf, 0.0f);
        }
        float* r0 = buf(n, 0.1f);
        float* gres = buf(n, 0.0f);
        float* bias = buf(F, 0.01f);
        float* dg = buf(C, 0.0f);
        float* db = buf(C, 0.0f);
        float* dbias = buf(F, 0.0f);
        CK(hipDeviceSynchronize());
        rec("block12_floor", [&](int) {
            const float* r = r0;
            for (Layer& e : ly) {
                add2(r, e.a, e.r1, e.y1, n);
                add2(e.r1, e.m, e.r2, e.y2, n);
                copy(e.h, e.o, nf);
                r = e.r2;
            }
            for (int l = L - 1; l >= 0; --l) {
                Layer& e = ly[l];
                add(e.h, e.gh, e.gin, nf);
                empty(96);
                add3(e.gy2, e.r2, gres, n);
                empty(48);
                add3(e.gy1, e.r1, gres, n);
                empty(48);
            }
        }, 20 * scale);
        rec("block12_step", [&](int) {
            const float* r = r0;
            for (Layer& e : ly) {
                residual_layernorm_forward_save(r, e.a, gamma, beta, e.r1, e.y1, e.m1, e.s1, R,
                                                C);
                residual_layernorm_forward_save(e.r1, e.m, gamma, beta, e.r2, e.y2, e.m2, e.s2,
                                                R, C);
                bias_gelu_forward(e.h, bias, e.o, R, F);
                r = e.r2;
            }
            for (int l = L - 1; l >= 0; --l) {
                Layer& e = ly[l];
                gelu_backward_with_bias_backward(e.h, bias, e.gh, e.gin, dbias, R, F);
                layernorm_backward_residual(e.gy2, e.r2, e.m2, e.s2, gamma, gres, dg, db, R, C);
                layernorm_backward_residual(e.gy1, e.r1, e.m1, e.s1, gamma, gres, dg, db, R, C);
            }
        }, 20 * scale);
        CK(hipDeviceSynchronize());
        for (Layer& e : ly)
            for (float* p : {e.a, e.m, e.h, e.gy1, e.gy2, e.gh, e.r1, e.r2, e.y1, e.y2, e.m1,
                             e.s1, e.m2, e.s2, e.o, e.gin})
                CK(hipFree(p));
        for (float* p : {r0, gres, bias, dg, db, dbias}) CK(hipFree(p));
    }
    CK(hipFree(gamma));
    CK(hipFree(beta));

    std::printf("{");
    for (size_t i = 0; i < out.size(); ++i)
        std::printf("%s\"%s\": %.4f", i ? ", " : "", out[i].first.c_str(), out[i].second);
    std::printf("}\n");
    return 0;
}
