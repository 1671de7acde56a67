// Caller-integration check: the non-GEMM call sequence of the reference's
// training step, issued through include/kernels.h exactly as
// FINAL_CLEAN_CODE/src/model/transformer.cu issues it:
//
//   forward  (transformer.cu:265-327): embedding_forward, pos_embedding_forward,
//            layernorm_forward_save (LN1), [QKV GEMM, attention, Wo GEMM],
//            residual_layernorm_forward_save (LN2), [W1 GEMM],
//            bias_relu_forward, [W2 GEMM], residual_add_with_bias;
//   backward (transformer.cu:475-584): [logits GEMM bwd], bias_backward (db2),
//            [W2 GEMM bwd], relu_backward_with_bias_backward (db1),
//            [W1 GEMM bwd], layernorm_backward_residual (LN2),
//            [Wo GEMM bwd, attention bwd, QKV GEMM bwd],
//            layernorm_backward_residual (LN1), embedding_backward,
//            pos_embedding_backward.
//
// Every bracketed GEMM / attention step is replaced by a fixed stand-in
// tensor that a small copy kernel writes where the GEMM would write its
// output.  With "gelu" the bias+ReLU pair is replaced by bias_gelu_forward /
// gelu_backward_with_bias_backward (the activation this library adds).  With
// "fp16" the reference's CME213_FP16_STORAGE_ONLY path runs instead
// (transformer.cu:293-324, 490-518): bias_relu_forward in place on
// ff_hidden, a float_to_half_buffer / half_to_float_buffer round trip
// through the half copy of the activation, half_to_float_buffer again at the
// start of the FFN backward, and relu_backward_with_bias_backward_half_mask
// with the half activation as the mask.
//
// Like main.cu:264-320 (CME213_USE_CUDA_GRAPH=1), three eager warm-up steps
// run first; then zero_grad + forward + backward is captured on the
// per-thread default stream into a graph and replayed.  zero_grad clears the
// flat gradient buffer with a fill kernel (graphs here must not record
// memsets).  Each replay, with host syncs and an eager step in between, must
// reproduce the eager step bit for bit.  The inputs and outputs of the eager
// step are written to DIR as raw little-endian arrays for the CPU oracle
// comparison in tests/test_gpu_transformer_nongemm.py.
//
// usage: transformer_nongemm DIR relu|gelu|fp16 [B T D FF V]
// exit status: 0 = ran and every replay matched, 1 = replay mismatch,
// 2 = HIP error or bad arguments.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "kernels.h"

extern "C" {
void orc_fill_pattern(float* v, long n, float scale, float shift);
}

#define HIPCHECK(x)                                                                  \
    do {                                                                             \
        hipError_t e_ = (x);                                                         \
        if (e_ != hipSuccess) {                                                      \
            std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_),   \
                         __FILE__, __LINE__);                                        \
            std::exit(2);                                                            \
        }                                                                            \
    } while (0)

__global__ void fill_zero_kernel(float* p, long n) {
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<long>(gridDim.x) * blockDim.x)
        p[i] = 0.0f;
}

__global__ void copy_kernel(const float* __restrict__ src, float* __restrict__ dst, long n) {
    for (long i = blockIdx.x * static_cast<long>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<long>(gridDim.x) * blockDim.x)
        dst[i] = src[i];
}

static unsigned grid_for(long n) {
    long g = (n + 255) / 256;
    return static_cast<unsigned>(g < 4096 ? (g < 1 ? 1 : g) : 4096);
}

struct Buf {
    std::string name;
    float* d = nullptr;
    long n = 0;
    bool output = false;  // written by the step (disturbed before each replay)
};

static std::vector<Buf*> g_all;

static Buf* make(const char* name, long n, bool output = true) {
    Buf* b = new Buf{name, nullptr, n, output};
    HIPCHECK(hipMalloc(&b->d, (n > 0 ? n : 1) * sizeof(float)));
    g_all.push_back(b);
    return b;
}

static Buf* make_pattern(const char* name, long n, float scale, float shift) {
    Buf* b = make(name, n, false);
    std::vector<float> h(n);
    orc_fill_pattern(h.data(), n, scale, shift);
    HIPCHECK(hipMemcpy(b->d, h.data(), n * sizeof(float), hipMemcpyHostToDevice));
    return b;
}

static std::vector<float> fetch(const Buf* b) {
    std::vector<float> h(b->n);
    HIPCHECK(hipMemcpy(h.data(), b->d, b->n * sizeof(float), hipMemcpyDeviceToHost));
    return h;
}

static void dump(const std::string& dir, const std::string& name, const void* p, size_t bytes) {
    const std::string path = dir + "/" + name + ".bin";
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f || std::fwrite(p, 1, bytes, f) != bytes) {
        std::fprintf(stderr, "cannot write %s\n", path.c_str());
        std::exit(2);
    }
    std::fclose(f);
}

int main(int argc, char** argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s DIR relu|gelu|fp16 [B T D FF V]\n", argv[0]);
        return 2;
    }
    const std::string dir = argv[1];
    const bool gelu = std::strcmp(argv[2], "gelu") == 0;
    const bool fp16 = std::strcmp(argv[2], "fp16") == 0;
    const int B = argc > 3 ? std::atoi(argv[3]) : 4;
    const int T = argc > 4 ? std::atoi(argv[4]) : 128;
    const int D = argc > 5 ? std::atoi(argv[5]) : 768;
    const int FF = argc > 6 ? std::atoi(argv[6]) : 4 * D;
    const int V = argc > 7 ? std::atoi(argv[7]) : 4096;
    if (B <= 0 || T <= 0 || D <= 0 || FF <= 0 || V <= 0) return 2;
    const int BT = B * T;
    std::printf("transformer non-GEMM sequence: %s B=%d T=%d D=%d FF=%d V=%d\n",
                gelu ? "gelu" : (fp16 ? "fp16" : "relu"), B, T, D, FF, V);

    // Parameters (fixed) and the flat gradient buffer (zero_grad clears it
    // in one pass, transformer.cu:260-263).
    Buf* tok_embed = make_pattern("tok_embed", static_cast<long>(V) * D, 0.02f, 0.0f);
    Buf* pos_embed = make_pattern("pos_embed", static_cast<long>(T) * D, 0.01f, 0.0f);
    Buf* ln1_g = make_pattern("ln1_gamma", D, 0.05f, 1.0f);
    Buf* ln1_b = make_pattern("ln1_beta", D, 0.02f, 0.0f);
    Buf* ln2_g = make_pattern("ln2_gamma", D, 0.04f, 1.0f);
    Buf* ln2_b = make_pattern("ln2_beta", D, 0.03f, 0.0f);
    Buf* b1 = make_pattern("b1", FF, 0.05f, 0.0f);
    Buf* b2 = make_pattern("b2", D, 0.05f, 0.0f);
    const long n_grads = static_cast<long>(V) * D + static_cast<long>(T) * D + 4L * D + FF + D;
    Buf* grads = make("all_grads", n_grads);
    float* dtok = grads->d;
    float* dpos = dtok + static_cast<long>(V) * D;
    float* dln1_g = dpos + static_cast<long>(T) * D;
    float* dln1_b = dln1_g + D;
    float* dln2_g = dln1_b + D;
    float* dln2_b = dln2_g + D;
    float* db1 = dln2_b + D;
    float* db2 = db1 + FF;

    // Tokens: a deterministic sequence that repeats every 300 positions, so
    // several positions share a table row.
    std::vector<int> h_tok(BT);
    for (int i = 0; i < BT; ++i)
        h_tok[i] = static_cast<int>((static_cast<long>(i % 300) * 7919 + 13) % V);
    int* d_tok = nullptr;
    HIPCHECK(hipMalloc(&d_tok, BT * sizeof(int)));
    HIPCHECK(hipMemcpy(d_tok, h_tok.data(), BT * sizeof(int), hipMemcpyHostToDevice));

    // Stand-ins for the GEMM / attention outputs.
    const long nD = static_cast<long>(BT) * D, nF = static_cast<long>(BT) * FF;
    Buf* s_attn_proj = make_pattern("s_attn_proj", nD, 0.8f, 0.0f);
    Buf* s_ff_hidden = make_pattern("s_ff_hidden", nF, 1.5f, 0.1f);
    Buf* s_ff_out = make_pattern("s_ff_out", nD, 0.6f, 0.0f);
    Buf* s_grad_res2 = make_pattern("s_grad_residual2", nD, 0.3f, 0.0f);
    Buf* s_grad_ff_act = make_pattern("s_grad_ff_act", nF, 0.2f, 0.0f);
    Buf* s_grad_ln2_out = make_pattern("s_grad_ln2_out", nD, 0.25f, 0.0f);
    Buf* s_grad_ln1_out = make_pattern("s_grad_ln1_out", nD, 0.15f, 0.0f);

    // Activations.
    Buf* embedded = make("embedded", nD);
    Buf* ln1_out = make("ln1_out", nD);
    Buf* ln1_mean = make("ln1_mean", BT);
    Buf* ln1_inv = make("ln1_inv_std", BT);
    Buf* attn_proj = make("attn_proj", nD);
    Buf* residual1 = make("residual1", nD);
    Buf* ln2_out = make("ln2_out", nD);
    Buf* ln2_mean = make("ln2_mean", BT);
    Buf* ln2_inv = make("ln2_inv_std", BT);
    Buf* ff_hidden = make("ff_hidden", nF);
    // fp16 storage: the activation lives in ff_hidden (in place) and in a
    // half copy (nF halves held in a float-sized buffer).
    Buf* ff_act = fp16 ? nullptr : make("ff_act", nF);
    Buf* ff_relu_half = fp16 ? make("ff_relu_half", (nF + 1) / 2) : nullptr;
    __half* act_half = fp16 ? reinterpret_cast<__half*>(ff_relu_half->d) : nullptr;
    Buf* ff_out = make("ff_out", nD);
    Buf* residual2 = make("residual2", nD);
    Buf* grad_res2 = make("grad_residual2", nD);
    Buf* grad_ff_act = make("grad_ff_act", nF);
    Buf* grad_ff_hidden = make("grad_ff_hidden", nF);
    Buf* grad_ln2_out = make("grad_ln2_out", nD);
    Buf* grad_ln1_out = make("grad_ln1_out", nD);

    hipStream_t st = hipStreamPerThread;
    auto gemm_standin = [&](const Buf* src, Buf* dst) {
        hipLaunchKernelGGL(copy_kernel, dim3(grid_for(src->n)), dim3(256), 0, st, src->d, dst->d,
                           src->n);
    };

    auto step = [&]() {
        hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(n_grads)), dim3(256), 0, st, grads->d,
                           n_grads);
        // forward
        embedding_forward(tok_embed->d, d_tok, embedded->d, BT, D);
        pos_embedding_forward(pos_embed->d, embedded->d, B, T, D);
        layernorm_forward_save(embedded->d, ln1_g->d, ln1_b->d, ln1_out->d, ln1_mean->d,
                               ln1_inv->d, BT, D);
        gemm_standin(s_attn_proj, attn_proj);
        residual_layernorm_forward_save(embedded->d, attn_proj->d, ln2_g->d, ln2_b->d,
                                        residual1->d, ln2_out->d, ln2_mean->d, ln2_inv->d, BT, D);
        gemm_standin(s_ff_hidden, ff_hidden);
        if (gelu) {
            bias_gelu_forward(ff_hidden->d, b1->d, ff_act->d, BT, FF);
        } else if (fp16) {
            bias_relu_forward(ff_hidden->d, b1->d, ff_hidden->d, BT, FF);
            float_to_half_buffer(ff_hidden->d, act_half, static_cast<int>(nF));
            half_to_float_buffer(act_half, ff_hidden->d, static_cast<int>(nF));
        } else {
            bias_relu_forward(ff_hidden->d, b1->d, ff_act->d, BT, FF);
        }
        gemm_standin(s_ff_out, ff_out);
        residual_add_with_bias(residual1->d, ff_out->d, b2->d, residual2->d, BT, D);
        // backward
        gemm_standin(s_grad_res2, grad_res2);
        if (fp16) half_to_float_buffer(act_half, ff_hidden->d, static_cast<int>(nF));
        bias_backward(grad_res2->d, db2, BT, D);
        gemm_standin(s_grad_ff_act, grad_ff_act);
        if (gelu)
            gelu_backward_with_bias_backward(ff_hidden->d, b1->d, grad_ff_act->d,
                                             grad_ff_hidden->d, db1, BT, FF);
        else if (fp16)
            relu_backward_with_bias_backward_half_mask(act_half, grad_ff_act->d,
                                                       grad_ff_hidden->d, db1, BT, FF);
        else
            relu_backward_with_bias_backward(ff_act->d, grad_ff_act->d, grad_ff_hidden->d, db1,
                                             BT, FF);
        gemm_standin(s_grad_ln2_out, grad_ln2_out);
        layernorm_backward_residual(grad_ln2_out->d, residual1->d, ln2_mean->d, ln2_inv->d,
                                    ln2_g->d, grad_res2->d, dln2_g, dln2_b, BT, D);
        gemm_standin(s_grad_ln1_out, grad_ln1_out);
        layernorm_backward_residual(grad_ln1_out->d, embedded->d, ln1_mean->d, ln1_inv->d,
                                    ln1_g->d, grad_res2->d, dln1_g, dln1_b, BT, D);
        embedding_backward(grad_res2->d, d_tok, dtok, BT, D);
        pos_embedding_backward(grad_res2->d, dpos, B, T, D);
    };

    // Three eager warm-up steps (main.cu:272,294), then the reference step.
    for (int i = 0; i < 3; ++i) step();
    step();
    HIPCHECK(hipStreamSynchronize(st));
    HIPCHECK(hipGetLastError());
    std::vector<std::vector<float>> eager;
    for (const Buf* b : g_all) eager.push_back(fetch(b));

    // Capture zero_grad + forward + backward on the per-thread stream.
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    HIPCHECK(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
    step();
    HIPCHECK(hipStreamEndCapture(st, &graph));
    HIPCHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));

    int mismatches = 0;
    for (int replay = 0; replay < 3; ++replay) {
        // Disturb every output first so that a replay which skipped a write
        // cannot pass by leaving the eager result in place.
        for (const Buf* b : g_all)
            if (b->output)
                hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(b->n)), dim3(256), 0, st,
                                   b->d, b->n);
        HIPCHECK(hipStreamSynchronize(st));
        HIPCHECK(hipGraphLaunch(exec, st));
        HIPCHECK(hipStreamSynchronize(st));
        for (size_t k = 0; k < g_all.size(); ++k) {
            const std::vector<float> h = fetch(g_all[k]);
            if (std::memcmp(h.data(), eager[k].data(), h.size() * sizeof(float)) != 0) {
                std::printf("  replay %d: %s differs from the eager step\n", replay,
                            g_all[k]->name.c_str());
                ++mismatches;
            }
        }
        step();  // eager work between replays
        HIPCHECK(hipStreamSynchronize(st));
    }
    std::printf("graph replays: %s\n", mismatches ? "MISMATCH" : "bit-identical to eager (3/3)");

    // Inputs and eager outputs for the oracle comparison.
    for (size_t k = 0; k < g_all.size(); ++k)
        dump(dir, g_all[k]->name, eager[k].data(), eager[k].size() * sizeof(float));
    dump(dir, "tokens", h_tok.data(), h_tok.size() * sizeof(int));
    const int shape[5] = {B, T, D, FF, V};
    dump(dir, "shape", shape, sizeof(shape));

    HIPCHECK(hipGraphExecDestroy(exec));
    HIPCHECK(hipGraphDestroy(graph));
    for (Buf* b : g_all) {
        HIPCHECK(hipFree(b->d));
        delete b;
    }
    HIPCHECK(hipFree(d_tok));
    return mismatches ? 1 : 0;
}
