// Row softmax and softmax cross-entropy for gfx950.
//
// Reference behaviour: FINAL_CLEAN_CODE/src/kernels/activations.cu:394-532.
//  * softmax_forward (:394-435): out = e / sum with e = expf(x - max), one
//    block per row walking the row three times in global memory.
//  * cross_entropy_kernel (:438-477): p = e * (1 / (sum + 1e-9)),
//    loss = -logf(p[t] + 1e-9), grad = (p - onehot(t)) * scale; one 32-lane
//    warp per row.
//  * cross_entropy_forward (:479-499): scale 1; the per-row losses are
//    copied to the host and summed there in order; returns the mean.
//  * cross_entropy_forward_v2 (:517-532): scale 1 / batch; the mean loss
//    stays on the device (memset + atomicAdd tree + a divide kernel).
//
// Here a "row group" of G waves holds a row in registers (K elements per
// lane), so the row is read from HBM once and the output written once.  The
// row maximum and sum are wave reductions (DPP) combined across the G waves
// in a fixed order through LDS.  Rows longer than 65536 use a block-per-row
// kernel that streams the row three times, as the reference does.  The
// device mean loss is one single-workgroup reduction in a fixed order: no
// memset (graph-capture safe) and bitwise reproducible.
#include <cfloat>
#include <vector>

#include "mi_common.hpp"

namespace mi {

namespace {

constexpr float kCeEps = 1e-9f;  // activations.cu:461,470
constexpr float kLog2e = 1.4426950408889634f;

// Raw buffer resource over one row of `cols` floats (word 3 as for every
// gfx9 raw buffer: 32-bit data, no swizzle).  Loads past the end return 0 and
// stores past the end are dropped, which bounds the row in hardware.
constexpr int kBufWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const float* p, int cols) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), 0, cols * 4, kBufWord3);
}

// G waves per row, K elements per lane.  Workgroups hold 4 waves (4 / G
// rows) for G < 4, otherwise one row of G waves.
template <int G>
constexpr int sm_threads() {
    return (G < 4 ? 4 : G) * kWave;
}

template <int G, int K, bool CE>
__global__ __launch_bounds__(sm_threads<G>()) void row_softmax_kernel(
    const float* __restrict__ x, float* __restrict__ out, int rows, int cols,
    const int* __restrict__ targets, float* __restrict__ losses, float scale) {
    constexpr int GPB = G < 4 ? 4 / G : 1;  // row groups per workgroup
    constexpr int GT = G * kWave;            // lanes per row
    __shared__ float red_max[GPB][G];
    __shared__ float red_sum[GPB][G];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int grp = wave / G;
    const int wig = wave % G;
    const int t = wig * kWave + lane;
    const int row = blockIdx.x * GPB + grp;
    // Groups past the last row process a copy of the last row and store
    // nothing, so every wave reaches the barriers.
    const bool valid = row < rows;
    const int rr = valid ? row : rows - 1;
    const float* xr = x + static_cast<size_t>(rr) * cols;

    // Raw buffer loads bounded by the row length: slots past the end read 0
    // in hardware, so no index is clamped and every load shares one lane
    // offset (t * 4) plus a per-slot scalar offset.  Masked slots then take
    // -FLT_MAX, the reference's initial maximum, and give exp(.) = 0 below.
    const __amdgpu_buffer_rsrc_t rin = row_rsrc(xr, cols);
    float v[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const float a = __int_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(rin, t * 4, k * GT * 4, 0));
        v[k] = (t + k * GT) < cols ? a : -FLT_MAX;
    }
    float m = -FLT_MAX;
#pragma unroll
    for (int k = 0; k < K; ++k) m = fmaxf(m, v[k]);
    m = wave_max(m);
    if constexpr (G > 1) {
        if (lane == 0) red_max[grp][wig] = m;
        __syncthreads();
        m = red_max[grp][0];
#pragma unroll
        for (int w = 1; w < G; ++w) m = fmaxf(m, red_max[grp][w]);
    }

    // e = exp(x - m) as 2^(x log2 e - m log2 e) on v_exp_f32, the exponent
    // formed by one FMA.  The rounding of m log2 e scales every e of the row
    // by the same factor, which cancels in the normalisation; masked slots
    // (-FLT_MAX) give 2^-inf = 0.
    const float mL = m * kLog2e;
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const float e = __builtin_amdgcn_exp2f(fmaf(v[k], kLog2e, -mL));
        v[k] = e;
        s += e;
    }
    s = wave_sum(s);
    if constexpr (G > 1) {
        if (lane == 0) red_sum[grp][wig] = s;
        __syncthreads();
        s = red_sum[grp][0];
#pragma unroll
        for (int w = 1; w < G; ++w) s += red_sum[grp][w];
    }
    if (!valid) return;  // after the last barrier

    // Buffer stores past the row end are dropped in hardware.
    const __amdgpu_buffer_rsrc_t rout = row_rsrc(out + static_cast<size_t>(row) * cols, cols);
    if constexpr (!CE) {
        const float inv = 1.0f / s;
#pragma unroll
        for (int k = 0; k < K; ++k)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(v[k] * inv), rout, t * 4,
                                                  k * GT * 4, 0);
    } else {
        const float inv = 1.0f / (s + kCeEps);
        const int tgt = targets[row];
        float pt = 0.0f;
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const float p = v[k] * inv;
            const bool hit = (t + k * GT) == tgt;
            pt = hit ? p : pt;
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_int((hit ? p - 1.0f : p) * scale),
                                                  rout, t * 4, k * GT * 4, 0);
        }
        // One lane owns the target and writes the loss; an invalid target
        // gives NaN (written by lane 0 of the group).
        if (tgt >= 0 && tgt < cols) {
            if (tgt % GT == t) losses[row] = -logf(pt + kCeEps);
        } else if (t == 0) {
            losses[row] = __int_as_float(0x7fc00000);
        }
    }
}

// Block-per-row fallback for rows longer than the register-resident shapes:
// max, sum of exponentials and the output are three passes over the row.
constexpr int kLongThreads = 1024;

template <int NW>
__device__ __forceinline__ float block_reduce(float v, float* red, bool is_max) {
    v = is_max ? wave_max(v) : wave_sum(v);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) r = is_max ? fmaxf(r, red[i]) : r + red[i];
    __syncthreads();
    return r;
}

template <bool CE>
__global__ __launch_bounds__(kLongThreads) void long_row_softmax_kernel(
    const float* __restrict__ x, float* __restrict__ out, int cols,
    const int* __restrict__ targets, float* __restrict__ losses, float scale) {
    constexpr int NW = kLongThreads / kWave;
    __shared__ float red[NW];
    const int row = blockIdx.x;
    const float* xr = x + static_cast<size_t>(row) * cols;
    float* orow = out + static_cast<size_t>(row) * cols;
    float m = -FLT_MAX;
    for (int j = threadIdx.x; j < cols; j += kLongThreads) m = fmaxf(m, xr[j]);
    m = block_reduce<NW>(m, red, true);
    float s = 0.0f;
    for (int j = threadIdx.x; j < cols; j += kLongThreads) s += expf(xr[j] - m);
    s = block_reduce<NW>(s, red, false);
    if constexpr (!CE) {
        for (int j = threadIdx.x; j < cols; j += kLongThreads) orow[j] = expf(xr[j] - m) / s;
    } else {
        const float inv = 1.0f / (s + kCeEps);
        const int tgt = targets[row];
        if ((tgt < 0 || tgt >= cols) && threadIdx.x == 0) losses[row] = __int_as_float(0x7fc00000);
        for (int j = threadIdx.x; j < cols; j += kLongThreads) {
            float p = expf(xr[j] - m) * inv;
            if (j == tgt) {
                losses[row] = -logf(p + kCeEps);
                p -= 1.0f;
            }
            orow[j] = p * scale;
        }
    }
}

// Mean of n per-row losses into *out, in a fixed order: thread i sums
// elements i, i + 1024, ... sequentially, the waves reduce with DPP and the
// 16 wave totals are added in wave order.
__global__ __launch_bounds__(kLongThreads) void loss_mean_kernel(const float* __restrict__ losses,
                                                                 int n, float* __restrict__ out) {
    constexpr int NW = kLongThreads / kWave;
    __shared__ float red[NW];
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += kLongThreads) s += losses[i];
    s = wave_sum(s);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        float total = red[0];
#pragma unroll
        for (int i = 1; i < NW; ++i) total += red[i];
        *out = total / static_cast<float>(n);
    }
}

struct SmPlan {
    int G = 0, K = 0;  // G == 0: long-row kernel
};

SmPlan plan_softmax(int cols) {
    const int slots = (cols + kWave - 1) / kWave;  // lane slots for one wave
    if (slots <= 16) {
        int k = 1;
        while (k < slots) k *= 2;
        return {1, k};
    }
    if (cols <= 2 * kWave * 16) return {2, 16};
    if (cols <= 4 * kWave * 16) return {4, 16};
    if (cols <= 8 * kWave * 16) return {8, 16};
    for (int k = 16; k <= 64; k += 8)
        if (cols <= 16 * kWave * k) return {16, k};
    return {};
}

template <int G, int K, bool CE>
void launch_rows(int rows, int cols, hipStream_t st, const float* x, float* out, const int* tg,
                 float* losses, float scale) {
    constexpr int GPB = G < 4 ? 4 / G : 1;
    const dim3 grid(static_cast<unsigned>((static_cast<long long>(rows) + GPB - 1) / GPB));
    hipLaunchKernelGGL((row_softmax_kernel<G, K, CE>), grid, dim3(sm_threads<G>()), 0, st, x, out,
                       rows, cols, tg, losses, scale);
}

template <bool CE>
void launch_softmax(int rows, int cols, hipStream_t st, const float* x, float* out, const int* tg,
                    float* losses, float scale) {
    const SmPlan p = plan_softmax(cols);
#define MI_SM_CASE(GG, KK)                                                       \
    if (p.G == GG && p.K == KK) {                                                \
        launch_rows<GG, KK, CE>(rows, cols, st, x, out, tg, losses, scale);      \
        return;                                                                  \
    }
    MI_SM_CASE(1, 1)
    MI_SM_CASE(1, 2)
    MI_SM_CASE(1, 4)
    MI_SM_CASE(1, 8)
    MI_SM_CASE(1, 16)
    MI_SM_CASE(2, 16)
    MI_SM_CASE(4, 16)
    MI_SM_CASE(8, 16)
    MI_SM_CASE(16, 16)
    MI_SM_CASE(16, 24)
    MI_SM_CASE(16, 32)
    MI_SM_CASE(16, 40)
    MI_SM_CASE(16, 48)
    MI_SM_CASE(16, 56)
    MI_SM_CASE(16, 64)
#undef MI_SM_CASE
    hipLaunchKernelGGL((long_row_softmax_kernel<CE>), dim3(rows), dim3(kLongThreads), 0, st, x,
                       out, cols, tg, losses, scale);
}

int check_ce_args(const char* name, const float* logits, const int* targets, const float* grad,
                  int batch, int vocab) {
    if (batch < 0 || vocab <= 0)
        return set_error(MI_ERR_INVALID_ARG, "%s: invalid shape batch=%d vocab=%d", name, batch,
                         vocab);
    if (batch > 0 && (!logits || !targets || !grad))
        return set_error(MI_ERR_INVALID_ARG, "%s: NULL pointer", name);
    return MI_OK;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" {

int mi_softmax_forward(const float* x, float* out, int rows, int cols, void* stream) {
    const char* name = "mi_softmax_forward";
    if (rows < 0 || cols <= 0)
        return set_error(MI_ERR_INVALID_ARG, "%s: invalid shape rows=%d cols=%d", name, rows,
                         cols);
    if (rows == 0) return MI_OK;
    if (!x || !out) return set_error(MI_ERR_INVALID_ARG, "%s: NULL pointer", name);
    launch_softmax<false>(rows, cols, to_stream(stream), x, out, nullptr, nullptr, 1.0f);
    return check_launch(name);
}

int mi_cross_entropy_forward(const float* logits, const int* targets, float* grad, int batch,
                             int vocab, float* loss, void* stream) {
    const char* name = "mi_cross_entropy_forward";
    int rc = check_ce_args(name, logits, targets, grad, batch, vocab);
    if (rc != MI_OK) return rc;
    if (!loss) return set_error(MI_ERR_INVALID_ARG, "%s: NULL loss pointer", name);
    if (batch == 0) {
        *loss = 0.0f / static_cast<float>(batch);  // the reference's total / batch
        return MI_OK;
    }
    hipStream_t st = to_stream(stream);
    int err = MI_OK;
    char* ws = static_cast<char*>(
        workspace_get(colsum_part_offset() + static_cast<size_t>(batch) * sizeof(float), st, &err));
    if (!ws) return err;
    float* losses = reinterpret_cast<float*>(ws + colsum_part_offset());
    launch_softmax<true>(batch, vocab, st, logits, grad, targets, losses, 1.0f);
    rc = check_launch(name);
    if (rc != MI_OK) return rc;
    // As the reference: the per-row losses come back to the host and are
    // summed there in row order.
    std::vector<float> h(static_cast<size_t>(batch));
    hipError_t e = hipMemcpyAsync(h.data(), losses, h.size() * sizeof(float),
                                  hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess)
        return set_error(static_cast<int>(e), "%s: copying the losses failed: %s", name,
                         hipGetErrorString(e));
    float total = 0.0f;
    for (float l : h) total += l;
    *loss = total / static_cast<float>(batch);
    return MI_OK;
}

int mi_cross_entropy_forward_v2(const float* logits, const int* targets, float* grad,
                                float* losses, float* loss_out, int batch, int vocab,
                                void* stream) {
    const char* name = "mi_cross_entropy_forward_v2";
    int rc = check_ce_args(name, logits, targets, grad, batch, vocab);
    if (rc != MI_OK) return rc;
    if (!loss_out || (batch > 0 && !losses))
        return set_error(MI_ERR_INVALID_ARG, "%s: NULL pointer", name);
    hipStream_t st = to_stream(stream);
    if (batch > 0) {
        launch_softmax<true>(batch, vocab, st, logits, grad, targets, losses,
                             1.0f / static_cast<float>(batch));
        rc = check_launch(name);
        if (rc != MI_OK) return rc;
    }
    hipLaunchKernelGGL(loss_mean_kernel, dim3(1), dim3(kLongThreads), 0, st, losses, batch,
                       loss_out);
    return check_launch(name);
}

size_t mi_cross_entropy_workspace(int batch) {
    return batch > 0 ? colsum_part_offset() + static_cast<size_t>(batch) * sizeof(float) : 0;
}

}  // extern "C"
