// Second pass of the deterministic column reductions.
//
// The first pass (LN backward, bias / ReLU / GELU backward) leaves one
// partial row per workgroup in the workspace: part[p][c], p < P.  This
// kernel adds the P partials of every column in a fixed order and
// accumulates the total into the caller's gradient (the reference's `+=`
// contract, e.g. FINAL_CLEAN_CODE/src/kernels/layernorm.cu:266-267).
//
// Layout: one workgroup owns 64 consecutive columns (one per lane, so each
// partial row is read as a coalesced 256-byte segment); its 16 waves each
// sum a contiguous slice of the P partial rows sequentially, and wave 0
// adds the 16 slice totals in wave order.  The slice bounds depend only on
// P, so the association order, and hence every bit of the result, is fixed.
#include "mi_common.hpp"

namespace mi {

namespace {

constexpr int kFinWaves = 16;
constexpr int kChunk = 32;

__global__ __launch_bounds__(kFinWaves * kWave) void colsum_finalize_kernel(
    const float* __restrict__ part, int P, int ncols, float* __restrict__ out0, int split,
    float* __restrict__ out1) {
    __shared__ float tot[kFinWaves][kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int c = blockIdx.x * kWave + lane;
    const int p0 = static_cast<int>(static_cast<long long>(wave) * P / kFinWaves);
    const int p1 = static_cast<int>(static_cast<long long>(wave + 1) * P / kFinWaves);
    // All loads of a chunk are issued before the first add, so a wave waits
    // for one memory round trip per kChunk partial rows.
    float s = 0.0f;
    if (c < ncols) {
        const float* col = part + c;
        for (int pb = p0; pb < p1; pb += kChunk) {
            float v[kChunk];
#pragma unroll
            for (int k = 0; k < kChunk; ++k)
                v[k] = (pb + k < p1) ? col[static_cast<size_t>(pb + k) * ncols] : 0.0f;
#pragma unroll
            for (int k = 0; k < kChunk; ++k)
                if (pb + k < p1) s += v[k];
        }
    }
    tot[wave][lane] = s;
    __syncthreads();
    if (wave == 0 && c < ncols) {
        float t = tot[0][lane];
#pragma unroll
        for (int w = 1; w < kFinWaves; ++w) t += tot[w][lane];
        float* o = (c < split) ? (out0 + c) : (out1 + (c - split));
        *o = *o + t;
    }
}

}  // namespace

int launch_colsum_finalize(const float* part, int P, int ncols, float* out0, int split,
                           float* out1, hipStream_t stream) {
    if (ncols <= 0 || P <= 0) return MI_OK;
    const int grid = (ncols + kWave - 1) / kWave;
    hipLaunchKernelGGL(colsum_finalize_kernel, dim3(grid), dim3(kFinWaves * kWave), 0, stream,
                       part, P, ncols, out0, split, out1);
    return check_launch("colsum_finalize");
}

}  // namespace mi
