// Second pass of the deterministic column reductions.
//
// The first pass (LN backward, bias / ReLU / GELU backward) leaves one
// partial row per workgroup in the workspace: part[p][c], p < P.  This
// kernel adds the P partials of every column in a fixed order and
// accumulates the total into the caller's gradient (the reference's `+=`
// contract, e.g. FINAL_CLEAN_CODE/src/kernels/layernorm.cu:266-267).
//
// Layout: one workgroup owns kFinCols consecutive columns; its threads are
// split into kFinSlices row slices, each summing a contiguous slice of the P
// partial rows sequentially, and the first slice adds the slice totals in
// slice order.  The slice bounds depend only on P, so the association order,
// and hence every bit of the result, is fixed.
//
// The kernel is latency-bound (one round trip for the partial rows, one for
// the store).  Measured in the headline step on MI355X (two finalizes per
// step, 256 partial rows of 1536 and 3072 columns): 512-thread workgroups of
// 32 columns x 16 slices 113.5 us per step; 1024 x (64 x 16) 114.3 us;
// 512 x (64 x 8) 114.1 us; 256 x (16 x 16) 113.9 us; 512 x (16 x 32)
// 114.2 us; 1024 x (128 x 8) 115.2 us; 256 x (64 x 4), two round trips per
// slice, 116.3 us.  Four adjacent columns per thread (16-byte loads, a
// quarter of the workgroups) measured 1.1 us slower per finalize.
#include "mi_common.hpp"

namespace mi {

namespace {

#ifndef MI_FIN_WAVES
#define MI_FIN_WAVES 8
#endif
#ifndef MI_FIN_COLS
#define MI_FIN_COLS 32
#endif
constexpr int kFinWaves = MI_FIN_WAVES;
constexpr int kFinThreads = kFinWaves * kWave;
constexpr int kFinCols = MI_FIN_COLS;                 // columns per workgroup
constexpr int kFinSlices = kFinThreads / kFinCols;    // row slices per workgroup
constexpr int kChunk = 32;

__global__ __launch_bounds__(kFinThreads) void colsum_finalize_kernel(
    const float* __restrict__ part, int P, int ncols, float* __restrict__ out0, int split,
    float* __restrict__ out1) {
    __shared__ float tot[kFinSlices][kFinCols];
    const int cl = threadIdx.x % kFinCols;
    const int slice = threadIdx.x / kFinCols;
    const int c = blockIdx.x * kFinCols + cl;
    const int p0 = static_cast<int>(static_cast<long long>(slice) * P / kFinSlices);
    const int p1 = static_cast<int>(static_cast<long long>(slice + 1) * P / kFinSlices);
    // The accumulated output's old value is loaded first, so its round trip
    // overlaps the partial-row loads instead of following the LDS combine.
    float* o = nullptr;
    float old = 0.0f;
    if (slice == 0 && c < ncols) {
        o = (c < split) ? (out0 + c) : (out1 + (c - split));
        old = *o;
    }
    // All loads of a chunk are issued before the first add, so a thread waits
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
    tot[slice][cl] = s;
    __syncthreads();
    if (slice == 0 && c < ncols) {
        float t = tot[0][cl];
#pragma unroll
        for (int w = 1; w < kFinSlices; ++w) t += tot[w][cl];
        *o = old + t;
    }
}

}  // namespace

int launch_colsum_finalize(const float* part, int P, int ncols, float* out0, int split,
                           float* out1, hipStream_t stream) {
    if (ncols <= 0 || P <= 0) return MI_OK;
    const int grid = (ncols + kFinCols - 1) / kFinCols;
    hipLaunchKernelGGL(colsum_finalize_kernel, dim3(grid), dim3(kFinThreads), 0, stream,
                       part, P, ncols, out0, split, out1);
    return check_launch("colsum_finalize");
}

}  // namespace mi
