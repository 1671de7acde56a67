// LayerNorm forward / backward for gfx950.
//
// Reference behaviour: FINAL_CLEAN_CODE/src/kernels/layernorm.cu.  The
// reference runs one 256-thread block per row and walks the row three times
// from global memory (sum, variance, normalise); the backward re-reads
// grad_out and x a second time, column-strided, for dgamma / dbeta.
//
// Here:
//  * forward: one wave64 per row, the row held in registers as W-wide
//    vectors (W = 4 -> global_load_dwordx4), so x is read from HBM once;
//    mean and variance are two wave reductions over the registers.
//  * backward: a "row group" of G waves owns a row (G = 1 up to 2048
//    columns, 4 beyond); grad_out and x are read once per row.  dx is
//    written in the same pass, and each thread keeps running dgamma/dbeta
//    sums for the columns it owns across all rows its group visits.  At the
//    end the groups of a workgroup combine through LDS (fixed tree order)
//    and the workgroup writes one partial row; colsum_finalize adds the
//    partial rows in a fixed order.  No float atomics: bitwise reproducible.
//  * rows wider than the register-resident templates fall back to
//    block-per-row kernels that stream the row from global memory.
#include <climits>
#include <mutex>

#include "mi_common.hpp"

#ifndef MI_LN_BWD_MAX_BLOCKS
#define MI_LN_BWD_MAX_BLOCKS 256
#endif

namespace mi {

namespace {

#ifndef MI_LN_FWD_WAVES
#define MI_LN_FWD_WAVES 4
#endif
constexpr int kFwdWaves = MI_LN_FWD_WAVES;  // waves per forward workgroup
#ifndef MI_LN_FWD_GB_LDS
#define MI_LN_FWD_GB_LDS 1
#endif

// gamma and beta staged in LDS once per workgroup wherever a wave stores
// before it needs them (the residual form, or a second row): read from
// global memory after a store, they waited for that store (the
// vector-memory counter retires in order); LDS reads wait on their own
// counter.  Block x12 1986-1987 -> 1972-1974 us, block x48 8538-8544 ->
// 8395-8403 us, wide sweep 449.0-449.3 -> 447.8-448.2 us; at the headline
// shape (two rows of 3 vectors) it also beats holding them in registers
// (LN forward 11.64-11.77 -> 11.45-11.56 us by events, five A/B rounds).
template <int W, int N, int R, bool RESID>
__host__ __device__ constexpr bool ln_fwd_gb_lds() {
    return MI_LN_FWD_GB_LDS && (RESID || R > 1);
}
#ifndef MI_LN_BWD_WAVES
#define MI_LN_BWD_WAVES 8
#endif
constexpr int kBwdWaves = MI_LN_BWD_WAVES;  // waves per backward workgroup
constexpr int kBlockThreads = 256;  // generic block-per-row kernels

// ---------------------------------------------------------------------------
// Forward: each wave normalises R consecutive rows, held in registers.  All
// loads of those rows are issued first (column indices clamped into the row,
// masked slots zeroed afterwards), then each row is reduced and written.
// ---------------------------------------------------------------------------
template <int W, int N, int R, bool SAVE, bool RESID>
__global__ __launch_bounds__(kFwdWaves * kWave) void ln_fwd_wave_kernel(
    int rows, int cols, float eps, const float* __restrict__ a, const float* __restrict__ b,
    const float* __restrict__ gamma, const float* __restrict__ beta, float* __restrict__ resid_out,
    float* __restrict__ out, float* __restrict__ mean_out, float* __restrict__ rstd_out) {
    const int lane = threadIdx.x & (kWave - 1);
    const int row0 = (blockIdx.x * kFwdWaves + static_cast<int>(threadIdx.x / kWave)) * R;
    if (!ln_fwd_gb_lds<W, N, R, RESID>() && row0 >= rows) return;  // wave-uniform
    const int nv = cols / W;

    fvec<W> v[R][N];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int rr = row0 + r < rows ? row0 + r : rows - 1;
        const size_t base = static_cast<size_t>(rr) * cols;
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const int j = lane + k * kWave;
            const int jj = j < nv ? j : nv - 1;
            v[r][k] = sload<W>(a + base, jj);
            if constexpr (RESID) {
                const fvec<W> w = sload<W>(b + base, jj);
#pragma unroll
                for (int e = 0; e < W; ++e) v[r][k].v[e] = v[r][k].v[e] + w.v[e];
            }
        }
    }
    // Where a row's stores precede its gamma/beta reads (ln_fwd_gb_lds),
    // gamma and beta come from LDS, filled once per workgroup; waves past
    // the last row then stay to the barrier and store nothing.  Elsewhere
    // (one plain row per wave) they are read from global memory after the
    // statistics, with no store in front of them.
    constexpr bool kLds = ln_fwd_gb_lds<W, N, R, RESID>();
    [[maybe_unused]] float* sgb = nullptr;
    if constexpr (kLds) {
        extern __shared__ __align__(16) float lds_gb[];
        sgb = lds_gb;
        const int nv2 = 2 * nv;
        for (int i = threadIdx.x; i < nv2; i += kFwdWaves * kWave) {
            const fvec<W> g = i < nv ? vload<W>(gamma, i) : vload<W>(beta, i - nv);
            vstore<W>(sgb, i, g);
        }
        __syncthreads();
    }

#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = row0 + r;
        if (row >= rows) break;  // wave-uniform
        const size_t base = static_cast<size_t>(row) * cols;
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const bool ok = (lane + k * kWave) < nv;
            if constexpr (RESID) {
                if (ok) sstore<W>(resid_out + base, lane + k * kWave, v[r][k]);
            }
#pragma unroll
            for (int e = 0; e < W; ++e) v[r][k].v[e] = ok ? v[r][k].v[e] : 0.0f;
        }

        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < N; ++k)
#pragma unroll
            for (int e = 0; e < W; ++e) s += v[r][k].v[e];
        const float mean = wave_sum(s) / static_cast<float>(cols);

        float q = 0.0f;
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const bool ok = (lane + k * kWave) < nv;
#pragma unroll
            for (int e = 0; e < W; ++e) {
                const float d = ok ? (v[r][k].v[e] - mean) : 0.0f;
                q += d * d;
            }
        }
        const float var = wave_sum(q) / static_cast<float>(cols);
        const float rstd = 1.0f / sqrtf(var + eps);
        if constexpr (SAVE) {
            if (lane == 0) {
                mean_out[row] = mean;
                rstd_out[row] = rstd;
            }
        }

#pragma unroll
        for (int k = 0; k < N; ++k) {
            const int j = lane + k * kWave;
            if (j < nv) {
                const fvec<W> g = kLds ? vload<W>(sgb, j) : vload<W>(gamma, j);
                const fvec<W> bt = kLds ? vload<W>(sgb, nv + j) : vload<W>(beta, j);
                fvec<W> y;
#pragma unroll
                for (int e = 0; e < W; ++e)
                    y.v[e] = (v[r][k].v[e] - mean) * rstd * g.v[e] + bt.v[e];
                sstore<W>(out + base, j, y);
            }
        }
    }
}

// Sum over the block; every thread returns the same value.  `red` holds one
// float per wave.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
    const float w = wave_sum(v);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = w;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) t += red[i];
    __syncthreads();
    return t;
}

// Forward, one block per row, any width (streams the row three times).
template <bool SAVE, bool RESID>
__global__ __launch_bounds__(kBlockThreads) void ln_fwd_block_kernel(
    int rows, int cols, float eps, const float* __restrict__ a, const float* __restrict__ b,
    const float* __restrict__ gamma, const float* __restrict__ beta, float* __restrict__ resid_out,
    float* __restrict__ out, float* __restrict__ mean_out, float* __restrict__ rstd_out) {
    constexpr int NW = kBlockThreads / kWave;
    __shared__ float red[NW];
    const int row = blockIdx.x;
    const size_t base = static_cast<size_t>(row) * cols;
    const float* src = RESID ? resid_out + base : a + base;
    float s = 0.0f;
    for (int i = threadIdx.x; i < cols; i += kBlockThreads) {
        float r = a[base + i];
        if constexpr (RESID) {
            r = r + b[base + i];
            resid_out[base + i] = r;  // re-read below by this same thread
        }
        s += r;
    }
    const float mean = block_sum<NW>(s, red) / static_cast<float>(cols);
    float q = 0.0f;
    for (int i = threadIdx.x; i < cols; i += kBlockThreads) {
        const float d = src[i] - mean;
        q += d * d;
    }
    const float var = block_sum<NW>(q, red) / static_cast<float>(cols);
    const float rstd = 1.0f / sqrtf(var + eps);
    if constexpr (SAVE) {
        if (threadIdx.x == 0) {
            mean_out[row] = mean;
            rstd_out[row] = rstd;
        }
    }
    for (int i = threadIdx.x; i < cols; i += kBlockThreads)
        out[base + i] = (src[i] - mean) * rstd * gamma[i] + beta[i];
}

// ---------------------------------------------------------------------------
// Backward, G waves per row, NWV waves per workgroup (kBwdWaves; 4 for
// 4-wave rows of 4 vectors per lane; 16 for the residual-accumulate form
// at C <= 768 and at four waves per row up to C = 2048, see plan_bwd).
// Dynamic LDS for the final combine of the GPB = NWV / G row groups:
// GPB rows of 2*cols floats for the one-barrier combine (used for GPB >= 4
// when that fits in 64 KB, 128 KB for 16 groups), else (GPB/2) slots of
// 2*N*W*64*G floats for the binary tree.  With GPB = 2 the tree is a single
// step and measured faster ([32768, 4096]: 457.3 against 458.5 us per LN
// fwd+bwd step).
// ---------------------------------------------------------------------------
#ifndef MI_LN_BWD_FLAT_LDS
#define MI_LN_BWD_FLAT_LDS (64 * 1024)
#endif
constexpr size_t kFlatCombineLds = MI_LN_BWD_FLAT_LDS;

__host__ __device__ constexpr size_t ln_bwd_flat_lds(int gpb) {
    return gpb >= 16 ? 2 * kFlatCombineLds : kFlatCombineLds;
}

__host__ __device__ inline bool ln_bwd_flat_combine(int gpb, int cols) {
    return gpb >= 4 && static_cast<size_t>(gpb) * 2 * static_cast<size_t>(cols) *
                               sizeof(float) <= ln_bwd_flat_lds(gpb);
}

template <int W, int N, int G, bool ADD, int NWV>
__global__ __launch_bounds__(NWV * kWave) void ln_bwd_group_kernel(
    int rows, int cols, int nblk, const float* __restrict__ gout, const float* __restrict__ x,
    const float* __restrict__ gamma, float* __restrict__ gx, const float* __restrict__ mean,
    const float* __restrict__ rstd, float* __restrict__ part) {
    // Argument order: the first 14 dwords (rows .. mean) are preloaded into
    // SGPRs.  They hold everything the first row's loads and the loop's
    // hoisted addresses need (gx's base address is set up before the loop);
    // rstd is first read after the row's data loads are issued, and part at
    // the end, so their scalar loads are off the critical path.
    constexpr int GPB = NWV / G;  // row groups per workgroup
    constexpr int GT = G * kWave;       // threads per group
    extern __shared__ float lds[];
    __shared__ float red[2][NWV][2];

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int grp = wave / G;
    const int wig = wave % G;
    const int t = wig * kWave + lane;
    const int nv = cols / W;

    fvec<W> gm[N], ag[N], ab[N];
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const int j = t + k * GT;
        gm[k] = (j < nv) ? vload<W>(gamma, j) : vzero<W>();
        ag[k] = vzero<W>();
        ab[k] = vzero<W>();
    }

    // nblk = gridDim.x, passed (and preloaded) with the other arguments: read
    // through the dispatch it is a scalar load in front of the first row.
    const int stride = nblk * GPB;
    // One row's inputs.  Every load is unconditional (row and column indices
    // are clamped into the tensor, masked slots are zeroed after the load),
    // so the loads carry no branches.
    struct RowIn {
        fvec<W> go[N], xv[N];
        float mu, is;
    };
    auto load_row = [&](long long row, RowIn& d) {
        const int rr = row < rows ? static_cast<int>(row) : rows - 1;
        const size_t off = static_cast<size_t>(rr) * cols;
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const int j = t + k * GT;
            const int jj = j < nv ? j : nv - 1;
            d.go[k] = sload<W>(gout + off, jj);
            d.xv[k] = sload<W>(x + off, jj);
        }
        d.mu = mean[rr];
        d.is = rstd[rr];
    };
    auto process = [&](const RowIn& cur, long long row, int parity) {
        const bool valid = row < rows;
        const size_t off = static_cast<size_t>(valid ? row : 0) * cols;
        const float mu = cur.mu;
        const float is = cur.is;
        // Masked slots (past the row end, or a group with no row) get
        // go = 0, so they add exact zeros to every sum.
        fvec<W> go[N];
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const bool ok = valid && (t + k * GT) < nv;
#pragma unroll
            for (int e = 0; e < W; ++e) go[k].v[e] = ok ? cur.go[k].v[e] : 0.0f;
        }
        // The accumulated gradient's vectors (ADD), requested together once
        // the row's inputs have arrived (clamped, unconditional), so that the
        // row's stores wait for one round trip.  Loaded one by one in the
        // store loop, each load also waited for the previous vector's store
        // (the vector-memory counter retires in order): block x48 8339-8348
        // -> 8247-8257 us, block x12 unchanged (1936 us), same box, three
        // A/B rounds.
        [[maybe_unused]] fvec<W> acc_in[N];
        if constexpr (ADD) {
#pragma unroll
            for (int k = 0; k < N; ++k) {
                const int j = t + k * GT;
                acc_in[k] = sload<W>(gx + off, j < nv ? j : nv - 1);
            }
        }
        float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
        for (int k = 0; k < N; ++k)
#pragma unroll
            for (int e = 0; e < W; ++e) {
                const float xh = (cur.xv[k].v[e] - mu) * is;
                const float dh = go[k].v[e] * gm[k].v[e];
                s1 += dh;
                s2 += dh * xh;
            }
        float S1 = wave_sum(s1);
        float S2 = wave_sum(s2);
        if constexpr (G > 1) {
            // red alternates with the row parity, so the next row's writes
            // cannot race these reads.
            float(*r)[2] = red[parity];
            if (lane == 0) {
                r[wave][0] = S1;
                r[wave][1] = S2;
            }
            __syncthreads();
            const int w0 = grp * G;
            S1 = r[w0][0];
            S2 = r[w0][1];
#pragma unroll
            for (int i = 1; i < G; ++i) {
                S1 += r[w0 + i][0];
                S2 += r[w0 + i][1];
            }
        }
        const float m1 = S1 / static_cast<float>(cols);
        const float m2 = S2 / static_cast<float>(cols);

#pragma unroll
        for (int k = 0; k < N; ++k) {
#pragma unroll
            for (int e = 0; e < W; ++e) {
                const float xh = (cur.xv[k].v[e] - mu) * is;
                ag[k].v[e] += go[k].v[e] * xh;
                ab[k].v[e] += go[k].v[e];
            }
        }
        if (valid) {
            if constexpr (ADD) {
#pragma unroll
                for (int k = 0; k < N; ++k) consume(acc_in[k]);
            }
#pragma unroll
            for (int k = 0; k < N; ++k) {
                const int j = t + k * GT;
                if (j < nv) {
                    fvec<W> d;
                    if constexpr (ADD) d = acc_in[k];
#pragma unroll
                    for (int e = 0; e < W; ++e) {
                        const float xh = (cur.xv[k].v[e] - mu) * is;
                        const float dh = go[k].v[e] * gm[k].v[e];
                        const float dx = is * (dh - m1 - xh * m2);
                        if constexpr (ADD)
                            d.v[e] = d.v[e] + rounded(dx);
                        else
                            d.v[e] = dx;
                    }
                    sstore<W>(gx + off, j, d);
                }
            }
        }
    };

    // The trip count is uniform across the workgroup (groups past the last
    // row process a masked row), so the barriers in process() are reached by
    // every wave.  RF rows are loaded before the first is processed; rows
    // are still processed, and summed into ag/ab, in increasing order.  With
    // one wave per row (G = 1) one row in flight measured fastest ([8192,
    // 768]: 2 or 4 rows were 0.4-0.5 us slower).  With several waves per row
    // and at most 2 vectors per lane, two rows in flight were faster ([8192,
    // 1600]: 34.0 against 36.7 us; [32768, 1600]: 109.0 against 124.1 us);
    // with 4 vectors per lane the second row costs occupancy ([32768, 4096]:
    // 290 against 269 us).
    constexpr int RF = (G > 1 && N <= 2) ? 2 : 1;
    const int first = blockIdx.x * GPB;
    const unsigned iters = strided_trips(static_cast<unsigned>(first), static_cast<unsigned>(rows),
                                         static_cast<unsigned>(stride));
    // Row numbers are 64-bit: with rows near INT_MAX, row + r * stride may
    // exceed the int range for the masked tail.
    long long row = first + grp;
    // At least one trip: every launched workgroup has a row (the grid is at
    // most ceil(rows / GPB) workgroups), and a trip over masked rows only
    // adds zeros.  With a possible zero-trip path the compiler kept gamma's
    // loads outstanding past the loop and waited for every store (vmcnt(0))
    // before the combine below.
    unsigned i = 0;
    do {
        RowIn cur[RF];
#pragma unroll
        for (int r = 0; r < RF; ++r) load_row(row + r * stride, cur[r]);
#pragma unroll
        for (int r = 0; r < RF; ++r) process(cur[r], row + r * stride, static_cast<int>((i + r) & 1u));
        i += RF;
        row += static_cast<long long>(RF) * stride;
    } while (i < iters);

    // Combine the GPB groups' running sums in a fixed binary-tree order
    // (level h adds group g + h into group g, for h = GPB/2 ... 1).
    // Every width this instantiation handles (at most N*W*GT columns) may
    // fit the staging; then the choice needs no run-time test.
    constexpr bool kFlatAll = GPB >= 4 && static_cast<size_t>(GPB) * 2 * N * W * GT *
                                              sizeof(float) <= ln_bwd_flat_lds(GPB);
    if (kFlatAll || ln_bwd_flat_combine(GPB, cols)) {
        // One barrier: every group stages its sums as a [2*cols] row
        // (dgamma then dbeta) in LDS, then each thread finishes a few
        // columns of the partial row, adding the GPB staged values in the
        // tree order.  Bit-identical to the tree below, which it replaces
        // where the staging fits; the tree needs log2(GPB) barrier pairs
        // (at [8192, 768] the kernel ran 14.89 -> 14.59 us).
        float* mine = lds + static_cast<size_t>(grp) * 2 * cols;
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const int j = t + k * GT;
            if (j < nv) {
                vstore<W>(mine, j, ag[k]);
                vstore<W>(mine + cols, j, ab[k]);
            }
        }
        __syncthreads();
        float* prow = part + static_cast<size_t>(blockIdx.x) * 2 * cols;
        const int tot = 2 * cols;
        for (int c = threadIdx.x; c < tot; c += NWV * kWave) {
            float v[GPB];
#pragma unroll
            for (int gi = 0; gi < GPB; ++gi) v[gi] = lds[static_cast<size_t>(gi) * tot + c];
#pragma unroll
            for (int h = GPB / 2; h >= 1; h /= 2)
#pragma unroll
                for (int gi = 0; gi < h; ++gi) v[gi] = v[gi] + v[gi + h];
            prow[c] = v[0];
        }
        return;
    }
    constexpr int SLOT = 2 * N * W * GT;
#pragma unroll
    for (int h = GPB / 2; h >= 1; h /= 2) {
        if (grp >= h && grp < 2 * h) {
            float* s = lds + (grp - h) * SLOT;
#pragma unroll
            for (int k = 0; k < N; ++k)
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    s[((0 * N + k) * W + e) * GT + t] = ag[k].v[e];
                    s[((1 * N + k) * W + e) * GT + t] = ab[k].v[e];
                }
        }
        __syncthreads();
        if (grp < h) {
            const float* s = lds + grp * SLOT;
#pragma unroll
            for (int k = 0; k < N; ++k)
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    ag[k].v[e] += s[((0 * N + k) * W + e) * GT + t];
                    ab[k].v[e] += s[((1 * N + k) * W + e) * GT + t];
                }
        }
        __syncthreads();
    }
    if (grp == 0) {
        float* pg = part + static_cast<size_t>(blockIdx.x) * 2 * cols;
        float* pb = pg + cols;
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const int j = t + k * GT;
            if (j < nv) {
                vstore<W>(pg, j, ag[k]);
                vstore<W>(pb, j, ab[k]);
            }
        }
    }
}

// Backward, one block per row group, any width.  Each thread owns columns
// c = tid + i*256 and keeps its dgamma/dbeta running sums directly in the
// block's partial row (only this block touches it, so plain loads/stores).
template <bool ADD>
__global__ __launch_bounds__(kBlockThreads) void ln_bwd_block_kernel(
    int rows, int cols, float* __restrict__ part, const float* __restrict__ gout,
    const float* __restrict__ x, const float* __restrict__ mean, const float* __restrict__ rstd,
    const float* __restrict__ gamma, float* __restrict__ gx) {
    constexpr int NW = kBlockThreads / kWave;
    __shared__ float red[NW];
    float* pg = part + static_cast<size_t>(blockIdx.x) * 2 * cols;
    float* pb = pg + cols;
    for (int c = threadIdx.x; c < cols; c += kBlockThreads) {
        pg[c] = 0.0f;
        pb[c] = 0.0f;
    }
    // unsigned: row + gridDim.x may pass INT_MAX when rows is near it
    for (unsigned row = blockIdx.x; row < static_cast<unsigned>(rows); row += gridDim.x) {
        const size_t off = static_cast<size_t>(row) * cols;
        const float mu = mean[row];
        const float is = rstd[row];
        float s1 = 0.0f, s2 = 0.0f;
        for (int c = threadIdx.x; c < cols; c += kBlockThreads) {
            const float xh = (x[off + c] - mu) * is;
            const float dh = gout[off + c] * gamma[c];
            s1 += dh;
            s2 += dh * xh;
        }
        const float m1 = block_sum<NW>(s1, red) / static_cast<float>(cols);
        const float m2 = block_sum<NW>(s2, red) / static_cast<float>(cols);
        for (int c = threadIdx.x; c < cols; c += kBlockThreads) {
            const float g = gout[off + c];
            const float xh = (x[off + c] - mu) * is;
            const float dh = g * gamma[c];
            const float dx = is * (dh - m1 - xh * m2);
            if constexpr (ADD)
                gx[off + c] = gx[off + c] + rounded(dx);
            else
                gx[off + c] = dx;
            pg[c] = pg[c] + g * xh;
            pb[c] = pb[c] + g;
        }
    }
}

// ---------------------------------------------------------------------------
// Host dispatch.
// ---------------------------------------------------------------------------

// Smallest supported vectors-per-lane count >= need, or 0 if none.
int pick_n(int need) {
    static const int kN[] = {1, 2, 3, 4, 6, 8, 12, 16};
    for (int n : kN)
        if (n >= need) return n;
    return 0;
}

// Rows per wave of the forward kernel, from a sweep over rows x {768, 1600,
// 4096} on MI355X.  Two rows per wave measured faster for 6M-16M elements
// when there are at least 6144 rows ([8192, 768]: 9.2 against 9.6 us;
// [6144, 1600]: 14.6 against 16.5 us; [8192, 1600]: 18.4 against 21.2 us),
// and for 4096-wide rows from 8192 rows ([8192, 4096]: 48.1 against 50.4
// us; [32768, 4096]: 184.3 against 189.4 us); one row per wave elsewhere
// ([4096, 768]: 5.5 against 6.8 us; [4096, 1600]: 9.8 against 10.6 us;
// [12288, 1600]: 29.5 against 32.0 us; [65536, 768]: 67.4 against 70.5 us;
// [2048, 4096]: 12.9 against 14.5 us).
int fwd_rows_per_wave(int rows, int cols) {
    const long long elems = static_cast<long long>(rows) * cols;
    if (cols >= 4096) return rows >= 8192 ? 2 : 1;
    return (rows >= 6144 && elems >= (6ll << 20) && elems <= (16ll << 20)) ? 2 : 1;
}

template <int W, int R, bool SAVE, bool RESID>
void launch_fwd_wave(int n, hipStream_t st, const float* a, const float* b, const float* gamma,
                     const float* beta, float* ro, float* out, float* mo, float* so, int rows,
                     int cols, float eps) {
    const long long waves = (static_cast<long long>(rows) + R - 1) / R;
    const dim3 grid(static_cast<unsigned>((waves + kFwdWaves - 1) / kFwdWaves));
    const dim3 block(kFwdWaves * kWave);
#define MI_LN_FWD_CASE(NN)                                                                     \
    case NN:                                                                                   \
        hipLaunchKernelGGL((ln_fwd_wave_kernel<W, NN, R, SAVE, RESID>), grid, block,              \
                           (ln_fwd_gb_lds<W, NN, R, RESID>() ? 2 * cols * sizeof(float) : 0), st,    \
                           rows, cols, eps, a, b, gamma, beta, ro, out, mo, so);               \
        break;
    switch (n) {
        MI_LN_FWD_CASE(1)
        MI_LN_FWD_CASE(2)
        MI_LN_FWD_CASE(3)
        MI_LN_FWD_CASE(4)
        MI_LN_FWD_CASE(6)
        MI_LN_FWD_CASE(8)
        MI_LN_FWD_CASE(12)
        MI_LN_FWD_CASE(16)
        default:
            break;
    }
#undef MI_LN_FWD_CASE
}

template <bool SAVE, bool RESID>
int ln_forward_impl(const char* name, const float* a, const float* b, const float* gamma,
                    const float* beta, float* ro, float* out, float* mo, float* so, int rows,
                    int cols, float eps, hipStream_t st) {
    if (rows < 0 || cols <= 0)
        return set_error(MI_ERR_INVALID_ARG, "%s: invalid shape rows=%d cols=%d", name, rows,
                         cols);
    if (rows == 0) return MI_OK;
    if (!a || !gamma || !beta || !out || (RESID && (!b || !ro)) || (SAVE && (!mo || !so)))
        return set_error(MI_ERR_INVALID_ARG, "%s: NULL pointer", name);
    const bool vec4 = (cols % 4 == 0) && aligned16(a) && aligned16(gamma) && aligned16(beta) &&
                      aligned16(out) && (!RESID || (aligned16(b) && aligned16(ro)));
    const int W = vec4 ? 4 : 1;
    const int need = (cols / W + kWave - 1) / kWave;
    const int n = pick_n(need);
    if (n != 0) {
        const bool two = fwd_rows_per_wave(rows, cols) == 2;
        if (vec4 && two)
            launch_fwd_wave<4, 2, SAVE, RESID>(n, st, a, b, gamma, beta, ro, out, mo, so, rows,
                                               cols, eps);
        else if (vec4)
            launch_fwd_wave<4, 1, SAVE, RESID>(n, st, a, b, gamma, beta, ro, out, mo, so, rows,
                                               cols, eps);
        else if (two)
            launch_fwd_wave<1, 2, SAVE, RESID>(n, st, a, b, gamma, beta, ro, out, mo, so, rows,
                                               cols, eps);
        else
            launch_fwd_wave<1, 1, SAVE, RESID>(n, st, a, b, gamma, beta, ro, out, mo, so, rows,
                                               cols, eps);
    } else {
        hipLaunchKernelGGL((ln_fwd_block_kernel<SAVE, RESID>), dim3(rows), dim3(kBlockThreads), 0,
                           st, rows, cols, eps, a, b, gamma, beta, ro, out, mo, so);
    }
    return check_launch(name);
}

struct BwdPlan {
    int W = 1, N = 0, G = 1;  // N == 0: block-per-row fallback
    int waves = kBwdWaves;    // waves per workgroup
    int blocks = 0;
    size_t lds = 0;
};

BwdPlan plan_bwd(int rows, int cols, bool vec4, bool add) {
    BwdPlan p;
    p.W = vec4 ? 4 : 1;
    const int nv = cols / p.W;
    // N <= 6 keeps the combine LDS at or under 48 KB (G = 1: 4 slots of
    // 2*N*W*64 floats; G = 4: 1 slot of 2*N*W*256 floats; G = 8: one group
    // per workgroup, no combine) and the registers within budget (N = 8 with
    // W = 4 spills).  Wider rows use the block-per-row kernel.
    static const int kG[] = {1, 4, 8};
    static const int kMaxN[] = {6, 6, 6};
    static const int kN[] = {1, 2, 3, 4, 6};
    for (int gi = 0; gi < 3 && !p.N; ++gi) {
        const int g = kG[gi];
        const int need = (nv + g * kWave - 1) / (g * kWave);
        for (int n : kN)
            if (n >= need && n <= kMaxN[gi]) {
                p.N = n;
                p.G = g;
                break;
            }
    }
    if (p.N) {
        // Rows of 4 waves with 4 vectors per lane (C around 3-4K) run one row
        // group per 4-wave workgroup, 512 workgroups: no barrier couples two
        // groups' rows ([32768, 4096] LN backward + residual 356.6 against
        // 369.5 us with 8-wave workgroups of two groups; 1600-wide rows are
        // slower that way, 28.2 against 27.1 us at [4096, 1600]).
        // The residual-accumulate form runs 16-wave workgroups at one wave
        // per row with up to 3 vectors per lane (C <= 768) and at four waves
        // per row with up to 2 (C <= 2048): with its third input stream,
        // twice the waves per CU pay off (GPT-2-small block x12 2011.6 ->
        // 1988.1 us; GPT-2-XL-shaped block x48 8.80 -> 8.55 ms), where the
        // plain form is 0.7 us slower that way at [8192, 768].
        p.waves = (p.G == 4 && p.N == 4)                ? 4
                  : (add && ((p.G == 1 && p.N <= 3) || (p.G == 4 && p.N <= 2))) ? 16
                                                         : kBwdWaves;
        const int maxb = p.waves == 4 ? 2 * MI_LN_BWD_MAX_BLOCKS : MI_LN_BWD_MAX_BLOCKS;
        const int gpb = p.waves / p.G;
        const long long groups = (static_cast<long long>(rows) + gpb - 1) / gpb;
        p.blocks = static_cast<int>(groups < maxb ? groups : maxb);
        p.lds = ln_bwd_flat_combine(gpb, cols)
                    ? static_cast<size_t>(gpb) * 2 * cols * sizeof(float)
                    : static_cast<size_t>(gpb / 2) * 2 * p.N * p.W * p.G * kWave * sizeof(float);
    } else {
        p.blocks = rows < MI_LN_BWD_MAX_BLOCKS ? rows : MI_LN_BWD_MAX_BLOCKS;
    }
    if (p.blocks < 1) p.blocks = 1;
    return p;
}

template <int W, int N, int G, bool ADD>
void launch_bwd_group(const BwdPlan& p, hipStream_t st, const float* g, const float* x,
                      const float* m, const float* s, const float* gamma, float* gx, float* part,
                      int rows, int cols) {
    if constexpr (ADD && ((G == 1 && N <= 3) || (G == 4 && N <= 2))) {
        if (p.waves == 16) {
            hipLaunchKernelGGL((ln_bwd_group_kernel<W, N, G, ADD, 16>), dim3(p.blocks),
                               dim3(16 * kWave), p.lds, st, rows, cols, p.blocks, g, x, gamma,
                               gx, m, s, part);
            return;
        }
    }
    if constexpr (G == 4 && N == 4) {
        if (p.waves == 4) {
            hipLaunchKernelGGL((ln_bwd_group_kernel<W, N, G, ADD, 4>), dim3(p.blocks),
                               dim3(4 * kWave), p.lds, st, rows, cols, p.blocks, g, x, gamma,
                               gx, m, s, part);
            return;
        }
    }
    hipLaunchKernelGGL((ln_bwd_group_kernel<W, N, G, ADD, kBwdWaves>), dim3(p.blocks),
                       dim3(kBwdWaves * kWave), p.lds, st, rows, cols, p.blocks, g, x, gamma,
                       gx, m, s, part);
}

template <int W, int G, bool ADD>
void dispatch_bwd_n(const BwdPlan& p, hipStream_t st, const float* g, const float* x,
                    const float* m, const float* s, const float* gamma, float* gx, float* part,
                    int rows, int cols) {
    switch (p.N) {
        case 1: launch_bwd_group<W, 1, G, ADD>(p, st, g, x, m, s, gamma, gx, part, rows, cols); break;
        case 2: launch_bwd_group<W, 2, G, ADD>(p, st, g, x, m, s, gamma, gx, part, rows, cols); break;
        case 3: launch_bwd_group<W, 3, G, ADD>(p, st, g, x, m, s, gamma, gx, part, rows, cols); break;
        case 4: launch_bwd_group<W, 4, G, ADD>(p, st, g, x, m, s, gamma, gx, part, rows, cols); break;
        case 6: launch_bwd_group<W, 6, G, ADD>(p, st, g, x, m, s, gamma, gx, part, rows, cols); break;
        default: break;
    }
}

template <int W, bool ADD>
void dispatch_bwd_g(const BwdPlan& p, hipStream_t st, const float* g, const float* x,
                    const float* m, const float* s, const float* gamma, float* gx, float* part,
                    int rows, int cols) {
    switch (p.G) {
        case 1: dispatch_bwd_n<W, 1, ADD>(p, st, g, x, m, s, gamma, gx, part, rows, cols); break;
        case 4: dispatch_bwd_n<W, 4, ADD>(p, st, g, x, m, s, gamma, gx, part, rows, cols); break;
        case 8: dispatch_bwd_n<W, 8, ADD>(p, st, g, x, m, s, gamma, gx, part, rows, cols); break;
        default: break;
    }
}

size_t bwd_workspace(const BwdPlan& p, int cols) { return colsum_bytes(p.blocks, 2 * cols); }

// Argument checks shared by the backward entry points; *done is set when the
// call is an empty no-op.
int ln_backward_check(const char* name, const float* g, const float* x, const float* m,
                      const float* s, const float* gamma, const float* gx, const float* dgamma,
                      const float* dbeta, int rows, int cols, bool* done) {
    *done = false;
    if (rows < 0 || cols <= 0)
        return set_error(MI_ERR_INVALID_ARG, "%s: invalid shape rows=%d cols=%d", name, rows,
                         cols);
    if (rows == 0) {
        *done = true;
        return MI_OK;
    }
    if (!g || !x || !m || !s || !gamma || !gx || !dgamma || !dbeta)
        return set_error(MI_ERR_INVALID_ARG, "%s: NULL pointer", name);
    return MI_OK;
}

bool ln_backward_vec4(const float* g, const float* x, const float* gamma, const float* gx,
                      int cols) {
    return (cols % 4 == 0) && aligned16(g) && aligned16(x) && aligned16(gamma) && aligned16(gx);
}

// Launches the backward's main pass and its column-sum finalize with the
// partial rows at `part` (at least p.blocks * 2 * cols floats).
template <bool ADD>
int ln_backward_launch(const char* name, const BwdPlan& p, const float* g, const float* x,
                       const float* m, const float* s, const float* gamma, float* gx,
                       float* dgamma, float* dbeta, float* part, int rows, int cols,
                       hipStream_t st) {
    if (p.N) {
        if (p.W == 4)
            dispatch_bwd_g<4, ADD>(p, st, g, x, m, s, gamma, gx, part, rows, cols);
        else
            dispatch_bwd_g<1, ADD>(p, st, g, x, m, s, gamma, gx, part, rows, cols);
    } else {
        hipLaunchKernelGGL((ln_bwd_block_kernel<ADD>), dim3(p.blocks), dim3(kBlockThreads), 0, st,
                           rows, cols, part, g, x, m, s, gamma, gx);
    }
    int rc = check_launch(name);
    if (rc != MI_OK) return rc;
    return launch_colsum_finalize(part, p.blocks, 2 * cols, dgamma, cols, dbeta, st);
}

template <bool ADD>
int ln_backward_impl(const char* name, const float* g, const float* x, const float* m,
                     const float* s, const float* gamma, float* gx, float* dgamma, float* dbeta,
                     int rows, int cols, hipStream_t st) {
    bool done = false;
    if (int rc = ln_backward_check(name, g, x, m, s, gamma, gx, dgamma, dbeta, rows, cols, &done))
        return rc;
    if (done) return MI_OK;
    const BwdPlan p = plan_bwd(rows, cols, ln_backward_vec4(g, x, gamma, gx, cols), ADD);
    int err = MI_OK;
    char* ws = static_cast<char*>(workspace_get(bwd_workspace(p, cols), st, &err));
    if (!ws) return err;
    float* part = reinterpret_cast<float*>(ws + colsum_part_offset());
    return ln_backward_launch<ADD>(name, p, g, x, m, s, gamma, gx, dgamma, dbeta, part, rows,
                                   cols, st);
}

// ---------------------------------------------------------------------------
// Allocation-free LayerNorm backward.  Its partial rows live in `scratch`, a
// file-scope device array of fixed size (each device the library runs on
// holds its own copy until the process ends).  Host code never passes the
// array's name to a kernel: in host code that name is a host-side stand-in,
// not a device address.  The device address of the current device's copy is
// looked up once per device with hipGetSymbolAddress and cached.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = MI_LN_BWD_NOALLOC_MAX_BYTES;
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};

int scratch_address(const char* name, char** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return set_error(static_cast<int>(e), "%s: hipGetDevice failed: %s", name,
                         hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxScratchDevices)
        return set_error(MI_ERR_INVALID_ARG, "%s: device %d out of range", name, dev);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr)
            return set_error(e != hipSuccess ? static_cast<int>(e) : MI_ERR_INVALID_ARG,
                             "%s: hipGetSymbolAddress(scratch) failed: %s", name,
                             hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = static_cast<char*>(g_scratch_ptr[dev]);
    return MI_OK;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" {

size_t mi_layernorm_backward_workspace(int rows, int cols) {
    if (rows <= 0 || cols <= 0) return 0;
    // The vec4 and scalar plans, plain and residual-accumulate, can differ;
    // report the largest.
    size_t most = 0;
    for (int add = 0; add < 2; ++add)
        for (int v4 = 0; v4 < 2; ++v4) {
            const size_t b = bwd_workspace(plan_bwd(rows, cols, v4 && cols % 4 == 0, add), cols);
            if (b > most) most = b;
        }
    return most;
}

int mi_layernorm_forward(const float* x, const float* gamma, const float* beta, float* out,
                         int rows, int cols, float eps, void* stream) {
    return ln_forward_impl<false, false>("mi_layernorm_forward", x, nullptr, gamma, beta, nullptr,
                                         out, nullptr, nullptr, rows, cols, eps,
                                         to_stream(stream));
}

int mi_layernorm_forward_save(const float* x, const float* gamma, const float* beta, float* out,
                              float* mean, float* inv_std, int rows, int cols, float eps,
                              void* stream) {
    return ln_forward_impl<true, false>("mi_layernorm_forward_save", x, nullptr, gamma, beta,
                                        nullptr, out, mean, inv_std, rows, cols, eps,
                                        to_stream(stream));
}

int mi_residual_layernorm_forward_save(const float* a, const float* b, const float* gamma,
                                       const float* beta, float* residual_out, float* out,
                                       float* mean, float* inv_std, int rows, int cols, float eps,
                                       void* stream) {
    return ln_forward_impl<true, true>("mi_residual_layernorm_forward_save", a, b, gamma, beta,
                                       residual_out, out, mean, inv_std, rows, cols, eps,
                                       to_stream(stream));
}

int mi_layernorm_backward(const float* grad_out, const float* x, const float* mean,
                          const float* inv_std, const float* gamma, float* grad_x, float* dgamma,
                          float* dbeta, int rows, int cols, void* stream) {
    return ln_backward_impl<false>("mi_layernorm_backward", grad_out, x, mean, inv_std, gamma,
                                   grad_x, dgamma, dbeta, rows, cols, to_stream(stream));
}

int mi_layernorm_backward_residual(const float* grad_out, const float* x, const float* mean,
                                   const float* inv_std, const float* gamma, float* grad_residual,
                                   float* dgamma, float* dbeta, int rows, int cols,
                                   void* stream) {
    return ln_backward_impl<true>("mi_layernorm_backward_residual", grad_out, x, mean, inv_std,
                                  gamma, grad_residual, dgamma, dbeta, rows, cols,
                                  to_stream(stream));
}

int mi_layernorm_backward_noalloc(const float* grad_out, const float* x, const float* mean,
                                  const float* inv_std, const float* gamma, float* grad_x,
                                  float* dgamma, float* dbeta, int rows, int cols,
                                  void* stream) {
    const char* name = "mi_layernorm_backward_noalloc";
    bool done = false;
    if (int rc = ln_backward_check(name, grad_out, x, mean, inv_std, gamma, grad_x, dgamma, dbeta,
                                   rows, cols, &done))
        return rc;
    if (done) return MI_OK;
    const BwdPlan p =
        plan_bwd(rows, cols, ln_backward_vec4(grad_out, x, gamma, grad_x, cols), false);
    const size_t need = bwd_workspace(p, cols);
    if (need > kScratchBytes)
        return set_error(MI_ERR_INVALID_ARG,
                         "%s: rows=%d cols=%d need %zu bytes of scratch, more than the static "
                         "%zu; use mi_layernorm_backward",
                         name, rows, cols, need, kScratchBytes);
    char* base = nullptr;
    if (int rc = scratch_address(name, &base)) return rc;
    float* part = reinterpret_cast<float*>(base + colsum_part_offset());
    return ln_backward_launch<false>(name, p, grad_out, x, mean, inv_std, gamma, grad_x, dgamma,
                                     dbeta, part, rows, cols, to_stream(stream));
}

}  // extern "C"
