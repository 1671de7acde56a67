// Token + position embedding for gfx950.
//
// Reference behaviour: FINAL_CLEAN_CODE/src/kernels/embedding.cu (gather,
// in-place position add, float-atomic scatter-add backward) and the CPU
// loops of NEW_code/tests/test_embedding.cu:16-41.
//
// Forward: one wave per token row, W-wide vector copies; the fused variant
// writes table[id] + pos[t] in one pass (one fp32 add, so bit-identical to
// the reference's gather followed by its in-place add).
//
// Token backward, deterministic and bit-identical to the CPU loop, which
// adds grad rows into grad_table in increasing token position:
//   1. keys = ids (invalid ids -> a sentinel that sorts last), vals = i;
//   2. stable LSD radix sort of (key, val), 8-bit digits, only as many
//      passes as the key range needs.  Each pass: per-tile digit histogram
//      (256-element tiles, LDS integer counters), a scan over tiles per
//      digit, and a stable scatter where one wave ranks its tile's
//      elements 64 at a time in index order (ballot-based digit match +
//      popcount).  Pass 0 reads the ids themselves;
//   3. one wave per run of equal keys: load grad_table[key] once, add the
//      run's grad rows in sorted (= increasing i) order, store once.
// Position backward: one thread per (t, column vector) adds grad_out[b, t]
// for b = 0, 1, ... in order onto grad_pos[t].
#include "mi_common.hpp"

namespace mi {

namespace {

constexpr int kRowWaves = 4;   // token rows per workgroup
constexpr int kTile = 256;     // radix tile: 4 batches of 64, one wave
constexpr int kDigits = 256;
constexpr unsigned kSentinel = 0xFFFFFFFFu;
static_assert(kTile == kDigits, "radix_hist_kernel uses one thread per digit and per element");
static_assert(kDigits == 4 * kWave, "radix_scatter_kernel scans four digit totals per lane");

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
template <int W, bool POS>
__global__ __launch_bounds__(kRowWaves * kWave) void emb_fwd_kernel(
    const float* __restrict__ table, const float* __restrict__ pos, const int* __restrict__ tokens,
    float* __restrict__ out, int batch_seq, int seq, int dim, int vocab) {
    const int lane = threadIdx.x & (kWave - 1);
    const int i = blockIdx.x * kRowWaves + static_cast<int>(threadIdx.x / kWave);
    if (i >= batch_seq) return;
    const int id = tokens[i];
    const bool ok = vocab <= 0 || (id >= 0 && id < vocab);
    const int nv = dim / W;
    const float* src = table + static_cast<size_t>(ok ? id : 0) * dim;
    const float* p = POS ? pos + static_cast<size_t>(i % seq) * dim : nullptr;
    float* dst = out + static_cast<size_t>(i) * dim;
#pragma unroll 4
    for (int j = lane; j < nv; j += kWave) {
        fvec<W> v = ok ? vload<W>(src, j) : vzero<W>();
        if constexpr (POS) {
            const fvec<W> q = vload<W>(p, j);
#pragma unroll
            for (int e = 0; e < W; ++e) v.v[e] = v.v[e] + q.v[e];
        }
        sstore<W>(dst, j, v);  // streamed out: measured 20.9 -> 16.0 us at config 2
    }
}

// embeddings[b, t, :] += pos[t, :], one wave per row.
template <int W>
__global__ __launch_bounds__(kRowWaves * kWave) void pos_add_kernel(const float* __restrict__ pos,
                                                                    float* __restrict__ emb,
                                                                    int rows, int seq, int dim) {
    const int lane = threadIdx.x & (kWave - 1);
    const int i = blockIdx.x * kRowWaves + static_cast<int>(threadIdx.x / kWave);
    if (i >= rows) return;
    const int nv = dim / W;
    const float* p = pos + static_cast<size_t>(i % seq) * dim;
    float* dst = emb + static_cast<size_t>(i) * dim;
#pragma unroll 4
    for (int j = lane; j < nv; j += kWave) {
        fvec<W> v = vload<W>(dst, j);
        const fvec<W> q = vload<W>(p, j);
#pragma unroll
        for (int e = 0; e < W; ++e) v.v[e] = v.v[e] + q.v[e];
        vstore<W>(dst, j, v);
    }
}

// grad_pos[t, j] += grad_out[b, t, j] for b = 0..batch-1 in order.
template <int W>
__global__ __launch_bounds__(256) void pos_bwd_kernel(const float* __restrict__ g,
                                                      float* __restrict__ gpos, int batch,
                                                      int seq, int dim) {
    const int nv = dim / W;
    const long long idx = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= static_cast<long long>(seq) * nv) return;
    const int t = static_cast<int>(idx / nv);
    const int j = static_cast<int>(idx % nv);
    const size_t row_stride = static_cast<size_t>(seq) * nv;  // in vectors
    const size_t base = static_cast<size_t>(t) * nv + j;
    fvec<W> acc = vload<W>(gpos, base);
    int b = 0;
    for (; b + 4 <= batch; b += 4) {
        fvec<W> q[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) q[u] = vload<W>(g, base + (b + u) * row_stride);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < W; ++e) acc.v[e] = acc.v[e] + q[u].v[e];
    }
    for (; b < batch; ++b) {
        const fvec<W> q = vload<W>(g, base + b * row_stride);
#pragma unroll
        for (int e = 0; e < W; ++e) acc.v[e] = acc.v[e] + q.v[e];
    }
    vstore<W>(gpos, base, acc);
}

// ---------------------------------------------------------------------------
// Stable LSD radix sort of (key, val) pairs.  Pass 0 reads the token ids
// directly (key = id, or the sentinel for an invalid id; val = position).
// ---------------------------------------------------------------------------
__device__ __forceinline__ unsigned token_key(int id, int vocab) {
    const bool ok = id >= 0 && (vocab <= 0 || id < vocab);
    return ok ? static_cast<unsigned>(id) : kSentinel;
}

// hist[d * ntiles + tile] = number of keys of the tile whose digit is d.
// One 256-thread workgroup per tile, one element per thread.
__global__ __launch_bounds__(kTile) void radix_hist_kernel(const unsigned* __restrict__ keys,
                                                           const int* __restrict__ ids, int vocab,
                                                           int n, int shift, int ntiles,
                                                           int* __restrict__ hist) {
    __shared__ int cnt[kDigits];
    cnt[threadIdx.x] = 0;
    __syncthreads();
    const int e = blockIdx.x * kTile + threadIdx.x;
    if (e < n) {
        const unsigned key = ids ? token_key(ids[e], vocab) : keys[e];
        atomicAdd(&cnt[(key >> shift) & (kDigits - 1)], 1);
    }
    __syncthreads();
    hist[threadIdx.x * ntiles + blockIdx.x] = cnt[threadIdx.x];
}

// Per-digit scan over tiles: hist[d * ntiles + t] becomes the number of
// digit-d keys in tiles before t, and total[d] the number of digit-d keys.
// One 256-thread workgroup per digit (the row of one digit is contiguous).
__global__ __launch_bounds__(256) void digit_scan_kernel(int* __restrict__ hist,
                                                         int* __restrict__ total, int ntiles) {
    __shared__ int wsum[4];
    __shared__ int carry_s;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    int* h = hist + static_cast<size_t>(blockIdx.x) * ntiles;
    if (threadIdx.x == 0) carry_s = 0;
    __syncthreads();
    for (int base = 0; base < ntiles; base += 256) {
        const int i = base + threadIdx.x;
        const int v = i < ntiles ? h[i] : 0;
        int x = v;  // inclusive scan over the wave
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            const int y = __shfl_up(x, off, kWave);
            if (lane >= off) x += y;
        }
        if (lane == kWave - 1) wsum[wave] = x;
        __syncthreads();
        int before = carry_s;
        for (int w = 0; w < wave; ++w) before += wsum[w];
        if (i < ntiles) h[i] = before + x - v;
        __syncthreads();
        if (threadIdx.x == 255) carry_s = before + x;
        __syncthreads();
    }
    if (threadIdx.x == 0) total[blockIdx.x] = carry_s;
}

// Stable scatter of one tile (kTile elements, 64 at a time in index order)
// by one wave.  The output position of digit d starts at
// (number of keys with a smaller digit) + offs[d * ntiles + tile]; the first
// term is an exclusive scan of the 256 digit totals, done by the wave (four
// digits per lane).
__global__ __launch_bounds__(kWave) void radix_scatter_kernel(
    const unsigned* __restrict__ kin, const int* __restrict__ vin, const int* __restrict__ ids,
    int vocab, unsigned* __restrict__ kout, int* __restrict__ vout, int n, int shift, int ntiles,
    const int* __restrict__ offs, const int* __restrict__ total) {
    __shared__ int run[kDigits];
    const int lane = threadIdx.x;
    const int tile = blockIdx.x;
    {
        int t[4], sum = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            t[k] = total[4 * lane + k];
            sum += t[k];
        }
        int x = sum;  // inclusive scan of the per-lane sums
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
            const int y = __shfl_up(x, off, kWave);
            if (lane >= off) x += y;
        }
        int base = x - sum;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int d = 4 * lane + k;
            run[d] = base + offs[d * ntiles + tile];
            base += t[k];
        }
    }
    // All of the tile's keys and values are loaded before the ranking.
    unsigned key[kTile / kWave];
    int val[kTile / kWave];
#pragma unroll
    for (int b = 0; b < kTile / kWave; ++b) {
        const int e = tile * kTile + b * kWave + lane;
        if (e < n) {
            key[b] = ids ? token_key(ids[e], vocab) : kin[e];
            val[b] = ids ? e : vin[e];
        } else {
            key[b] = 0u;
            val[b] = 0;
        }
    }
    __syncthreads();
    const unsigned long long below = (1ull << lane) - 1ull;
#pragma unroll
    for (int b = 0; b < kTile / kWave; ++b) {
        const int e = tile * kTile + b * kWave + lane;
        const bool valid = e < n;
        const int d = static_cast<int>((key[b] >> shift) & (kDigits - 1));
        unsigned long long peers = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 8; ++bit) {
            const bool set = (d >> bit) & 1;
            const unsigned long long msk = __ballot(set);
            peers &= set ? msk : ~msk;
        }
        const int rank = __popcll(peers & below);
        const int pos = run[d] + rank;
        const bool leader = valid && (63 - __clzll(peers)) == lane;
        __syncthreads();  // every lane has read run[] before the leaders update it
        if (valid) {
            kout[pos] = key[b];
            vout[pos] = val[b];
        }
        if (leader) run[d] += __popcll(peers);
        __syncthreads();
    }
}

// One wave per sorted position; the first position of each run of equal
// keys accumulates the run's grad rows, in sorted order, onto its table row.
// The table row, the run's keys and its values are requested together; the
// grad rows are then loaded kAccBatch at a time before being added in order.
constexpr int kAccBatch = 4;

template <int W, int NCH>
__global__ __launch_bounds__(kRowWaves * kWave) void emb_bwd_accum_kernel(
    const unsigned* __restrict__ keys, const int* __restrict__ vals, int n,
    const float* __restrict__ g, float* __restrict__ table, int dim) {
    const int lane = threadIdx.x & (kWave - 1);
    const int s = blockIdx.x * kRowWaves + static_cast<int>(threadIdx.x / kWave);
    if (s >= n) return;
    // One load covers the previous position (lane 0) and the first 63
    // positions from s (lanes 1..63): the run-start test, the run's extent
    // in this window and its grad row indices all come from one round trip,
    // and the table row and grad rows are then requested together.
    constexpr unsigned kNoKey = 0xFFFFFFFEu;  // no key takes this value
    const int e0 = s - 1 + lane;
    const bool in = e0 >= 0 && e0 < n;
    const unsigned kk = in ? keys[e0] : kNoKey;
    const int vv = (in && lane > 0) ? vals[e0] : 0;
    const unsigned key = __shfl(kk, 1, kWave);
    if (key == kSentinel || __shfl(kk, 0, kWave) == key) return;  // wave-uniform
    // Run length within the window: trailing set bits of the match mask of
    // positions s, s+1, ... (lanes 1..63).
    const unsigned long long m0 = __ballot(lane > 0 && kk == key) >> 1;
    const int cnt0 = (~m0 == 0ull) ? 64 : (__ffsll(static_cast<unsigned long long>(~m0)) - 1);
    const int nv = dim / W;
    float* trow = table + static_cast<size_t>(key) * dim;
    for (int c0 = 0; c0 < nv; c0 += NCH * kWave) {
        fvec<W> acc[NCH];
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            const int j = c0 + lane + k * kWave;
            acc[k] = j < nv ? vload<W>(trow, j) : vzero<W>();
        }
        // Adds `cnt` grad rows whose indices sit in lanes off, off+1, ... of
        // `idx`, in order, kAccBatch rows per group of loads.
        auto add_rows = [&](int idx, int off, int cnt) {
            int q = 0;
            for (; q + kAccBatch <= cnt; q += kAccBatch) {
                fvec<W> v[kAccBatch][NCH];
#pragma unroll
                for (int u = 0; u < kAccBatch; ++u) {
                    const float* grow =
                        g + static_cast<size_t>(__shfl(idx, off + q + u, kWave)) * dim;
#pragma unroll
                    for (int k = 0; k < NCH; ++k) {
                        const int j = c0 + lane + k * kWave;
                        v[u][k] = j < nv ? vload<W>(grow, j) : vzero<W>();
                    }
                }
#pragma unroll
                for (int u = 0; u < kAccBatch; ++u)
#pragma unroll
                    for (int k = 0; k < NCH; ++k)
#pragma unroll
                        for (int x = 0; x < W; ++x) acc[k].v[x] = acc[k].v[x] + v[u][k].v[x];
            }
            for (; q < cnt; ++q) {
                const float* grow = g + static_cast<size_t>(__shfl(idx, off + q, kWave)) * dim;
#pragma unroll
                for (int k = 0; k < NCH; ++k) {
                    const int j = c0 + lane + k * kWave;
                    if (j < nv) {
                        const fvec<W> v = vload<W>(grow, j);
#pragma unroll
                        for (int x = 0; x < W; ++x) acc[k].v[x] = acc[k].v[x] + v.v[x];
                    }
                }
            }
        };
        const int first = cnt0 < 63 ? cnt0 : 63;
        add_rows(vv, 1, first);
        if (cnt0 >= 63) {
            // Long runs: continue 64 positions at a time after the window.
            for (int b0 = s + 63;; b0 += kWave) {
                const int e = b0 + lane;
                const bool same = e < n && keys[e] == key;
                const int my_i = same ? vals[e] : 0;
                const unsigned long long m = __ballot(same);
                const int cnt =
                    (~m == 0ull) ? kWave : (__ffsll(static_cast<unsigned long long>(~m)) - 1);
                add_rows(my_i, 0, cnt);
                if (cnt < kWave) break;
            }
        }
#pragma unroll
        for (int k = 0; k < NCH; ++k) {
            const int j = c0 + lane + k * kWave;
            if (j < nv) vstore<W>(trow, j, acc[k]);
        }
    }
}

struct SortPlan {
    int ntiles;
    int passes;
    size_t bytes;
    size_t off_k0, off_k1, off_v0, off_v1, off_hist, off_total;
};

SortPlan plan_sort(int n, int vocab) {
    SortPlan p;
    p.ntiles = (n + kTile - 1) / kTile;
    int bits = 32;
    if (vocab > 0) {
        // Keys are ids in [0, vocab) or the sentinel, whose low `bits` bits
        // are all ones and so still sort after every id below 2^bits.
        bits = 1;
        while (bits < 32 && (1u << bits) <= static_cast<unsigned>(vocab)) ++bits;
    }
    p.passes = (bits + 7) / 8;
    // The first 256 bytes of the workspace are reserved.
    const size_t a = round_up(static_cast<size_t>(n) * 4, 256);
    p.off_k0 = 256;
    p.off_k1 = p.off_k0 + a;
    p.off_v0 = p.off_k0 + 2 * a;
    p.off_v1 = p.off_k0 + 3 * a;
    p.off_hist = p.off_k0 + 4 * a;
    p.off_total = p.off_hist + round_up(static_cast<size_t>(p.ntiles) * kDigits * 4, 256);
    p.bytes = p.off_total + kDigits * 4;
    return p;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" {

size_t mi_embedding_backward_workspace(int batch_seq) {
    if (batch_seq <= 0) return 0;
    return plan_sort(batch_seq, 0).bytes;
}

int mi_embedding_forward(const float* table, const int* tokens, float* out, int batch_seq,
                         int dim, int vocab, void* stream) {
    const char* name = "mi_embedding_forward";
    if (batch_seq < 0 || dim <= 0)
        return set_error(MI_ERR_INVALID_ARG, "%s: batch_seq=%d dim=%d", name, batch_seq, dim);
    if (batch_seq == 0) return MI_OK;
    if (!table || !tokens || !out) return set_error(MI_ERR_INVALID_ARG, "%s: NULL", name);
    const dim3 grid((batch_seq + kRowWaves - 1) / kRowWaves), block(kRowWaves * kWave);
    hipStream_t st = to_stream(stream);
    if (dim % 4 == 0 && aligned16(table) && aligned16(out))
        hipLaunchKernelGGL((emb_fwd_kernel<4, false>), grid, block, 0, st, table, nullptr, tokens,
                           out, batch_seq, 1, dim, vocab);
    else
        hipLaunchKernelGGL((emb_fwd_kernel<1, false>), grid, block, 0, st, table, nullptr, tokens,
                           out, batch_seq, 1, dim, vocab);
    return check_launch(name);
}

int mi_embedding_pos_forward(const float* table, const float* pos_table, const int* tokens,
                             float* out, int batch, int seq, int dim, int vocab, void* stream) {
    const char* name = "mi_embedding_pos_forward";
    if (batch < 0 || seq <= 0 || dim <= 0)
        return set_error(MI_ERR_INVALID_ARG, "%s: batch=%d seq=%d dim=%d", name, batch, seq, dim);
    const long long bt = static_cast<long long>(batch) * seq;
    if (bt == 0) return MI_OK;
    if (bt > INT32_MAX) return set_error(MI_ERR_INVALID_ARG, "%s: batch*seq too large", name);
    if (!table || !pos_table || !tokens || !out)
        return set_error(MI_ERR_INVALID_ARG, "%s: NULL", name);
    const dim3 grid(static_cast<unsigned>((bt + kRowWaves - 1) / kRowWaves)),
        block(kRowWaves * kWave);
    hipStream_t st = to_stream(stream);
    if (dim % 4 == 0 && aligned16(table) && aligned16(pos_table) && aligned16(out))
        hipLaunchKernelGGL((emb_fwd_kernel<4, true>), grid, block, 0, st, table, pos_table, tokens,
                           out, static_cast<int>(bt), seq, dim, vocab);
    else
        hipLaunchKernelGGL((emb_fwd_kernel<1, true>), grid, block, 0, st, table, pos_table, tokens,
                           out, static_cast<int>(bt), seq, dim, vocab);
    return check_launch(name);
}

int mi_pos_embedding_forward(const float* pos_table, float* embeddings, int batch, int seq,
                             int dim, void* stream) {
    const char* name = "mi_pos_embedding_forward";
    if (batch < 0 || seq <= 0 || dim <= 0)
        return set_error(MI_ERR_INVALID_ARG, "%s: batch=%d seq=%d dim=%d", name, batch, seq, dim);
    const long long rows = static_cast<long long>(batch) * seq;
    if (rows == 0) return MI_OK;
    if (rows > INT32_MAX) return set_error(MI_ERR_INVALID_ARG, "%s: batch*seq too large", name);
    if (!pos_table || !embeddings) return set_error(MI_ERR_INVALID_ARG, "%s: NULL", name);
    const dim3 grid(static_cast<unsigned>((rows + kRowWaves - 1) / kRowWaves)),
        block(kRowWaves * kWave);
    hipStream_t st = to_stream(stream);
    if (dim % 4 == 0 && aligned16(pos_table) && aligned16(embeddings))
        hipLaunchKernelGGL(pos_add_kernel<4>, grid, block, 0, st, pos_table, embeddings,
                           static_cast<int>(rows), seq, dim);
    else
        hipLaunchKernelGGL(pos_add_kernel<1>, grid, block, 0, st, pos_table, embeddings,
                           static_cast<int>(rows), seq, dim);
    return check_launch(name);
}

int mi_pos_embedding_backward(const float* grad_out, float* grad_pos_table, int batch, int seq,
                              int dim, void* stream) {
    const char* name = "mi_pos_embedding_backward";
    if (batch < 0 || seq <= 0 || dim <= 0)
        return set_error(MI_ERR_INVALID_ARG, "%s: batch=%d seq=%d dim=%d", name, batch, seq, dim);
    if (batch == 0) return MI_OK;
    if (!grad_out || !grad_pos_table) return set_error(MI_ERR_INVALID_ARG, "%s: NULL", name);
    hipStream_t st = to_stream(stream);
    const bool v4 = dim % 4 == 0 && aligned16(grad_out) && aligned16(grad_pos_table);
    const long long threads = static_cast<long long>(seq) * (v4 ? dim / 4 : dim);
    const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
    if (v4)
        hipLaunchKernelGGL(pos_bwd_kernel<4>, grid, dim3(256), 0, st, grad_out, grad_pos_table,
                           batch, seq, dim);
    else
        hipLaunchKernelGGL(pos_bwd_kernel<1>, grid, dim3(256), 0, st, grad_out, grad_pos_table,
                           batch, seq, dim);
    return check_launch(name);
}

int mi_embedding_backward(const float* grad_out, const int* tokens, float* grad_table,
                          int batch_seq, int dim, int vocab, void* stream) {
    const char* name = "mi_embedding_backward";
    if (batch_seq < 0 || dim <= 0)
        return set_error(MI_ERR_INVALID_ARG, "%s: batch_seq=%d dim=%d", name, batch_seq, dim);
    if (batch_seq == 0) return MI_OK;
    if (!grad_out || !tokens || !grad_table) return set_error(MI_ERR_INVALID_ARG, "%s: NULL", name);
    hipStream_t st = to_stream(stream);
    const SortPlan p = plan_sort(batch_seq, vocab);
    int err = MI_OK;
    char* ws = static_cast<char*>(workspace_get(p.bytes, st, &err));
    if (!ws) return err;
    unsigned* k[2] = {reinterpret_cast<unsigned*>(ws + p.off_k0),
                      reinterpret_cast<unsigned*>(ws + p.off_k1)};
    int* v[2] = {reinterpret_cast<int*>(ws + p.off_v0), reinterpret_cast<int*>(ws + p.off_v1)};
    int* hist = reinterpret_cast<int*>(ws + p.off_hist);
    int* total = reinterpret_cast<int*>(ws + p.off_total);
    const int n = batch_seq;

    int cur = 0;
    for (int pass = 0; pass < p.passes; ++pass) {
        const int shift = 8 * pass;
        const int* ids = pass == 0 ? tokens : nullptr;  // pass 0 keys come from the ids
        hipLaunchKernelGGL(radix_hist_kernel, dim3(p.ntiles), dim3(kTile), 0, st, k[cur], ids,
                           vocab, n, shift, p.ntiles, hist);
        hipLaunchKernelGGL(digit_scan_kernel, dim3(kDigits), dim3(256), 0, st, hist, total,
                           p.ntiles);
        hipLaunchKernelGGL(radix_scatter_kernel, dim3(p.ntiles), dim3(kWave), 0, st, k[cur],
                           v[cur], ids, vocab, k[cur ^ 1], v[cur ^ 1], n, shift, p.ntiles, hist,
                           total);
        cur ^= 1;
    }
    const dim3 grid((n + kRowWaves - 1) / kRowWaves), block(kRowWaves * kWave);
    if (dim % 4 == 0 && aligned16(grad_out) && aligned16(grad_table))
        hipLaunchKernelGGL((emb_bwd_accum_kernel<4, 4>), grid, block, 0, st, k[cur], v[cur], n,
                           grad_out, grad_table, dim);
    else
        hipLaunchKernelGGL((emb_bwd_accum_kernel<1, 4>), grid, block, 0, st, k[cur], v[cur], n,
                           grad_out, grad_table, dim);
    return check_launch(name);
}

}  // extern "C"
