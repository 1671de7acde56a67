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
// adds grad rows into grad_table in increasing token position: one kernel,
// no sort and no workspace (emb_bwd_owner_kernel below).  Each workgroup
// owns a slice of the ids, collects the positions of its ids from the
// whole id vector, sorts them by id in LDS and adds every id's rows in
// position order; exactly one wave updates a given table row.
// Position backward: one thread per (t, column vector) adds grad_out[b, t]
// for b = 0, 1, ... in order onto grad_pos[t]; the fused token + position
// backward does the same sums inside the token kernel's workgroups.
#include <type_traits>

#include "mi_common.hpp"

namespace mi {

namespace {

constexpr int kRowWaves = 4;   // token rows per workgroup

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
// Each wave gathers R consecutive token rows: the R ids are read first,
// then the loads of all R rows (table and position, NQ vectors per lane per
// row at a time) are issued before any row is stored, so that R row gathers
// are in flight per wave instead of one behind each id load.
template <int W, bool POS, int R, int NQ>
__global__ __launch_bounds__(kRowWaves * kWave) void emb_fwd_kernel(
    const float* __restrict__ table, const float* __restrict__ pos, const int* __restrict__ tokens,
    float* __restrict__ out, int batch_seq, int seq, int dim, int vocab) {
    const int lane = threadIdx.x & (kWave - 1);
    const int i0 = (blockIdx.x * kRowWaves + static_cast<int>(threadIdx.x / kWave)) * R;
    if (i0 >= batch_seq) return;  // wave-uniform
    const int nv = dim / W;
    int id[R];
    bool ok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = i0 + r < batch_seq ? i0 + r : batch_seq - 1;
        id[r] = tokens[i];
        ok[r] = i0 + r < batch_seq && (vocab <= 0 || (id[r] >= 0 && id[r] < vocab));
    }
    for (int j0 = lane; j0 < nv; j0 += NQ * kWave) {
        fvec<W> v[R][NQ];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float* src = table + static_cast<size_t>(ok[r] ? id[r] : 0) * dim;
            const float* p = POS ? pos + static_cast<size_t>((i0 + r) % seq) * dim : nullptr;
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                const int j = j0 + q * kWave;
                // Table rows are gathered with the non-temporal hint: in the
                // config-2 step (forward after the previous backward) it
                // measured 65.1 -> 64.1 us, although a forward repeated
                // alone, which finds the 154 MB table in the last-level
                // cache, is faster without it (15.9 us).
                v[r][q] = (ok[r] && j < nv) ? sload<W>(src, j) : vzero<W>();
                if constexpr (POS) {
                    if (j < nv && i0 + r < batch_seq) {
                        const fvec<W> t = vload<W>(p, j);
#pragma unroll
                        for (int e = 0; e < W; ++e) v[r][q].v[e] = v[r][q].v[e] + t.v[e];
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (i0 + r >= batch_seq) break;  // wave-uniform
            float* dst = out + static_cast<size_t>(i0 + r) * dim;
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                const int j = j0 + q * kWave;
                // streamed out: measured 20.9 -> 16.0 us at config 2
                if (j < nv) sstore<W>(dst, j, v[r][q]);
            }
        }
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
// Token backward, owner-computes form.  Workgroup k of K (a power of two)
// owns the valid ids with id % K == k, so no two workgroups touch the same
// table row.  Every workgroup reads the whole id vector (4 bytes per token,
// served from L2, against 3 KB of grad row per token) and keeps the
// positions of its own ids, in position order, in an LDS list (windows of
// kOwnCap entries).  The list is sorted by id in LDS, stably, so that each
// id's entries form a run in increasing position; the waves take runs from
// an LDS counter and add each run onto its table row (one load, the run's
// grad rows in order, one store).  Every row therefore receives its grad
// rows in increasing token position, as in the CPU loop, and the result is
// bit-identical whichever wave adds a run.  Measured at config 2 (16384
// tokens, D = 768): 34 us against 46.7 us for a six-launch radix sort plus
// an accumulate pass.
// ---------------------------------------------------------------------------
constexpr int kOwnWaves = 8;
constexpr int kOwnThreads = kOwnWaves * kWave;   // 512
constexpr int kOwnPer = 32;                      // ids per thread per pass
constexpr int kOwnGroups = kOwnPer / 4;          // 4-id groups per thread
constexpr int kOwnSpan = kOwnThreads * kOwnPer;  // positions per pass
constexpr int kOwnCap = 2048;                    // list entries per window
constexpr int kOwnBatch = 2;                     // grad rows per group of loads
constexpr int kOwnTake = 2;                      // sorted entries per claim
constexpr int kOwnMaxK = 512;                    // owning workgroups, at most
constexpr int kOwnTokens = 32;                   // tokens per owner, about

// Position gradient fused into the owner kernel (POS): the workgroups also
// share out the seq * nv position column vectors, one per thread per round;
// each is grad_pos[t, j] + grad_out[0, t, j] + grad_out[1, t, j] + ... in
// increasing b, the order of pos_bwd_kernel.  The old values and the first
// kPosPre batch rows of a thread's first vector are requested before the
// id scan and summed after it, so that they stream from HBM while the
// workgroup scans ids and builds its list (HBM is otherwise idle then); the
// partial sums wait in LDS, and the remaining rows are added after the
// token gradient.
constexpr int kPosPre = 7;   // batch rows in flight across the id scan, at most
constexpr int kPosChunk = 5; // batch rows per group of loads afterwards

// 128 VGPRs at most, so that two 8-wave workgroups fit on a CU.
template <int W, int NCH, bool POS>
__global__ __launch_bounds__(kOwnThreads) __attribute__((amdgpu_waves_per_eu(4))) void
emb_bwd_owner_kernel(int n, int vocab, int dim, int batch, int seq, int vec_ids, int nblk,
                     const int* __restrict__ ids, const float* __restrict__ g,
                     float* __restrict__ table, float* __restrict__ gpos) {
    __shared__ __align__(16) int s_id[kOwnCap];  // list in position order
    __shared__ int s_pos[kOwnCap];
    __shared__ int s_sid[kOwnCap];  // list sorted by id
    __shared__ int s_spos[kOwnCap];
    __shared__ int s_wsum[kOwnWaves];
    __shared__ int s_next;
    __shared__ fvec<W> s_pacc[POS ? kOwnThreads : 1];  // first position rows, summed
    const int lane = threadIdx.x & (kWave - 1);
    // Uniform over the wave; readfirstlane lets the compiler see that, so
    // branches on it are scalar branches, not exec-masked ones.
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
    // nblk (= gridDim.x, passed and preloaded with the other arguments) is a
    // power of two, so id % nblk is a mask.
    const unsigned kmask = static_cast<unsigned>(nblk) - 1u;
    const unsigned k = blockIdx.x;
    const int nv = dim / W;

    const unsigned long long below = (1ull << lane) - 1ull;

    // acc += the grad rows of sorted-list entries from, from + 1, ... while
    // they carry `id` (none if entry `from` does not), in list order, for
    // the column vectors c0 + lane + q * 64.
    auto add_entries = [&](int id, int from, int L, int c0, fvec<W>(&acc)[NCH]) __attribute__((always_inline)) {
        for (int off = from;; off += kWave) {
            const int e = off + lane;
            const bool same = e < L && s_sid[e] == id;
            const int pos_l = same ? s_spos[e] : 0;
            const unsigned long long m = __ballot(same);
            const int cnt =
                (~m == 0ull) ? kWave : (__ffsll(static_cast<unsigned long long>(~m)) - 1);
            for (int u0 = 0; u0 < cnt; u0 += kOwnBatch) {
                fvec<W> v[kOwnBatch][NCH];
#pragma unroll
                for (int u = 0; u < kOwnBatch; ++u) {
                    const int src = u0 + u < cnt ? u0 + u : 0;
                    const float* grow = g + static_cast<size_t>(__shfl(pos_l, src, kWave)) * dim;
#pragma unroll
                    for (int q = 0; q < NCH; ++q) {
                        const int j = c0 + lane + q * kWave;
                        v[u][q] = (u0 + u < cnt && j < nv) ? vload<W>(grow, j) : vzero<W>();
                    }
                }
#pragma unroll
                for (int u = 0; u < kOwnBatch; ++u)
                    if (u0 + u < cnt) {
#pragma unroll
                        for (int q = 0; q < NCH; ++q)
#pragma unroll
                            for (int x = 0; x < W; ++x) acc[q].v[x] = acc[q].v[x] + v[u][q].v[x];
                    }
            }
            if (cnt < kWave) break;
        }
    };

    // Adds the run starting at sorted-list entry s0 (entries s0, s0 + 1, ...
    // with the id of s0, in position order) onto that id's table row.
    auto add_run = [&](int s0, int L) __attribute__((always_inline)) {
        const int id = s_sid[s0];
        float* row = table + static_cast<size_t>(id) * dim;
        for (int c0 = 0; c0 < nv; c0 += NCH * kWave) {
            fvec<W> acc[NCH];
#pragma unroll
            for (int q = 0; q < NCH; ++q) {
                const int j = c0 + lane + q * kWave;
                acc[q] = j < nv ? vload<W>(row, j) : vzero<W>();
            }
            add_entries(id, s0, L, c0, acc);
#pragma unroll
            for (int q = 0; q < NCH; ++q) {
                const int j = c0 + lane + q * kWave;
                if (j < nv) vstore<W>(row, j, acc[q]);
            }
        }
    };

    // Adds the runs starting at sorted-list entries sa and sb together: the
    // two table rows and the first grad row of each run are requested at
    // once; the rest of each run (if any) follows.
    auto add_pair = [&](int sa, int sb, int L) __attribute__((always_inline)) {
        const int ida = s_sid[sa];
        const int idb = s_sid[sb];
        float* ra = table + static_cast<size_t>(ida) * dim;
        float* rb = table + static_cast<size_t>(idb) * dim;
        const float* ga = g + static_cast<size_t>(s_spos[sa]) * dim;
        const float* gb = g + static_cast<size_t>(s_spos[sb]) * dim;
        for (int c0 = 0; c0 < nv; c0 += NCH * kWave) {
            fvec<W> A[NCH], B[NCH];
            {
                fvec<W> GA[NCH], GB[NCH];
#pragma unroll
                for (int q = 0; q < NCH; ++q) {
                    const int j = c0 + lane + q * kWave;
                    const bool ok = j < nv;
                    A[q] = ok ? vload<W>(ra, j) : vzero<W>();
                    B[q] = ok ? vload<W>(rb, j) : vzero<W>();
                    GA[q] = ok ? vload<W>(ga, j) : vzero<W>();
                    GB[q] = ok ? vload<W>(gb, j) : vzero<W>();
                }
#pragma unroll
                for (int q = 0; q < NCH; ++q)
#pragma unroll
                    for (int x = 0; x < W; ++x) {
                        A[q].v[x] = A[q].v[x] + GA[q].v[x];
                        B[q].v[x] = B[q].v[x] + GB[q].v[x];
                    }
            }
            add_entries(ida, sa + 1, L, c0, A);
            add_entries(idb, sb + 1, L, c0, B);
#pragma unroll
            for (int q = 0; q < NCH; ++q) {
                const int j = c0 + lane + q * kWave;
                if (j < nv) {
                    vstore<W>(ra, j, A[q]);
                    vstore<W>(rb, j, B[q]);
                }
            }
        }
    };

    // Sorts list entries [0, L) by id into s_sid / s_spos (a rank sort over
    // 4-entry LDS reads; equal ids keep their position order).  The waves
    // then take sorted entries from an LDS counter, one at a time, and the
    // taker of an entry that starts a run of equal ids adds the whole run.
    // Each run is added by one wave, whichever it is, so the result does
    // not depend on the assignment.
    auto process = [&](int L) __attribute__((always_inline)) {
        for (int i = static_cast<int>(threadIdx.x); i < L; i += kOwnThreads) {
            const int me = s_id[i];
            int r = 0;
            int j = 0;
            for (; j + 4 <= L; j += 4) {
                const int4 o = *reinterpret_cast<const int4*>(&s_id[j]);
                r += (o.x < me || (o.x == me && j < i)) ? 1 : 0;
                r += (o.y < me || (o.y == me && j + 1 < i)) ? 1 : 0;
                r += (o.z < me || (o.z == me && j + 2 < i)) ? 1 : 0;
                r += (o.w < me || (o.w == me && j + 3 < i)) ? 1 : 0;
            }
            for (; j < L; ++j) {
                const int o = s_id[j];
                r += (o < me || (o == me && j < i)) ? 1 : 0;
            }
            s_sid[r] = me;
            s_spos[r] = s_pos[i];
        }
        if (threadIdx.x == 0) s_next = 0;
        __syncthreads();
        for (;;) {
            int e = 0;
            if (lane == 0) e = atomicAdd(&s_next, kOwnTake);
            e = __shfl(e, 0, kWave);
            if (e >= L) break;
            const bool sa = e == 0 || s_sid[e - 1] != s_sid[e];
            const bool sb = kOwnTake == 2 && e + 1 < L && s_sid[e] != s_sid[e + 1];
            if (sa && sb)
                add_pair(e, e + 1, L);
            else if (sa)
                add_run(e, L);
            else if (sb)
                add_run(e + 1, L);
        }
    };

    // Position gradient, first round: requests issued now, summed below.
    const long long pvec = POS ? static_cast<long long>(seq) * nv : 0;   // position vectors
    const long long pstride = static_cast<long long>(nblk) * kOwnThreads;
    // A thread's first position vector, below kOwnMaxK * kOwnThreads = 2^18:
    // 32 bits.  Held as a 64-bit value it was spilled to scratch, and its
    // reload waited for every outstanding load.
    const int pv0 = static_cast<int>(k) * kOwnThreads + wave * kWave + lane;
    const size_t bstride = static_cast<size_t>(seq) * nv;                // vectors per batch row
    // PRE batch rows of the first position vector are requested across the
    // id scan (7 for 2-3 column vectors per lane, 4 for one: more spills
    // registers in the scan); with 4 column vectors per lane none fit, and the
    // position sums run after the token gradient alone.  The position
    // bookkeeping kept across the token updates stays in registers (no
    // instantiation spills).
    constexpr int PRE = !POS ? 0 : NCH == 1 ? 4 : NCH <= 3 ? kPosPre : 0;
    constexpr int NPQ = PRE > 0 ? PRE : 1;
    // Adds batch rows b0, b0 + 1, ... of position vector pv onto acc, in
    // order, and stores the total.
    auto pos_rest = [&](long long pv, int b0, fvec<W> acc) __attribute__((always_inline)) {
        for (int b = b0; b < batch; b += kPosChunk) {
            fvec<W> q[kPosChunk];
#pragma unroll
            for (int u = 0; u < kPosChunk; ++u)
                q[u] = b + u < batch ? sload<W>(g, (b + u) * bstride + pv) : vzero<W>();
#pragma unroll
            for (int u = 0; u < kPosChunk; ++u)
                if (b + u < batch)
#pragma unroll
                    for (int x = 0; x < W; ++x) acc.v[x] = acc.v[x] + q[u].v[x];
        }
        vstore<W>(gpos, pv, acc);
    };
    // The position vectors after a thread's first one (pv0 + pstride, ...).
    auto pos_others = [&]() __attribute__((always_inline)) {
        for (long long pv = pv0 + pstride; pv < pvec; pv += pstride)
            pos_rest(pv, 0, vload<W>(gpos, pv));
    };

    // One pass over kOwnSpan positions of the id vector.  The first pass is
    // a separate instantiation (FIRST) so that the position registers live
    // only inside it.  This lambda and those it calls are inlined: an
    // out-of-line call keeps the captured locals in scratch memory.
    auto pass = [&](long long base, auto first_tag) __attribute__((always_inline)) {
        constexpr bool first = decltype(first_tag)::value && PRE > 0;
        [[maybe_unused]] fvec<W> pacc, pq[NPQ];
        // Wave w reads positions base + w * kOwnPer * 64 + [0, kOwnPer * 64):
        // group j (4 ids per lane) covers 256 consecutive positions, lane l
        // takes positions 4l .. 4l + 3 of it, so every load instruction of
        // the wave reads one contiguous KiB.  bits marks the ids this
        // workgroup owns.
        const long long wpos = base + static_cast<long long>(wave) * kOwnPer * kWave;
        int my[kOwnPer];
        unsigned bits = 0;
        // Either the wave's whole span is in range with 16-byte aligned ids
        // (one 16-byte load per group) or every id is a 4-byte load at a
        // clamped position, masked after the load.  The choice is uniform
        // over the wave and no load sits under a per-lane branch, so the
        // waits that follow count these loads exactly: with per-lane
        // branches the compiler waited for all but one of the position loads
        // issued below before the first id was tested, which serialised
        // them with the scan.
        if (vec_ids && wpos + kOwnPer * kWave <= n) {
#pragma unroll
            for (int j = 0; j < kOwnGroups; ++j) {
                const long long p4 = wpos + j * 4 * kWave + 4 * lane;
                const int4 v = *reinterpret_cast<const int4*>(ids + p4);
                my[4 * j] = v.x;
                my[4 * j + 1] = v.y;
                my[4 * j + 2] = v.z;
                my[4 * j + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < kOwnGroups; ++j) {
                const long long p4 = wpos + j * 4 * kWave + 4 * lane;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const long long p = p4 + e;
                    const int v = ids[p < n ? p : n - 1];
                    my[4 * j + e] = p < n ? v : -1;
                }
            }
        }
        if constexpr (first) {
            // Issued after the id loads: loads complete in issue order, so
            // the scan can use its ids while these are still in flight.
            // Unconditional loads, issued back to back on every lane: rows
            // past the batch are clamped to its last row and lanes past the
            // last position vector to that vector, and neither is added.
            // With the loads under a per-lane branch the compiler's wait
            // counts for the ids below had to allow for a path without
            // them, and each id group then waited for one more of these.
            const long long pvc = pv0 < pvec ? pv0 : pvec - 1;
            pacc = vload<W>(gpos, static_cast<size_t>(pvc));
#pragma unroll
            for (int u = 0; u < PRE; ++u)
                pq[u] = sload<W>(g, static_cast<size_t>(u < batch ? u : batch - 1) * bstride +
                                        static_cast<size_t>(pvc));
        }
#pragma unroll
        for (int j = 0; j < kOwnGroups; ++j) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int id = my[4 * j + e];
                const bool ok = id >= 0 && (vocab <= 0 || id < vocab) &&
                                (static_cast<unsigned>(id) & kmask) == k;
                bits |= static_cast<unsigned>(ok) << (4 * j + e);
            }
        }
        // List slots in position order: within the wave from ballots
        // (group, then lane, then element), across waves from their totals.
        int lane_off[kOwnGroups];
        int wtot = 0;
#pragma unroll
        for (int j = 0; j < kOwnGroups; ++j) {
            int pre = 0, tot = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const unsigned long long b = __ballot((bits >> (4 * j + e)) & 1u);
                pre += __popcll(b & below);
                tot += __popcll(b);
            }
            lane_off[j] = wtot + pre;
            wtot += tot;
        }
        if (lane == 0) s_wsum[wave] = wtot;
        __syncthreads();
        int before = 0, total = 0;
#pragma unroll
        for (int w = 0; w < kOwnWaves; ++w) {
            const int t = s_wsum[w];
            before += w < wave ? t : 0;
            total += t;
        }
        __syncthreads();  // s_wsum is rewritten by the next pass
        // Windows of kOwnCap list entries (one window unless this
        // workgroup's ids are very frequent in this span).  The first window
        // is written from the ids in registers; later windows read their ids
        // again, one at a time, so that no id registers stay live while the
        // windows are processed.
        if (total > 0) {
#pragma unroll
            for (int j = 0; j < kOwnGroups; ++j) {
                int slot = before + lane_off[j];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if ((bits >> (4 * j + e)) & 1u) {
                        if (slot < kOwnCap) {
                            s_id[slot] = my[4 * j + e];
                            s_pos[slot] = static_cast<int>(wpos + j * 4 * kWave + 4 * lane + e);
                        }
                        ++slot;
                    }
                }
            }
        }
        if constexpr (first) {
            if (pv0 < pvec) {
#pragma unroll
                for (int u = 0; u < PRE; ++u)
                    if (u < batch)
#pragma unroll
                        for (int x = 0; x < W; ++x) pacc.v[x] = pacc.v[x] + pq[u].v[x];
                s_pacc[threadIdx.x] = pacc;  // finished after the token gradient
            }
        }
        for (int w0 = 0; w0 < total; w0 += kOwnCap) {
            if (w0 > 0) {
#pragma unroll 1
                for (int j = 0; j < kOwnGroups; ++j) {
                    int slot = before + lane_off[j];
#pragma unroll 1
                    for (int e = 0; e < 4; ++e) {
                        if ((bits >> (4 * j + e)) & 1u) {
                            if (slot >= w0 && slot < w0 + kOwnCap) {
                                const long long p = wpos + j * 4 * kWave + 4 * lane + e;
                                s_id[slot - w0] = ids[p];
                                s_pos[slot - w0] = static_cast<int>(p);
                            }
                            ++slot;
                        }
                    }
                }
            }
            __syncthreads();
            process(total - w0 < kOwnCap ? total - w0 : kOwnCap);
            __syncthreads();
        }
    };
    if constexpr (PRE > 0) {
        pass(0, std::true_type{});
        for (long long base = kOwnSpan; base < n; base += kOwnSpan) pass(base, std::false_type{});
    } else {
        for (long long base = 0; base < n; base += kOwnSpan) pass(base, std::false_type{});
    }
    // The rest of the position sums follow the token gradient: the table-row
    // updates start as soon as the list is built (config-2 step 58.8 ->
    // 58.3 us against finishing the position sums first).
    if constexpr (POS) {
        if (pv0 < pvec) {
            if constexpr (PRE > 0)
                pos_rest(pv0, PRE, s_pacc[threadIdx.x]);
            else
                pos_rest(pv0, 0, vload<W>(gpos, pv0));
        }
        pos_others();
    }
}

#ifndef MI_EMB_ROWS
#define MI_EMB_ROWS 4
#endif
// Token rows per wave in the forward gather.  Config 2 step (V = 50257,
// D = 768, 16384 tokens): 1 row 60.1 us, 2 rows 60.7, 4 rows 59.1, 8 rows 63.8.
constexpr int kEmbRows = MI_EMB_ROWS;

// Forward gather launch: kEmbRows rows per wave, NQ = vectors per lane per
// row at a time (just enough for the row, at most 4).
template <bool POS>
void launch_emb_fwd(const float* table, const float* pos, const int* tokens, float* out,
                    int batch_seq, int seq, int dim, int vocab, hipStream_t st) {
    const bool v4 = dim % 4 == 0 && aligned16(table) && aligned16(out) && (!POS || aligned16(pos));
    const int nv = v4 ? dim / 4 : dim;
    const int nq = nv <= kWave ? 1 : nv <= 2 * kWave ? 2 : nv <= 3 * kWave ? 3 : 4;
    const long long waves = (static_cast<long long>(batch_seq) + kEmbRows - 1) / kEmbRows;
    const dim3 grid(static_cast<unsigned>((waves + kRowWaves - 1) / kRowWaves)),
        block(kRowWaves * kWave);
#define MI_FWD_CASE(WW, QQ)                                                                     \
    hipLaunchKernelGGL((emb_fwd_kernel<WW, POS, kEmbRows, QQ>), grid, block, 0, st, table, pos, \
                       tokens, out, batch_seq, seq, dim, vocab)
    switch ((v4 ? 10 : 0) + nq) {
        case 11: MI_FWD_CASE(4, 1); break;
        case 12: MI_FWD_CASE(4, 2); break;
        case 13: MI_FWD_CASE(4, 3); break;
        case 14: MI_FWD_CASE(4, 4); break;
        case 1: MI_FWD_CASE(1, 1); break;
        case 2: MI_FWD_CASE(1, 2); break;
        case 3: MI_FWD_CASE(1, 3); break;
        default: MI_FWD_CASE(1, 4); break;
    }
#undef MI_FWD_CASE
}

// One launch of the owner kernel: K = 2^log2k owning workgroups, about
// kOwnTokens tokens each.  The position gradient (POS) needs 16-byte
// alignment of grad_pos as well for the vector path.
template <bool POS>
void launch_owner(const float* grad_out, const int* tokens, float* grad_table, float* grad_pos,
                  int batch_seq, int batch, int seq, int dim, int vocab, hipStream_t st) {
    int log2k = 0;
    while ((2 << log2k) <= kOwnMaxK && (2ll << log2k) * kOwnTokens <= batch_seq) ++log2k;
    const dim3 grid(1u << log2k), block(kOwnThreads);
    const bool vec_ids = aligned16(tokens);
    const bool v4 = dim % 4 == 0 && aligned16(grad_out) && aligned16(grad_table) &&
                    (!POS || aligned16(grad_pos));
    const int nv = v4 ? dim / 4 : dim;
    // Column vectors per lane held at once: just enough for the row, at most
    // 4 (wider rows loop over column chunks).
    const int nch = nv <= kWave ? 1 : nv <= 2 * kWave ? 2 : nv <= 3 * kWave ? 3 : 4;
#define MI_OWNER_CASE(WW, NN)                                                                  \
    hipLaunchKernelGGL((emb_bwd_owner_kernel<WW, NN, POS>), grid, block, 0, st, batch_seq,    \
                       vocab, dim, batch, seq, vec_ids ? 1 : 0, 1 << log2k, tokens, grad_out, \
                       grad_table, grad_pos)
    switch ((v4 ? 10 : 0) + nch) {
        case 11: MI_OWNER_CASE(4, 1); break;
        case 12: MI_OWNER_CASE(4, 2); break;
        case 13: MI_OWNER_CASE(4, 3); break;
        case 14: MI_OWNER_CASE(4, 4); break;
        case 1: MI_OWNER_CASE(1, 1); break;
        case 2: MI_OWNER_CASE(1, 2); break;
        case 3: MI_OWNER_CASE(1, 3); break;
        default: MI_OWNER_CASE(1, 4); break;
    }
#undef MI_OWNER_CASE
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" {

size_t mi_embedding_backward_workspace(int) { return 0; }

int mi_embedding_forward(const float* table, const int* tokens, float* out, int batch_seq,
                         int dim, int vocab, void* stream) {
    const char* name = "mi_embedding_forward";
    if (batch_seq < 0 || dim <= 0)
        return set_error(MI_ERR_INVALID_ARG, "%s: batch_seq=%d dim=%d", name, batch_seq, dim);
    if (batch_seq == 0) return MI_OK;
    if (!table || !tokens || !out) return set_error(MI_ERR_INVALID_ARG, "%s: NULL", name);
    launch_emb_fwd<false>(table, nullptr, tokens, out, batch_seq, 1, dim, vocab,
                          to_stream(stream));
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
    launch_emb_fwd<true>(table, pos_table, tokens, out, static_cast<int>(bt), seq, dim, vocab,
                         to_stream(stream));
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
    launch_owner<false>(grad_out, tokens, grad_table, nullptr, batch_seq, 0, 1, dim, vocab,
                        to_stream(stream));
    return check_launch(name);
}

int mi_embedding_pos_backward(const float* grad_out, const int* tokens, float* grad_table,
                              float* grad_pos_table, int batch, int seq, int dim, int vocab,
                              void* stream) {
    const char* name = "mi_embedding_pos_backward";
    if (batch < 0 || seq <= 0 || dim <= 0)
        return set_error(MI_ERR_INVALID_ARG, "%s: batch=%d seq=%d dim=%d", name, batch, seq, dim);
    const long long bt = static_cast<long long>(batch) * seq;
    if (bt == 0) return MI_OK;
    if (bt > INT32_MAX) return set_error(MI_ERR_INVALID_ARG, "%s: batch*seq too large", name);
    if (!grad_out || !tokens || !grad_table || !grad_pos_table)
        return set_error(MI_ERR_INVALID_ARG, "%s: NULL", name);
    launch_owner<true>(grad_out, tokens, grad_table, grad_pos_table, static_cast<int>(bt), batch,
                       seq, dim, vocab, to_stream(stream));
    return check_launch(name);
}

}  // extern "C"
