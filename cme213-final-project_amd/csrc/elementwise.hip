// Residual adds, bias broadcast, ReLU and tanh-GELU (forward and backward
// with the bias gradient) for gfx950.
//
// Reference behaviour: FINAL_CLEAN_CODE/src/kernels/activations.cu:5-283
// (residual_add, residual_add_with_bias, bias_add, bias_relu_forward,
// relu_forward / relu_backward, relu_backward_with_bias_backward,
// bias_backward).  GELU has no reference; it takes the bias+ReLU slots.
//
// Layout, measured on MI355X at [8192, 3072]:
//  * non-reducing bias operators (bias+GELU / bias+ReLU forward, bias add,
//    residual+bias) run flat: a grid-stride loop of 256-thread workgroups, one
//    16-byte vector per thread per step, the bias column found by a
//    multiply-high division.  Many short-lived workgroups stream HBM best
//    (6.0 TB/s for bias+GELU forward vs 5.6 TB/s for the row-band form);
//  * reducing operators (bias / ReLU / GELU backward with dbias) use "row
//    bands": a workgroup covers whole rows, each thread owns fixed column
//    vectors (bias and column sums in registers), and rows are interleaved
//    over the workgroups so the resident workgroups stream one contiguous
//    band of memory at a time.  A 2-D tiling (column tiles x row blocks)
//    measured 28% slower (concurrent 4 KiB pieces at a 12 KiB stride spread
//    over the whole tensor); splitting a band into row lanes combined in LDS
//    measured 3-15% slower.
//
// Column reductions (dbias) are deterministic: each thread sums its columns
// over the workgroup's rows in row order and the workgroup writes one
// partial row; colsum_finalize adds the partial rows in a fixed order.  The
// reference uses float atomicAdd here (activations.cu:231,271).
#include <cstring>
#include <type_traits>

#include "mi_common.hpp"

#ifndef MI_REDUCE_TILES
#define MI_REDUCE_TILES 256
#endif

namespace mi {

namespace {

constexpr int kThreads = 256;
#ifndef MI_EW_UNROLL
#define MI_EW_UNROLL 1
#endif
#ifndef MI_FLAT_MAX_GRID
#define MI_FLAT_MAX_GRID 16384
#endif
#ifndef MI_FWD_BANDS
#define MI_FWD_BANDS 512
#endif
constexpr int kUnroll = MI_EW_UNROLL;

// ---------------------------------------------------------------------------
// tanh-approximation GELU (Hendrycks & Gimpel 2016):
//   gelu(u) = 0.5 u (1 + tanh z),  z = sqrt(2/pi) (u + 0.044715 u^3).
// With s = 0.5 (1 + tanh z) = 1 / (1 + e^{-2z}) (logistic of 2z):
//   gelu(u)  = u s
//   gelu'(u) = s + 2 u s (1 - s) z',  z' = sqrt(2/pi) (1 + 3*0.044715 u^2)
//            = s (1 + 2 u (e s) z'),  since 1 - s = e s with e = e^{-2z}.
// Neither form has the cancellation of 1 + tanh z for very negative u.
// e^{-2z} is one v_exp_f32 (2^x) on -2 z log2(e), its exponent clamped at
// 126 so that e, s and e*s stay finite; 1 / (1 + e) is one v_rcp_f32.
// Where the exponent reaches 126 (u below about -10, and u = -inf) gelu and
// gelu' are below 1e-36 in magnitude and are returned as 0, their limit: u*s
// with the clamped s = 2^-126 would grow like u (gelu(-1e38) = -1.2) and the
// derivative like u^3.  Where e underflows to 0 (u above about 10.5, and
// u = +inf) gelu' is exactly 1 = s, and the u*(e*s)*z' term, 0 * inf for
// |u| > 1.8e19, is skipped.  NaN propagates through both.
// ---------------------------------------------------------------------------
// Folded constants: -2 z log2(e) = u * (kT0 + kT1 u^2), and
// 2 z' = kD0 + kD1 u^2.
constexpr float kT0 = -2.302208198144325f;    // -2 * sqrt(2/pi) * log2(e)
constexpr float kT1 = -0.1029432395800235f;   // -2 * sqrt(2/pi) * 0.044715 * log2(e)
constexpr float kD0 = 1.5957691216057308f;    // 2 * sqrt(2/pi)
constexpr float kD1 = 0.21406444881780076f;   // 2 * sqrt(2/pi) * 3 * 0.044715
constexpr float kTMax = 126.0f;

struct GeluTerms {
    float s;     // 1 / (1 + e^{-2z})
    float e;     // e^{-2z}, exponent clamped at kTMax
    bool zero;   // the exponent reached kTMax: gelu and gelu' are 0
};

__device__ __forceinline__ GeluTerms gelu_terms(float u, float u2) {
    const float t = u * fmaf(kT1, u2, kT0);
    const float e = __builtin_amdgcn_exp2f(fminf(t, kTMax));
    return {__builtin_amdgcn_rcpf(1.0f + e), e, t >= kTMax};
}

__device__ __forceinline__ float gelu_fwd(float u) {
    const GeluTerms g = gelu_terms(u, u * u);
    return g.zero ? 0.0f : u * g.s;
}

__device__ __forceinline__ float gelu_grad(float u) {
    const float u2 = u * u;
    const GeluTerms g = gelu_terms(u, u2);
    // s (1 + 2 u (1 - s) z') with 1 - s = e s
    const float d = g.s * fmaf(u * (g.e * g.s), fmaf(kD1, u2, kD0), 1.0f);
    return g.zero ? 0.0f : (g.e == 0.0f ? g.s : d);
}

// ---------------------------------------------------------------------------
// Operator arguments.  An Op (at most three pointers) reaches the kernels as
// three pointer arguments, not as a struct argument.  The library is built
// with kernel-argument preloading: the first 14 dwords of the argument
// segment arrive in SGPRs when a wave starts, and the compiler preloads
// scalar and pointer arguments only, not aggregates.  Passed as a struct, the
// Op's pointers would cost each kernel a scalar-memory round trip before its
// first load.  They travel as pointers (not as integers) so that the
// compiler still knows they address global memory and emits global, not
// flat, loads and stores.
// ---------------------------------------------------------------------------
struct OpWords {
    const void* w0;
    const void* w1;
    const void* w2;
};

template <class Op>
OpWords op_words(const Op& op) {
    static_assert(sizeof(Op) <= sizeof(OpWords), "an Op holds at most three pointers");
    static_assert(std::is_trivially_copyable<Op>::value, "an Op is a plain pointer struct");
    const void* w[3] = {nullptr, nullptr, nullptr};
    std::memcpy(w, &op, sizeof(Op));
    return {w[0], w[1], w[2]};
}

template <class Op>
__device__ __forceinline__ Op op_from(const void* w0, const void* w1, const void* w2) {
    const void* const w[3] = {w0, w1, w2};
    Op op;
    __builtin_memcpy(&op, w, sizeof(Op));
    return op;
}

// ---------------------------------------------------------------------------
// Flat element-wise kernels (no broadcast).  Pointers may alias (the
// reference allows residual_add(a, b, a)); each element is read and written
// by one thread, so aliasing is safe without __restrict__.
// ---------------------------------------------------------------------------
template <int W>
struct AddOp {
    const float* a;
    const float* b;
    float* out;
    __device__ void operator()(size_t i) const {
        const fvec<W> x = sload<W>(a, i), y = sload<W>(b, i);
        fvec<W> o;
#pragma unroll
        for (int e = 0; e < W; ++e) o.v[e] = x.v[e] + y.v[e];
        sstore<W>(out, i, o);
    }
};

template <int W>
struct ReluOp {
    const float* in;
    float* out;
    __device__ void operator()(size_t i) const {
        const fvec<W> x = sload<W>(in, i);
        fvec<W> o;
#pragma unroll
        for (int e = 0; e < W; ++e) o.v[e] = (x.v[e] > 0.0f) ? x.v[e] : 0.0f;
        sstore<W>(out, i, o);
    }
};

template <int W>
struct ReluBwdOp {
    const float* in;
    const float* g;
    float* gin;
    __device__ void operator()(size_t i) const {
        const fvec<W> x = sload<W>(in, i), d = sload<W>(g, i);
        fvec<W> o;
#pragma unroll
        for (int e = 0; e < W; ++e) o.v[e] = (x.v[e] > 0.0f) ? d.v[e] : 0.0f;
        sstore<W>(gin, i, o);
    }
};

template <class Op>
__global__ __launch_bounds__(kThreads) void flat_kernel(const void* w0, const void* w1,
                                                        const void* w2, long long nvec) {
    const Op op = op_from<Op>(w0, w1, w2);
    const long long stride = static_cast<long long>(gridDim.x) * kThreads;
    for (long long i = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; i < nvec;
         i += stride)
        op(static_cast<size_t>(i));
}

template <class Op>
int launch_flat(const char* name, Op op, long long nvec, hipStream_t st) {
    if (nvec <= 0) return MI_OK;
    long long grid = (nvec + kThreads - 1) / kThreads;
    if (grid > MI_FLAT_MAX_GRID) grid = MI_FLAT_MAX_GRID;
    const OpWords ow = op_words(op);
    hipLaunchKernelGGL(flat_kernel<Op>, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, st,
                       ow.w0, ow.w1, ow.w2, nvec);
    return check_launch(name);
}

// ---------------------------------------------------------------------------
// Row-band broadcast kernels.  An Op provides
//   In load(size_t vec_index) const;          // HBM loads of one vector
//   fvec<W> apply(size_t vec_index, const In&, const fvec<W>& bias,
//                 bool store = true) const;
// apply() writes the output vector (if any, and if `store`) and returns the
// vector that contributes to the column sum (ignored by the non-reducing
// kernel).
//
// A workgroup of T threads covers whole rows: thread t owns the column
// vectors j = t + k*T, k < NC, and keeps their bias vectors and column sums
// in registers.  Workgroup b handles rows b, b + G, b + 2G, ... (G = grid
// size), so at any moment the resident workgroups stream one contiguous band
// of rows and HBM sees a linear sweep.  Rows are processed in batches of U
// (default 1): the batch's loads are issued together, then the batch is
// computed and stored.  On the [8192, 3072] GELU backward, one row per batch
// measured 49.5 us against 50.8 / 53.5 / 54.1 us for 2 / 3 / 4 rows, and
// keeping a second batch in flight during the computation was about 3 us
// slower still.  Rows wider than 4 x 1024 vectors use the column-slice
// fallback below.
// ---------------------------------------------------------------------------
template <int W, int NC, class Op, bool REDUCE>
__global__ __launch_bounds__(1024) void rowband_kernel(const void* w0, const void* w1,
                                                       const void* w2,
                                                       const float* __restrict__ bias,
                                                       float* __restrict__ part, int rows, int nv,
                                                       int T, int G) {
    const Op op = op_from<Op>(w0, w1, w2);
    // Rows per batch (MI_EW_UNROLL, default 1); widths of 3+ vectors per
    // thread use single rows to stay within the 128 VGPRs a 1024-thread
    // workgroup allows (no spills).
    constexpr int U = NC <= 2 ? kUnroll : 1;
    // T and G (blockDim.x and gridDim.x) arrive as arguments, preloaded with
    // the others: read through the dispatch they are scalar loads in front
    // of the first row's loads.
    fvec<W> bv[NC], acc[NC];
#pragma unroll
    for (int k = 0; k < NC; ++k) {
        const int j = threadIdx.x + k * T;
        bv[k] = (bias && j < nv) ? vload<W>(bias, j) : vzero<W>();
        acc[k] = vzero<W>();
    }
    // Loads are unconditional: row and column indices are clamped into the
    // tensor and the results of clamped slots are discarded, so the loads
    // carry no branches and the compiler waits for each row just before it
    // is used.
    using In = typename Op::In;
    auto load_batch = [&](unsigned r, In (&d)[U][NC]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const unsigned row = r + static_cast<unsigned>(u * G);
            const int rr = row < static_cast<unsigned>(rows) ? static_cast<int>(row) : rows - 1;
#pragma unroll
            for (int k = 0; k < NC; ++k) {
                const int j = threadIdx.x + k * T;
                const int jj = j < nv ? j : nv - 1;
                d[u][k] = op.load(static_cast<size_t>(rr) * nv + jj);
            }
        }
    };
    // Clamped slots compute a discarded value; only the store and the
    // column-sum update are predicated.  The batch's inputs are consumed
    // unconditionally before the first store, so no load is sunk into a
    // predicated store and no wait has to cover a store.
    auto run_batch = [&](unsigned r, const In (&d)[U][NC]) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int k = 0; k < NC; ++k) d[u][k].consume();
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const unsigned row = r + static_cast<unsigned>(u * G);
            const bool row_ok = row < static_cast<unsigned>(rows);
            const size_t rb = static_cast<size_t>(row_ok ? row : 0) * nv;
#pragma unroll
            for (int k = 0; k < NC; ++k) {
                const int j = threadIdx.x + k * T;
                const bool ok = row_ok && j < nv;
                const fvec<W> c = op.apply(rb + (j < nv ? j : 0), d[u][k], bv[k], ok);
                if constexpr (REDUCE) {
#pragma unroll
                    for (int e = 0; e < W; ++e) acc[k].v[e] += ok ? c.v[e] : 0.0f;
                }
            }
        }
    };
    // Row numbers and the trip count are unsigned: with rows near INT_MAX,
    // the last batch's row numbers and rows - first + step - 1 exceed the
    // int range (rows < 2^31 and step <= 2^20 keep them below 2^32).
    const unsigned step = static_cast<unsigned>(U * G);
    const unsigned first = blockIdx.x;
    const unsigned iters = strided_trips(first, static_cast<unsigned>(rows), step);
    In A[U][NC];
    unsigned r = first;
    for (unsigned i = 0; i < iters; ++i, r += step) {
        load_batch(r, A);
        run_batch(r, A);
    }
    if constexpr (REDUCE) {
        float* prow = part + static_cast<size_t>(blockIdx.x) * nv * W;
#pragma unroll
        for (int k = 0; k < NC; ++k) {
            const int j = threadIdx.x + k * T;
            if (j < nv) vstore<W>(prow, j, acc[k]);
        }
    }
}

template <int W>
struct ResidBiasOp {  // out = (a + x) + bias
    const float* a;
    const float* x;
    float* out;
    struct In {
        fvec<W> a, x;
        __device__ void consume() const {
            mi::consume(a);
            mi::consume(x);
        }
    };
    __device__ In load(size_t i) const { return {sload<W>(a, i), sload<W>(x, i)}; }
    __device__ fvec<W> apply(size_t i, const In& in, const fvec<W>& b, bool store = true) const {
        fvec<W> o;
#pragma unroll
        for (int e = 0; e < W; ++e) o.v[e] = in.a.v[e] + in.x.v[e] + b.v[e];
        if (store) sstore<W>(out, i, o);
        return o;
    }
};

template <int W>
struct BiasAddOp {  // out += bias (in place)
    float* out;
    struct In {
        fvec<W> o;
        __device__ void consume() const { mi::consume(o); }
    };
    __device__ In load(size_t i) const { return {sload<W>(out, i)}; }
    __device__ fvec<W> apply(size_t i, const In& in, const fvec<W>& b, bool store = true) const {
        fvec<W> o;
#pragma unroll
        for (int e = 0; e < W; ++e) o.v[e] = in.o.v[e] + b.v[e];
        if (store) sstore<W>(out, i, o);
        return o;
    }
};

template <int W>
struct BiasReluOp {  // out = max(in + bias, 0)
    const float* in;
    float* out;
    struct In {
        fvec<W> x;
        __device__ void consume() const { mi::consume(x); }
    };
    __device__ In load(size_t i) const { return {sload<W>(in, i)}; }
    __device__ fvec<W> apply(size_t i, const In& v, const fvec<W>& b, bool store = true) const {
        fvec<W> o;
#pragma unroll
        for (int e = 0; e < W; ++e) {
            const float t = v.x.v[e] + b.v[e];
            o.v[e] = (t > 0.0f) ? t : 0.0f;
        }
        if (store) sstore<W>(out, i, o);
        return o;
    }
};

template <int W>
struct BiasGeluOp {  // out = gelu(in + bias)
    const float* in;
    float* out;
    struct In {
        fvec<W> x;
        __device__ void consume() const { mi::consume(x); }
    };
    __device__ In load(size_t i) const { return {sload<W>(in, i)}; }
    __device__ fvec<W> apply(size_t i, const In& v, const fvec<W>& b, bool store = true) const {
        fvec<W> o;
#pragma unroll
        for (int e = 0; e < W; ++e) o.v[e] = gelu_fwd(v.x.v[e] + b.v[e]);
        if (store) sstore<W>(out, i, o);
        return o;
    }
};

template <int W>
struct ColSumOp {  // dbias partials of grad
    const float* g;
    struct In {
        fvec<W> g;
        __device__ void consume() const { mi::consume(g); }
    };
    __device__ In load(size_t i) const { return {sload<W>(g, i)}; }
    __device__ fvec<W> apply(size_t, const In& v, const fvec<W>&, bool = true) const {
        return v.g;
    }
};

template <int W>
struct ReluBwdBiasOp {  // gin = mask > 0 ? g : 0
    const float* mask;
    const float* g;
    float* gin;
    struct In {
        fvec<W> m, g;
        __device__ void consume() const {
            mi::consume(m);
            mi::consume(g);
        }
    };
    __device__ In load(size_t i) const { return {sload<W>(mask, i), sload<W>(g, i)}; }
    __device__ fvec<W> apply(size_t i, const In& v, const fvec<W>&, bool store = true) const {
        fvec<W> o;
#pragma unroll
        for (int e = 0; e < W; ++e) o.v[e] = (v.m.v[e] > 0.0f) ? v.g.v[e] : 0.0f;
        if (store) sstore<W>(gin, i, o);
        return o;
    }
};

template <int W>
struct GeluBwdBiasOp {  // gin = g * gelu'(in + bias)
    const float* in;
    const float* g;
    float* gin;
    struct In {
        fvec<W> x, g;
        __device__ void consume() const {
            mi::consume(x);
            mi::consume(g);
        }
    };
    __device__ In load(size_t i) const { return {sload<W>(in, i), sload<W>(g, i)}; }
    __device__ fvec<W> apply(size_t i, const In& v, const fvec<W>& b, bool store = true) const {
        fvec<W> o;
#pragma unroll
        for (int e = 0; e < W; ++e) o.v[e] = v.g.v[e] * gelu_grad(v.x.v[e] + b.v[e]);
        if (store) sstore<W>(gin, i, o);
        return o;
    }
};

// ----- 16-bit storage variants (the reference's fp16 storage path,
// activations.cu:199-217,285-347, plus bf16) --------------------------------

template <int W, Fmt16 T>
struct BiasRelu16Op {  // out16 = to16(max(in + bias, 0))
    const float* in;
    uint16_t* out;
    struct In {
        fvec<W> x;
        __device__ void consume() const { mi::consume(x); }
    };
    __device__ In load(size_t i) const { return {sload<W>(in, i)}; }
    __device__ fvec<W> apply(size_t i, const In& v, const fvec<W>& b, bool store = true) const {
        fvec<W> o;
#pragma unroll
        for (int e = 0; e < W; ++e) {
            const float t = v.x.v[e] + b.v[e];
            o.v[e] = (t > 0.0f) ? t : 0.0f;
        }
        if (store) store16<W, T>(out, i, o);
        return o;
    }
};

template <int W, Fmt16 T>
struct BiasGelu16Op {  // out16 = to16(gelu(in + bias))
    const float* in;
    uint16_t* out;
    struct In {
        fvec<W> x;
        __device__ void consume() const { mi::consume(x); }
    };
    __device__ In load(size_t i) const { return {sload<W>(in, i)}; }
    __device__ fvec<W> apply(size_t i, const In& v, const fvec<W>& b, bool store = true) const {
        fvec<W> o;
#pragma unroll
        for (int e = 0; e < W; ++e) o.v[e] = gelu_fwd(v.x.v[e] + b.v[e]);
        if (store) store16<W, T>(out, i, o);
        return o;
    }
};

template <int W, Fmt16 T>
struct ReluBwdMask16Op {  // gin = from16(mask) > 0 ? g : 0
    const uint16_t* mask;
    const float* g;
    float* gin;
    struct In {
        fvec<W> m, g;
        __device__ void consume() const {
            mi::consume(m);
            mi::consume(g);
        }
    };
    __device__ In load(size_t i) const { return {load16<W, T>(mask, i), sload<W>(g, i)}; }
    __device__ fvec<W> apply(size_t i, const In& v, const fvec<W>&, bool store = true) const {
        fvec<W> o;
#pragma unroll
        for (int e = 0; e < W; ++e) o.v[e] = (v.m.v[e] > 0.0f) ? v.g.v[e] : 0.0f;
        if (store) sstore<W>(gin, i, o);
        return o;
    }
};

template <int W, Fmt16 T>
struct To16Op {
    const float* in;
    uint16_t* out;
    __device__ void operator()(size_t i) const { store16<W, T>(out, i, sload<W>(in, i)); }
};

template <int W, Fmt16 T>
struct From16Op {
    const uint16_t* in;
    float* out;
    __device__ void operator()(size_t i) const { sstore<W>(out, i, load16<W, T>(in, i)); }
};

int check_shape(const char* name, int rows, int cols) {
    if (rows < 0 || cols <= 0)
        return set_error(MI_ERR_INVALID_ARG, "%s: invalid shape rows=%d cols=%d", name, rows,
                         cols);
    return MI_OK;
}

// Fallback for rows wider than the row-band kernels cover (more than
// kMaxNC*1024 vectors): thread j of column block blockIdx.x owns one column
// vector and walks the rows of slice blockIdx.y in order; one partial row per
// slice.  Used only for very wide rows, where it is still coalesced.
template <int W, class Op, bool REDUCE>
__global__ __launch_bounds__(kThreads) void colslice_kernel(const void* w0,
                                                            const void* w1,
                                                            const void* w2,
                                                            const float* __restrict__ bias,
                                                            float* __restrict__ part, int rows,
                                                            int nv, int rps) {
    const Op op = op_from<Op>(w0, w1, w2);
    const int j = blockIdx.x * kThreads + threadIdx.x;
    if (j >= nv) return;
    const int r0 = blockIdx.y * rps;
    const int r1 = min(r0 + rps, rows);
    const fvec<W> bv = bias ? vload<W>(bias, j) : vzero<W>();
    fvec<W> acc = vzero<W>();
    for (int r = r0; r < r1; ++r) {
        const typename Op::In in = op.load(static_cast<size_t>(r) * nv + j);
        const fvec<W> c = op.apply(static_cast<size_t>(r) * nv + j, in, bv);
        if constexpr (REDUCE) {
#pragma unroll
            for (int e = 0; e < W; ++e) acc.v[e] += c.v[e];
        }
    }
    if constexpr (REDUCE) vstore<W>(part + static_cast<size_t>(blockIdx.y) * nv * W, j, acc);
}

constexpr int kSlices = 64;

// Unsigned 32-bit division by a run-time constant d with a precomputed
// multiplier (Granlund & Montgomery 1994): l = ceil(log2 d),
// m = floor(2^32 (2^l - d) / d) + 1, q = (t + ((n - t) >> 1)) >> (l - 1) with
// t = umulhi(n, m); exact for every n < 2^32 and d >= 2 (d = 1 handled apart).
struct UDiv {
    unsigned m;
    int l;
    unsigned d;
};

inline UDiv make_udiv(unsigned d) {
    UDiv u{0u, 0, d};
    if (d > 1) {
        int l = 0;
        while ((1ull << l) < d) ++l;
        u.l = l;
        u.m = static_cast<unsigned>((((1ull << 32) * ((1ull << l) - d)) / d) + 1);
    }
    return u;
}

__device__ __forceinline__ unsigned udiv(unsigned n, const UDiv& u) {
    if (u.d == 1) return n;
    const unsigned t = __umulhi(n, u.m);
    return (t + ((n - t) >> 1)) >> (u.l - 1);
}

// Flat grid-stride variant of the non-reducing broadcast kernels: thread i
// takes vectors i, i + stride, ...; the bias column is i mod nv.
template <int W, class Op>
__global__ __launch_bounds__(kThreads) void flatbias_kernel(const void* w0,
                                                            const void* w1,
                                                            const void* w2,
                                                            const float* __restrict__ bias,
                                                            unsigned nvec, unsigned div_m,
                                                            int div_l, unsigned div_d) {
    const Op op = op_from<Op>(w0, w1, w2);
    const UDiv row_div{div_m, div_l, div_d};
    const unsigned stride = gridDim.x * kThreads;
    for (unsigned i = blockIdx.x * kThreads + threadIdx.x; i < nvec; i += stride) {
        const unsigned j = i - udiv(i, row_div) * row_div.d;
        const fvec<W> b = vload<W>(bias, j);
        const typename Op::In in = op.load(i);
        (void)op.apply(i, in, b);
    }
}

// The same walk with a stride that is a multiple of nv: every vector a
// thread visits is in the same bias column, so the bias vector is loaded
// once per thread and no division runs in the loop ([8192, 3072]: bias+ReLU
// 33.1 -> 32.6 us, bias+GELU 33.1 -> 32.8 us, against 31.7 us for a plain
// copy of the same bytes).
//
// The first data load is issued before the column is worked out, and the
// column comes from the workgroup's base (uniform: one scalar division per
// wave) plus the thread index, wrapped once when nv >= kThreads, instead of
// a per-lane division: these workgroups live for one or two vectors, so the
// prologue's latency sits in front of every thread's first load ([8192,
// 3072] bias+GELU and bias+ReLU measured 1.45 us slower than a plain copy of
// the same bytes with the division and bias load first).
template <int W, class Op>
__global__ __launch_bounds__(kThreads) void flatcol_kernel(const void* w0,
                                                           const void* w1,
                                                           const void* w2,
                                                           const float* __restrict__ bias,
                                                           unsigned nvec, unsigned nv) {
    const Op op = op_from<Op>(w0, w1, w2);
    const unsigned stride = gridDim.x * kThreads;
    const unsigned base = blockIdx.x * kThreads;
    unsigned i = base + threadIdx.x;
    if (i >= nvec) return;
    typename Op::In in = op.load(i);
    unsigned j;
    if (nv >= kThreads) {
        j = base % nv + threadIdx.x;
        if (j >= nv) j -= nv;
    } else {
        j = i % nv;
    }
    const fvec<W> b = vload<W>(bias, j);
    for (;;) {
        (void)op.apply(i, in, b);
        i += stride;
        if (i >= nvec) break;
        in = op.load(i);
    }
}

// Workgroups of the column-fixed walk.  Up to MI_FLAT_MAX_GRID workgroups
// every thread takes at most one vector, so any grid will do; beyond that
// the grid is a multiple of q = nv / gcd(nv, kThreads), so that
// grid * kThreads is a multiple of nv, at most MI_FLAT_MAX_GRID; 0 when q
// itself is larger.
long long flatcol_grid(unsigned long long nvec, int nv) {
    const long long want = (static_cast<long long>(nvec) + kThreads - 1) / kThreads;
    if (want <= MI_FLAT_MAX_GRID) return want;
    int a = nv, b = kThreads;
    while (b != 0) {
        const int t = a % b;
        a = b;
        b = t;
    }
    const long long q = nv / a;
    return q <= MI_FLAT_MAX_GRID ? MI_FLAT_MAX_GRID / q * q : 0;
}

#ifndef MI_FWD_FLAT
#define MI_FWD_FLAT 1
#endif

// Workgroup shape: NC column vectors per thread, T threads (a multiple of
// 64, at most 1024) so that NC * T covers the row with the least padding.
struct BandShape {
    int nc;
    int threads;
};

constexpr int kMaxNC = 4;

BandShape band_shape(int nv) {
    int nc = (nv + 1023) / 1024;
    if (nc > kMaxNC) nc = kMaxNC;
    const int per = (nv + nc - 1) / nc;
    int threads = ((per + kWave - 1) / kWave) * kWave;
    if (threads > 1024) threads = 1024;
    return {nc, threads};
}

// Workgroups of the non-reducing kernels: enough for about two resident
// workgroups per CU on a 256-CU device.
constexpr int kFwdBands = MI_FWD_BANDS;

template <int W, class Op, bool REDUCE>
void launch_band(const BandShape& b, int grid, Op op, const float* bias, float* part, int rows,
                 int nv, hipStream_t st) {
#define MI_BAND_CASE(NN)                                                                   \
    case NN:                                                                               \
        hipLaunchKernelGGL((rowband_kernel<W, NN, Op, REDUCE>), dim3(grid), dim3(b.threads), \
                           0, st, ow.w0, ow.w1, ow.w2, bias, part, rows, nv, b.threads,    \
                           grid);                                                          \
        break;
    const OpWords ow = op_words(op);
    switch (b.nc) {
        MI_BAND_CASE(1)
        MI_BAND_CASE(2)
        MI_BAND_CASE(3)
        MI_BAND_CASE(4)
        default:
            break;
    }
#undef MI_BAND_CASE
}

bool band_fits(int nv) { return nv <= kMaxNC * 1024; }

template <int W, class Op>
int launch_rowtile(const char* name, Op op, const float* bias, int rows, int cols,
                   hipStream_t st) {
    const int nv = cols / W;
    const unsigned long long nvec = static_cast<unsigned long long>(rows) * nv;
    // The flat kernel walks 32-bit vector indices: below 2^31 vectors,
    // i + stride (stride <= MI_FLAT_MAX_GRID * kThreads) cannot wrap past
    // 2^32 and restart the walk.  Larger tensors take the row bands, whose
    // offsets are 64-bit.
    const long long cgrid = nvec < (1ull << 31) ? flatcol_grid(nvec, nv) : 0;
    const OpWords ow = op_words(op);
    if (MI_FWD_FLAT && cgrid > 0) {
        hipLaunchKernelGGL((flatcol_kernel<W, Op>), dim3(static_cast<unsigned>(cgrid)),
                           dim3(kThreads), 0, st, ow.w0, ow.w1, ow.w2, bias,
                           static_cast<unsigned>(nvec), static_cast<unsigned>(nv));
    } else if (MI_FWD_FLAT && nvec < (1ull << 31)) {
        long long grid = (static_cast<long long>(nvec) + kThreads - 1) / kThreads;
        if (grid > MI_FLAT_MAX_GRID) grid = MI_FLAT_MAX_GRID;
        const UDiv dv = make_udiv(static_cast<unsigned>(nv));
        hipLaunchKernelGGL((flatbias_kernel<W, Op>), dim3(static_cast<unsigned>(grid)),
                           dim3(kThreads), 0, st, ow.w0, ow.w1, ow.w2, bias,
                           static_cast<unsigned>(nvec), dv.m, dv.l, dv.d);
    } else if (band_fits(nv)) {
        const BandShape b = band_shape(nv);
        const int grid = rows < kFwdBands ? rows : kFwdBands;
        launch_band<W, Op, false>(b, grid, op, bias, nullptr, rows, nv, st);
    } else {
        const int rps = static_cast<int>((static_cast<long long>(rows) + kSlices - 1) / kSlices);
        const dim3 grid((nv + kThreads - 1) / kThreads,
                        static_cast<unsigned>((static_cast<long long>(rows) + rps - 1) / rps));
        hipLaunchKernelGGL((colslice_kernel<W, Op, false>), grid, dim3(kThreads), 0, st, ow.w0,
                           ow.w1, ow.w2, bias, nullptr, rows, nv, rps);
    }
    return check_launch(name);
}

// Partial rows of the reducing kernels: one per row-band workgroup (at most
// MI_REDUCE_TILES), or one per row slice in the wide-row fallback.  Depends
// only on the shape, so the summation order is fixed for a given shape.
int plan_reduce_parts(int rows, int nv) {
    if (!band_fits(nv)) {
        const int rps = static_cast<int>((static_cast<long long>(rows) + kSlices - 1) / kSlices);
        return static_cast<int>((static_cast<long long>(rows) + rps - 1) / rps);
    }
    return rows < MI_REDUCE_TILES ? rows : MI_REDUCE_TILES;
}

template <int W, class Op>
int launch_rowtile_reduce(const char* name, Op op, const float* bias, float* dbias, int rows,
                          int cols, hipStream_t st) {
    const int nv = cols / W;
    const int P = plan_reduce_parts(rows, nv);
    int err = MI_OK;
    char* ws = static_cast<char*>(workspace_get(colsum_bytes(P, cols), st, &err));
    if (!ws) return err;
    float* part = reinterpret_cast<float*>(ws + colsum_part_offset());
    if (band_fits(nv)) {
        launch_band<W, Op, true>(band_shape(nv), P, op, bias, part, rows, nv, st);
    } else {
        const int rps = static_cast<int>((static_cast<long long>(rows) + kSlices - 1) / kSlices);
        const dim3 grid((nv + kThreads - 1) / kThreads, P);
        const OpWords ow = op_words(op);
        hipLaunchKernelGGL((colslice_kernel<W, Op, true>), grid, dim3(kThreads), 0, st, ow.w0,
                           ow.w1, ow.w2, bias, part, rows, nv, rps);
    }
    int rc = check_launch(name);
    if (rc != MI_OK) return rc;
    return launch_colsum_finalize(part, P, cols, dbias, cols, nullptr, st);
}

bool all_aligned(std::initializer_list<const void*> ps) {
    for (const void* p : ps)
        if (p && !aligned16(p)) return false;
    return true;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" {

size_t mi_bias_backward_workspace(int rows, int cols) {
    if (rows <= 0 || cols <= 0) return 0;
    // the vec4 and scalar plans can differ; report the larger
    const size_t a = colsum_bytes(plan_reduce_parts(rows, cols / 4), cols);
    const size_t b = colsum_bytes(plan_reduce_parts(rows, cols), cols);
    return a > b ? a : b;
}

int mi_residual_add(const float* a, const float* b, float* out, long long n, void* stream) {
    if (n < 0) return set_error(MI_ERR_INVALID_ARG, "mi_residual_add: n=%lld", n);
    if (n == 0) return MI_OK;
    if (!a || !b || !out) return set_error(MI_ERR_INVALID_ARG, "mi_residual_add: NULL pointer");
    if (n % 4 == 0 && all_aligned({a, b, out}))
        return launch_flat("mi_residual_add", AddOp<4>{a, b, out}, n / 4, to_stream(stream));
    return launch_flat("mi_residual_add", AddOp<1>{a, b, out}, n, to_stream(stream));
}

int mi_relu_forward(const float* in, float* out, long long n, void* stream) {
    if (n < 0) return set_error(MI_ERR_INVALID_ARG, "mi_relu_forward: n=%lld", n);
    if (n == 0) return MI_OK;
    if (!in || !out) return set_error(MI_ERR_INVALID_ARG, "mi_relu_forward: NULL pointer");
    if (n % 4 == 0 && all_aligned({in, out}))
        return launch_flat("mi_relu_forward", ReluOp<4>{in, out}, n / 4, to_stream(stream));
    return launch_flat("mi_relu_forward", ReluOp<1>{in, out}, n, to_stream(stream));
}

int mi_relu_backward(const float* in, const float* grad_out, float* grad_in, long long n,
                     void* stream) {
    if (n < 0) return set_error(MI_ERR_INVALID_ARG, "mi_relu_backward: n=%lld", n);
    if (n == 0) return MI_OK;
    if (!in || !grad_out || !grad_in)
        return set_error(MI_ERR_INVALID_ARG, "mi_relu_backward: NULL pointer");
    if (n % 4 == 0 && all_aligned({in, grad_out, grad_in}))
        return launch_flat("mi_relu_backward", ReluBwdOp<4>{in, grad_out, grad_in}, n / 4,
                           to_stream(stream));
    return launch_flat("mi_relu_backward", ReluBwdOp<1>{in, grad_out, grad_in}, n,
                       to_stream(stream));
}

int mi_residual_add_with_bias(const float* residual, const float* x, const float* bias,
                              float* out, int rows, int cols, void* stream) {
    const char* name = "mi_residual_add_with_bias";
    if (int rc = check_shape(name, rows, cols)) return rc;
    if (rows == 0) return MI_OK;
    if (!residual || !x || !bias || !out) return set_error(MI_ERR_INVALID_ARG, "%s: NULL", name);
    if (cols % 4 == 0 && all_aligned({residual, x, bias, out}))
        return launch_rowtile<4>(name, ResidBiasOp<4>{residual, x, out}, bias, rows, cols,
                                 to_stream(stream));
    return launch_rowtile<1>(name, ResidBiasOp<1>{residual, x, out}, bias, rows, cols,
                             to_stream(stream));
}

int mi_bias_add(float* out, const float* bias, int rows, int cols, void* stream) {
    const char* name = "mi_bias_add";
    if (int rc = check_shape(name, rows, cols)) return rc;
    if (rows == 0) return MI_OK;
    if (!bias || !out) return set_error(MI_ERR_INVALID_ARG, "%s: NULL", name);
    if (cols % 4 == 0 && all_aligned({bias, out}))
        return launch_rowtile<4>(name, BiasAddOp<4>{out}, bias, rows, cols, to_stream(stream));
    return launch_rowtile<1>(name, BiasAddOp<1>{out}, bias, rows, cols, to_stream(stream));
}

int mi_bias_relu_forward(const float* in, const float* bias, float* out, int rows, int cols,
                         void* stream) {
    const char* name = "mi_bias_relu_forward";
    if (int rc = check_shape(name, rows, cols)) return rc;
    if (rows == 0) return MI_OK;
    if (!in || !bias || !out) return set_error(MI_ERR_INVALID_ARG, "%s: NULL", name);
    if (cols % 4 == 0 && all_aligned({in, bias, out}))
        return launch_rowtile<4>(name, BiasReluOp<4>{in, out}, bias, rows, cols,
                                 to_stream(stream));
    return launch_rowtile<1>(name, BiasReluOp<1>{in, out}, bias, rows, cols, to_stream(stream));
}

int mi_bias_gelu_forward(const float* in, const float* bias, float* out, int rows, int cols,
                         void* stream) {
    const char* name = "mi_bias_gelu_forward";
    if (int rc = check_shape(name, rows, cols)) return rc;
    if (rows == 0) return MI_OK;
    if (!in || !bias || !out) return set_error(MI_ERR_INVALID_ARG, "%s: NULL", name);
    if (cols % 4 == 0 && all_aligned({in, bias, out}))
        return launch_rowtile<4>(name, BiasGeluOp<4>{in, out}, bias, rows, cols,
                                 to_stream(stream));
    return launch_rowtile<1>(name, BiasGeluOp<1>{in, out}, bias, rows, cols, to_stream(stream));
}

int mi_bias_backward(const float* grad, float* dbias, int rows, int cols, void* stream) {
    const char* name = "mi_bias_backward";
    if (int rc = check_shape(name, rows, cols)) return rc;
    if (rows == 0) return MI_OK;
    if (!grad || !dbias) return set_error(MI_ERR_INVALID_ARG, "%s: NULL", name);
    if (cols % 4 == 0 && all_aligned({grad}))
        return launch_rowtile_reduce<4>(name, ColSumOp<4>{grad}, nullptr, dbias, rows, cols,
                                        to_stream(stream));
    return launch_rowtile_reduce<1>(name, ColSumOp<1>{grad}, nullptr, dbias, rows, cols,
                                    to_stream(stream));
}

int mi_relu_backward_with_bias_backward(const float* mask, const float* grad_out, float* grad_in,
                                        float* dbias, int rows, int cols, void* stream) {
    const char* name = "mi_relu_backward_with_bias_backward";
    if (int rc = check_shape(name, rows, cols)) return rc;
    if (rows == 0) return MI_OK;
    if (!mask || !grad_out || !grad_in || !dbias)
        return set_error(MI_ERR_INVALID_ARG, "%s: NULL", name);
    if (cols % 4 == 0 && all_aligned({mask, grad_out, grad_in}))
        return launch_rowtile_reduce<4>(name, ReluBwdBiasOp<4>{mask, grad_out, grad_in}, nullptr,
                                        dbias, rows, cols, to_stream(stream));
    return launch_rowtile_reduce<1>(name, ReluBwdBiasOp<1>{mask, grad_out, grad_in}, nullptr,
                                    dbias, rows, cols, to_stream(stream));
}

int mi_gelu_backward_with_bias_backward(const float* in, const float* bias,
                                        const float* grad_out, float* grad_in, float* dbias,
                                        int rows, int cols, void* stream) {
    const char* name = "mi_gelu_backward_with_bias_backward";
    if (int rc = check_shape(name, rows, cols)) return rc;
    if (rows == 0) return MI_OK;
    if (!in || !bias || !grad_out || !grad_in || !dbias)
        return set_error(MI_ERR_INVALID_ARG, "%s: NULL", name);
    if (cols % 4 == 0 && all_aligned({in, bias, grad_out, grad_in}))
        return launch_rowtile_reduce<4>(name, GeluBwdBiasOp<4>{in, grad_out, grad_in}, bias,
                                        dbias, rows, cols, to_stream(stream));
    return launch_rowtile_reduce<1>(name, GeluBwdBiasOp<1>{in, grad_out, grad_in}, bias, dbias,
                                    rows, cols, to_stream(stream));
}

}  // extern "C"

// ----- 16-bit storage ---------------------------------------------------------

namespace {

template <Fmt16 T>
int convert_to16(const char* name, const float* in, void* out, long long n, void* stream) {
    if (n < 0) return set_error(MI_ERR_INVALID_ARG, "%s: n=%lld", name, n);
    if (n == 0) return MI_OK;
    if (!in || !out) return set_error(MI_ERR_INVALID_ARG, "%s: NULL pointer", name);
    uint16_t* o = static_cast<uint16_t*>(out);
    if (n % 4 == 0 && aligned16(in) && aligned8(o))
        return launch_flat(name, To16Op<4, T>{in, o}, n / 4, to_stream(stream));
    return launch_flat(name, To16Op<1, T>{in, o}, n, to_stream(stream));
}

template <Fmt16 T>
int convert_from16(const char* name, const void* in, float* out, long long n, void* stream) {
    if (n < 0) return set_error(MI_ERR_INVALID_ARG, "%s: n=%lld", name, n);
    if (n == 0) return MI_OK;
    if (!in || !out) return set_error(MI_ERR_INVALID_ARG, "%s: NULL pointer", name);
    const uint16_t* i16 = static_cast<const uint16_t*>(in);
    if (n % 4 == 0 && aligned8(i16) && aligned16(out))
        return launch_flat(name, From16Op<4, T>{i16, out}, n / 4, to_stream(stream));
    return launch_flat(name, From16Op<1, T>{i16, out}, n, to_stream(stream));
}

template <Fmt16 T, bool GELU>
int bias_act_to16(const char* name, const float* in, const float* bias, void* out, int rows,
                  int cols, void* stream) {
    if (int rc = check_shape(name, rows, cols)) return rc;
    if (rows == 0) return MI_OK;
    if (!in || !bias || !out) return set_error(MI_ERR_INVALID_ARG, "%s: NULL", name);
    uint16_t* o = static_cast<uint16_t*>(out);
    const bool vec4 = cols % 4 == 0 && aligned16(in) && aligned16(bias) && aligned8(o);
    if constexpr (GELU) {
        if (vec4)
            return launch_rowtile<4>(name, BiasGelu16Op<4, T>{in, o}, bias, rows, cols,
                                     to_stream(stream));
        return launch_rowtile<1>(name, BiasGelu16Op<1, T>{in, o}, bias, rows, cols,
                                 to_stream(stream));
    } else {
        if (vec4)
            return launch_rowtile<4>(name, BiasRelu16Op<4, T>{in, o}, bias, rows, cols,
                                     to_stream(stream));
        return launch_rowtile<1>(name, BiasRelu16Op<1, T>{in, o}, bias, rows, cols,
                                 to_stream(stream));
    }
}

template <Fmt16 T>
int relu_bwd_mask16(const char* name, const void* mask, const float* grad_out, float* grad_in,
                    float* dbias, int rows, int cols, void* stream) {
    if (int rc = check_shape(name, rows, cols)) return rc;
    if (rows == 0) return MI_OK;
    if (!mask || !grad_out || !grad_in || !dbias)
        return set_error(MI_ERR_INVALID_ARG, "%s: NULL", name);
    const uint16_t* m = static_cast<const uint16_t*>(mask);
    if (cols % 4 == 0 && aligned8(m) && all_aligned({grad_out, grad_in}))
        return launch_rowtile_reduce<4>(name, ReluBwdMask16Op<4, T>{m, grad_out, grad_in},
                                        nullptr, dbias, rows, cols, to_stream(stream));
    return launch_rowtile_reduce<1>(name, ReluBwdMask16Op<1, T>{m, grad_out, grad_in}, nullptr,
                                    dbias, rows, cols, to_stream(stream));
}

}  // namespace

extern "C" {

int mi_float_to_half(const float* in, void* out, long long n, void* stream) {
    return convert_to16<Fmt16::Half>("mi_float_to_half", in, out, n, stream);
}

int mi_half_to_float(const void* in, float* out, long long n, void* stream) {
    return convert_from16<Fmt16::Half>("mi_half_to_float", in, out, n, stream);
}

int mi_float_to_bf16(const float* in, void* out, long long n, void* stream) {
    return convert_to16<Fmt16::BF16>("mi_float_to_bf16", in, out, n, stream);
}

int mi_bf16_to_float(const void* in, float* out, long long n, void* stream) {
    return convert_from16<Fmt16::BF16>("mi_bf16_to_float", in, out, n, stream);
}

int mi_bias_relu_forward_to_half(const float* in, const float* bias, void* out, int rows,
                                 int cols, void* stream) {
    return bias_act_to16<Fmt16::Half, false>("mi_bias_relu_forward_to_half", in, bias, out, rows,
                                             cols, stream);
}

int mi_bias_gelu_forward_to_half(const float* in, const float* bias, void* out, int rows,
                                 int cols, void* stream) {
    return bias_act_to16<Fmt16::Half, true>("mi_bias_gelu_forward_to_half", in, bias, out, rows,
                                            cols, stream);
}

int mi_bias_gelu_forward_to_bf16(const float* in, const float* bias, void* out, int rows,
                                 int cols, void* stream) {
    return bias_act_to16<Fmt16::BF16, true>("mi_bias_gelu_forward_to_bf16", in, bias, out, rows,
                                            cols, stream);
}

int mi_relu_backward_with_bias_backward_half_mask(const void* mask, const float* grad_out,
                                                  float* grad_in, float* dbias, int rows,
                                                  int cols, void* stream) {
    return relu_bwd_mask16<Fmt16::Half>("mi_relu_backward_with_bias_backward_half_mask", mask,
                                        grad_out, grad_in, dbias, rows, cols, stream);
}

}  // extern "C"
