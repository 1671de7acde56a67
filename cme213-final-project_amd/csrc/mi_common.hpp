// Shared device helpers and host plumbing for the gfx950 layer kernels.
//
// Device side: wave64 reductions built from DPP row operations plus
// v_readlane, 4-wide vector load/store types, and the launch-shape
// constants.  Host side: the error slot returned through mi_last_error(),
// stream conversion, and the per-device workspace used by the deterministic
// two-pass column reductions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "mi_index.hpp"
#include "mi_kernels.h"

namespace mi {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Vector types.  fvec<4> is 16-byte aligned so a load through it becomes one
// global_load_dwordx4; fvec<1> is the scalar fallback for widths that are not
// a multiple of 4 or pointers that are not 16-byte aligned.
// ---------------------------------------------------------------------------
template <int W>
struct alignas(4 * W) fvec {
    float v[W];
};

template <int W>
__device__ __forceinline__ fvec<W> vzero() {
    fvec<W> r;
#pragma unroll
    for (int e = 0; e < W; ++e) r.v[e] = 0.0f;
    return r;
}

template <int W>
__device__ __forceinline__ fvec<W> vload(const float* base, size_t vec_index) {
    return reinterpret_cast<const fvec<W>*>(base)[vec_index];
}

template <int W>
__device__ __forceinline__ void vstore(float* base, size_t vec_index, const fvec<W>& x) {
    reinterpret_cast<fvec<W>*>(base)[vec_index] = x;
}

// Loads / stores of activation tensors that are touched once per call carry
// the non-temporal hint (global_load/store ... nt): the lines are streamed
// rather than kept in L2 / the last-level cache, which measured faster for
// every operation of the headline step on MI355X (about 8% on the step).
// Parameters (gamma, beta, bias) and partial sums use ordinary accesses.
// Set MI_STREAM_NT_LOAD / MI_STREAM_NT_STORE to 0 to build without the hint.
#ifndef MI_STREAM_NT_LOAD
#define MI_STREAM_NT_LOAD 1
#endif
#ifndef MI_STREAM_NT_STORE
#define MI_STREAM_NT_STORE 1
#endif

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int W>
__device__ __forceinline__ fvec<W> sload(const float* base, size_t vec_index) {
    if constexpr (W == 4 && MI_STREAM_NT_LOAD) {
        const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(base) + vec_index);
        return fvec<4>{{t.x, t.y, t.z, t.w}};
    } else {
        return vload<W>(base, vec_index);
    }
}

template <int W>
__device__ __forceinline__ void sstore(float* base, size_t vec_index, const fvec<W>& x) {
    if constexpr (W == 4 && MI_STREAM_NT_STORE) {
        const f32x4 t = {x.v[0], x.v[1], x.v[2], x.v[3]};
        __builtin_nontemporal_store(t, reinterpret_cast<f32x4*>(base) + vec_index);
    } else {
        vstore<W>(base, vec_index, x);
    }
}

// ---------------------------------------------------------------------------
// 16-bit storage.  Half is IEEE binary16 through the hardware conversion
// (round to nearest even, overflow to inf); BF16 keeps the upper 16 bits of
// the fp32 pattern, rounded to nearest even, with NaN kept a quiet NaN.
// Vectors of 4 move as one 8-byte access.
// ---------------------------------------------------------------------------
enum class Fmt16 { Half, BF16 };

template <Fmt16 T>
__device__ __forceinline__ uint16_t to16(float x) {
    if constexpr (T == Fmt16::Half) {
        return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
    } else {
        const uint32_t u = __float_as_uint(x);
        if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
        return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    }
}

template <Fmt16 T>
__device__ __forceinline__ float from16(uint16_t h) {
    if constexpr (T == Fmt16::Half)
        return static_cast<float>(__builtin_bit_cast(_Float16, h));
    else
        return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int W, Fmt16 T>
__device__ __forceinline__ fvec<W> load16(const uint16_t* base, size_t vec_index) {
    fvec<W> r;
    if constexpr (W == 4) {
        const u32x2 p = reinterpret_cast<const u32x2*>(base)[vec_index];
        r.v[0] = from16<T>(static_cast<uint16_t>(p.x & 0xffffu));
        r.v[1] = from16<T>(static_cast<uint16_t>(p.x >> 16));
        r.v[2] = from16<T>(static_cast<uint16_t>(p.y & 0xffffu));
        r.v[3] = from16<T>(static_cast<uint16_t>(p.y >> 16));
    } else {
#pragma unroll
        for (int e = 0; e < W; ++e) r.v[e] = from16<T>(base[vec_index * W + e]);
    }
    return r;
}

template <int W, Fmt16 T>
__device__ __forceinline__ void store16(uint16_t* base, size_t vec_index, const fvec<W>& x) {
    if constexpr (W == 4) {
        u32x2 p;
        p.x = static_cast<uint32_t>(to16<T>(x.v[0])) | (static_cast<uint32_t>(to16<T>(x.v[1])) << 16);
        p.y = static_cast<uint32_t>(to16<T>(x.v[2])) | (static_cast<uint32_t>(to16<T>(x.v[3])) << 16);
        reinterpret_cast<u32x2*>(base)[vec_index] = p;
    } else {
#pragma unroll
        for (int e = 0; e < W; ++e) base[vec_index * W + e] = to16<T>(x.v[e]);
    }
}

inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

// ---------------------------------------------------------------------------
// Wave64 sum.  Four DPP steps reduce each 16-lane row (quad xor-1, quad
// xor-2, half-row mirror, row mirror); the four row totals are then read
// with v_readlane and added in a fixed order.  Every lane returns the same
// bit pattern, and the association order is fixed by the code, so the
// result is deterministic.  All 64 lanes must be active at the call.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __int_as_float(
        __builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float readlane(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Returns v unchanged but hides how it was computed, so that an add which
// consumes it is rounded on its own instead of being contracted into an FMA
// with the multiply that produced v.  Fused "out += f(...)" paths use it to
// give the same bits as computing f and then adding.
__device__ __forceinline__ float rounded(float v) {
    asm("" : "+v"(v));
    return v;
}

// Marks a loaded vector as used at this point, unconditionally.  Without it
// the compiler may sink a load whose only uses sit under a predicated store
// into that branch, which serialises the loads of a batch and adds full
// memory-queue waits.
template <int W>
__device__ __forceinline__ void consume(const fvec<W>& x) {
#pragma unroll
    for (int e = 0; e < W; ++e) asm volatile("" ::"v"(x.v[e]));
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
    v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
    v += dpp_move<0x141>(v);  // row_half_mirror: 8-lane groups
    v += dpp_move<0x140>(v);  // row_mirror: 16-lane rows
    const float r0 = readlane(v, 0);
    const float r1 = readlane(v, 16);
    const float r2 = readlane(v, 32);
    const float r3 = readlane(v, 48);
    return (r0 + r1) + (r2 + r3);
}

// Wave64 maximum with the same DPP pattern; every lane returns the result.
// (fmaxf is exact and order-independent, so only NaN handling matters: NaN
// operands are ignored, as fmaxf ignores them.)  All 64 lanes must be active.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_move<0xB1>(v));
    v = fmaxf(v, dpp_move<0x4E>(v));
    v = fmaxf(v, dpp_move<0x141>(v));
    v = fmaxf(v, dpp_move<0x140>(v));
    return fmaxf(fmaxf(readlane(v, 0), readlane(v, 16)), fmaxf(readlane(v, 32), readlane(v, 48)));
}

// ---------------------------------------------------------------------------
// Host plumbing (defined in runtime.hip).
// ---------------------------------------------------------------------------
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
inline hipStream_t to_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Returns a device buffer of at least `bytes` for the current device (the
// library-owned workspace), growing it if needed.  Growth is refused while
// `stream` is being captured into a graph.  On failure returns nullptr and
// stores the error code in *err.
void* workspace_get(size_t bytes, hipStream_t stream, int* err);

// out0[c] += sum_p part[p * ncols + c] for c < split, out1[c - split] for
// c >= split; fixed summation order (reduce.hip).
int launch_colsum_finalize(const float* part, int P, int ncols, float* out0, int split,
                           float* out1, hipStream_t stream);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Workspace layout of a two-pass column reduction with P partial rows of
// ncols floats.  The first 256 bytes of the workspace are reserved.
inline size_t colsum_part_offset() { return 256; }

inline size_t colsum_bytes(int P, int ncols) {
    return colsum_part_offset() + static_cast<size_t>(P) * ncols * sizeof(float);
}
}  // namespace mi
