// Device runtime of the kernels that the general lowering (stade_hip.lower) writes for
// generated STADE text: Julia's arithmetic semantics and the accumulation primitives.
//
// Julia semantics kept (1-based indexing is applied by the generated code itself):
//   mod floored (sign of the divisor), div truncated, `x^2` = x*x (Base.literal_pow),
//   max / min on floats propagate NaN and order -0.0 < 0.0, sign(0) = 0.
// Accumulation into a shadow array at an index that other threads may share:
//   wave_add: if the whole wave is active and every lane adds into the same element, the
//   wave's values are summed across lanes and one lane makes the atomic addition (the
//   wave-aggregated atomic); otherwise each lane adds atomically.  Floating-point atomics
//   use the hardware instructions (unsafeAtomicAdd): the order of the additions is left to
//   the hardware, as the generated adjoint's `@atomic` leaves it.
//   block_add: a value a thread has summed in a register over its iterations (a loop's sum
//   into a scalar, or into an array element whose index does not change over the loop: the
//   reference's hoisted atomic), added once per block.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

namespace stade_lowered {

__device__ __forceinline__ int64_t jl_mod(int64_t a, int64_t b) {
    int64_t r = a % b;
    return (r != 0 && ((r < 0) != (b < 0))) ? r + b : r;
}
__device__ __forceinline__ double jl_mod(double a, double b) {
    double r = fmod(a, b);
    return (r != 0.0 && ((r < 0.0) != (b < 0.0))) ? r + b : r;
}
__device__ __forceinline__ float jl_mod(float a, float b) {
    float r = fmodf(a, b);
    return (r != 0.0f && ((r < 0.0f) != (b < 0.0f))) ? r + b : r;
}
__device__ __forceinline__ int64_t jl_fld(int64_t a, int64_t b) {
    int64_t q = a / b;
    return (q * b != a && ((a < 0) != (b < 0))) ? q - 1 : q;
}
__device__ __forceinline__ int64_t jl_cld(int64_t a, int64_t b) {
    int64_t q = a / b;
    return (q * b != a && ((a < 0) == (b < 0))) ? q + 1 : q;
}
// number of values of lo:step:hi
__device__ __host__ __forceinline__ int64_t jl_trip(int64_t lo, int64_t step, int64_t hi) {
    int64_t t = (hi - lo + step) / step;
    return t > 0 ? t : 0;
}

template <class T>
__device__ __forceinline__ T jl_maxf(T a, T b) {
    if (a != a) return a;
    if (b != b) return b;
    if (a == b) return signbit(a) ? b : a;  // max(-0.0, 0.0) = 0.0
    return a > b ? a : b;
}
template <class T>
__device__ __forceinline__ T jl_minf(T a, T b) {
    if (a != a) return a;
    if (b != b) return b;
    if (a == b) return signbit(a) ? a : b;
    return a < b ? a : b;
}
__device__ __forceinline__ int64_t jl_max(int64_t a, int64_t b) { return a > b ? a : b; }
__device__ __forceinline__ int64_t jl_min(int64_t a, int64_t b) { return a < b ? a : b; }
__device__ __forceinline__ double jl_max(double a, double b) { return jl_maxf(a, b); }
__device__ __forceinline__ double jl_min(double a, double b) { return jl_minf(a, b); }
__device__ __forceinline__ float jl_max(float a, float b) { return jl_maxf(a, b); }
__device__ __forceinline__ float jl_min(float a, float b) { return jl_minf(a, b); }

template <class T>
__device__ __forceinline__ T jl_sign(T x) {
    return x > T(0) ? T(1) : (x < T(0) ? T(-1) : x);
}
__device__ __forceinline__ int64_t jl_ipow(int64_t b, int64_t e) {
    int64_t r = 1;
    while (e > 0) {
        if (e & 1) r *= b;
        b *= b;
        e >>= 1;
    }
    return r;
}

// ---- wave reductions (full wave, 64 lanes) ------------------------------------------------
template <class T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// The lanes-over-iterations form: lane l of every wave holds a partial of the same outer
// iteration, each wave over a share of the inner loop; the block's NW partials of a lane,
// added in wave order through `lds` (NW x 64 slots), in every wave.  Every thread of the
// block must call it.
template <int NW, class T>
__device__ __forceinline__ T xwave_sum(T v, T* lds) {
    const int ln = threadIdx.x & 63, wv = threadIdx.x >> 6;
    lds[wv * 64 + ln] = v;
    __syncthreads();
    T s = lds[ln];
#pragma unroll
    for (int w = 1; w < NW; ++w) s += lds[w * 64 + ln];
    __syncthreads();  // (the slots are reused by the next call)
    return s;
}

__device__ __forceinline__ void atomic_add(double* p, double v) { unsafeAtomicAdd(p, v); }
__device__ __forceinline__ void atomic_add(float* p, float v) { unsafeAtomicAdd(p, v); }
__device__ __forceinline__ void atomic_add(int64_t* p, int64_t v) {
    atomicAdd(reinterpret_cast<unsigned long long*>(p), (unsigned long long)v);
}

// Path statistics (optional; `st` is null unless a caller asked for them, see the
// `_set_stats` entry point of a lowered function): a 64-bit counter per accumulation path,
// counted once per wave or block, so that a test can tell which path a launch took.
enum : int {
    ST_WAVE_AGG = 0,     // wave_add calls that made one atomic for the whole wave
    ST_WAVE_LANE = 1,    // wave_add calls that made one atomic per lane
    ST_PRIV_BLOCK = 2,   // blocks that accumulated into an LDS-privatised copy
    ST_SPLIT_BLOCK = 3,  // blocks of the wave-per-iteration (narrow-output) form
    ST_BLOCK_ADD = 4,    // block_add calls that added a nonzero block total
    ST_ROW_BLOCK = 5,    // blocks of a flat loop's row-block twin
    ST_COL_BLOCK = 6,    // blocks of a flat loop's column-block twin
    ST_XSPLIT_BLOCK = 7, // blocks of the lanes-over-iterations form (waves share the inner loops)
    ST_N = 8,
};

__device__ __forceinline__ void count(unsigned long long* st, int k) {
    if (st) atomicAdd(&st[k], 1ull);
}

template <class T>
__device__ __forceinline__ void wave_add(T* p, T v, unsigned long long* st) {
    const uint64_t active = __ballot(1);
    if (active == ~0ull) {
        const uint64_t u = reinterpret_cast<uint64_t>(p);
        const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u), hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
        T* p0 = reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
        if (__ballot(p == p0) == ~0ull) {
            v = wave_sum(v);
            if ((threadIdx.x & 63) == 0) {
                atomic_add(p0, v);
                count(st, ST_WAVE_AGG);
            }
            return;
        }
    }
    atomic_add(p, v);
    if (st && (threadIdx.x & 63) == (unsigned)__builtin_ctzll(active)) count(st, ST_WAVE_LANE);
}

// One atomic addition per block of the block's values (a loop's sum into a scalar, or its
// accumulations into one array element at an index that does not change over the loop): the
// wave's DPP-free butterfly sum, the waves' sums in order through `lds` (one slot per wave),
// then thread 0 adds the total if it is nonzero.  Every thread of the block must call it;
// `p` may be null only when the block's values are all zero.
template <class T>
__device__ __forceinline__ void block_add(T* p, T v, T* lds, unsigned long long* st) {
    v = wave_sum(v);
    const int nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        T s = lds[0];
        for (int w = 1; w < nw; ++w) s += lds[w];
        if (s != (T)0 && p) {
            atomic_add(p, s);
            count(st, ST_BLOCK_ADD);
        }
    }
    __syncthreads();
}

// LDS-privatised accumulation: the block's copy, then one global atomic per nonzero element
template <class T>
__device__ __forceinline__ void lds_add(T* p, T v) {
    atomicAdd(p, v);
}
__device__ __forceinline__ void lds_add(int64_t* p, int64_t v) {
    atomicAdd(reinterpret_cast<unsigned long long*>(p), (unsigned long long)v);
}

}  // namespace stade_lowered
