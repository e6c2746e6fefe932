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
//   reference's hoisted atomic), added once per block (the row-block twin's rows).
//   block_part + fold_load / fold_sum: the same block sums in a loop's one-thread-per-
//   iteration grid, stored per block and added in a fixed order by a one-block kernel after
//   the loop.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include <cstring>
#include <mutex>

namespace stade_lowered {

// (an argument within one period of [0, b) -- a periodic neighbour's index, `mod(i - 2, n)` with
// i in 1:n -- by compares and an add, the reference's mod-reduced form (`cgen_mod_reduce_body`
// /root/reference/src/STADE.jl:8126-8169) taken at run time; the division otherwise)
__device__ __forceinline__ int64_t jl_mod(int64_t a, int64_t b) {
    if (b > 0) {
        if (a >= 0 && a < b) return a;
        if (a < 0 && a >= -b) return a + b;
        if (a >= b && a - b < b) return a - b;
    }
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

// The same with G outer iterations a block (G = 16, 32 or 64): lane l of wave w takes
// iteration l % G and share l / G + (64 / G) w of the shared inner loops, so that a block has
// 64 / G x NW shares.  An iteration's partials: the wave's 64 / G groups added by xor shuffles,
// then the waves' sums in wave order through `lds` (NW x G slots), in every lane.  With G = 64
// it is xwave_sum.
template <int NW, int G, class T>
__device__ __forceinline__ T xgroup_sum(T v, T* lds) {
#pragma unroll
    for (int o = G; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
    const int ln = threadIdx.x & 63, wv = threadIdx.x >> 6, r = ln & (G - 1);
    if (ln < G) lds[wv * G + r] = v;
    __syncthreads();
    T s = lds[r];
#pragma unroll
    for (int w = 1; w < NW; ++w) s += lds[w * G + r];
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
    ST_WAVE_AGG = 0,     // wave_add (group_add) calls that made one atomic for the whole wave (group)
    ST_WAVE_LANE = 1,    // wave_add calls that made one atomic per lane
    ST_PRIV_BLOCK = 2,   // blocks that accumulated into an LDS-privatised copy
    ST_SPLIT_BLOCK = 3,  // blocks of the wave-per-iteration (narrow-output) form
    ST_BLOCK_ADD = 4,    // block sums (block_add, block_part) that were nonzero
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

// wave_add for the lanes-over-iterations form with G iterations a block: the lanes of a
// G-lane group share an inner-loop iteration, and so, typically, an accumulation target (a
// column's shadow updated by every row).  If the whole wave is active and each group's lanes
// add into their group's first lane's element, each group's values are summed (xor shuffles)
// and its first lane makes one atomic addition (counted as aggregated); otherwise each lane
// adds atomically.  G = 64 is wave_add.
template <int G, class T>
__device__ __forceinline__ void group_add(T* p, T v, unsigned long long* st) {
    if constexpr (G == 64) {
        wave_add(p, v, st);
    } else {
        const uint64_t active = __ballot(1);
        const int ln = threadIdx.x & 63;
        if (active == ~0ull) {
            const uint64_t u = reinterpret_cast<uint64_t>(p);
            const int g0 = ln & ~(G - 1);
            const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)u, g0, 64);
            const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(u >> 32), g0, 64);
            if (__ballot(u == (((uint64_t)hi << 32) | lo)) == ~0ull) {
#pragma unroll
                for (int o = 1; o < G; o <<= 1) v += __shfl_xor(v, o, 64);
                if ((ln & (G - 1)) == 0) {
                    atomic_add(p, v);
                    count(st, ST_WAVE_AGG);
                }
                return;
            }
        }
        atomic_add(p, v);
        if (st && ln == __builtin_ctzll(active)) count(st, ST_WAVE_LANE);
    }
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

// The block's sum of its threads' values (a loop's sum into a scalar, or its accumulations
// into one array element whose index does not change over the loop), stored by thread 0 into
// slots[blockIdx.x]: no atomic.  A one-block fold launched after the loop (fold_load, fold_sum) adds
// the launch's slots in block order into the target, so that the sum's order is fixed and no
// address takes one atomic per block (thousands of same-address device atomics serialise).
// Every thread of the block must call it.
template <class T>
__device__ __forceinline__ void block_part(T* slots, T v, T* lds, unsigned long long* st) {
    v = wave_sum(v);
    const int nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        T s = lds[0];
        for (int w = 1; w < nw; ++w) s += lds[w];
        slots[blockIdx.x] = s;
        if (s != (T)0) count(st, ST_BLOCK_ADD);
    }
    __syncthreads();
}

// The fold, run by one block of FOLD_NT threads: fold_load issues the loads of a thread's
// slots (b = threadIdx.x + u FOLD_NT, zero past nb) all at once, so that a fold costs one
// memory round trip whatever nb; fold_sum adds them in a fixed tree, then the waves' sums in
// wave order, and returns the total to thread 0 (the other threads get 0).  Every thread of the
// block must call fold_sum.
constexpr int FOLD_NT = 1024, FOLD_PER = 8;  // at most FOLD_NT x FOLD_PER = 8192 slots
template <class T>
__device__ __forceinline__ void fold_load(const T* slots, unsigned nb, T (&v)[FOLD_PER]) {
#pragma unroll
    for (int u = 0; u < FOLD_PER; ++u) {
        const unsigned b = threadIdx.x + (unsigned)u * FOLD_NT;
        v[u] = b < nb ? slots[b] : (T)0;
    }
}
template <class T>
__device__ __forceinline__ T fold_sum(const T (&v)[FOLD_PER], T* lds) {
    T s = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
    s = wave_sum(s);
    const int nw = blockDim.x >> 6;
    __syncthreads();  // (the slots of lds are reused by the next call)
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = s;
    __syncthreads();
    T t = 0;
    if (threadIdx.x == 0) {
        t = lds[0];
        for (int w = 1; w < nw; ++w) t += lds[w];
    }
    return t;
}

// LDS-privatised accumulation: the block's copy, then one global atomic per nonzero element
template <class T>
__device__ __forceinline__ void lds_add(T* p, T v) {
    atomicAdd(p, v);
}
__device__ __forceinline__ void lds_add(int64_t* p, int64_t v) {
    atomicAdd(reinterpret_cast<unsigned long long*>(p), (unsigned long long)v);
}

// ------------------------------------------------------------------------------------------
// Host side: replays of a lowered function's launch sequence as a HIP graph.
//
// The host part of a generated function reads and writes nothing but its frame `a` (array
// pointers and sizes, scalar arguments, host loop variables, its local arrays' addresses), and
// its kernels take `a` by value, so two calls whose frames are byte-identical issue the same
// launches with the same arguments.  A function with host loops (a time loop: thousands of
// small dependent launches, each paying the host's launch cost) runs a frame by direct
// launches the first time it sees it; when the same frame comes back (same device, arrays,
// sizes and scalars), its sequence is captured once, on a private stream, into a HIP graph,
// which that call and every later call with that frame launch onto the caller's stream.  A
// few frames are kept (the least recently used is dropped); every graph is dropped when one of
// the function's local arrays is reallocated, since the graphs hold its old address.  A frame
// whose capture fails runs by direct launches from then on.  The lock is recursive: a direct
// run (under it) that reallocates a local array drops the graphs through clear().
// ------------------------------------------------------------------------------------------
template <class A>
class LaunchGraphs {
  public:
    using Fn = int32_t (*)(A, hipStream_t);

    int32_t run(const A& a, hipStream_t stream, Fn fn) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kDevices) {
            (void)hipGetLastError();
            return fn(a, stream);
        }
        // on a stream the caller is capturing: launched directly, with no second capture, graph
        // launch or device synchronisation inside the caller's capture (the generated function's
        // own stream synchronisation then fails the call)
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) != hipSuccess) {
            (void)hipGetLastError();
            return fn(a, stream);
        }
        if (cs != hipStreamCaptureStatusNone) return fn(a, stream);
        std::lock_guard<std::recursive_mutex> lk(mu_);
        ++tick_;
        Slot* s = find(a, dev);
        if (!s) {
            s = oldest();
            drop(*s);
            std::memcpy(&s->key, &a, sizeof(A));
            s->dev = dev;
            s->used = true;
            s->tick = tick_;
            return fn(a, stream);
        }
        s->tick = tick_;
        if (!s->exec && !s->failed) capture(*s, a, fn, dev);
        if (s->exec) {
            if (hipGraphLaunch(s->exec, stream) == hipSuccess) {
                ++replays_;
                return 0;
            }
            (void)hipGetLastError();
            drop(*s);
            s->failed = true;
        }
        return fn(a, stream);
    }

    // every graph dropped (the caller has synchronised the device)
    void clear() {
        std::lock_guard<std::recursive_mutex> lk(mu_);
        for (Slot& s : slots_) {
            drop(s);
            s.used = false;
        }
    }

    void counts(int64_t* out) const {
        out[0] = captures_;
        out[1] = replays_;
    }

  private:
    static constexpr int kSlots = 4, kDevices = 64;
    struct Slot {
        A key;
        int dev;
        bool used, failed;
        hipGraphExec_t exec;
        unsigned long long tick;
    };
    Slot slots_[kSlots] = {};
    hipStream_t cap_[kDevices] = {};
    std::recursive_mutex mu_;
    unsigned long long tick_ = 0;
    int64_t captures_ = 0, replays_ = 0;

    Slot* find(const A& a, int dev) {
        for (Slot& s : slots_)
            if (s.used && s.dev == dev && std::memcmp(&s.key, &a, sizeof(A)) == 0) return &s;
        return nullptr;
    }
    Slot* oldest() {
        Slot* o = &slots_[0];
        for (Slot& s : slots_) {
            if (!s.used) return &s;
            if (s.tick < o->tick) o = &s;
        }
        return o;
    }
    void drop(Slot& s) {
        if (s.exec) {
            // a launch of the graph may still run: the exec is destroyed after the device is idle
            (void)hipDeviceSynchronize();
            (void)hipGraphExecDestroy(s.exec);
            s.exec = nullptr;
        }
        s.failed = false;
    }
    void capture(Slot& s, const A& a, Fn fn, int dev) {
        s.failed = true;
        if (!cap_[dev] && hipStreamCreateWithFlags(&cap_[dev], hipStreamNonBlocking) != hipSuccess) {
            cap_[dev] = nullptr;
            (void)hipGetLastError();
            return;
        }
        if (hipStreamBeginCapture(cap_[dev], hipStreamCaptureModeThreadLocal) != hipSuccess) {
            (void)hipGetLastError();
            return;
        }
        const int32_t rc = fn(a, cap_[dev]);
        hipGraph_t g = nullptr;
        const hipError_t e = hipStreamEndCapture(cap_[dev], &g);
        if (rc != 0 || e != hipSuccess || !g) {
            if (g) (void)hipGraphDestroy(g);
            (void)hipGetLastError();
            return;
        }
        hipGraphExec_t x = nullptr;
        const hipError_t ei = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (ei != hipSuccess || !x) {
            (void)hipGetLastError();
            return;
        }
        s.exec = x;
        s.failed = false;
        ++captures_;
    }
};

}  // namespace stade_lowered
