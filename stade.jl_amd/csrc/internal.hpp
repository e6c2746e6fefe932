// Shared internals of libstade_hip: error state, per-device workspace, wave64/block reductions.
//
// Everything here is CDNA (gfx950) code: 64-lane wavefronts, DPP row operations inside a
// 16-lane row, LDS trees across waves, and a sync-free last-block second pass for grid-wide
// sums (the design the reference keeps CUDA-only: `cgen_reduce_block_kernel`
// /root/reference/src/STADE.jl:10333-10354, `sync_free_reduce` 10303-10316).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <utility>

#define STADE_HIP_OK 0
#define STADE_HIP_EINVAL (-1)
#define STADE_HIP_ENOMEM (-2)
#define STADE_HIP_ERANGE (-3)

namespace stade {

// ------------------------------------------------------------------------------------------
// error state (host)
// ------------------------------------------------------------------------------------------
int32_t set_error(int32_t code, const char* fmt, ...);
int32_t check_hip(hipError_t e, const char* what);
#define STADE_TRY_HIP(expr)                                              \
    do {                                                                 \
        hipError_t _e = (expr);                                          \
        if (_e != hipSuccess) return ::stade::check_hip(_e, #expr);     \
    } while (0)
#define STADE_LAUNCHED(what)                                             \
    do {                                                                 \
        hipError_t _e = hipGetLastError();                               \
        if (_e != hipSuccess) return ::stade::check_hip(_e, what);       \
    } while (0)

// ------------------------------------------------------------------------------------------
// per-device workspace: grid-reduction partials, device scalars and scratch owned by the
// library.  Calls that share a device must be stream-ordered with respect to each other.
// ------------------------------------------------------------------------------------------
struct Workspace {
    double* partials;       // per-block partial sums, kPartialSlots doubles
    double* dscalars;       // small device scalars handed back to the host
    uint32_t* sync;         // ticket counters (kSyncSlots), zero between calls: a kernel's last
                            // block resets the one it used
    void* scratch;          // grows on demand
    size_t scratch_bytes;
    bool scratch_captured;  // a graph captured since `scratch` was allocated may hold its address
};
constexpr int kPartialSlots = 1 << 22;
constexpr int kDeviceScalars = 64;
constexpr int kSyncSlots = 64;
// the device error flag (an int32 in the device scalars), raised with kErrIndex by a kernel
// that sees an index the generated code would reject
constexpr int kErrFlagSlot = 16;
constexpr int kErrIndex = 1;

// Workspace of the current device; nullptr (with the error set) on failure.
Workspace* workspace();
// Scratch of at least `bytes`; nullptr (with the error set) on failure.  Only valid under a
// WsCall of the current device.  Under graph capture it does not grow (the graph would keep
// the address of a buffer the growth replaces): it fails with STADE_HIP_ESTATE.  A buffer a
// graph may still use is never freed; a growth outside capture retires it instead.
void* scratch(size_t bytes);
// The code of the last scratch() failure on this thread (STADE_HIP_ENOMEM or STADE_HIP_ESTATE).
int32_t scratch_error();

// The workspace of the current device for one library call that enqueues on `stream`.
// While the guard lives, the calling thread holds the device's library lock, so calls from
// other host threads wait (scratch cannot be regrown under a call that is enqueuing into it).
// If the previous call on the device used another stream, `stream` first waits for an event
// that call recorded at its end, so calls on different streams that share the workspace run
// one after the other on the device instead of racing.  The destructor records this call's
// event on `stream` (a stream that may be destroyed later is never touched again).  A
// stream under graph capture is neither ordered nor recorded: the caller's graph orders it.
class WsCall {
  public:
    // with_workspace = false: the lock and the ordering only (the allocation-free entry
    // point); `ws` then stays null and ok() tells success
    explicit WsCall(hipStream_t stream, bool with_workspace = true);
    bool ok() const { return ok_; }
    int32_t error() const { return err_; }   // the failure's code when !ok()
    ~WsCall();
    WsCall(const WsCall&) = delete;
    WsCall& operator=(const WsCall&) = delete;
    bool capturing() const { return capturing_; }
    Workspace* ws;  // nullptr (with the error set) on failure
  private:
    int dev_;
    hipStream_t stream_;
    bool capturing_;
    bool ok_;
    int32_t err_;
};
// Create the current device's call-order event now (the allocation-free entry point's
// one-time set-up, so that its calls create nothing); 0 or a hipError_t.
int32_t call_order_setup();

// ------------------------------------------------------------------------------------------
// kernel timing: when enabled (stade_hip_profile_start), every launch made through
// STADE_TIMED is bracketed by HIP events recorded on the launch's own stream; the elapsed
// times are summed per kernel name when read (stade_hip_profile_read).
// ------------------------------------------------------------------------------------------
bool prof_enabled();
void prof_begin(const char* kernel, hipStream_t s);
void prof_end(hipStream_t s);
#define STADE_TIMED(name, stream, ...)                                   \
    do {                                                                 \
        const bool _p = ::stade::prof_enabled();                        \
        if (_p) ::stade::prof_begin(name, stream);                      \
        __VA_ARGS__;                                                     \
        if (_p) ::stade::prof_end(stream);                              \
    } while (0)

// ------------------------------------------------------------------------------------------
// device: wave64 and block reductions
// ------------------------------------------------------------------------------------------

// DPP move of a 64-bit value: both 32-bit halves go through the same lane permutation.
template <int Ctrl>
__device__ __forceinline__ double dpp_f64(double v) {
    int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), Ctrl, 0xF, 0xF, false);
    int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), Ctrl, 0xF, 0xF, false);
    return __hiloint2double(hi, lo);
}
template <int Ctrl>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), Ctrl, 0xF, 0xF, false));
}

// DPP controls (gfx9): quad_perm and row rotate
constexpr int kDppQuadSwap1 = 0xB1;   // quad_perm:[1,0,3,2]
constexpr int kDppQuadSwap2 = 0x4E;   // quad_perm:[2,3,0,1]
constexpr int kDppRowRor4 = 0x124;    // row_ror:4
constexpr int kDppRowRor8 = 0x128;    // row_ror:8

// DPP wavefront shifts (gfx9 family): neighbour values across the 64 lanes of a wave.
constexpr int kDppWaveShl1 = 0x130;  // wave_shl:1, lane l <- lane l+1
constexpr int kDppWaveShr1 = 0x138;  // wave_shr:1, lane l <- lane l-1

// v of the lane to the west (lane l-1); lane 0 gets `edge`
__device__ __forceinline__ double from_west(double v, double edge) {
    const int lo = __builtin_amdgcn_update_dpp(__double2loint(edge), __double2loint(v), kDppWaveShr1, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(__double2hiint(edge), __double2hiint(v), kDppWaveShr1, 0xF, 0xF, false);
    return __hiloint2double(hi, lo);
}
// v of the lane to the east (lane l+1); lane 63 gets `edge`
__device__ __forceinline__ double from_east(double v, double edge) {
    const int lo = __builtin_amdgcn_update_dpp(__double2loint(edge), __double2loint(v), kDppWaveShl1, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(__double2hiint(edge), __double2hiint(v), kDppWaveShl1, 0xF, 0xF, false);
    return __hiloint2double(hi, lo);
}
// v of lane l, in every lane
__device__ __forceinline__ double lane_val(double v, int l) {
    return __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), l), __builtin_amdgcn_readlane(__double2loint(v), l));
}

// Sum over the 64 lanes; every lane gets the total.  Inside a 16-lane row: two quad
// permutations and two row rotations (DPP, no LDS traffic); across rows: two xor shuffles.
__device__ __forceinline__ double wave_sum(double v) {
    v += dpp_f64<kDppQuadSwap1>(v);
    v += dpp_f64<kDppQuadSwap2>(v);
    v += dpp_f64<kDppRowRor4>(v);
    v += dpp_f64<kDppRowRor8>(v);
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<kDppQuadSwap1>(v);
    v += dpp_f32<kDppQuadSwap2>(v);
    v += dpp_f32<kDppRowRor4>(v);
    v += dpp_f32<kDppRowRor8>(v);
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// Block sum of NV values per thread (blockDim.x a multiple of 64, at most 1024).  The
// result is valid in thread 0.  `lds` holds 16 * NV slots.
template <int NV, typename T>
__device__ __forceinline__ void block_sum(T (&v)[NV], T* lds) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k] = wave_sum(v[k]);
    if (lane == 0) {
#pragma unroll
        for (int k = 0; k < NV; ++k) lds[wave * NV + k] = v[k];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            T s = lds[k];
            for (int w = 1; w < nw; ++w) s += lds[w * NV + k];
            v[k] = s;
        }
    }
    __syncthreads();
}

// Destinations of a grid-wide sum: out.p[k][0] += total of value k.
struct SumOuts {
    double* p[4];
};

// Grid-wide sums in two stages, with no fence and no host synchronisation.
//
// Stage 1 (every block of the producing kernel): the block's sums go to
// partials[bid * NV + k] with plain stores.
// Stage 2 (one block of a kernel launched after it on the same stream, so the producer's
// stores are visible at the kernel boundary): the partials are added in a fixed order --
// a strided in-order walk per thread, then a fixed-shape tree -- so the result does not
// depend on scheduling, and `out.p[k][0] += total`.
//
// The single-kernel alternative (each block fences, takes a ticket, the last block sums)
// needs a device-scope release fence per block; on MI355X that writes back the XCD's L2
// and measured 2.8-4.1x slower for the diffusion kernels, so it is not used.
template <int NV>
__device__ __forceinline__ void block_partials(double (&v)[NV], double* lds, double* partials) {
    block_sum<NV>(v, lds);
    const unsigned bid = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    if (threadIdx.x == 0) {
#pragma unroll
        for (int k = 0; k < NV; ++k) partials[(size_t)bid * NV + k] = v[k];
    }
}

// Stage 2, run by all threads of one block.
template <int NV>
__device__ __forceinline__ void finalize_partials(const double* partials, int nparts, double* lds, SumOuts out) {
    double acc[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) acc[k] = 0.0;
    // unrolled so that several partials' loads are in flight (the sums keep their order)
#pragma unroll 8
    for (int b = threadIdx.x; b < nparts; b += blockDim.x) {
#pragma unroll
        for (int k = 0; k < NV; ++k) acc[k] += partials[(size_t)b * NV + k];
    }
    block_sum<NV>(acc, lds);
    if (threadIdx.x == 0) {
        // every destination read before any is written (they may alias as far as the compiler
        // knows, and interleaving would cost a memory round trip per destination)
        double old[NV];
#pragma unroll
        for (int k = 0; k < NV; ++k) old[k] = out.p[k][0];
#pragma unroll
        for (int k = 0; k < NV; ++k) out.p[k][0] = old[k] + acc[k];
    }
}

// Stage 2 as its own launch (one block of THREADS, at most 1024), for a producer with no
// follow-on kernel.  More threads keep more partials' loads in flight: a 1024-thread block
// reads tens of thousands of partials in a few microseconds.
template <int NV, int THREADS = 256>
__global__ __launch_bounds__(THREADS) void finalize_kernel(const double* partials, int nparts, SumOuts out) {
    __shared__ double lds[16 * NV];
    finalize_partials<NV>(partials, nparts, lds, out);
}

// f(std::integral_constant<int, I>{}) for I = 0 .. N-1 in order: an unroll that does not
// depend on the compiler's unroll threshold (a long register-resident loop that stays rolled
// moves its arrays to scratch memory)
template <typename F, int... I>
__device__ __forceinline__ void static_for_seq(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_seq(f, std::make_integer_sequence<int, N>{});
}

// Periodic wrap of a coordinate that is at most one period outside [0, n).
__device__ __forceinline__ int wrap1(int x, int n) { return x < 0 ? x + n : (x >= n ? x - n : x); }
// Periodic wrap of any coordinate (floored modulus).
__device__ __forceinline__ int wrapn(int x, int n) {
    int r = x % n;
    return r < 0 ? r + n : r;
}

}  // namespace stade
