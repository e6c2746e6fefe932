// diffusion2d: tangent, adjoint and HVP of one explicit periodic 5-point diffusion step
// followed by loss += sum(un .^ 2), on an n x n column-major grid (i fastest).
//
// Generated code this replaces: stade.jl_amd/corpus/diffusion2d_{b,d,hv}.jl, the STADE
// adjoint/tangent/HVP of diffusion2d.jl (`agen_emit` /root/reference/src/STADE.jl:3390-3419,
// `tgen_emit` 3271-3278, `hvp_emit` 6729-6782), which `stade_amdgpu_file` (18604) runs as one
// launch per loop plus a host mapreduce for the loss (10519-10571) and the periodic
// owner-computes gather (`cgen_gather_periodic_inverse` 7343-7529) for the adjoint scatter.
//
// Layout and work per launch:
//   * 64 x 32 output tiles per 256-thread block: lane = i offset (one 512-byte row segment
//     per wave load), wave = j offset modulo 4.  u is staged in LDS with a 2-cell periodic
//     halo, unb with a 1-cell halo.  The adjoint needs the new state at the neighbours of a
//     cell, so the block recomputes un on its 1-cell halo instead of reading it back.
//   * adjoint, pass 1: un, loss, w = unb + (2 un) lossb on tile+halo, then the gather
//     ub[c] += w_c + 0.1 (w_E + w_W + w_N + w_S) + 4 (-(0.1 w_c)): each cell owns its ub, no
//     atomics.  ub is prefetched into registers before the first barrier.  Pass 1 reads unb
//     but never writes it, so the halo reads cannot race with the reset.  Pass 2 streams the
//     reset unb = 0 and, in its first block, adds the per-block loss partials of pass 1 (the
//     second stage of the grid sum).  HBM traffic = 48 B/cell, the algorithmic figure
//     (u R, un W, unb R+W, ub R+W): 40 B/cell in pass 1, 8 B/cell in pass 2.
//   * blockIdx -> tile is row-major over tiles with 64-cell-wide tiles along i, so the
//     blocks that share a j-halo row are a multiple of 8 launches apart whenever the tile
//     count along i is a multiple of 8, and land on the same XCD (round-robin dispatch).
#include "internal.hpp"
#include "../../include/stade_hip.h"

namespace stade {
namespace {

constexpr int TI = 64, TJ = 32, NT = 256, NW = NT / 64;
constexpr int UI = TI + 4, UJ = TJ + 4;  // 2-cell halo
constexpr int WI = TI + 2, WJ = TJ + 2;  // 1-cell halo
constexpr int RPT = TJ / NW;             // owned rows per thread

__device__ __forceinline__ int wrap_any(int x, int n, bool small) { return small ? wrapn(x, n) : wrap1(x, n); }

// un at LDS position (b, a) in the operation order of the generated text:
// u + 0.1 * (u[W] + u[E] + u[S] + u[N] - 4.0 * u)
template <int W>
__device__ __forceinline__ double step5(const double (*s)[W], int b, int a) {
    double c = s[b][a];
    double t = s[b][a - 1] + s[b][a + 1];
    t = t + s[b - 1][a];
    t = t + s[b + 1][a];
    t = t - 4.0 * c;
    return c + 0.1 * t;
}
// tangent form: ud + 0.1 * ((((ud[W] + ud[E]) + ud[S]) + ud[N]) + -(4.0 * ud))
template <int W>
__device__ __forceinline__ double step5d(const double (*s)[W], int b, int a) {
    double c = s[b][a];
    double t = s[b][a - 1] + s[b][a + 1];
    t = t + s[b - 1][a];
    t = t + s[b + 1][a];
    t = t + -(4.0 * c);
    return c + 0.1 * t;
}

// Stage a (TI + 2h) x (TJ + 2h) periodic tile of src into dst (row stride W), halo h:
// the 64 interior columns one row per wave instruction, the 2h halo columns separately.
template <int W>
__device__ __forceinline__ void stage(double (*dst)[W], const double* __restrict__ src, int i0, int j0, int h, int n,
                                      bool small) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rows = TJ + 2 * h;
    const int gi = wrap_any(i0 + lane, n, small);
    for (int b = wave; b < rows; b += NW) {
        const int gj = wrap_any(j0 - h + b, n, small);
        dst[b][lane + h] = src[(size_t)gj * n + gi];
    }
    for (int q = threadIdx.x; q < rows * 2 * h; q += NT) {
        const int b = q / (2 * h), c = q % (2 * h);
        const int col = c < h ? c : TI + c;  // 0..h-1 and TI+h..TI+2h-1
        const int gj = wrap_any(j0 - h + b, n, small), gx = wrap_any(i0 - h + col, n, small);
        dst[b][col] = src[(size_t)gj * n + gx];
    }
}

// ---------------------------------------------------------------------------------------
// tangent: un, und, loss += sum un^2, lossd += sum (2 un) und
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(NT) void diffusion_d_kernel(const double* __restrict__ u, const double* __restrict__ ud,
                                                         double* __restrict__ un, double* __restrict__ und, int n,
                                                         int tiles_i, double* partials) {
    __shared__ double su[WJ][WI];
    __shared__ double sud[WJ][WI];
    __shared__ double red[32];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i0 = (blockIdx.x % tiles_i) * TI, j0 = (blockIdx.x / tiles_i) * TJ;
    const bool small = n < UJ;
    stage<WI>(su, u, i0, j0, 1, n, small);
    stage<WI>(sud, ud, i0, j0, 1, n, small);
    __syncthreads();
    double acc[2] = {0.0, 0.0};
    const int gi = i0 + lane;
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
        const int b = wave + NW * r, gj = j0 + b;
        if (gi < n && gj < n) {
            double v = step5<WI>(su, b + 1, lane + 1);
            double vd = step5d<WI>(sud, b + 1, lane + 1);
            size_t g = (size_t)gj * n + gi;
            und[g] = vd;
            un[g] = v;
            acc[1] += (2.0 * v) * vd;
            acc[0] += v * v;
        }
    }
    block_partials<2>(acc, red, partials);
}

// ---------------------------------------------------------------------------------------
// adjoint pass 1 (HV = false) and its tangent (HV = true, forward over reverse): un (+ und),
// loss partials, gather of w = unb + (2 un) lossb (+ wd) into ub (+ ubd); unb not written
// ---------------------------------------------------------------------------------------
template <bool HV>
__global__ __launch_bounds__(NT) void diffusion_b_kernel(const double* __restrict__ u, const double* __restrict__ ud,
                                                         double* __restrict__ un, double* __restrict__ und,
                                                         const double* __restrict__ unb, const double* __restrict__ unbd,
                                                         double* __restrict__ ub, double* __restrict__ ubd,
                                                         const double* __restrict__ lossb, const double* __restrict__ lossbd,
                                                         int n, int tiles_i, double* partials) {
    __shared__ double su[UJ][UI];
    __shared__ double sw[WJ][WI];
    __shared__ double sud[HV ? UJ : 1][HV ? UI : 1];
    __shared__ double swd[HV ? WJ : 1][HV ? WI : 1];
    __shared__ double red[32];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i0 = (blockIdx.x % tiles_i) * TI, j0 = (blockIdx.x / tiles_i) * TJ;
    const bool small = n < UJ;
    const int gi = i0 + lane;
    // prefetch the owned ub (+ ubd): their latency overlaps the LDS phases
    double pub[RPT], pubd[RPT];
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
        const int gj = j0 + wave + NW * r;
        const bool live = gi < n && gj < n;
        pub[r] = live ? ub[(size_t)gj * n + gi] : 0.0;
        pubd[r] = (HV && live) ? ubd[(size_t)gj * n + gi] : 0.0;
    }
    stage<UI>(su, u, i0, j0, 2, n, small);
    stage<WI>(sw, unb, i0, j0, 1, n, small);
    if constexpr (HV) {
        stage<UI>(sud, ud, i0, j0, 2, n, small);
        stage<WI>(swd, unbd, i0, j0, 1, n, small);
    }
    __syncthreads();
    const double lb = lossb[0];
    const double lbd = HV ? lossbd[0] : 0.0;
    double acc[2] = {0.0, 0.0};
    // un and w on the 1-cell halo region: interior columns by lane, then the two halo columns
    for (int q = threadIdx.x; q < WJ * WI; q += NT) {
        int b, a;
        if (q < WJ * TI) {
            b = q >> 6;
            a = (q & 63) + 1;
        } else {
            int h = q - WJ * TI;
            b = h >> 1;
            a = (h & 1) ? WI - 1 : 0;
        }
        double v = step5<UI>(su, b + 1, a + 1);
        double vd = 0.0;
        if constexpr (HV) {
            vd = step5d<UI>(sud, b + 1, a + 1);
            swd[b][a] = swd[b][a] + (lb * (2.0 * vd) + (2.0 * v) * lbd);
        }
        sw[b][a] = sw[b][a] + (2.0 * v) * lb;
        const int oi = i0 + a - 1, oj = j0 + b - 1;
        if (a >= 1 && a <= TI && b >= 1 && b <= TJ && oi < n && oj < n) {
            size_t g = (size_t)oj * n + oi;
            if (HV) {
                und[g] = vd;
                acc[1] += (2.0 * v) * vd;
            }
            un[g] = v;
            acc[0] += v * v;
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
        const int b = wave + NW * r, gj = j0 + b;
        if (gi >= n || gj >= n) continue;
        const int A = lane + 1, B = b + 1;
        double wc = sw[B][A];
        double s = wc;
        s = s + 0.1 * sw[B][A + 1];
        s = s + 0.1 * sw[B][A - 1];
        s = s + 0.1 * sw[B + 1][A];
        s = s + 0.1 * sw[B - 1][A];
        s = s + 4.0 * -(0.1 * wc);
        size_t g = (size_t)gj * n + gi;
        if constexpr (HV) {
            double wcd = swd[B][A];
            double sd = wcd;
            sd = sd + 0.1 * swd[B][A + 1];
            sd = sd + 0.1 * swd[B][A - 1];
            sd = sd + 0.1 * swd[B + 1][A];
            sd = sd + 0.1 * swd[B - 1][A];
            sd = sd + 4.0 * -(0.1 * wcd);
            ubd[g] = pubd[r] + sd;
        }
        ub[g] = pub[r] + s;
    }
    if (HV) {
        block_partials<2>(acc, red, partials);
    } else {
        double v1[1] = {acc[0]};
        block_partials<1>(v1, red, partials);
    }
}

// pass 2 of the adjoint: the statement reset unb[idx] = 0.0 (and unbd) for every cell; the
// first block also finishes the loss sum of pass 1
template <int NV>
__global__ __launch_bounds__(NT) void zero2_kernel(double* __restrict__ a, double* __restrict__ b, size_t count,
                                                   const double* partials, int nparts, SumOuts outs) {
    __shared__ double red[16 * NV];
    if (blockIdx.x == 0) finalize_partials<NV>(partials, nparts, red, outs);
    const size_t stride = (size_t)gridDim.x * NT * 2;
    // 16-byte stores need 16-byte aligned bases (a view into a larger allocation may not be)
    const bool vec = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) == 0;
    for (size_t k = ((size_t)blockIdx.x * NT + threadIdx.x) * 2; k < count; k += stride) {
        if (vec && k + 1 < count) {
            *reinterpret_cast<double2*>(a + k) = make_double2(0.0, 0.0);
            if (b) *reinterpret_cast<double2*>(b + k) = make_double2(0.0, 0.0);
        } else {
            a[k] = 0.0;
            if (b) b[k] = 0.0;
            if (k + 1 < count) {
                a[k + 1] = 0.0;
                if (b) b[k + 1] = 0.0;
            }
        }
    }
}

int32_t check_n(int64_t n, const char* fn) {
    if (n < 0) return set_error(STADE_HIP_EINVAL, "%s: n = %lld is negative", fn, (long long)n);
    if (n > 46340) return set_error(STADE_HIP_ERANGE, "%s: n = %lld exceeds 46340 (n*n must fit Int32 cell indices)", fn, (long long)n);
    int64_t tiles = ((n + TI - 1) / TI) * ((n + TJ - 1) / TJ);
    if (tiles * 2 > kPartialSlots) return set_error(STADE_HIP_ERANGE, "%s: n = %lld needs more reduction slots than the workspace holds", fn, (long long)n);
    return STADE_HIP_OK;
}

unsigned zero_blocks(int64_t count) {
    int64_t per = (int64_t)NT * 2 * 8;
    int64_t blocks = (count + per - 1) / per;
    return (unsigned)(blocks > 65536 ? 65536 : (blocks < 1 ? 1 : blocks));
}

}  // namespace
}  // namespace stade

using namespace stade;

extern "C" {

int32_t stade_hip_diffusion2d_d(double* loss, double* lossd, const double* u, const double* ud, double* un, double* und,
                                int64_t n, hipStream_t stream) {
    if (int32_t rc = check_n(n, "stade_hip_diffusion2d_d")) return rc;
    if (n == 0) return STADE_HIP_OK;
    if (!loss || !lossd || !u || !ud || !un || !und) return set_error(STADE_HIP_EINVAL, "stade_hip_diffusion2d_d: null pointer");
    Workspace* ws = workspace();
    if (!ws) return STADE_HIP_ENOMEM;
    int ti = (int)((n + TI - 1) / TI), tj = (int)((n + TJ - 1) / TJ);
    STADE_TIMED("diffusion2d_d", stream,
                diffusion_d_kernel<<<ti * tj, NT, 0, stream>>>(u, ud, un, und, (int)n, ti, ws->partials));
    STADE_LAUNCHED("diffusion_d_kernel");
    STADE_TIMED("finalize", stream, finalize_kernel<2><<<1, NT, 0, stream>>>(ws->partials, ti * tj, SumOuts{{loss, lossd}}));
    STADE_LAUNCHED("finalize_kernel");
    return STADE_HIP_OK;
}

int32_t stade_hip_diffusion2d_b(double* loss, const double* lossb, const double* u, double* ub, double* un, double* unb,
                                int64_t n, hipStream_t stream) {
    if (int32_t rc = check_n(n, "stade_hip_diffusion2d_b")) return rc;
    if (n == 0) return STADE_HIP_OK;
    if (!loss || !lossb || !u || !ub || !un || !unb) return set_error(STADE_HIP_EINVAL, "stade_hip_diffusion2d_b: null pointer");
    Workspace* ws = workspace();
    if (!ws) return STADE_HIP_ENOMEM;
    int ti = (int)((n + TI - 1) / TI), tj = (int)((n + TJ - 1) / TJ);
    STADE_TIMED("diffusion2d_b", stream,
                diffusion_b_kernel<false><<<ti * tj, NT, 0, stream>>>(u, nullptr, un, nullptr, unb, nullptr, ub, nullptr, lossb,
                                                                      nullptr, (int)n, ti, ws->partials));
    STADE_LAUNCHED("diffusion_b_kernel");
    STADE_TIMED("zero", stream,
                zero2_kernel<1><<<zero_blocks(n * n), NT, 0, stream>>>(unb, nullptr, (size_t)(n * n), ws->partials, ti * tj,
                                                                       SumOuts{{loss}}));
    STADE_LAUNCHED("zero2_kernel");
    return STADE_HIP_OK;
}

int32_t stade_hip_diffusion2d_hv(double* loss, const double* lossb, const double* u, double* ub, double* un, double* unb,
                                 int64_t n, double* lossd, const double* lossbd, const double* ud, double* ubd, double* und,
                                 double* unbd, hipStream_t stream) {
    if (int32_t rc = check_n(n, "stade_hip_diffusion2d_hv")) return rc;
    if (n == 0) return STADE_HIP_OK;
    if (!loss || !lossb || !u || !ub || !un || !unb || !lossd || !lossbd || !ud || !ubd || !und || !unbd)
        return set_error(STADE_HIP_EINVAL, "stade_hip_diffusion2d_hv: null pointer");
    Workspace* ws = workspace();
    if (!ws) return STADE_HIP_ENOMEM;
    int ti = (int)((n + TI - 1) / TI), tj = (int)((n + TJ - 1) / TJ);
    STADE_TIMED("diffusion2d_hv", stream,
                diffusion_b_kernel<true><<<ti * tj, NT, 0, stream>>>(u, ud, un, und, unb, unbd, ub, ubd, lossb, lossbd, (int)n,
                                                                     ti, ws->partials));
    STADE_LAUNCHED("diffusion_b_kernel<hv>");
    STADE_TIMED("zero", stream,
                zero2_kernel<2><<<zero_blocks(n * n), NT, 0, stream>>>(unb, unbd, (size_t)(n * n), ws->partials, ti * tj,
                                                                       SumOuts{{loss, lossd}}));
    STADE_LAUNCHED("zero2_kernel");
    return STADE_HIP_OK;
}

}  // extern "C"
