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
//   * 64 x 32 output tiles per 256-thread block; u is staged in LDS with a 2-cell periodic
//     halo, unb with a 1-cell halo.  The adjoint needs the new state at the neighbours of a
//     cell, so the block recomputes un on its 1-cell halo instead of reading it back.
//   * adjoint, pass 1: un, loss, w = unb + (2 un) lossb on tile+halo, then the gather
//     ub[c] += w_c + 0.1 (w_E + w_W + w_N + w_S) + 4 (-(0.1 w_c)): each cell owns its ub, no
//     atomics.  Pass 1 reads unb but never writes it, so the halo reads cannot race with the
//     reset.  Pass 2 streams the reset unb = 0.  HBM traffic = 48 B/cell, the algorithmic
//     figure (u R, un W, unb R+W, ub R+W).
//   * the loss is a grid sum: DPP wave sum -> LDS block tree -> sync-free last block.
//   * blockIdx -> tile is row-major over tiles with 64-cell-wide tiles along i, so the
//     blocks that share a j-halo row are 64/32 tiles apart in launch order and land on the
//     same XCD (8 XCDs, round-robin dispatch) whenever the tile count along i is a multiple
//     of 8.
#include "internal.hpp"
#include "../../include/stade_hip.h"

namespace stade {
namespace {

constexpr int TI = 64, TJ = 32, NT = 256;
constexpr int UI = TI + 4, UJ = TJ + 4;  // 2-cell halo
constexpr int WI = TI + 2, WJ = TJ + 2;  // 1-cell halo

__device__ __forceinline__ int wrap_any(int x, int n, bool small) { return small ? wrapn(x, n) : wrap1(x, n); }

// un at LDS position (b, a) of a halo-2 tile, in the operation order of the generated text:
// u + 0.1 * (u[W] + u[E] + u[S] + u[N] - 4.0 * u)
__device__ __forceinline__ double step5(const double (*s)[UI], int b, int a) {
    double c = s[b][a];
    double t = s[b][a - 1] + s[b][a + 1];
    t = t + s[b - 1][a];
    t = t + s[b + 1][a];
    t = t - 4.0 * c;
    return c + 0.1 * t;
}
// tangent form: ud + 0.1 * ((((ud[W] + ud[E]) + ud[S]) + ud[N]) + -(4.0 * ud))
__device__ __forceinline__ double step5d(const double (*s)[UI], int b, int a) {
    double c = s[b][a];
    double t = s[b][a - 1] + s[b][a + 1];
    t = t + s[b - 1][a];
    t = t + s[b + 1][a];
    t = t + -(4.0 * c);
    return c + 0.1 * t;
}

template <typename T>
__device__ __forceinline__ void load_tile(T (*dst)[UI], const double* __restrict__ src, int ni, int nj, int i0, int j0,
                                          int halo, int n, bool small) {
    for (int e = threadIdx.x; e < ni * nj; e += NT) {
        int a = e % ni, b = e / ni;
        int gi = wrap_any(i0 - halo + a, n, small), gj = wrap_any(j0 - halo + b, n, small);
        dst[b][a] = src[(size_t)gj * n + gi];
    }
}

// ---------------------------------------------------------------------------------------
// tangent: un, und, loss += sum un^2, lossd += sum (2 un) und
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(NT) void diffusion_d_kernel(const double* __restrict__ u, const double* __restrict__ ud,
                                                         double* __restrict__ un, double* __restrict__ und,
                                                         double* loss, double* lossd, int n, int tiles_i,
                                                         double* partials, unsigned* ticket) {
    __shared__ double su[UJ][UI];
    __shared__ double sud[UJ][UI];
    __shared__ double red[32];
    const int ti = blockIdx.x % tiles_i, tj = blockIdx.x / tiles_i;
    const int i0 = ti * TI, j0 = tj * TJ;
    const bool small = n < UJ;
    // 1-cell halo is enough here; store it at offset 1 so step5 sees the same indexing
    for (int e = threadIdx.x; e < WI * WJ; e += NT) {
        int a = e % WI, b = e / WI;
        int gi = wrap_any(i0 - 1 + a, n, small), gj = wrap_any(j0 - 1 + b, n, small);
        size_t g = (size_t)gj * n + gi;
        su[b + 1][a + 1] = u[g];
        sud[b + 1][a + 1] = ud[g];
    }
    __syncthreads();
    double acc[2] = {0.0, 0.0};
    for (int e = threadIdx.x; e < TI * TJ; e += NT) {
        int a = e % TI, b = e / TI;
        int gi = i0 + a, gj = j0 + b;
        if (gi >= n || gj >= n) continue;
        double v = step5(su, b + 2, a + 2);
        double vd = step5d(sud, b + 2, a + 2);
        size_t g = (size_t)gj * n + gi;
        und[g] = vd;
        un[g] = v;
        acc[1] += (2.0 * v) * vd;
        acc[0] += v * v;
    }
    grid_sum_into<2>(acc, red, partials, ticket, SumOuts{{loss, lossd}});
}

// ---------------------------------------------------------------------------------------
// adjoint pass 1: un, loss, gather of w = unb + (2 un) lossb into ub (unb not written)
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(NT) void diffusion_b_kernel(const double* __restrict__ u, double* __restrict__ un,
                                                         const double* __restrict__ unb, double* __restrict__ ub,
                                                         const double* __restrict__ lossb, double* loss, int n,
                                                         int tiles_i, double* partials, unsigned* ticket) {
    __shared__ double su[UJ][UI];
    __shared__ double sw[WJ][UI];
    __shared__ double red[16];
    const int ti = blockIdx.x % tiles_i, tj = blockIdx.x / tiles_i;
    const int i0 = ti * TI, j0 = tj * TJ;
    const bool small = n < UJ;
    load_tile(su, u, UI, UJ, i0, j0, 2, n, small);
    for (int e = threadIdx.x; e < WI * WJ; e += NT) {
        int a = e % WI, b = e / WI;
        int gi = wrap_any(i0 - 1 + a, n, small), gj = wrap_any(j0 - 1 + b, n, small);
        sw[b][a] = unb[(size_t)gj * n + gi];
    }
    __syncthreads();
    const double lb = lossb[0];
    double acc[1] = {0.0};
    for (int e = threadIdx.x; e < WI * WJ; e += NT) {
        int a = e % WI, b = e / WI;
        double v = step5(su, b + 1, a + 1);
        sw[b][a] = sw[b][a] + (2.0 * v) * lb;
        int gi = i0 + a - 1, gj = j0 + b - 1;
        if (a >= 1 && a <= TI && b >= 1 && b <= TJ && gi < n && gj < n) {
            un[(size_t)gj * n + gi] = v;
            acc[0] += v * v;
        }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < TI * TJ; e += NT) {
        int a = e % TI, b = e / TI;
        int gi = i0 + a, gj = j0 + b;
        if (gi >= n || gj >= n) continue;
        const int A = a + 1, B = b + 1;
        double wc = sw[B][A];
        double s = wc;
        s = s + 0.1 * sw[B][A + 1];
        s = s + 0.1 * sw[B][A - 1];
        s = s + 0.1 * sw[B + 1][A];
        s = s + 0.1 * sw[B - 1][A];
        s = s + 4.0 * -(0.1 * wc);
        size_t g = (size_t)gj * n + gi;
        ub[g] = ub[g] + s;
    }
    grid_sum_into<1>(acc, red, partials, ticket, SumOuts{{loss}});
}

// ---------------------------------------------------------------------------------------
// HVP pass 1: adjoint pass 1 and its tangent (forward over reverse)
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(NT) void diffusion_hv_kernel(const double* __restrict__ u, const double* __restrict__ ud,
                                                          double* __restrict__ un, double* __restrict__ und,
                                                          const double* __restrict__ unb, const double* __restrict__ unbd,
                                                          double* __restrict__ ub, double* __restrict__ ubd,
                                                          const double* __restrict__ lossb, const double* __restrict__ lossbd,
                                                          double* loss, double* lossd, int n, int tiles_i,
                                                          double* partials, unsigned* ticket) {
    __shared__ double su[UJ][UI];
    __shared__ double sud[UJ][UI];
    __shared__ double sw[WJ][UI];
    __shared__ double swd[WJ][UI];
    __shared__ double red[32];
    const int ti = blockIdx.x % tiles_i, tj = blockIdx.x / tiles_i;
    const int i0 = ti * TI, j0 = tj * TJ;
    const bool small = n < UJ;
    load_tile(su, u, UI, UJ, i0, j0, 2, n, small);
    load_tile(sud, ud, UI, UJ, i0, j0, 2, n, small);
    for (int e = threadIdx.x; e < WI * WJ; e += NT) {
        int a = e % WI, b = e / WI;
        int gi = wrap_any(i0 - 1 + a, n, small), gj = wrap_any(j0 - 1 + b, n, small);
        size_t g = (size_t)gj * n + gi;
        sw[b][a] = unb[g];
        swd[b][a] = unbd[g];
    }
    __syncthreads();
    const double lb = lossb[0], lbd = lossbd[0];
    double acc[2] = {0.0, 0.0};
    for (int e = threadIdx.x; e < WI * WJ; e += NT) {
        int a = e % WI, b = e / WI;
        double v = step5(su, b + 1, a + 1);
        double vd = step5d(sud, b + 1, a + 1);
        double h4 = 2.0 * v;
        swd[b][a] = swd[b][a] + (lb * (2.0 * vd) + h4 * lbd);
        sw[b][a] = sw[b][a] + h4 * lb;
        int gi = i0 + a - 1, gj = j0 + b - 1;
        if (a >= 1 && a <= TI && b >= 1 && b <= TJ && gi < n && gj < n) {
            size_t g = (size_t)gj * n + gi;
            und[g] = vd;
            un[g] = v;
            acc[1] += (2.0 * v) * vd;
            acc[0] += v * v;
        }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < TI * TJ; e += NT) {
        int a = e % TI, b = e / TI;
        int gi = i0 + a, gj = j0 + b;
        if (gi >= n || gj >= n) continue;
        const int A = a + 1, B = b + 1;
        double wc = sw[B][A], wcd = swd[B][A];
        double s = wc, sd = wcd;
        s = s + 0.1 * sw[B][A + 1];
        sd = sd + 0.1 * swd[B][A + 1];
        s = s + 0.1 * sw[B][A - 1];
        sd = sd + 0.1 * swd[B][A - 1];
        s = s + 0.1 * sw[B + 1][A];
        sd = sd + 0.1 * swd[B + 1][A];
        s = s + 0.1 * sw[B - 1][A];
        sd = sd + 0.1 * swd[B - 1][A];
        s = s + 4.0 * -(0.1 * wc);
        sd = sd + 4.0 * -(0.1 * wcd);
        size_t g = (size_t)gj * n + gi;
        ubd[g] = ubd[g] + sd;
        ub[g] = ub[g] + s;
    }
    grid_sum_into<2>(acc, red, partials, ticket, SumOuts{{loss, lossd}});
}

// pass 2 of the adjoint: the statement reset unb[idx] = 0.0 for every cell
__global__ __launch_bounds__(NT) void zero2_kernel(double* __restrict__ a, double* __restrict__ b, size_t count) {
    size_t stride = (size_t)gridDim.x * NT * 2;
    // 16-byte stores need 16-byte aligned bases (a view into a larger allocation may not be)
    const bool vec = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) & 15) == 0;
    for (size_t k = ((size_t)blockIdx.x * NT + threadIdx.x) * 2; k < count; k += stride) {
        if (!vec) {
            a[k] = 0.0;
            if (b) b[k] = 0.0;
            if (k + 1 < count) {
                a[k + 1] = 0.0;
                if (b) b[k + 1] = 0.0;
            }
        } else if (k + 1 < count) {
            *reinterpret_cast<double2*>(a + k) = make_double2(0.0, 0.0);
            if (b) *reinterpret_cast<double2*>(b + k) = make_double2(0.0, 0.0);
        } else {
            a[k] = 0.0;
            if (b) b[k] = 0.0;
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

int32_t launch_zero2(double* a, double* b, int64_t count, hipStream_t stream) {
    if (count <= 0) return STADE_HIP_OK;
    int64_t per = (int64_t)NT * 2 * 8;
    int64_t blocks = (count + per - 1) / per;
    if (blocks > 65536) blocks = 65536;
    STADE_TIMED("zero", stream, zero2_kernel<<<(unsigned)blocks, NT, 0, stream>>>(a, b, (size_t)count));
    STADE_LAUNCHED("zero2_kernel");
    return STADE_HIP_OK;
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
                diffusion_d_kernel<<<ti * tj, NT, 0, stream>>>(u, ud, un, und, loss, lossd, (int)n, ti, ws->partials, ws->tickets + 0));
    STADE_LAUNCHED("diffusion_d_kernel");
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
                diffusion_b_kernel<<<ti * tj, NT, 0, stream>>>(u, un, unb, ub, lossb, loss, (int)n, ti, ws->partials, ws->tickets + 0));
    STADE_LAUNCHED("diffusion_b_kernel");
    return launch_zero2(unb, nullptr, n * n, stream);
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
                diffusion_hv_kernel<<<ti * tj, NT, 0, stream>>>(u, ud, un, und, unb, unbd, ub, ubd, lossb, lossbd, loss, lossd,
                                                                 (int)n, ti, ws->partials, ws->tickets + 0));
    STADE_LAUNCHED("diffusion_hv_kernel");
    return launch_zero2(unb, unbd, n * n, stream);
}

}  // extern "C"
