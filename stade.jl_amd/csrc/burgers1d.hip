// burgers1d: tangent, adjoint and HVP of explicit 1-D viscous Burgers time stepping with a
// counted, guarded time loop, then loss += sum(u_T .^ 2).
//
// Generated code this replaces: stade.jl_amd/corpus/burgers1d_{b,d,hv}.jl.  Under
// `stade_amdgpu_file` the time loop stays on the host (a loop containing stack operations is
// not split, /root/reference/src/STADE.jl:8212-8225, 10613-10615) and issues one launch per
// inner loop per step: about 2 x 2 x nsteps launches per adjoint, each moving one 8 MiB row.
//
// Tape: u_stack[((x - 1) + (t - 1) * n) + 1] (the cell loop is the fastest digit,
// `agen_local_position` 4867-4881) holds the state at the start of step t; branch_stack[t]
// holds the guard's outcome (Int64, bit-exact).  The guard `tc < tend` with tc += dt only on
// taken steps is evaluated on the host with the same IEEE double operations, so the taken
// steps are a prefix 1..nrun of the loop.
//
// Kernels (one block owns S consecutive cells and carries a K-cell halo on each side):
//   * forward chunk: K time steps with the state in registers and neighbours by DPP (the
//     valid region shrinks by one cell per step), the owned part of every state written to
//     the tape; HBM traffic is the tape rows (written once) plus one state read and write per
//     chunk.
//   * backward init: w = unb + (ub + (2 u_T) lossb), loss += sum u_T^2, unb = 0 (pointwise).
//   * backward chunk: K steps of the transposed stencil in gathered (owner-computes) form,
//     reading tape rows.  The generated per-cell update is evaluated in a factored form with
//     fused multiply-adds (the same sum, about half the fp64 operations; results agree with
//     the generated order to rounding).  The scalar shadows of the two coefficients are
//     per-thread sums over owned cells and steps, then a deterministic grid sum.  Full
//     chunks (K = 32 steps) keep the state in registers with DPP neighbours
//     (bwd_reg_kernel); a shorter last chunk uses the LDS form (bwd_kernel).
#include "internal.hpp"
#include "../../include/stade_hip.h"

#include <math.h>

#include <algorithm>

namespace stade {
namespace {

constexpr int NT = 256, KMAX = 32;
constexpr int kInitBlockCells = NT * 8;  // cells per block of the backward init kernel
#ifndef STADE_BURG_FT
#define STADE_BURG_FT 512
#endif
#ifndef STADE_BURG_FS
#define STADE_BURG_FS 4096
#endif
#ifndef STADE_BURG_FS_NOTAPE
#define STADE_BURG_FS_NOTAPE 960
#endif
#ifndef STADE_BURG_FT_NOTAPE
#define STADE_BURG_FT_NOTAPE 256
#endif
#ifndef STADE_BURG_FC
#define STADE_BURG_FC 1
#endif
#ifndef STADE_BURG_FC_NOTAPE
#define STADE_BURG_FC_NOTAPE 4
#endif
// forward chunk kernel (register form): threads, owned cells and cells per lane of a block.
// With a tape row to write every step (adjoint, HVP, the checkpoint policy's recomputed
// segments) 512 / 4096 / 1: against the LDS form it
// replaced (1024 / 4096), the HVP 3-6 % faster and the adjoint 0-2 %; 1024 / 4096, 256 / 4096
// and 512 / 2048 measured between the two; two cells a lane (512 / 4032 / 2) halved both
// rates (its tape stores cover every other element).  The tangent, which writes no tape and is
// bound by its instruction issue (fp64 arithmetic and the neighbour shifts), 256 / 960 / 4:
// the region of 1024 cells is one slot of four cells a lane, every wave does the same work,
// and a lane shifts two values an array a step for four cells; 18 % faster than 512 / 1024 /
// 1 (one cell a lane, wave 0 computing a third slot the others skip).  Measured at 2^20 cells:
// 512 / 960 / 2 +9 %, 256 / 448 / 2 +11 %, 128 / 448 / 4 +7 %, 64 / 448 / 8 +7 %, 512 / 1984 /
// 4 +5 %, 64 / 960 / 16 (137 registers) -15 %.  The checkpoint policy's first sweep, which
// writes a row every `every` >= KMAX steps (at most one a launch), takes the tangent's form.
constexpr int BNT = STADE_BURG_FT, BNT_NOTAPE = STADE_BURG_FT_NOTAPE;
constexpr int FWD_S = STADE_BURG_FS, FWD_C = STADE_BURG_FC;
constexpr int FWD_S_NOTAPE = STADE_BURG_FS_NOTAPE, FWD_C_NOTAPE = STADE_BURG_FC_NOTAPE;
#ifndef STADE_BURG_BT
#define STADE_BURG_BT 512
#endif
#ifndef STADE_BURG_BS
#define STADE_BURG_BS 2048
#endif
#ifndef STADE_BURG_BT_HV
#define STADE_BURG_BT_HV 512
#endif
#ifndef STADE_BURG_BS_HV
#define STADE_BURG_BS_HV 1024
#endif
// backward chunk kernels: threads and owned cells per block (adjoint; HVP).  Each step of a
// chunk ends in a block barrier, and the step is bound by its chain of barrier, edge loads,
// DPP moves and arithmetic: two 512-thread blocks per CU (two barrier domains, the same 16
// waves) measured 2-3 % faster than one 1024-thread block.
constexpr int BWD_T = STADE_BURG_BT, BWD_S = STADE_BURG_BS, BWD_T_HV = STADE_BURG_BT_HV, BWD_S_HV = STADE_BURG_BS_HV;

struct Coef {
    double cadv, cdif, cadvd, cdifd;
};

// The generated step  un = uc - cadv * uc * (u[ip] - u[im]) + cdif * (u[ip] - 2.0 * uc + u[im])
// and its tangent (cadv, cdif and u all carry tangents), with fused multiply-adds: 6 and 11
// fp64 operations instead of 8 and 19; results agree with the generated order to rounding.
__device__ __forceinline__ double step_u(double um, double uc, double up, const Coef& c) {
    const double h1 = up - um, h2 = fma(-2.0, uc, up) + um;
    return fma(c.cdif, h2, fma(-(c.cadv * uc), h1, uc));
}

__device__ __forceinline__ double step_ud(double um, double uc, double up, double dm, double dc, double dp, const Coef& c) {
    const double h1 = up - um, h2 = fma(-2.0, uc, up) + um;
    const double dh1 = dp - dm, dh2 = fma(-2.0, dc, dp) + dm;
    // t = d(cadv uc h1) = cadvd uc h1 + cadv (dc h1 + uc dh1)
    const double t = fma(c.cadvd * uc, h1, c.cadv * fma(dc, h1, uc * dh1));
    return fma(c.cdif, dh2, fma(c.cdifd, h2, dc - t));
}

// ---------------------------------------------------------------------------------------
// forward: `nk` steps starting at 0-based step t0, from src (+ srcd) to dst (+ dstd), with the
// state in registers.  Thread t holds the C consecutive positions e = C (t + i T) + j, j < C
// (slot i) of the extended region [x0 - KMAX, x0 + S + KMAX).  A position's neighbours are the
// lane's own registers except at the lane's two ends: e - 1 of its first position and e + 1 of
// its last come from the adjacent lanes (DPP wavefront shifts), and a wave's two end lanes take
// theirs from the end values the waves publish in a small LDS array, double buffered by step:
// one barrier a step and no LDS traffic for the interior.  C cells a lane make C - 1 of every C
// neighbour pairs register reads: two shifts per array a step for C cells instead of 2 C.
// Any nk <= KMAX (the owned cells stay valid for KMAX steps; the region's ends go stale one
// cell a step, and the lanes past its end, in a wave that starts inside it, hold copies of the
// last position that nothing stores).
// ---------------------------------------------------------------------------------------
template <bool TAN, int S, int T, int C>
__global__ __launch_bounds__(T) void fwd_reg_kernel(const double* __restrict__ src, const double* __restrict__ srcd,
                                                    double* __restrict__ dst, double* __restrict__ dstd,
                                                    double* __restrict__ tape, double* __restrict__ taped, int n, int64_t t0,
                                                    int nk, Coef c, int64_t row0, int every) {
    constexpr int L = S + 2 * KMAX;
    constexpr int SP = C * T;  // positions per slot
    constexpr int M = (L + SP - 1) / SP, NWV = T / 64;
    constexpr int NA = TAN ? 2 : 1;  // exchanged arrays: u (+ ud)
    static_assert(S % 64 == 0 && T % 64 == 0, "whole waves");
    __shared__ double edge[2][NA][M][NWV][2];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int x0 = blockIdx.x * S;
    const int own = min(S, n - x0);
    int xc[M][C], eo[M];
    bool owned[M][C];
#pragma unroll
    for (int i = 0; i < M; ++i) {
#pragma unroll
        for (int j = 0; j < C; ++j) {
            const int e = C * (threadIdx.x + i * T) + j;
            xc[i][j] = wrapn(x0 - KMAX + min(e, L - 1), n);
            owned[i][j] = e >= KMAX && e < KMAX + own;
        }
        int si, sv, ss;
        if (lane == 0) {
            ss = 1;
            sv = wave > 0 ? wave - 1 : NWV - 1;
            si = wave > 0 ? i : max(i - 1, 0);
        } else {
            ss = 0;
            sv = wave < NWV - 1 ? wave + 1 : 0;
            si = wave < NWV - 1 ? i : min(i + 1, M - 1);
        }
        eo[i] = (si * NWV + sv) * 2 + ss;
    }
    // a wave whose first position of slot i lies past the region computes nothing there (uniform)
    auto past = [&](int i) { return C * (i * T + wave * 64) >= L; };
    auto edge_at = [&](int buf, int a, int i) { return (&edge[buf][a][0][0][0])[eo[i]]; };
    double u[M][C], ud[M][C];
#pragma unroll
    for (int i = 0; i < M; ++i) {
#pragma unroll
        for (int j = 0; j < C; ++j) {
            u[i][j] = src[xc[i][j]];
            ud[i][j] = TAN ? srcd[xc[i][j]] : 0.0;
        }
    }
    // lane 0 publishes its first position (the west wave's east neighbour), lane 63 its last
    auto publish = [&](int buf) {
        if (lane == 0 || lane == 63) {
            const int side = lane == 63;
#pragma unroll
            for (int i = 0; i < M; ++i) {
                edge[buf][0][i][wave][side] = side ? u[i][C - 1] : u[i][0];
                if constexpr (TAN) edge[buf][1][i][wave][side] = side ? ud[i][C - 1] : ud[i][0];
            }
        }
    };
    publish(0);
    __syncthreads();
    for (int k = 0; k < nk; ++k) {
        const int buf = k & 1;
        // the state at the start of step t0 + k goes to tape row (t0 + k - row0) / every when
        // every divides t0 + k - row0 (every = 1, row0 = 0: the generated stack's layout);
        // streaming stores: a tape row is read back only by the reverse sweep
        const int64_t tr = t0 + k - row0;
        if (tape && tr % every == 0) {
            const size_t row = (size_t)(tr / every) * (size_t)n + (size_t)(x0 - KMAX);
#pragma unroll
            for (int i = 0; i < M; ++i) {
#pragma unroll
                for (int j = 0; j < C; ++j) {
                    if (owned[i][j]) {
                        const size_t g = row + (size_t)(C * (threadIdx.x + i * T) + j);
                        __builtin_nontemporal_store(u[i][j], &tape[g]);
                        if (TAN && taped) __builtin_nontemporal_store(ud[i][j], &taped[g]);
                    }
                }
            }
        }
        double un[M][C], udn[M][C];
#pragma unroll
        for (int i = 0; i < M; ++i) {
#pragma unroll
            for (int j = 0; j < C; ++j) {
                un[i][j] = u[i][j];
                udn[i][j] = ud[i][j];
            }
            if (past(i)) continue;
            const double eu = edge_at(buf, 0, i);
            const double uw = from_west(u[i][C - 1], eu), ue = from_east(u[i][0], eu);
            double dw = 0.0, de = 0.0;
            if constexpr (TAN) {
                const double ed = edge_at(buf, 1, i);
                dw = from_west(ud[i][C - 1], ed);
                de = from_east(ud[i][0], ed);
            }
#pragma unroll
            for (int j = 0; j < C; ++j) {
                const double um = j > 0 ? u[i][j - 1] : uw, up = j < C - 1 ? u[i][j + 1] : ue;
                if constexpr (TAN) {
                    const double dm = j > 0 ? ud[i][j - 1] : dw, dp = j < C - 1 ? ud[i][j + 1] : de;
                    udn[i][j] = step_ud(um, u[i][j], up, dm, ud[i][j], dp, c);
                }
                un[i][j] = step_u(um, u[i][j], up, c);
            }
        }
#pragma unroll
        for (int i = 0; i < M; ++i) {
#pragma unroll
            for (int j = 0; j < C; ++j) {
                u[i][j] = un[i][j];
                ud[i][j] = udn[i][j];
            }
        }
        publish(buf ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < M; ++i) {
#pragma unroll
        for (int j = 0; j < C; ++j) {
            if (owned[i][j]) {
                const int x = x0 + C * (threadIdx.x + i * T) + j - KMAX;
                dst[x] = u[i][j];
                if (TAN) dstd[x] = ud[i][j];
            }
        }
    }
}

// ---------------------------------------------------------------------------------------
// backward init: loss (+ lossd), the first adjoint state w (+ wd), unb (+ unbd) reset.
// When no step ran (nrun = 0) this is the whole reverse sweep: ub += (2 u) lossb.
// ---------------------------------------------------------------------------------------
template <bool HV>
__global__ __launch_bounds__(NT) void bwd_init_kernel(const double* __restrict__ uT, const double* __restrict__ udT,
                                                      double* __restrict__ ub, double* __restrict__ ubd,
                                                      double* __restrict__ unb, double* __restrict__ unbd,
                                                      double* __restrict__ w, double* __restrict__ wd,
                                                      const double* __restrict__ lossb, const double* __restrict__ lossbd,
                                                      int n, int ran, double* dscal, double* partials) {
    __shared__ double red[32];
    if (blockIdx.x == 0 && threadIdx.x < 4) dscal[threadIdx.x] = 0.0;
    const double lb = lossb[0];
    const double lbd = HV ? lossbd[0] : 0.0;
    double acc[2] = {0.0, 0.0};
    // the thread's cells x, x + stride, ... in groups of CPT: every read of a group (clamped,
    // unconditional) before its first store, the sums in the same cell order
    constexpr int CPT = kInitBlockCells / NT;
    const int stride = gridDim.x * NT;
    for (int x0 = blockIdx.x * NT + threadIdx.x; x0 < n; x0 += stride * CPT) {
        double uv[CPT], ubv[CPT], unbv[CPT], udv[CPT], ubdv[CPT], unbdv[CPT];
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int xc = min(x0 + k * stride, n - 1);
            uv[k] = uT[xc];
            ubv[k] = ub[xc];
            unbv[k] = ran ? unb[xc] : 0.0;
            udv[k] = HV ? udT[xc] : 0.0;
            ubdv[k] = HV ? ubd[xc] : 0.0;
            unbdv[k] = (HV && ran) ? unbd[xc] : 0.0;
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
            const int x = x0 + k * stride;
            if (x >= n) break;
            const double u = uv[k];
            acc[0] += u * u;
            const double g = ubv[k] + (2.0 * u) * lb;
            double gd = 0.0;
            if (HV) {
                const double ud = udv[k];
                acc[1] += (2.0 * u) * ud;
                gd = ubdv[k] + (lb * (2.0 * ud) + (2.0 * u) * lbd);
            }
            if (ran) {
                w[x] = unbv[k] + g;
                unb[x] = 0.0;
                if (HV) {
                    wd[x] = unbdv[k] + gd;
                    unbd[x] = 0.0;
                }
            } else {
                ub[x] = g;
                if (HV) ubd[x] = gd;
            }
        }
    }
    if (HV) {
        block_partials<2>(acc, red, partials);
    } else {
        double v[1] = {acc[0]};
        block_partials<1>(v, red, partials);
    }
}

// ---------------------------------------------------------------------------------------
// backward chunk: nk steps, descending from 0-based step t_hi.  Per cell y of the new state:
//   ub[y] = B(y+1) + C(y+1) + own(y) + A(y-1) + C(y-1)   (the generated statement order of
// the interior, with A/B/C the contributions a cell sends to its east/west neighbours)
// ---------------------------------------------------------------------------------------

// One backward step k on the extended region: reads the tape row in U (+ UD) and the adjoint
// state in Wc (+ WDc), writes the next adjoint state to Wn (+ WDn) on [k+1, len-k-1), and adds
// the owned cells' coefficient-shadow terms to acc.
template <bool HV, int M, int T>
__device__ __forceinline__ void bwd_step(int k, int len, int nk, int own, const double* U, const double* UD, const double* Wc,
                                         const double* WDc, double* Wn, double* WDn, const Coef& c, double (&acc)[4]) {
#pragma unroll
    for (int i = 0; i < M; ++i) {
        const int e = threadIdx.x + i * T;
        if (e < k + 1 || e >= len - k - 1) continue;
        // the update in its factored form (as in bwd_reg_kernel)
        const double um1 = U[e - 1], uc = U[e], up1 = U[e + 1];
        const double wm = Wc[e - 1], wc = Wc[e], wp = Wc[e + 1];
        const double dp = wp - wc, dm = wm - wc;
        const double lap = dp + dm;
        const double adv = fma(up1, dp, -(um1 * dm));
        const double c3 = up1 - um1;
        const double h6 = uc * c3;
        const double h9 = fma(-2.0, uc, up1) + um1;
        const bool owned = e >= nk && e < nk + own;
        if (owned) {
            acc[0] = fma(-h6, wc, acc[0]);
            acc[1] = fma(h9, wc, acc[1]);
        }
        if (HV) {
            const double dm1 = UD[e - 1], dc = UD[e], dp1 = UD[e + 1];
            const double wdm = WDc[e - 1], wdc = WDc[e], wdp = WDc[e + 1];
            const double ddp = wdp - wdc, ddm = wdm - wdc;
            const double lapd = ddp + ddm;
            const double advd = fma(dp1, dp, fma(up1, ddp, fma(-dm1, dm, -(um1 * ddm))));
            WDn[e] = fma(c.cadv, advd, fma(c.cadvd, adv, fma(c.cdif, lapd, fma(c.cdifd, lap, wdc))));
            if (owned) {
                const double c3d = dp1 - dm1;
                const double h6d = fma(uc, c3d, c3 * dc);
                acc[2] = fma(-h6, wdc, fma(-h6d, wc, acc[2]));
                const double h9d = fma(-2.0, dc, dp1) + dm1;
                acc[3] = fma(h9, wdc, fma(wc, h9d, acc[3]));
            }
        }
        Wn[e] = fma(c.cadv, adv, fma(c.cdif, lap, wc));
    }
}

// the chunk's final adjoint state and its coefficient-shadow partials
template <bool HV, int T>
__device__ __forceinline__ void bwd_finish(const double* Wc, const double* WDc, double* __restrict__ vout,
                                           double* __restrict__ voutd, int x0, int nk, int own, double (&acc)[4], double* red,
                                           double* partials) {
    for (int e = threadIdx.x; e < own; e += T) {
        vout[x0 + e] = Wc[nk + e];
        if (HV) voutd[x0 + e] = WDc[nk + e];
    }
    if (HV) {
        block_partials<4>(acc, red, partials);
    } else {
        double v[2] = {acc[0], acc[1]};
        block_partials<2>(v, red, partials);
    }
}

// any nk <= KMAX: the tape row of the next step is fetched one step ahead
template <bool HV, int S, int T>
__global__ __launch_bounds__(T) void bwd_kernel(const double* __restrict__ win, const double* __restrict__ wind,
                                                  double* __restrict__ vout, double* __restrict__ voutd,
                                                  const double* __restrict__ tape, const double* __restrict__ taped, int n,
                                                  int64_t t_hi, int nk, Coef c, double* partials, int64_t row0) {
    constexpr int L = S + 2 * KMAX;
    constexpr int M = (L + T - 1) / T;  // extended-region positions per thread
    __shared__ double W[2][L];
    __shared__ double U[L];
    __shared__ double WD[HV ? 2 : 1][HV ? L : 1];
    __shared__ double UD[HV ? L : 1];
    __shared__ double red[16 * 4];
    const int x0 = blockIdx.x * S;
    const int len = S + 2 * nk;
    const int own = min(S, n - x0);
    // the thread's positions e = threadIdx.x + i * T and their (periodic) columns
    int xcol[M];
#pragma unroll
    for (int i = 0; i < M; ++i) {
        const int e = threadIdx.x + i * T;
        xcol[i] = e < len ? wrapn(x0 - nk + e, n) : 0;
        if (e < len) {
            W[0][e] = win[xcol[i]];
            if (HV) WD[0][e] = wind[xcol[i]];
        }
    }
    // tape row of backward step k (state at the start of step t_hi - k), on [k, len - k):
    // held in registers from one step ahead
    double pre[M], pred[M];
    auto fetch = [&](int k) {
        const size_t row = (size_t)(t_hi - k - row0) * (size_t)n;
#pragma unroll
        for (int i = 0; i < M; ++i) {
            const int e = threadIdx.x + i * T;
            if (e >= k && e < len - k) {
                pre[i] = __builtin_nontemporal_load(&tape[row + xcol[i]]);
                if (HV) pred[i] = __builtin_nontemporal_load(&taped[row + xcol[i]]);
            }
        }
    };
    fetch(0);
    double acc[4] = {0.0, 0.0, 0.0, 0.0};  // cadvb, cdifb, cadvbd, cdifbd
    int cur = 0;
    for (int k = 0; k < nk; ++k) {
#pragma unroll
        for (int i = 0; i < M; ++i) {
            const int e = threadIdx.x + i * T;
            if (e >= k && e < len - k) {
                U[e] = pre[i];
                if (HV) UD[e] = pred[i];
            }
        }
        if (k + 1 < nk) fetch(k + 1);
        __syncthreads();
        bwd_step<HV, M, T>(k, len, nk, own, U, UD, W[cur], WD[HV ? cur : 0], W[cur ^ 1], WD[HV ? cur ^ 1 : 0], c, acc);
        __syncthreads();
        cur ^= 1;
    }
    bwd_finish<HV, T>(W[cur], WD[HV ? cur : 0], vout, voutd, x0, nk, own, acc, red, partials);
}

// ---------------------------------------------------------------------------------------
// A full chunk of KMAX steps with the state in registers.  Thread t holds positions
// e = t + i * T (slot i) of the extended region; its neighbours e -/+ 1 are the adjacent
// lanes of the same slot, taken by DPP wavefront shifts.  Only a wave's two end lanes need a
// value from another wave (lane 0: the previous wave's lane 63, or slot i-1's last lane for
// wave 0; lane 63: the next wave's lane 0, or slot i+1's first lane for the last wave): every
// wave publishes its end lanes' tape value and adjoint state in a small LDS array, double
// buffered by step, so a step needs one barrier and almost no LDS traffic.  The tape row of
// step k+1 is published at the end of step k, so the prefetch ring of PD rows keeps PD - 1
// rows in flight.  The arithmetic per position is bwd_step's, in the same order.  A ring of 2
// measured faster than 4 (537 against 526 adjoint evals/s); loading the tape shifted by -/+1
// instead of taking neighbours by DPP needed more registers than a 1024-thread block allows
// and ran at 392.
// ---------------------------------------------------------------------------------------
template <bool HV, int S, int PD, int T>
__global__ __launch_bounds__(T) void bwd_reg_kernel(const double* __restrict__ win, const double* __restrict__ wind,
                                                      double* __restrict__ vout, double* __restrict__ voutd,
                                                      const double* __restrict__ tape, const double* __restrict__ taped, int n,
                                                      int64_t t_hi, Coef c, double* partials, int64_t row0) {
    constexpr int nk = KMAX, L = S + 2 * KMAX;
    constexpr int M = (L + T - 1) / T, NWV = T / 64;
    constexpr int NA = HV ? 4 : 2;  // exchanged arrays: u, w (+ ud, wd)
    static_assert(KMAX % PD == 0, "full chunks are whole rounds of the prefetch ring");
    static_assert(L - (M - 1) * T <= 64, "the last slot belongs to wave 0 alone");
    __shared__ double edge[2][NA][M][NWV][2];
    __shared__ double red[16 * 4];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int x0 = blockIdx.x * S;
    const int own = min(S, n - x0);
    // columns, ownership, and where an end lane finds its outside neighbour (slot, wave, side)
    int xc[M], eo[M];
    bool owned[M];
#pragma unroll
    for (int i = 0; i < M; ++i) {
        const int e = threadIdx.x + i * T;
        xc[i] = wrapn(x0 - nk + min(e, L - 1), n);
        owned[i] = e >= nk && e < nk + own;
        int si, sv, ss;
        if (lane == 0) {
            ss = 1;
            sv = wave > 0 ? wave - 1 : NWV - 1;
            si = wave > 0 ? i : max(i - 1, 0);
        } else {
            ss = 0;
            sv = wave < NWV - 1 ? wave + 1 : 0;
            si = wave < NWV - 1 ? i : min(i + 1, M - 1);
        }
        eo[i] = (si * NWV + sv) * 2 + ss;
    }
    auto edge_at = [&](int buf, int a, int i) { return (&edge[buf][a][0][0][0])[eo[i]]; };
    double w[M], wd[M];
#pragma unroll
    for (int i = 0; i < M; ++i) {
        w[i] = win[xc[i]];
        wd[i] = HV ? wind[xc[i]] : 0.0;
    }
    double pu[PD][M], pud[HV ? PD : 1][M];
    auto fetch = [&](int slot, int k) {
        const size_t row = (size_t)(t_hi - (k < nk ? k : nk - 1) - row0) * (size_t)n;
#pragma unroll
        for (int i = 0; i < M; ++i) {
            pu[slot][i] = __builtin_nontemporal_load(&tape[row + xc[i]]);
            if constexpr (HV) pud[slot][i] = __builtin_nontemporal_load(&taped[row + xc[i]]);
        }
    };
    // the end lanes' adjoint state and the tape row of the next step (ring slot `nxt`)
    auto publish = [&](int buf, int nxt) {
        if (lane == 0 || lane == 63) {
            const int side = lane == 63;
#pragma unroll
            for (int i = 0; i < M; ++i) {
                edge[buf][0][i][wave][side] = pu[nxt][i];
                edge[buf][1][i][wave][side] = w[i];
                if constexpr (HV) {
                    edge[buf][2][i][wave][side] = pud[nxt][i];
                    edge[buf][3][i][wave][side] = wd[i];
                }
            }
        }
    };
#pragma unroll
    for (int j = 0; j < PD; ++j) fetch(j, j);
    publish(0, 0);
    __syncthreads();
    double acc[4] = {0.0, 0.0, 0.0, 0.0};  // cadvb, cdifb, cadvbd, cdifbd
    for (int k0 = 0; k0 < nk; k0 += PD) {
#pragma unroll
        for (int j = 0; j < PD; ++j) {
            const int k = k0 + j, buf = k & 1;
            double wn[M], wdn[M];
#pragma unroll
            for (int i = 0; i < M; ++i) {
                wn[i] = w[i];
                wdn[i] = wd[i];
                if (i == M - 1 && wave != 0) continue;  // past the extended region (uniform)
                const double uc = pu[j][i], eu = edge_at(buf, 0, i);
                const double um1 = from_west(uc, eu), up1 = from_east(uc, eu);
                const double wc = w[i], ew = edge_at(buf, 1, i);
                const double wm = from_west(wc, ew), wp = from_east(wc, ew);
                // The generated update, collected by the cell's own stencil:
                //   wn = wc + cdif (wp - 2 wc + wm) + cadv (up1 (wp - wc) - um1 (wm - wc))
                // (the sum of the contributions B, C of cell e+1, A, C of cell e-1 and the
                // cell's own term), and the shadows' summands
                //   cadvb += -(uc (up1 - um1)) wc,   cdifb += (up1 - 2 uc + um1) wc,
                // with fused multiply-adds: 13 fp64 operations instead of 24, equal to the
                // generated order up to rounding.
                const double dp = wp - wc, dm = wm - wc;
                const double lap = dp + dm;
                const double adv = fma(up1, dp, -(um1 * dm));
                wn[i] = fma(c.cadv, adv, fma(c.cdif, lap, wc));
                const double c3 = up1 - um1;
                const double h6 = uc * c3;
                const double h9 = fma(-2.0, uc, up1) + um1;
                if (owned[i]) {
                    acc[0] = fma(-h6, wc, acc[0]);
                    acc[1] = fma(h9, wc, acc[1]);
                }
                if constexpr (HV) {
                    const double dc = pud[j][i], eud = edge_at(buf, 2, i);
                    const double dm1 = from_west(dc, eud), dp1 = from_east(dc, eud);
                    const double wdc = wd[i], ewd = edge_at(buf, 3, i);
                    const double wdm = from_west(wdc, ewd), wdp = from_east(wdc, ewd);
                    // tangent of the update above (cadv, cdif, u and w all carry tangents)
                    const double ddp = wdp - wdc, ddm = wdm - wdc;
                    const double lapd = ddp + ddm;
                    const double advd = fma(dp1, dp, fma(up1, ddp, fma(-dm1, dm, -(um1 * ddm))));
                    wdn[i] = fma(c.cadv, advd, fma(c.cadvd, adv, fma(c.cdif, lapd, fma(c.cdifd, lap, wdc))));
                    if (owned[i]) {
                        const double c3d = dp1 - dm1;
                        const double h6d = fma(uc, c3d, c3 * dc);
                        acc[2] = fma(-h6, wdc, fma(-h6d, wc, acc[2]));
                        const double h9d = fma(-2.0, dc, dp1) + dm1;
                        acc[3] = fma(h9, wdc, fma(wc, h9d, acc[3]));
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < M; ++i) {
                w[i] = wn[i];
                wd[i] = wdn[i];
            }
            publish(buf ^ 1, (j + 1) % PD);
            fetch(j, k + PD);
            __syncthreads();
        }
    }
#pragma unroll
    for (int i = 0; i < M; ++i) {
        const int e = threadIdx.x + i * T;
        if (owned[i]) {
            vout[x0 + e - nk] = w[i];
            if (HV) voutd[x0 + e - nk] = wd[i];
        }
    }
    if (HV) {
        block_partials<4>(acc, red, partials);
    } else {
        double v[2] = {acc[0], acc[1]};
        block_partials<2>(v, red, partials);
    }
}

// second stage of the reverse sweep's sums: block 0 the loss (init kernel's partials),
// block 1 the coefficient shadows (all backward chunks' partials, in chunk order); 1024
// threads a block, so that a few partials a thread are all in flight at once
constexpr int FNT = 1024;
template <bool HV>
__global__ __launch_bounds__(FNT) void bwd_finalize_kernel(const double* pinit, int ninit, SumOuts loss_out,
                                                          const double* pbwd, int nbwd, SumOuts scal_out) {
    __shared__ double red[64];
    if (blockIdx.x == 0) {
        if (HV)
            finalize_partials<2>(pinit, ninit, red, loss_out);
        else
            finalize_partials<1>(pinit, ninit, red, loss_out);
    } else {
        if (HV)
            finalize_partials<4>(pbwd, nbwd, red, scal_out);
        else
            finalize_partials<2>(pbwd, nbwd, red, scal_out);
    }
}

// tangent: loss += sum u^2, lossd += sum (2 u) ud over the final state
__global__ __launch_bounds__(NT) void loss2_kernel(const double* __restrict__ u, const double* __restrict__ ud, int n,
                                                   double* partials) {
    __shared__ double red[32];
    double acc[2] = {0.0, 0.0};
    for (int x = blockIdx.x * NT + threadIdx.x; x < n; x += gridDim.x * NT) {
        double v = u[x];
        acc[1] += (2.0 * v) * ud[x];
        acc[0] += v * v;
    }
    block_partials<2>(acc, red, partials);
}

__global__ __launch_bounds__(NT) void branch_kernel(int64_t* __restrict__ b, int64_t nsteps, int64_t nrun) {
    for (int64_t t = (int64_t)blockIdx.x * NT + threadIdx.x; t < nsteps; t += (int64_t)gridDim.x * NT) b[t] = t < nrun ? 1 : 0;
}

__global__ __launch_bounds__(NT) void copy2_kernel(const double* __restrict__ a, double* __restrict__ ao,
                                                   const double* __restrict__ b, double* __restrict__ bo, int n) {
    for (int x = blockIdx.x * NT + threadIdx.x; x < n; x += gridDim.x * NT) {
        ao[x] = a[x];
        if (b) bo[x] = b[x];
    }
}

// the guard: how many leading steps run (tc < tend, tc += dt on taken steps), as the text does
int64_t taken_steps(double dt, double tend, int64_t nsteps) {
    double tc = 0.0;
    int64_t k = 0;
    for (int64_t t = 0; t < nsteps; ++t) {
        if (tc < tend) {
            tc = tc + dt;
            ++k;
        }
    }
    return k;
}

double* g_host_scal = nullptr;

int32_t host_scalars(double** out) {
    if (!g_host_scal) {
        hipError_t e = hipHostMalloc((void**)&g_host_scal, 8 * sizeof(double), hipHostMallocDefault);
        if (e != hipSuccess) return check_hip(e, "hipHostMalloc");
    }
    *out = g_host_scal;
    return STADE_HIP_OK;
}

unsigned grid_for(int n, int per_block) { return (unsigned)((n + per_block - 1) / per_block); }

int32_t check(int64_t n, int64_t nsteps, const char* fn) {
    if (n < 0 || nsteps < 0) return set_error(STADE_HIP_EINVAL, "%s: negative size (n = %lld, nsteps = %lld)", fn, (long long)n, (long long)nsteps);
    if (n > (1LL << 30)) return set_error(STADE_HIP_ERANGE, "%s: n = %lld exceeds 2^30 cells", fn, (long long)n);
    if (grid_for((int)n, BWD_S_HV) * 4 > (unsigned)kPartialSlots) return set_error(STADE_HIP_ERANGE, "%s: n too large for the workspace", fn);
    return STADE_HIP_OK;
}

// forward sweep over steps [t_begin, t_end): src (+d) -> final state in fin (+d); the state at
// the start of step t goes to tape row (t - row0) / every when every divides t - row0
template <bool TAN>
int32_t forward(const double* src, const double* srcd, double* fin, double* find, double* tape, double* taped, int n,
                int64_t t_begin, int64_t t_end, const Coef& c, double* P, double* Q, double* Pd, double* Qd, hipStream_t stream,
                int64_t row0 = 0, int every = 1) {
    // the four-cell form also where the tape is sparse: at most one row a launch (the checkpoint
    // policy's first sweep, a row every `every` >= KMAX steps)
    const bool notape = tape == nullptr || every >= KMAX;
    const unsigned nb = grid_for(n, notape ? FWD_S_NOTAPE : FWD_S);
    const double *cs = src, *csd = srcd;
    int64_t t0 = t_begin;
    int flip = 0;
    while (t0 < t_end) {
        int nk = (int)((t_end - t0) < KMAX ? (t_end - t0) : KMAX);
        bool last = t0 + nk >= t_end;
        double* d = last ? fin : (flip ? Q : P);
        double* dd = last ? find : (flip ? Qd : Pd);
        if (notape) {
            STADE_TIMED(TAN ? "burgers1d_fwd_tan" : "burgers1d_fwd", stream,
                        fwd_reg_kernel<TAN, FWD_S_NOTAPE, BNT_NOTAPE, FWD_C_NOTAPE><<<nb, BNT_NOTAPE, 0, stream>>>(cs, csd, d, dd, tape, taped, n, t0, nk, c,
                                                                                        row0, every));
        } else {
            STADE_TIMED(TAN ? "burgers1d_fwd_tan" : "burgers1d_fwd", stream,
                        fwd_reg_kernel<TAN, FWD_S, BNT, FWD_C><<<nb, BNT, 0, stream>>>(cs, csd, d, dd, tape, taped, n, t0, nk, c, row0,
                                                                                 every));
        }
        STADE_LAUNCHED("burgers1d fwd_reg_kernel");
        cs = d;
        csd = dd;
        flip ^= 1;
        t0 += nk;
    }
    return STADE_HIP_OK;
}

// reduction partials: the init kernel's at offset 0, the backward chunks' after it
int init_blocks(int64_t n) { return (int)grid_for((int)n, kInitBlockCells); }
size_t bwd_offset(int64_t n) { return ((size_t)init_blocks(n) * 2 + 1023) / 1024 * 1024; }
template <bool HV>
int bwd_blocks(int64_t n) { return (int)grid_for((int)n, HV ? BWD_S_HV : BWD_S); }
// (every > 1: the checkpoint policy's reverse sweep, whose segments of `every` steps are
// chunked separately)
template <bool HV>
int32_t check_partials(int64_t n, int64_t nrun, const char* fn, int64_t every = 1) {
    const int64_t chunks = every > 1 ? (nrun + every - 1) / every * ((every + KMAX - 1) / KMAX) : (nrun + KMAX - 1) / KMAX;
    const int64_t need = (int64_t)bwd_offset(n) + chunks * bwd_blocks<HV>(n) * (HV ? 4 : 2);
    if (need > kPartialSlots)
        return set_error(STADE_HIP_ERANGE, "%s: n * nsteps too large for the reduction workspace (%lld slots needed)", fn, (long long)need);
    return STADE_HIP_OK;
}

// The reverse sweep's state: the adjoint state (+d) in cw, the other buffer of the pair in ow,
// and the chunks done so far (each writes nb * NV partials).
struct BwdState {
    double *cw, *cwd, *ow, *owd;
    int chunk;
};

// reverse sweep over steps t_hi, t_hi - 1, ..., t_lo, reading tape row t - row0 for step t;
// when `final` the last chunk writes its state to ub (+d); *nparts = partial blocks so far
template <bool HV>
int32_t backward_range(BwdState& st, double* ub, double* ubd, const double* tape, const double* taped, int n, int64_t t_hi,
                       int64_t t_lo, int64_t row0, bool final, const Coef& c, double* pbwd, int* nparts, hipStream_t stream) {
    constexpr int S = HV ? BWD_S_HV : BWD_S, T = HV ? BWD_T_HV : BWD_T;
    constexpr int NV = HV ? 4 : 2;
    const unsigned nb = grid_for(n, S);
    int64_t t = t_hi;
    while (t >= t_lo) {
        int nk = (int)((t - t_lo + 1) < KMAX ? (t - t_lo + 1) : KMAX);
        bool last = final && t - nk < t_lo;
        double* d = last ? ub : st.ow;
        double* dd = last ? ubd : st.owd;
        if (nk == KMAX) {
            STADE_TIMED(HV ? "burgers1d_bwd_hv" : "burgers1d_bwd", stream,
                        bwd_reg_kernel<HV, S, 2, T><<<nb, T, 0, stream>>>(st.cw, st.cwd, d, dd, tape, taped, n, t, c,
                                                                      pbwd + (size_t)st.chunk * nb * NV, row0));
        } else {
            STADE_TIMED(HV ? "burgers1d_bwd_hv" : "burgers1d_bwd", stream,
                        bwd_kernel<HV, S, T><<<nb, T, 0, stream>>>(st.cw, st.cwd, d, dd, tape, taped, n, t, nk, c,
                                                                 pbwd + (size_t)st.chunk * nb * NV, row0));
        }
        STADE_LAUNCHED("burgers1d bwd_kernel");
        ++st.chunk;
        *nparts = st.chunk * (int)nb;
        std::swap(st.cw, st.ow);
        std::swap(st.cwd, st.owd);
        t -= nk;
    }
    return STADE_HIP_OK;
}

// reverse sweep over steps nrun..1 from w (+d) with the whole tape; the final state goes to
// ub (+d); returns the number of partial blocks written at pbwd
template <bool HV>
int32_t backward(double* w, double* wd, double* W2, double* W2d, double* ub, double* ubd, const double* tape, const double* taped,
                 int n, int64_t nrun, const Coef& c, double* pbwd, int* nparts, hipStream_t stream) {
    BwdState st{w, wd, W2, W2d, 0};
    return backward_range<HV>(st, ub, ubd, tape, taped, n, nrun - 1, 0, 0, true, c, pbwd, nparts, stream);
}

// The reverse sweep under the checkpoint policy: the forward kept the state at the start of
// every `every`-th step (rows ck, and ckd for the HVP); each segment [s0, s1), last first, is
// recomputed from its checkpoint into the segment tape seg (+ segd, `every` rows), then swept
// back.  The recomputed states are those the full forward produced (the same kernels, the
// same steps), so the reverse sweep reads the tape it would have read.
template <bool HV>
int32_t backward_ckpt(double* w, double* wd, double* W2, double* W2d, double* ub, double* ubd, const double* ck,
                      const double* ckd, double* seg, double* segd, double* R, int n, int64_t nrun, int every, const Coef& c,
                      double* pbwd, int* nparts, hipStream_t stream) {
    BwdState st{w, wd, W2, W2d, 0};
    double *R1 = R, *R2 = R + n, *R1d = R + 2 * (size_t)n, *R2d = R + 3 * (size_t)n, *Rf = R + 4 * (size_t)n,
           *Rfd = R + 5 * (size_t)n;
    const int64_t nseg = (nrun + every - 1) / every;
    for (int64_t k = nseg - 1; k >= 0; --k) {
        const int64_t s0 = k * every, s1 = std::min<int64_t>(s0 + every, nrun);
        const double* src = ck + (size_t)k * n;
        const double* srcd = HV ? ckd + (size_t)k * n : nullptr;
        if (int32_t rc = forward<HV>(src, srcd, Rf, HV ? Rfd : nullptr, seg, HV ? segd : nullptr, n, s0, s1, c, R1, R2,
                                     HV ? R1d : nullptr, HV ? R2d : nullptr, stream, s0, 1))
            return rc;
        if (int32_t rc = backward_range<HV>(st, ub, ubd, seg, HV ? segd : nullptr, n, s1 - 1, s0, s0, k == 0, c, pbwd, nparts,
                                            stream))
            return rc;
    }
    return STADE_HIP_OK;
}

}  // namespace
}  // namespace stade

using namespace stade;

namespace stade {
namespace {

template <bool CK>
int32_t adjoint_impl(const char* fn, int64_t every, double* loss, const double* lossb, const double* u, double* ub, double* un, double* unb,
                              double nu, double* nub, double dt, double* dtb, double dx, double* dxb, double tend, double* tendb,
                              int64_t n, int64_t nsteps, int64_t* branch_stack, double* u_stack, hipStream_t stream) {
    if (int32_t rc = check(n, nsteps, fn)) return rc;
    if (!nub || !dtb || !dxb || !tendb) return set_error(STADE_HIP_EINVAL, "%s: null scalar shadow", fn);
    if ((n > 0 && (!loss || !lossb || !u || !ub || !un || !unb)) || (nsteps > 0 && (!branch_stack || (n > 0 && !u_stack))))
        return set_error(STADE_HIP_EINVAL, "%s: null pointer", fn);
    const double cadv = 0.5 * dt / dx;
    const double cdif = nu * dt / (dx * dx);
    const int64_t nrun = taken_steps(dt, tend, nsteps);
    if (int32_t rc = check_partials<false>(n, nrun, fn, CK ? every : 1)) return rc;
    Coef c{cadv, cdif, 0.0, 0.0};
    WsCall call_(stream);
    Workspace* ws = call_.ws;
    if (!ws) return STADE_HIP_ENOMEM;
    if (nsteps > 0) {
        STADE_TIMED("burgers1d_branch", stream, branch_kernel<<<grid_for((int)(nsteps < (1 << 20) ? nsteps : (1 << 20)), NT), NT, 0, stream>>>(branch_stack, nsteps, nrun));
        STADE_LAUNCHED("burgers1d branch_kernel");
    }
    double cadvb = 0.0, cdifb = 0.0;
    if (n > 0) {
        // checkpoint policy: the segment tape (`every` rows) and the recompute states follow
        const size_t seg_len = CK ? (size_t)every * (size_t)n : 0;
        double* P = (double*)scratch(sizeof(double) * (2 * (size_t)n + (CK ? seg_len + 6 * (size_t)n : 0)));
        if (!P) return scratch_error();
        double* Q = P + n;
        double* seg = Q + n;
        double* R = seg + seg_len;
        if (int32_t rc = forward<false>(u, nullptr, un, nullptr, u_stack, nullptr, (int)n, 0, nrun, c, P, Q, nullptr, nullptr, stream,
                                        0, CK ? (int)every : 1))
            return rc;
        const double* uT = nrun > 0 ? un : u;
        const int gi = init_blocks(n);
        STADE_TIMED("burgers1d_init", stream,
                    bwd_init_kernel<false><<<gi, NT, 0, stream>>>(uT, nullptr, ub, nullptr, unb, nullptr, P, nullptr, lossb, nullptr,
                                                                  (int)n, nrun > 0, ws->dscalars, ws->partials));
        STADE_LAUNCHED("burgers1d bwd_init_kernel");
        int nparts = 0;
        double* pbwd = ws->partials + bwd_offset(n);
        if (nrun > 0) {
            int32_t rc = CK ? backward_ckpt<false>(P, nullptr, Q, nullptr, ub, nullptr, u_stack, nullptr, seg, nullptr, R, (int)n, nrun,
                                                   (int)every, c, pbwd, &nparts, stream)
                            : backward<false>(P, nullptr, Q, nullptr, ub, nullptr, u_stack, nullptr, (int)n, nrun, c, pbwd, &nparts,
                                              stream);
            if (rc) return rc;
        }
        STADE_TIMED("finalize", stream,
                    bwd_finalize_kernel<false><<<2, FNT, 0, stream>>>(ws->partials, gi, SumOuts{{loss}}, pbwd, nparts,
                                                                     SumOuts{{ws->dscalars + 0, ws->dscalars + 1}}));
        STADE_LAUNCHED("burgers1d bwd_finalize_kernel");
        double* hs;
        if (int32_t rc = host_scalars(&hs)) return rc;
        STADE_TRY_HIP(hipMemcpyAsync(hs, ws->dscalars, 2 * sizeof(double), hipMemcpyDeviceToHost, stream));
        STADE_TRY_HIP(hipStreamSynchronize(stream));
        cadvb = hs[0];
        cdifb = hs[1];
    } else {
        STADE_TRY_HIP(hipStreamSynchronize(stream));
    }
    // the statements after the time loop, on the host in the generated order
    double nub_ = *nub, dtb_ = *dtb, dxb_ = *dxb;
    if (nrun > 0) dtb_ = dtb_ + 0.0;  // dtb = dtb + tcb on each taken step; tcb is never seeded
    const double o8 = cdifb;
    const double c9 = dx * dx;
    nub_ = nub_ + (dt / c9) * o8;
    dtb_ = dtb_ + (nu / c9) * o8;
    const double c10 = -((nu * dt) / (c9 * c9)) * o8;
    dxb_ = dxb_ + dx * c10;
    dxb_ = dxb_ + dx * c10;
    const double o11 = cadvb;
    dtb_ = dtb_ + (0.5 / dx) * o11;
    dxb_ = dxb_ + -((0.5 * dt) / (dx * dx)) * o11;
    *nub = nub_;
    *dtb = dtb_;
    *dxb = dxb_;
    return STADE_HIP_OK;
}

template <bool CK>
int32_t hvp_impl(const char* fn, int64_t every, double* loss, const double* lossb, const double* u, double* ub, double* un, double* unb,
                               double nu, double* nub, double dt, double* dtb, double dx, double* dxb, double tend, double* tendb,
                               int64_t n, int64_t nsteps, double* lossd, const double* lossbd, const double* ud, double* ubd,
                               double* und, double* unbd, double nud, double* nubd, double dtd, double* dtbd, double dxd,
                               double* dxbd, double tendd, double* tendbd, int64_t* branch_stack, double* u_stack,
                               hipStream_t stream) {
    (void)tendd;
    if (int32_t rc = check(n, nsteps, fn)) return rc;
    if (!nub || !dtb || !dxb || !tendb || !nubd || !dtbd || !dxbd || !tendbd)
        return set_error(STADE_HIP_EINVAL, "%s: null scalar shadow", fn);
    if ((n > 0 && (!loss || !lossb || !u || !ub || !un || !unb || !lossd || !lossbd || !ud || !ubd || !und || !unbd)) ||
        (nsteps > 0 && (!branch_stack || (n > 0 && !u_stack))))
        return set_error(STADE_HIP_EINVAL, "%s: null pointer", fn);
    const double c0 = dx * dx;
    Coef c{0.5 * dt / dx, nu * dt / c0, (0.5 * dtd) / dx + -((0.5 * dt) / (dx * dx)) * dxd,
           (dt * nud + nu * dtd) / c0 + -((nu * dt) / (c0 * c0)) * (dx * dxd + dx * dxd)};
    const int64_t nrun = taken_steps(dt, tend, nsteps);
    if (int32_t rc = check_partials<true>(n, nrun, fn, CK ? every : 1)) return rc;
    WsCall call_(stream);
    Workspace* ws = call_.ws;
    if (!ws) return STADE_HIP_ENOMEM;
    if (nsteps > 0) {
        STADE_TIMED("burgers1d_branch", stream, branch_kernel<<<grid_for((int)(nsteps < (1 << 20) ? nsteps : (1 << 20)), NT), NT, 0, stream>>>(branch_stack, nsteps, nrun));
        STADE_LAUNCHED("burgers1d branch_kernel");
    }
    double sc[4] = {0.0, 0.0, 0.0, 0.0};  // cadvb, cdifb, cadvbd, cdifbd
    if (n > 0) {
        // u_stack_d: allocated inside the generated _hv (Vector{Float64}(undef, length(u_stack)));
        // here a library scratch region, reused across calls
        // (checkpoint policy: u_stack_d holds the checkpoints of ud, and the two segment tapes
        // and the recompute states follow)
        const size_t rows = CK ? (size_t)((nrun + every - 1) / every) : (size_t)nrun;
        const size_t tape_len = rows * (size_t)n;
        const size_t seg_len = CK ? (size_t)every * (size_t)n : 0;
        double* P = (double*)scratch(sizeof(double) * (4 * (size_t)n + tape_len + (CK ? 2 * seg_len + 6 * (size_t)n : 0)));
        if (!P) return scratch_error();
        double *Q = P + n, *Pd = Q + n, *Qd = Pd + n, *taped = Qd + n;
        double *seg = taped + tape_len, *segd = seg + seg_len, *R = segd + seg_len;
        if (int32_t rc = forward<true>(u, ud, un, und, u_stack, taped, (int)n, 0, nrun, c, P, Q, Pd, Qd, stream, 0,
                                       CK ? (int)every : 1))
            return rc;
        const double* uT = nrun > 0 ? un : u;
        const double* udT = nrun > 0 ? und : ud;
        const int gi = init_blocks(n);
        STADE_TIMED("burgers1d_init", stream,
                    bwd_init_kernel<true><<<gi, NT, 0, stream>>>(uT, udT, ub, ubd, unb, unbd, P, Pd, lossb, lossbd, (int)n,
                                                                 nrun > 0, ws->dscalars, ws->partials));
        STADE_LAUNCHED("burgers1d bwd_init_kernel");
        int nparts = 0;
        double* pbwd = ws->partials + bwd_offset(n);
        if (nrun > 0) {
            int32_t rc = CK ? backward_ckpt<true>(P, Pd, Q, Qd, ub, ubd, u_stack, taped, seg, segd, R, (int)n, nrun, (int)every, c,
                                                  pbwd, &nparts, stream)
                            : backward<true>(P, Pd, Q, Qd, ub, ubd, u_stack, taped, (int)n, nrun, c, pbwd, &nparts, stream);
            if (rc) return rc;
        }
        STADE_TIMED("finalize", stream,
                    bwd_finalize_kernel<true><<<2, FNT, 0, stream>>>(ws->partials, gi, SumOuts{{loss, lossd}}, pbwd, nparts,
                                                                    SumOuts{{ws->dscalars + 0, ws->dscalars + 1,
                                                                             ws->dscalars + 2, ws->dscalars + 3}}));
        STADE_LAUNCHED("burgers1d bwd_finalize_kernel");
        double* hs;
        if (int32_t rc = host_scalars(&hs)) return rc;
        STADE_TRY_HIP(hipMemcpyAsync(hs, ws->dscalars, 4 * sizeof(double), hipMemcpyDeviceToHost, stream));
        STADE_TRY_HIP(hipStreamSynchronize(stream));
        for (int k = 0; k < 4; ++k) sc[k] = hs[k];
    } else {
        STADE_TRY_HIP(hipStreamSynchronize(stream));
    }
    // the statements after the time loop of the generated _hv, on the host in their order
    double nb_ = *nub, nbd_ = *nubd, db_ = *dtb, dbd_ = *dtbd, xb_ = *dxb, xbd_ = *dxbd;
    if (nrun > 0) {
        dbd_ = dbd_ + 0.0;
        db_ = db_ + 0.0;
    }
    const double o8d = sc[3], o8 = sc[1];
    const double c9d = dx * dxd + dx * dxd, c9 = dx * dx;
    const double h10d = dtd / c9 + -(dt / (c9 * c9)) * c9d, h10 = dt / c9;
    nbd_ = nbd_ + (o8 * h10d + h10 * o8d);
    nb_ = nb_ + h10 * o8;
    const double h11d = nud / c9 + -(nu / (c9 * c9)) * c9d, h11 = nu / c9;
    dbd_ = dbd_ + (o8 * h11d + h11 * o8d);
    db_ = db_ + h11 * o8;
    const double h12d = dt * nud + nu * dtd, h12 = nu * dt;
    const double h13d = (2 * c9) * c9d, h13 = c9 * c9;
    const double c10d = -(h12 / h13) * o8d + -(h12d / h13 + -(h12 / (h13 * h13)) * h13d) * o8;
    const double c10 = -(h12 / h13) * o8;
    xbd_ = xbd_ + (c10 * dxd + dx * c10d);
    xb_ = xb_ + dx * c10;
    xbd_ = xbd_ + (c10 * dxd + dx * c10d);
    xb_ = xb_ + dx * c10;
    const double o11d = sc[2], o11 = sc[0];
    const double h14d = -(0.5 / (dx * dx)) * dxd, h14 = 0.5 / dx;
    dbd_ = dbd_ + (o11 * h14d + h14 * o11d);
    db_ = db_ + h14 * o11;
    const double dx2 = dx * dx;
    const double h15d = -((0.5 * dtd) / dx2 + -((0.5 * dt) / (dx2 * dx2)) * ((2 * dx) * dxd));
    const double h15 = -((0.5 * dt) / dx2);
    xbd_ = xbd_ + (o11 * h15d + h15 * o11d);
    xb_ = xb_ + h15 * o11;
    *nub = nb_;
    *nubd = nbd_;
    *dtb = db_;
    *dtbd = dbd_;
    *dxb = xb_;
    *dxbd = xbd_;
    return STADE_HIP_OK;
}

}  // namespace
}  // namespace stade

extern "C" {

int32_t stade_hip_burgers1d_stack_lengths(int64_t n, int64_t nsteps, int64_t lengths[2]) {
    // initstacks_burgers1d_b: branch_stack max(0, div(nsteps - 1, 1) + 1),
    // u_stack max(0, div(nsteps - 1, 1) + 1) * max(0, div(n - 1, 1) + 1)   (Julia div truncates)
    if (!lengths) return set_error(STADE_HIP_EINVAL, "stade_hip_burgers1d_stack_lengths: null lengths");
    int64_t a = (nsteps - 1) / 1 + 1, b = (n - 1) / 1 + 1;
    a = a > 0 ? a : 0;
    b = b > 0 ? b : 0;
    lengths[0] = a;
    lengths[1] = a * b;
    return STADE_HIP_OK;
}

int32_t stade_hip_initstacks_burgers1d_b(int64_t n, int64_t nsteps, int64_t** branch_stack, double** u_stack) {
    int64_t len[2];
    if (int32_t rc = stade_hip_burgers1d_stack_lengths(n, nsteps, len)) return rc;
    if (!branch_stack || !u_stack) return set_error(STADE_HIP_EINVAL, "stade_hip_initstacks_burgers1d_b: null output");
    *branch_stack = nullptr;
    *u_stack = nullptr;
    STADE_TRY_HIP(hipMalloc((void**)branch_stack, (size_t)(len[0] > 0 ? len[0] : 1) * sizeof(int64_t)));
    hipError_t e = hipMalloc((void**)u_stack, (size_t)(len[1] > 0 ? len[1] : 1) * sizeof(double));
    if (e != hipSuccess) {
        (void)hipFree(*branch_stack);  // the allocation error is the one reported
        *branch_stack = nullptr;
        return check_hip(e, "hipMalloc(u_stack)");
    }
    return STADE_HIP_OK;
}

int32_t stade_hip_burgers1d_b(double* loss, const double* lossb, const double* u, double* ub, double* un, double* unb,
                              double nu, double* nub, double dt, double* dtb, double dx, double* dxb, double tend, double* tendb,
                              int64_t n, int64_t nsteps, int64_t* branch_stack, double* u_stack, hipStream_t stream) {
    return adjoint_impl<false>("stade_hip_burgers1d_b", 1, loss, lossb, u, ub, un, unb, nu, nub, dt, dtb, dx, dxb, tend, tendb, n,
                               nsteps, branch_stack, u_stack, stream);
}

int32_t stade_hip_burgers1d_ckpt_lengths(int64_t n, int64_t nsteps, int64_t every, int64_t lengths[2]) {
    if (!lengths) return set_error(STADE_HIP_EINVAL, "stade_hip_burgers1d_ckpt_lengths: null lengths");
    if (every < 1 || every > (1 << 20)) return set_error(STADE_HIP_ERANGE, "stade_hip_burgers1d_ckpt_lengths: every = %lld out of range", (long long)every);
    const int64_t a = nsteps > 0 ? nsteps : 0, b = n > 0 ? n : 0;
    lengths[0] = a;
    lengths[1] = (a + every - 1) / every * b;
    return STADE_HIP_OK;
}

int32_t stade_hip_burgers1d_b_ckpt(double* loss, const double* lossb, const double* u, double* ub, double* un, double* unb,
                                   double nu, double* nub, double dt, double* dtb, double dx, double* dxb, double tend,
                                   double* tendb, int64_t n, int64_t nsteps, int64_t* branch_stack, double* u_ckpt, int64_t every,
                                   hipStream_t stream) {
    if (every < 1 || every > (1 << 20)) return set_error(STADE_HIP_ERANGE, "stade_hip_burgers1d_b_ckpt: every = %lld out of range", (long long)every);
    return adjoint_impl<true>("stade_hip_burgers1d_b_ckpt", every, loss, lossb, u, ub, un, unb, nu, nub, dt, dtb, dx, dxb, tend,
                              tendb, n, nsteps, branch_stack, u_ckpt, stream);
}

int32_t stade_hip_burgers1d_d(double* loss, double* lossd, double* u, double* ud, double* un, double* und, double nu, double nud,
                              double dt, double dtd, double dx, double dxd, double tend, double tendd, int64_t n, int64_t nsteps,
                              hipStream_t stream) {
    (void)tendd;
    if (int32_t rc = check(n, nsteps, "stade_hip_burgers1d_d")) return rc;
    if (n == 0) return STADE_HIP_OK;
    if (!loss || !lossd || !u || !ud || !un || !und) return set_error(STADE_HIP_EINVAL, "stade_hip_burgers1d_d: null pointer");
    const double c0 = dx * dx;
    Coef c{0.5 * dt / dx, nu * dt / c0, (0.5 * dtd) / dx + -((0.5 * dt) / (dx * dx)) * dxd,
           (dt * nud + nu * dtd) / c0 + -((nu * dt) / (c0 * c0)) * (dx * dxd + dx * dxd)};
    const int64_t nrun = taken_steps(dt, tend, nsteps);
    WsCall call_(stream);
    Workspace* ws = call_.ws;
    if (!ws) return STADE_HIP_ENOMEM;
    double* P = (double*)scratch(sizeof(double) * 4 * (size_t)n);
    if (!P) return scratch_error();
    double *Q = P + n, *Pd = Q + n, *Qd = Pd + n;
    if (nrun > 0) {
        if (int32_t rc = forward<true>(u, ud, un, und, nullptr, nullptr, (int)n, 0, nrun, c, P, Q, Pd, Qd, stream)) return rc;
        STADE_TIMED("burgers1d_copy", stream, copy2_kernel<<<grid_for((int)n, NT * 8), NT, 0, stream>>>(un, u, und, ud, (int)n));
        STADE_LAUNCHED("burgers1d copy2_kernel");
    }
    // loss and lossd from the final state, now in u and ud
    const int gl = init_blocks(n);
    STADE_TIMED("burgers1d_loss", stream, loss2_kernel<<<gl, NT, 0, stream>>>(u, ud, (int)n, ws->partials));
    STADE_LAUNCHED("burgers1d loss2_kernel");
    STADE_TIMED("finalize", stream, finalize_kernel<2><<<1, NT, 0, stream>>>(ws->partials, gl, SumOuts{{loss, lossd}}));
    STADE_LAUNCHED("burgers1d finalize_kernel");
    return STADE_HIP_OK;
}

int32_t stade_hip_burgers1d_hv(double* loss, const double* lossb, const double* u, double* ub, double* un, double* unb,
                               double nu, double* nub, double dt, double* dtb, double dx, double* dxb, double tend, double* tendb,
                               int64_t n, int64_t nsteps, double* lossd, const double* lossbd, const double* ud, double* ubd,
                               double* und, double* unbd, double nud, double* nubd, double dtd, double* dtbd, double dxd,
                               double* dxbd, double tendd, double* tendbd, int64_t* branch_stack, double* u_stack,
                               hipStream_t stream) {
    return hvp_impl<false>("stade_hip_burgers1d_hv", 1, loss, lossb, u, ub, un, unb, nu, nub, dt, dtb, dx, dxb, tend, tendb, n, nsteps,
                           lossd, lossbd, ud, ubd, und, unbd, nud, nubd, dtd, dtbd, dxd, dxbd, tendd, tendbd, branch_stack, u_stack,
                           stream);
}

int32_t stade_hip_burgers1d_hv_ckpt(double* loss, const double* lossb, const double* u, double* ub, double* un, double* unb,
                                    double nu, double* nub, double dt, double* dtb, double dx, double* dxb, double tend, double* tendb,
                                    int64_t n, int64_t nsteps, double* lossd, const double* lossbd, const double* ud, double* ubd,
                                    double* und, double* unbd, double nud, double* nubd, double dtd, double* dtbd, double dxd,
                                    double* dxbd, double tendd, double* tendbd, int64_t* branch_stack, double* u_ckpt, int64_t every,
                                    hipStream_t stream) {
    if (every < 1 || every > (1 << 20)) return set_error(STADE_HIP_ERANGE, "stade_hip_burgers1d_hv_ckpt: every = %lld out of range", (long long)every);
    return hvp_impl<true>("stade_hip_burgers1d_hv_ckpt", every, loss, lossb, u, ub, un, unb, nu, nub, dt, dtb, dx, dxb, tend, tendb, n,
                          nsteps, lossd, lossbd, ud, ubd, und, unbd, nud, nubd, dtd, dtbd, dxd, dxbd, tendd, tendbd, branch_stack,
                          u_ckpt, stream);
}

}  // extern "C"
