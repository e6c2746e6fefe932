// diffusion2d: tangent, adjoint and HVP of one explicit periodic 5-point diffusion step
// followed by loss += sum(un .^ 2), on an n x n column-major grid (i fastest).
//
// Generated code this replaces: stade.jl_amd/corpus/diffusion2d_{b,d,hv}.jl, the STADE
// adjoint/tangent/HVP of diffusion2d.jl (`agen_emit` /root/reference/src/STADE.jl:3390-3419,
// `tgen_emit` 3271-3278, `hvp_emit` 6729-6782), which `stade_amdgpu_file` (18604) runs as one
// launch per loop plus a host mapreduce for the loss (10519-10571) and the periodic
// owner-computes gather (`cgen_gather_periodic_inverse` 7343-7529) for the adjoint scatter.
//
// Two kernel families:
//   * wave-strip kernels: one wavefront per strip of 128 columns (n a multiple of 128, the
//     benchmark grids; 16-byte accesses) or of 64 columns (n a multiple of 64 only) and a chunk
//     of rows, no LDS and no barriers (described at their definition);
//   * row-streaming kernels (every other n), described next.
//
// Row-streaming layout and work per launch:
//   * A 256-thread block owns a strip of 256 columns (i) and a chunk of CH rows (j); thread t
//     owns column c0 + t.  It marches down its rows keeping ring buffers of whole strip rows
//     in LDS (u: 5 rows, the new state's adjoint seed w: 3 rows), each row with a periodic
//     halo of 2 columns a side.  Every array element of the chunk is loaded once (plus the
//     2-row / 2-column halo), and the loads for two rows ahead are issued before the current
//     row is computed (two register sets, the row loop unrolled by two), so each wave keeps
//     reads in flight across the barriers.
//   * adjoint, pass 1, for output row j: un on row j+1 (interior and the 1-column halo),
//     w = unb + (2 un) lossb there, then the owner-computes gather
//     ub[c] += w_c + 0.1 (w_E + w_W + w_N + w_S) + 4 (-(0.1 w_c)): each cell owns its ub, no
//     atomics.  Pass 1 reads unb but never writes it, so the halo reads cannot race with the
//     reset.  Pass 2 streams the reset unb = 0 and, in its first block, adds the per-block
//     loss partials of pass 1 (the second stage of the grid sum).  HBM traffic = 48 B/cell,
//     the algorithmic figure (u R, un W, unb R+W, ub R+W): 40 B/cell in pass 1, 8 in pass 2.
//   * tangent: un, und for row j from u, ud rows j-1..j+1 (3-row rings), loss partials.
//   * blockIdx = chunk * strips + strip: the blocks that share a halo row are `strips`
//     launches apart, on the same XCD (round-robin dispatch) when strips is a multiple of 8.
#include "internal.hpp"

#include <mutex>
#include <initializer_list>
#include <type_traits>
#include "../../include/stade_hip.h"

namespace stade {
namespace {

typedef double dvec2 __attribute__((ext_vector_type(2)));
// streaming (nontemporal) 16-byte access to a pair, for data read or written once by a pass:
// the hint keeps these streams from displacing the halo lines that neighbouring waves re-read
// from L2 (the adjoint pass went from 137 to 108 us with it)
__device__ __forceinline__ double2 nt_load2(const double2* p) {
    const dvec2 v = __builtin_nontemporal_load(reinterpret_cast<const dvec2*>(p));
    return make_double2(v.x, v.y);
}
__device__ __forceinline__ void nt_store2(double2 v, double2* p) {
    const dvec2 w = {v.x, v.y};
    __builtin_nontemporal_store(w, reinterpret_cast<dvec2*>(p));
}
constexpr int SW = 256, NT = SW;  // strip width = threads per block
constexpr int RW = SW + 4;        // LDS row: 2 halo columns each side (position k = column - c0 + 2)
constexpr int CH = 32;            // rows per block (measured best of 16 / 32 / 64 at n = 4096)

// Column geometry of a strip: wi columns c0 .. c0+wi-1; LDS positions 0, 1 hold columns
// c0-2, c0-1 and positions wi+2, wi+3 hold c0+wi, c0+wi+1 (periodic).  Threads 0..3 each
// carry one halo column (hcol) and its LDS position (hpos) in registers: a per-thread array
// indexed by the thread id would live in scratch memory and cost a load per row.
struct Strip {
    int c0, wi, j0, wj, n;
    int hcol, hpos;
};

__device__ __forceinline__ Strip strip_of(int n, int strips) {
    Strip s;
    const int sx = blockIdx.x % strips, cy = blockIdx.x / strips;
    const int t = threadIdx.x;
    s.c0 = sx * SW;
    s.wi = min(SW, n - s.c0);
    s.j0 = cy * CH;
    s.wj = min(CH, n - s.j0);
    s.n = n;
    const int off = t < 2 ? t - 2 : s.wi + (t & 3) - 2;  // t = 0..3: c0-2, c0-1, c0+wi, c0+wi+1
    s.hcol = wrapn(s.c0 + off, n);
    s.hpos = t < 2 ? t : s.wi + (t & 3);
    return s;
}

// One strip row of an array: the thread's own column and (threads 0..3) a halo column.
struct RowVal {
    double own, halo;
};

// halo = 2: all four halo columns (u, ud of the adjoint: the new state is formed on a
// 1-column halo); halo = 1: only columns c0-1 and c0+wi (threads 1 and 2)
__device__ __forceinline__ RowVal load_row(const double* __restrict__ a, const Strip& s, int r, int halo) {
    const int t = threadIdx.x;
    const size_t base = (size_t)wrapn(s.j0 + r, s.n) * s.n;
    RowVal v{0.0, 0.0};
    if (t < s.wi) v.own = a[base + s.c0 + t];
    if (halo == 2 ? t < 4 : (t == 1 || t == 2)) v.halo = a[base + s.hcol];
    return v;
}

__device__ __forceinline__ void put_row(double* row, const RowVal& v, const Strip& s) {
    const int t = threadIdx.x;
    if (t < s.wi) row[t + 2] = v.own;
    if (t < 4) row[s.hpos] = v.halo;
}

// un at LDS position k of the middle row, in the operation order of the generated text:
// u + 0.1 * (u[W] + u[E] + u[S] + u[N] - 4.0 * u)
__device__ __forceinline__ double step5(const double* up, const double* uc, const double* dn, int k) {
    const double c = uc[k];
    double t = uc[k - 1] + uc[k + 1];
    t = t + up[k];
    t = t + dn[k];
    t = t - 4.0 * c;
    return c + 0.1 * t;
}
// tangent form: ud + 0.1 * ((((ud[W] + ud[E]) + ud[S]) + ud[N]) + -(4.0 * ud))
__device__ __forceinline__ double step5d(const double* up, const double* uc, const double* dn, int k) {
    const double c = uc[k];
    double t = uc[k - 1] + uc[k + 1];
    t = t + up[k];
    t = t + dn[k];
    t = t + -(4.0 * c);
    return c + 0.1 * t;
}

// ---------------------------------------------------------------------------------------
// tangent: un, und, loss += sum un^2, lossd += sum (2 un) und
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(NT) void diffusion_d_kernel(const double* __restrict__ u, const double* __restrict__ ud,
                                                         double* __restrict__ un, double* __restrict__ und, int n,
                                                         int strips, double* partials) {
    __shared__ double su[3][RW];
    __shared__ double sud[3][RW];
    __shared__ double red[32];
    const Strip s = strip_of(n, strips);
    const int t = threadIdx.x, k = t + 2;
    double acc[2] = {0.0, 0.0};
    // rows -1, 0 staged; row 1 in flight
    put_row(su[0], load_row(u, s, -1, 1), s);
    put_row(sud[0], load_row(ud, s, -1, 1), s);
    put_row(su[1], load_row(u, s, 0, 1), s);
    put_row(sud[1], load_row(ud, s, 0, 1), s);
    // row r+1 is staged at step r: sets q[0], q[1] hold the rows of the next even / odd step
    struct Pref {
        RowVal u, ud;
    } q[2];
    auto fetch = [&](Pref& p, int r) {
        if (r < s.wj) {
            p.u = load_row(u, s, r + 1, 1);
            p.ud = load_row(ud, s, r + 1, 1);
        }
    };
    fetch(q[0], 0);
    fetch(q[1], 1);
    auto step = [&](int r, Pref& p) {
        const int sp = r % 3, sc = (r + 1) % 3, sn = (r + 2) % 3;  // rows r-1, r, r+1 (row q in slot (q+1) % 3)
        put_row(su[sn], p.u, s);
        put_row(sud[sn], p.ud, s);
        fetch(p, r + 2);
        __syncthreads();
        if (t < s.wi) {
            const double v = step5(su[sp], su[sc], su[sn], k);
            const double vd = step5d(sud[sp], sud[sc], sud[sn], k);
            const size_t g = (size_t)(s.j0 + r) * n + s.c0 + t;
            und[g] = vd;
            un[g] = v;
            acc[1] += (2.0 * v) * vd;
            acc[0] += v * v;
        }
        __syncthreads();
    };
    for (int r = 0; r < s.wj; r += 2) {
        step(r, q[0]);
        if (r + 1 < s.wj) step(r + 1, q[1]);
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
                                                         int n, int strips, double* partials) {
    __shared__ double su[5][RW];
    __shared__ double sw[3][RW];
    __shared__ double sud[HV ? 5 : 1][HV ? RW : 1];
    __shared__ double swd[HV ? 3 : 1][HV ? RW : 1];
    __shared__ double red[32];
    const Strip s = strip_of(n, strips);
    const int t = threadIdx.x, k = t + 2;
    const double lb = lossb[0];
    const double lbd = HV ? lossbd[0] : 0.0;
    double acc[2] = {0.0, 0.0};

    // un / w of strip row r (interior columns, then threads 0 and 1 the halo columns c0-1 and
    // c0+wi) from the u rings (rows r-1, r, r+1 in slots (r+1)%5, (r+2)%5, (r+3)%5), into w
    // slot (r+1)%3; the owned interior of rows 0..wj-1 is stored.  The unb halo values are
    // held by threads 1 (column c0-1) and 2 (column c0+wi) and shuffled to threads 0 and 1
    // by every lane, outside the branches.
    auto new_state_all = [&](int r, const RowVal& nb, const RowVal& nbd) {
        const double hb0 = __shfl(nb.halo, 1, 64), hb1 = __shfl(nb.halo, 2, 64);
        const double hbd0 = HV ? __shfl(nbd.halo, 1, 64) : 0.0, hbd1 = HV ? __shfl(nbd.halo, 2, 64) : 0.0;
        const int sp = (r + 1) % 5, sc = (r + 2) % 5, sn = (r + 3) % 5, sw_ = (r + 1) % 3;
        const bool own_row = r >= 0 && r < s.wj;
        auto one = [&](int kk, double b, double bd, bool store) {
            const double v = step5(su[sp], su[sc], su[sn], kk);
            double vd = 0.0;
            if constexpr (HV) {
                vd = step5d(sud[sp], sud[sc], sud[sn], kk);
                swd[sw_][kk] = bd + (lb * (2.0 * vd) + (2.0 * v) * lbd);
            }
            sw[sw_][kk] = b + (2.0 * v) * lb;
            if (store) {
                const size_t g = (size_t)(s.j0 + r) * n + s.c0 + t;
                if (HV) {
                    und[g] = vd;
                    acc[1] += (2.0 * v) * vd;
                }
                un[g] = v;
                acc[0] += v * v;
            }
        };
        if (t < s.wi) one(k, nb.own, nbd.own, own_row);
        if (t == 0) one(1, hb0, hbd0, false);
        if (t == 1) one(s.wi + 2, hb1, hbd1, false);
    };

    // prologue: u rows -2..1 and unb rows -1, 0 staged; w rows -1, 0 formed
    for (int r = -2; r <= 1; ++r) {
        put_row(su[(r + 2) % 5], load_row(u, s, r, 2), s);
        if constexpr (HV) put_row(sud[(r + 2) % 5], load_row(ud, s, r, 2), s);
    }
    RowVal b_m1 = load_row(unb, s, -1, 1), b_0 = load_row(unb, s, 0, 1);
    RowVal bd_m1{0.0, 0.0}, bd_0{0.0, 0.0};
    if constexpr (HV) {
        bd_m1 = load_row(unbd, s, -1, 1);
        bd_0 = load_row(unbd, s, 0, 1);
    }
    __syncthreads();
    new_state_all(-1, b_m1, bd_m1);
    new_state_all(0, b_0, bd_0);
    // step r stages u row r+2 and uses unb row r+1 and ub row r: sets q[0], q[1] hold those
    // of the next even / odd step, refilled two steps ahead
    struct Pref {
        RowVal u, ud, b, bd;
        double ub, ubd;
    } q[2];
    auto fetch = [&](Pref& p, int r) {
        if (r >= s.wj) return;
        p.u = load_row(u, s, r + 2, 2);
        p.b = load_row(unb, s, r + 1, 1);
        if (t < s.wi) p.ub = ub[(size_t)(s.j0 + r) * n + s.c0 + t];
        if constexpr (HV) {
            p.ud = load_row(ud, s, r + 2, 2);
            p.bd = load_row(unbd, s, r + 1, 1);
            if (t < s.wi) p.ubd = ubd[(size_t)(s.j0 + r) * n + s.c0 + t];
        }
    };
    q[0].ud = q[0].bd = q[1].ud = q[1].bd = RowVal{0.0, 0.0};
    q[0].ub = q[0].ubd = q[1].ub = q[1].ubd = 0.0;
    fetch(q[0], 0);
    fetch(q[1], 1);
    auto step = [&](int r, Pref& p) {
        // A: stage u row r+2; refill this set for step r+2
        put_row(su[(r + 4) % 5], p.u, s);
        if constexpr (HV) put_row(sud[(r + 4) % 5], p.ud, s);
        const RowVal cb = p.b, cbd = p.bd;
        const double cub = p.ub, cubd = p.ubd;
        fetch(p, r + 2);
        __syncthreads();
        // B: un and w of row r+1
        new_state_all(r + 1, cb, cbd);
        __syncthreads();
        // C: gather into ub of row r from w rows r-1, r, r+1
        if (t < s.wi) {
            const double* wm = sw[r % 3];
            const double* wc = sw[(r + 1) % 3];
            const double* wp = sw[(r + 2) % 3];
            const double c = wc[k];
            double a = c;
            a = a + 0.1 * wc[k + 1];
            a = a + 0.1 * wc[k - 1];
            a = a + 0.1 * wp[k];
            a = a + 0.1 * wm[k];
            a = a + 4.0 * -(0.1 * c);
            const size_t g = (size_t)(s.j0 + r) * n + s.c0 + t;
            if constexpr (HV) {
                const double* dm = swd[r % 3];
                const double* dc = swd[(r + 1) % 3];
                const double* dp = swd[(r + 2) % 3];
                const double cd = dc[k];
                double ad = cd;
                ad = ad + 0.1 * dc[k + 1];
                ad = ad + 0.1 * dc[k - 1];
                ad = ad + 0.1 * dp[k];
                ad = ad + 0.1 * dm[k];
                ad = ad + 4.0 * -(0.1 * cd);
                ubd[g] = cubd + ad;
            }
            ub[g] = cub + a;
        }
    };
    for (int r = 0; r < s.wj; r += 2) {
        step(r, q[0]);
        if (r + 1 < s.wj) step(r + 1, q[1]);
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
            // streaming stores: the zeros are not read again by this evaluation
            nt_store2(make_double2(0.0, 0.0), reinterpret_cast<double2*>(a + k));
            if (b) nt_store2(make_double2(0.0, 0.0), reinterpret_cast<double2*>(b + k));
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

// ---------------------------------------------------------------------------------------
// Wave-strip kernels: the fast path when n is a multiple of 64 and of the chunk height.
//
// One wavefront owns a strip of 64 columns (lane l: column c0 + l) and a chunk of WCH rows,
// and marches down it alone: no LDS, no barriers.  East / west neighbours come from the
// adjacent lanes by DPP wavefront shifts; the strip's two edge columns come from a second
// load per row ("halo" lanes 0..3 load columns c0-2, c0-1, c0+64, c0+65; lanes 4..63 repeat
// lane 3's address, a cache line already being fetched) and are broadcast with readlane.
// Rows above and below are held in registers.  The row loop is unrolled in full and every
// load is unconditional, so the loads of the next WD rows stay in flight while a row is
// computed (the compiler can count them exactly; a branch around a load would force it to
// wait for all of them).
// ---------------------------------------------------------------------------------------
#ifndef STADE_DIFF_WCH
#define STADE_DIFF_WCH 64
#endif
#ifndef STADE_DIFF_WCH_HV
#define STADE_DIFF_WCH_HV 32
#endif
#ifndef STADE_DIFF_WD
#define STADE_DIFF_WD 3
#endif
#ifndef STADE_DIFF_WD_HV
#define STADE_DIFF_WD_HV 4
#endif
#ifndef STADE_DIFF_WD2_HV
#define STADE_DIFF_WD2_HV 4
#endif
// rows per wave and rows of loads in flight ahead of the row being computed; measured at
// n = 4096: 64 rows beat 32 for the adjoint and the tangent (fewer halo rows), while the
// HVP, with twice the values per row, keeps 32 rows to stay in registers (at 64 it spills).
// Depths 3..6 measured within 2 % of each other; on the 128-column strips with streaming
// hints 3 is 1.6 % faster than 4 for the adjoint (6 and 32-row chunks slower).
constexpr int WS = 64;                      // columns per wave strip
constexpr int WCH = STADE_DIFF_WCH;         // adjoint, tangent
constexpr int WCH_HV = STADE_DIFF_WCH_HV;   // HVP
constexpr int WD = STADE_DIFF_WD;
constexpr int WD_HV = STADE_DIFF_WD_HV;
static_assert(WS % WCH == 0 && WS % WCH_HV == 0, "the wave-strip path requires n % 64 == 0 to imply n % rows == 0");
// the 5-point forms of step5 / step5d on values instead of LDS positions
__device__ __forceinline__ double step5v(double up, double c, double dn, double w, double e) {
    double t = w + e;
    t = t + up;
    t = t + dn;
    t = t - 4.0 * c;
    return c + 0.1 * t;
}
__device__ __forceinline__ double step5dv(double up, double c, double dn, double w, double e) {
    double t = w + e;
    t = t + up;
    t = t + dn;
    t = t + -(4.0 * c);
    return c + 0.1 * t;
}

struct WaveGeom {
    int c0, j0, oc, hc;
};
// wave `wid` = strip wid % nstrips, chunk wid / nstrips of `rows` rows
__device__ __forceinline__ WaveGeom wave_geom(int wid, int n, int nstrips, int rows) {
    const int lane = threadIdx.x & 63;
    WaveGeom g;
    g.c0 = (wid % nstrips) * WS;
    g.j0 = (wid / nstrips) * rows;
    g.oc = g.c0 + lane;
    const int hoff = lane == 0 ? -2 : (lane == 1 ? -1 : (lane == 2 ? WS : WS + 1));
    g.hc = wrap1(g.c0 + hoff, n);
    return g;
}

// tangent: un, und of rows j0 .. j0+ROWS-1 from u, ud rows j0-1 .. j0+ROWS
template <int ROWS, int D>
__global__ __launch_bounds__(256) void diffusion_d_wave(const double* __restrict__ u, const double* __restrict__ ud,
                                                        double* __restrict__ un, double* __restrict__ und, int n,
                                                        int nstrips, int nwaves, double* partials) {
    const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= nwaves) return;  // whole waves only; the kernel has no barrier
    const WaveGeom g = wave_geom(wid, n, nstrips, ROWS);
    double U[ROWS + 2], H[ROWS + 2], UD[ROWS + 2], HD[ROWS + 2];  // row q at index q + 1
    auto load = [&](int q) {
        const size_t rb = (size_t)wrap1(g.j0 + q, n) * n;
        U[q + 1] = u[rb + g.oc];
        H[q + 1] = u[rb + g.hc];
        UD[q + 1] = ud[rb + g.oc];
        HD[q + 1] = ud[rb + g.hc];
    };
    load(-1);
    load(0);
#pragma unroll
    for (int k = 1; k <= D; ++k) load(k);
    double acc[2] = {0.0, 0.0};
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        if (r + D + 1 <= ROWS) load(r + D + 1);
        const int i = r + 1;
        const double v = step5v(U[i - 1], U[i], U[i + 1], from_west(U[i], lane_val(H[i], 1)), from_east(U[i], lane_val(H[i], 2)));
        const double vd =
            step5dv(UD[i - 1], UD[i], UD[i + 1], from_west(UD[i], lane_val(HD[i], 1)), from_east(UD[i], lane_val(HD[i], 2)));
        const size_t gi = (size_t)(g.j0 + r) * n + g.oc;
        und[gi] = vd;
        un[gi] = v;
        acc[1] += (2.0 * v) * vd;
        acc[0] += v * v;
    }
    acc[0] = wave_sum(acc[0]);
    acc[1] = wave_sum(acc[1]);
    if ((threadIdx.x & 63) == 0) {
        partials[(size_t)wid * 2] = acc[0];
        partials[(size_t)wid * 2 + 1] = acc[1];
    }
}

// adjoint pass 1 (HV = false) and its tangent (HV = true): un (+ und) of the wave's rows,
// loss partials, and the gather of w = unb + (2 un) lossb (+ wd) into ub (+ ubd)
template <bool HV, int ROWS, int D>
__global__ __launch_bounds__(256) void diffusion_b_wave(const double* __restrict__ u, const double* __restrict__ ud,
                                                        double* __restrict__ un, double* __restrict__ und,
                                                        const double* __restrict__ unb, const double* __restrict__ unbd,
                                                        double* __restrict__ ub, double* __restrict__ ubd,
                                                        const double* __restrict__ lossb, const double* __restrict__ lossbd,
                                                        int n, int nstrips, int nwaves, double* partials) {
    const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wid >= nwaves) return;  // whole waves only; the kernel has no barrier
    const WaveGeom g = wave_geom(wid, n, nstrips, ROWS);
    const double lb = lossb[0];
    const double lbd = HV ? lossbd[0] : 0.0;
    // u rows -2 .. ROWS+1 at index q + 2; unb rows -1 .. ROWS at q + 1; ub rows 0 .. ROWS-1
    double U[ROWS + 4], H[ROWS + 4], B[ROWS + 2], BH[ROWS + 2], UB[ROWS];
    double UD[HV ? ROWS + 4 : 1], HD[HV ? ROWS + 4 : 1], BD[HV ? ROWS + 2 : 1], BHD[HV ? ROWS + 2 : 1], UBD[HV ? ROWS : 1];
    auto rowb = [&](int q) { return (size_t)wrap1(g.j0 + q, n) * n; };
    auto load_u = [&](int q) {
        const size_t rb = rowb(q);
        U[q + 2] = u[rb + g.oc];
        H[q + 2] = u[rb + g.hc];
        if constexpr (HV) {
            UD[q + 2] = ud[rb + g.oc];
            HD[q + 2] = ud[rb + g.hc];
        }
    };
    auto load_b = [&](int q) {
        const size_t rb = rowb(q);
        B[q + 1] = unb[rb + g.oc];
        BH[q + 1] = unb[rb + g.hc];
        if constexpr (HV) {
            BD[q + 1] = unbd[rb + g.oc];
            BHD[q + 1] = unbd[rb + g.hc];
        }
    };
    // the loads that step r consumes last: u row r+2, unb row r+1, ub row r
    auto load_group = [&](int r) {
        load_u(r + 2);
        load_b(r + 1);
        const size_t gi = (size_t)(g.j0 + r) * n + g.oc;
        UB[r] = ub[gi];
        if constexpr (HV) UBD[r] = ubd[gi];
    };
    // w of rows -1 .. ROWS (own column) and of the edge columns c0-1 (west) and c0+64 (east)
    double Wo[ROWS + 2], Ww[ROWS + 2], We[ROWS + 2];
    double WDo[HV ? ROWS + 2 : 1], WDw[HV ? ROWS + 2 : 1], WDe[HV ? ROWS + 2 : 1];
    double acc[2] = {0.0, 0.0};
    // un (+ und) and w (+ wd) of row q in the generated text's operation order; un stored
    // for the wave's own rows
    auto new_state = [&](int q) {
        const int i = q + 2;
        const double v = step5v(U[i - 1], U[i], U[i + 1], from_west(U[i], lane_val(H[i], 1)), from_east(U[i], lane_val(H[i], 2)));
        const double vw = step5v(lane_val(H[i - 1], 1), lane_val(H[i], 1), lane_val(H[i + 1], 1), lane_val(H[i], 0), lane_val(U[i], 0));
        const double ve = step5v(lane_val(H[i - 1], 2), lane_val(H[i], 2), lane_val(H[i + 1], 2), lane_val(U[i], 63), lane_val(H[i], 3));
        const int b = q + 1;
        Wo[b] = B[b] + (2.0 * v) * lb;
        Ww[b] = lane_val(BH[b], 1) + (2.0 * vw) * lb;
        We[b] = lane_val(BH[b], 2) + (2.0 * ve) * lb;
        double vd = 0.0;
        if constexpr (HV) {
            vd = step5dv(UD[i - 1], UD[i], UD[i + 1], from_west(UD[i], lane_val(HD[i], 1)), from_east(UD[i], lane_val(HD[i], 2)));
            const double vdw =
                step5dv(lane_val(HD[i - 1], 1), lane_val(HD[i], 1), lane_val(HD[i + 1], 1), lane_val(HD[i], 0), lane_val(UD[i], 0));
            const double vde =
                step5dv(lane_val(HD[i - 1], 2), lane_val(HD[i], 2), lane_val(HD[i + 1], 2), lane_val(UD[i], 63), lane_val(HD[i], 3));
            WDo[b] = BD[b] + (lb * (2.0 * vd) + (2.0 * v) * lbd);
            WDw[b] = lane_val(BHD[b], 1) + (lb * (2.0 * vdw) + (2.0 * vw) * lbd);
            WDe[b] = lane_val(BHD[b], 2) + (lb * (2.0 * vde) + (2.0 * ve) * lbd);
        }
        if (q >= 0 && q < ROWS) {
            const size_t gi = (size_t)(g.j0 + q) * n + g.oc;
            if constexpr (HV) {
                und[gi] = vd;
                acc[1] += (2.0 * v) * vd;
            }
            un[gi] = v;
            acc[0] += v * v;
        }
    };
    // ub[row r] += w_c + 0.1 w_E + 0.1 w_W + 0.1 w_S + 0.1 w_N + 4 (-(0.1 w_c))
    auto gather = [&](int r) {
        const int b = r + 1;
        const double c = Wo[b];
        double a = c;
        a = a + 0.1 * from_east(c, We[b]);
        a = a + 0.1 * from_west(c, Ww[b]);
        a = a + 0.1 * Wo[b + 1];
        a = a + 0.1 * Wo[b - 1];
        a = a + 4.0 * -(0.1 * c);
        const size_t gi = (size_t)(g.j0 + r) * n + g.oc;
        if constexpr (HV) {
            const double cd = WDo[b];
            double ad = cd;
            ad = ad + 0.1 * from_east(cd, WDe[b]);
            ad = ad + 0.1 * from_west(cd, WDw[b]);
            ad = ad + 0.1 * WDo[b + 1];
            ad = ad + 0.1 * WDo[b - 1];
            ad = ad + 4.0 * -(0.1 * cd);
            ubd[gi] = UBD[r] + ad;
        }
        ub[gi] = UB[r] + a;
    };
#pragma unroll
    for (int q = -2; q <= 1; ++q) load_u(q);
    load_b(-1);
    load_b(0);
#pragma unroll
    for (int k = 0; k < D; ++k) load_group(k);
    new_state(-1);
    new_state(0);
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        if (r + D < ROWS) load_group(r + D);
        new_state(r + 1);
        gather(r);
    }
    acc[0] = wave_sum(acc[0]);
    if constexpr (HV) acc[1] = wave_sum(acc[1]);
    if ((threadIdx.x & 63) == 0) {
        partials[(size_t)wid * (HV ? 2 : 1)] = acc[0];
        if constexpr (HV) partials[(size_t)wid * 2 + 1] = acc[1];
    }
}

// 128-column strips: lane l owns columns c0 + 2l and c0 + 2l + 1 and moves them as one
// 16-byte load or store, so a row of a strip is 1 KB (eight cache lines) and the strip's two
// halo lines add a quarter instead of a half.  East / west of the pair come from the pair
// itself and from the adjacent lane; the halo lanes are as in the 64-column kernels (columns
// c0-2, c0-1, c0+128, c0+129).  Operation order per cell is the same as there.  The row loops
// are unrolled by static_for: at 64 rows the bodies exceed the compiler's unroll threshold,
// and a rolled loop would move the register arrays to scratch memory.
constexpr int WS2 = 128;
// Rows per wave (16, 32 or 64; each divides 128, so n % 128 == 0 implies n % rows == 0),
// chosen by n from timings of the three heights on MI355X at n = 1024 .. 16384.  16 rows are
// within a few per cent of the best almost everywhere, and the only choice that holds up at
// large n: at n = 8192 the adjoint ran at 71 % of the HBM peak with 16 rows, 60 % with 32 and
// 48 % with 64 (power-of-two strides: a 64-row chunk of 64 KB rows starts 4 MB after the one
// above), and at 16384 68 / 60 / 58 %.  Two ranges measured faster with taller chunks: around
// n = 2048 (32 rows; 16-row chunks leave 20 % of each wave's rows to the halo) and, for the
// adjoint, n = 4096, where 64 rows make a grid of exactly two blocks a CU, all resident at
// once (77-81 % against 74 % with 16 rows).  The HVP, with twice the values per row, keeps
// four rows in flight (256 VGPRs, one wave a SIMD; 64 rows would spill) and takes the
// tangent's heights: 16 rows measured 1-7 points above 32 from n = 6144 to 12288 and 15 points
// above at n <= 1024, and within 2 points either way from 2048 to 4096.
constexpr int WD2_HV = STADE_DIFF_WD2_HV;
int rows_b2(int64_t n) { return n == 4096 ? 64 : (n >= 1536 && n <= 2560) ? 32 : 16; }
int rows_d2(int64_t n) { return (n >= 2048 && n <= 4096) ? 32 : 16; }
int rows_hv2(int64_t n) { return rows_d2(n); }
// calls f with the chunk height as a compile-time constant (heights above MAXR are not
// instantiated)
template <int MAXR, typename F>
void with_rows(int rows, F&& f) {
    if constexpr (MAXR >= 64) {
        if (rows == 64) return f(std::integral_constant<int, 64>{});
    }
    if (rows == 32) return f(std::integral_constant<int, 32>{});
    f(std::integral_constant<int, 16>{});
}

struct WaveGeom2 {
    int lane, c0, j0, oc, hc;
};
__device__ __forceinline__ WaveGeom2 wave_geom2(int wid, int n, int nstrips, int rows) {
    WaveGeom2 g;
    g.lane = threadIdx.x & 63;
    g.c0 = (wid % nstrips) * WS2;
    g.j0 = (wid / nstrips) * rows;
    g.oc = g.c0 + 2 * g.lane;
    g.hc = wrap1(g.c0 + (g.lane == 0 ? -2 : (g.lane == 1 ? -1 : (g.lane == 2 ? WS2 : WS2 + 1))), n);
    return g;
}
// the pair holding element (row base rb, column oc) of a double array; rb and oc are even
__device__ __forceinline__ size_t pair_of(size_t rb, int oc) { return (rb + oc) >> 1; }

// 5-point step of the pair (x: column oc, y: oc + 1) from the rows above and below and the
// halo columns hw (oc - 1 of lane 0) and he (oc + 2 of lane 63)
template <bool TANGENT>
__device__ __forceinline__ double2 step_pair(double2 up, double2 c, double2 dn, double hw, double he) {
    double2 v;
    if constexpr (TANGENT) {
        v.x = step5dv(up.x, c.x, dn.x, from_west(c.y, hw), c.y);
        v.y = step5dv(up.y, c.y, dn.y, c.x, from_east(c.x, he));
    } else {
        v.x = step5v(up.x, c.x, dn.x, from_west(c.y, hw), c.y);
        v.y = step5v(up.y, c.y, dn.y, c.x, from_east(c.x, he));
    }
    return v;
}

// tangent: un, und of rows j0 .. j0+ROWS-1 from u, ud rows j0-1 .. j0+ROWS
template <int ROWS, int D>
__global__ __launch_bounds__(256) void diffusion_d_wave2(const double* __restrict__ u, const double* __restrict__ ud,
                                                         double* __restrict__ un, double* __restrict__ und, int n,
                                                         int nstrips, int nwaves, double* partials) {
    __shared__ double red[4 * 2];
    const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
    double acc[2] = {0.0, 0.0};
    if (wid < nwaves) {  // whole waves; the four of a block meet at the barrier below
        const WaveGeom2 g = wave_geom2(wid, n, nstrips, ROWS);
        const double2* __restrict__ u2 = reinterpret_cast<const double2*>(u);
        const double2* __restrict__ ud2 = reinterpret_cast<const double2*>(ud);
        double2* __restrict__ un2 = reinterpret_cast<double2*>(un);
        double2* __restrict__ und2 = reinterpret_cast<double2*>(und);
        double2 U[ROWS + 2], UD[ROWS + 2];  // row q at index q + 1
        double H[ROWS + 2], HD[ROWS + 2];
        auto load = [&](int q) {
            const size_t rb = (size_t)wrap1(g.j0 + q, n) * n;
            U[q + 1] = u2[pair_of(rb, g.oc)];
            H[q + 1] = u[rb + g.hc];
            UD[q + 1] = ud2[pair_of(rb, g.oc)];
            HD[q + 1] = ud[rb + g.hc];
        };
        load(-1);
        load(0);
#pragma unroll
        for (int k = 1; k <= D; ++k) load(k);
        static_for<ROWS>([&](auto rc) {
            constexpr int r = decltype(rc)::value, i = r + 1;
            if constexpr (r + D + 1 <= ROWS) load(r + D + 1);
            const double2 v = step_pair<false>(U[i - 1], U[i], U[i + 1], lane_val(H[i], 1), lane_val(H[i], 2));
            const double2 vd = step_pair<true>(UD[i - 1], UD[i], UD[i + 1], lane_val(HD[i], 1), lane_val(HD[i], 2));
            const size_t gp = pair_of((size_t)(g.j0 + r) * n, g.oc);
            nt_store2(vd, &und2[gp]);
            nt_store2(v, &un2[gp]);
            acc[1] += (2.0 * v.x) * vd.x;
            acc[0] += v.x * v.x;
            acc[1] += (2.0 * v.y) * vd.y;
            acc[0] += v.y * v.y;
        });
    }
    // one partial pair per block: its four waves' sums added in wave order
    block_partials<2>(acc, red, partials);
}

// adjoint pass 1 (HV = false) and its tangent (HV = true): un (+ und) of the wave's rows,
// loss partials, and the gather of w = unb + (2 un) lossb (+ wd) into ub (+ ubd)
template <bool HV, int ROWS, int D>
__global__ __launch_bounds__(256) void diffusion_b_wave2(const double* __restrict__ u, const double* __restrict__ ud,
                                                         double* __restrict__ un, double* __restrict__ und,
                                                         const double* __restrict__ unb, const double* __restrict__ unbd,
                                                         double* __restrict__ ub, double* __restrict__ ubd,
                                                         const double* __restrict__ lossb, const double* __restrict__ lossbd,
                                                         int n, int nstrips, int nwaves, double* partials) {
    __shared__ double red[4 * (HV ? 2 : 1)];
    const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
    double acc[2] = {0.0, 0.0};
    if (wid < nwaves) {  // whole waves; the four of a block meet at the barrier below
        const WaveGeom2 g = wave_geom2(wid, n, nstrips, ROWS);
        const double lb = lossb[0];
        const double lbd = HV ? lossbd[0] : 0.0;
        const double2* __restrict__ u2 = reinterpret_cast<const double2*>(u);
        const double2* __restrict__ ud2 = reinterpret_cast<const double2*>(ud);
        const double2* __restrict__ unb2 = reinterpret_cast<const double2*>(unb);
        const double2* __restrict__ unbd2 = reinterpret_cast<const double2*>(unbd);
        double2* __restrict__ un2 = reinterpret_cast<double2*>(un);
        double2* __restrict__ und2 = reinterpret_cast<double2*>(und);
        double2* __restrict__ ub2 = reinterpret_cast<double2*>(ub);
        double2* __restrict__ ubd2 = reinterpret_cast<double2*>(ubd);
        // u rows -2 .. ROWS+1 at index q + 2; unb rows -1 .. ROWS at q + 1; ub rows 0 .. ROWS-1
        double2 U[ROWS + 4], B[ROWS + 2], UB[ROWS];
        double H[ROWS + 4], BH[ROWS + 2];
        double2 UD[HV ? ROWS + 4 : 1], BD[HV ? ROWS + 2 : 1], UBD[HV ? ROWS : 1];
        double HD[HV ? ROWS + 4 : 1], BHD[HV ? ROWS + 2 : 1];
        auto rowb = [&](int q) { return (size_t)wrap1(g.j0 + q, n) * n; };
        auto load_u = [&](int q) {
            const size_t rb = rowb(q);
            U[q + 2] = u2[pair_of(rb, g.oc)];
            H[q + 2] = u[rb + g.hc];
            if constexpr (HV) {
                UD[q + 2] = ud2[pair_of(rb, g.oc)];
                HD[q + 2] = ud[rb + g.hc];
            }
        };
        auto load_b = [&](int q) {
            const size_t rb = rowb(q);
            B[q + 1] = unb2[pair_of(rb, g.oc)];
            BH[q + 1] = unb[rb + g.hc];
            if constexpr (HV) {
                BD[q + 1] = unbd2[pair_of(rb, g.oc)];
                BHD[q + 1] = unbd[rb + g.hc];
            }
        };
        // the loads that step r consumes last: u row r+2, unb row r+1, ub row r
        auto load_group = [&](int r) {
            load_u(r + 2);
            load_b(r + 1);
            const size_t gp = pair_of((size_t)(g.j0 + r) * n, g.oc);
            UB[r] = nt_load2(&ub2[gp]);
            if constexpr (HV) UBD[r] = nt_load2(&ubd2[gp]);
        };
        // w of rows -1 .. ROWS (own pair) and of the edge columns c0-1 (west) and c0+128 (east)
        double2 Wo[ROWS + 2], WDo[HV ? ROWS + 2 : 1];
        double Ww[ROWS + 2], We[ROWS + 2], WDw[HV ? ROWS + 2 : 1], WDe[HV ? ROWS + 2 : 1];
        // un (+ und) and w (+ wd) of row q in the generated text's operation order; un stored
        // for the wave's own rows
        auto new_state = [&](int q) {
            const int i = q + 2, b = q + 1;
            const double hw = lane_val(H[i], 1), he = lane_val(H[i], 2);
            const double2 v = step_pair<false>(U[i - 1], U[i], U[i + 1], hw, he);
            const double vw = step5v(lane_val(H[i - 1], 1), hw, lane_val(H[i + 1], 1), lane_val(H[i], 0), lane_val(U[i].x, 0));
            const double ve = step5v(lane_val(H[i - 1], 2), he, lane_val(H[i + 1], 2), lane_val(U[i].y, 63), lane_val(H[i], 3));
            Wo[b].x = B[b].x + (2.0 * v.x) * lb;
            Wo[b].y = B[b].y + (2.0 * v.y) * lb;
            Ww[b] = lane_val(BH[b], 1) + (2.0 * vw) * lb;
            We[b] = lane_val(BH[b], 2) + (2.0 * ve) * lb;
            double2 vd = make_double2(0.0, 0.0);
            if constexpr (HV) {
                const double hdw = lane_val(HD[i], 1), hde = lane_val(HD[i], 2);
                vd = step_pair<true>(UD[i - 1], UD[i], UD[i + 1], hdw, hde);
                const double vdw =
                    step5dv(lane_val(HD[i - 1], 1), hdw, lane_val(HD[i + 1], 1), lane_val(HD[i], 0), lane_val(UD[i].x, 0));
                const double vde =
                    step5dv(lane_val(HD[i - 1], 2), hde, lane_val(HD[i + 1], 2), lane_val(UD[i].y, 63), lane_val(HD[i], 3));
                WDo[b].x = BD[b].x + (lb * (2.0 * vd.x) + (2.0 * v.x) * lbd);
                WDo[b].y = BD[b].y + (lb * (2.0 * vd.y) + (2.0 * v.y) * lbd);
                WDw[b] = lane_val(BHD[b], 1) + (lb * (2.0 * vdw) + (2.0 * vw) * lbd);
                WDe[b] = lane_val(BHD[b], 2) + (lb * (2.0 * vde) + (2.0 * ve) * lbd);
            }
            if (q >= 0 && q < ROWS) {
                const size_t gp = pair_of((size_t)(g.j0 + q) * n, g.oc);
                if constexpr (HV) {
                    nt_store2(vd, &und2[gp]);
                    acc[1] += (2.0 * v.x) * vd.x;
                    acc[1] += (2.0 * v.y) * vd.y;
                }
                nt_store2(v, &un2[gp]);
                acc[0] += v.x * v.x;
                acc[0] += v.y * v.y;
            }
        };
        // ub[row r] += w_c + 0.1 w_E + 0.1 w_W + 0.1 w_S + 0.1 w_N + 4 (-(0.1 w_c))
        auto gather1 = [](double c, double e, double w, double s, double nn) {
            double a = c;
            a = a + 0.1 * e;
            a = a + 0.1 * w;
            a = a + 0.1 * s;
            a = a + 0.1 * nn;
            a = a + 4.0 * -(0.1 * c);
            return a;
        };
        auto gather = [&](int r) {
            const int b = r + 1;
            const size_t gp = pair_of((size_t)(g.j0 + r) * n, g.oc);
            if constexpr (HV) {
                const double2 c = WDo[b];
                double2 o;
                o.x = UBD[r].x + gather1(c.x, c.y, from_west(c.y, WDw[b]), WDo[b + 1].x, WDo[b - 1].x);
                o.y = UBD[r].y + gather1(c.y, from_east(c.x, WDe[b]), c.x, WDo[b + 1].y, WDo[b - 1].y);
                nt_store2(o, &ubd2[gp]);
            }
            const double2 c = Wo[b];
            double2 o;
            o.x = UB[r].x + gather1(c.x, c.y, from_west(c.y, Ww[b]), Wo[b + 1].x, Wo[b - 1].x);
            o.y = UB[r].y + gather1(c.y, from_east(c.x, We[b]), c.x, Wo[b + 1].y, Wo[b - 1].y);
            nt_store2(o, &ub2[gp]);
        };
#pragma unroll
        for (int q = -2; q <= 1; ++q) load_u(q);
        load_b(-1);
        load_b(0);
#pragma unroll
        for (int k = 0; k < D; ++k) load_group(k);
        new_state(-1);
        new_state(0);
        static_for<ROWS>([&](auto rc) {
            constexpr int r = decltype(rc)::value;
            if constexpr (r + D < ROWS) load_group(r + D);
            new_state(r + 1);
            gather(r);
        });
    }
    // one partial (pair) per block: its four waves' sums added in wave order
    if constexpr (HV) {
        block_partials<2>(acc, red, partials);
    } else {
        double v1[1] = {acc[0]};
        block_partials<1>(v1, red, partials);
    }
}

struct WaveGrid {
    int nstrips, nwaves, blocks;
};
// the 128-column kernels move 16-byte pairs: every array they touch must be 16-byte aligned
// (an array that is a view into a larger allocation may be 8-byte aligned only)
bool pairs_ok(int64_t n, std::initializer_list<const void*> arrays) {
    if (n % WS2 != 0) return false;
    for (const void* p : arrays)
        if (reinterpret_cast<uintptr_t>(p) & 15) return false;
    return true;
}
// the wave-strip path applies when n is a multiple of the strip width (and so of the rows
// per wave)
bool wave_path(int64_t n) { return n >= WS && n % WS == 0; }
WaveGrid wave_grid_of(int64_t n, int rows) {
    const int nstrips = (int)(n / WS), nwaves = nstrips * (int)(n / rows);
    return WaveGrid{nstrips, nwaves, (nwaves + 3) / 4};
}

int32_t check_n(int64_t n, const char* fn) {
    if (n < 0) return set_error(STADE_HIP_EINVAL, "%s: n = %lld is negative", fn, (long long)n);
    if (n > 46340) return set_error(STADE_HIP_ERANGE, "%s: n = %lld exceeds 46340 (n*n must fit Int32 cell indices)", fn, (long long)n);
    return STADE_HIP_OK;
}

// two 16-byte stores per thread; measured fastest for a 128 MiB fill on MI355X
unsigned zero_blocks(int64_t count) {
    int64_t per = (int64_t)NT * 2 * 2;
    int64_t blocks = (count + per - 1) / per;
    return (unsigned)(blocks > 65536 ? 65536 : (blocks < 1 ? 1 : blocks));
}

struct Grid {
    int strips, blocks;
};
Grid grid_of(int64_t n) {
    const int strips = (int)((n + SW - 1) / SW), chunks = (int)((n + CH - 1) / CH);
    return Grid{strips, strips * chunks};
}

// the adjoint's reduction partials: one per block of pass 1 (one per wave on the 64-column
// strips)
int64_t adjoint_partials(int64_t n, bool pairs) {
    if (pairs) return ((n / WS2) * (n / rows_b2(n)) + 3) / 4;
    if (wave_path(n)) return (n / WS) * (n / WCH);
    const Grid g = grid_of(n);
    return g.blocks;
}

// the adjoint: pass 1 (un, the loss partials and the owner-computes gather into ub), then
// pass 2 (the unb reset, with the loss sum of the partials); `partials` holds at least
// adjoint_partials(n, pairs_ok(...)) doubles
int32_t adjoint(double* loss, const double* lossb, const double* u, double* ub, double* un, double* unb, int64_t n,
                double* partials, hipStream_t stream) {
    int nparts;
    if (pairs_ok(n, {u, un, unb, ub})) {
        const int rows = rows_b2(n), nstrips = (int)(n / WS2), nwaves = nstrips * (int)(n / rows);
        STADE_TIMED("diffusion2d_b", stream, with_rows<64>(rows, [&](auto rc) {
                        diffusion_b_wave2<false, decltype(rc)::value, WD><<<(nwaves + 3) / 4, 256, 0, stream>>>(
                            u, nullptr, un, nullptr, unb, nullptr, ub, nullptr, lossb, nullptr, (int)n, nstrips, nwaves, partials);
                    }));
        STADE_LAUNCHED("diffusion_b_wave2");
        nparts = (nwaves + 3) / 4;
    } else if (wave_path(n)) {
        const WaveGrid w = wave_grid_of(n, WCH);
        STADE_TIMED("diffusion2d_b", stream,
                    diffusion_b_wave<false, WCH, WD><<<w.blocks, 256, 0, stream>>>(u, nullptr, un, nullptr, unb, nullptr, ub, nullptr,
                                                                              lossb, nullptr, (int)n, w.nstrips, w.nwaves, partials));
        STADE_LAUNCHED("diffusion_b_wave");
        nparts = w.nwaves;
    } else {
        const Grid g = grid_of(n);
        STADE_TIMED("diffusion2d_b", stream,
                    diffusion_b_kernel<false><<<g.blocks, NT, 0, stream>>>(u, nullptr, un, nullptr, unb, nullptr, ub, nullptr,
                                                                           lossb, nullptr, (int)n, g.strips, partials));
        STADE_LAUNCHED("diffusion_b_kernel");
        nparts = g.blocks;
    }
    STADE_TIMED("zero", stream,
                zero2_kernel<1><<<zero_blocks(n * n), NT, 0, stream>>>(unb, nullptr, (size_t)(n * n), partials, nparts,
                                                                       SumOuts{{loss}}));
    STADE_LAUNCHED("zero2_kernel");
    return STADE_HIP_OK;
}

// ------------------------------------------------------------------------------------------
// Scratch of the allocation-free adjoint (stade_hip_diffusion2d_b_noalloc): the pass-1 loss
// partials in a static device array, one copy per GPU, held until the process ends.  Host
// code never passes `scratch` itself (in host code the name is a stand-in, not a device
// address): each device's address is looked up once with hipGetSymbolAddress and kept.
// ------------------------------------------------------------------------------------------
constexpr int64_t kNoAllocPartials = 131072;  // 1 MiB of doubles
static __device__ __align__(256) double scratch[kNoAllocPartials];
static std::mutex g_scratch_mu;
static double* g_scratch_ptr[64];

int32_t noalloc_scratch(double** out) {
    int dev = 0;
    STADE_TRY_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return set_error(STADE_HIP_ERANGE, "device ordinal %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        STADE_TRY_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (!ptr) return set_error(STADE_HIP_ENOMEM, "hipGetSymbolAddress returned no address for the scratch array");
        // the event that orders calls on different streams, made here once so that no call
        // creates anything
        if (int32_t rc = call_order_setup()) return rc;
        g_scratch_ptr[dev] = (double*)ptr;
    }
    *out = g_scratch_ptr[dev];
    return STADE_HIP_OK;
}

}  // namespace
}  // namespace stade

using namespace stade;

extern "C" {

int32_t stade_hip_diffusion2d_b_noalloc(double* loss, const double* lossb, const double* u, double* ub, double* un,
                                        double* unb, int64_t n, hipStream_t stream) {
    if (int32_t rc = check_n(n, "stade_hip_diffusion2d_b_noalloc")) return rc;
    if (n == 0) return STADE_HIP_OK;
    if (!loss || !lossb || !u || !ub || !un || !unb)
        return set_error(STADE_HIP_EINVAL, "stade_hip_diffusion2d_b_noalloc: null pointer");
    const int64_t need = adjoint_partials(n, pairs_ok(n, {u, un, unb, ub}));
    if (need > kNoAllocPartials)
        return set_error(STADE_HIP_ERANGE,
                         "stade_hip_diffusion2d_b_noalloc: n = %lld needs %lld partial sums, above the %lld of the static "
                         "scratch (use stade_hip_diffusion2d_b)",
                         (long long)n, (long long)need, (long long)kNoAllocPartials);
    double* partials = nullptr;
    if (int32_t rc = noalloc_scratch(&partials)) return rc;
    // ordered like every other call (the device's lock while enqueueing, then a wait for the
    // previous call's stream), without the allocating workspace: calls on different streams
    // run one after the other; a replay of a captured call is ordered by the caller
    WsCall call_(stream, false);
    if (!call_.ok()) return call_.error();
    return adjoint(loss, lossb, u, ub, un, unb, n, partials, stream);
}

int32_t stade_hip_diffusion2d_d(double* loss, double* lossd, const double* u, const double* ud, double* un, double* und,
                                int64_t n, hipStream_t stream) {
    if (int32_t rc = check_n(n, "stade_hip_diffusion2d_d")) return rc;
    if (n == 0) return STADE_HIP_OK;
    if (!loss || !lossd || !u || !ud || !un || !und) return set_error(STADE_HIP_EINVAL, "stade_hip_diffusion2d_d: null pointer");
    WsCall call_(stream);
    Workspace* ws = call_.ws;
    if (!ws) return STADE_HIP_ENOMEM;
    int nparts;
    if (pairs_ok(n, {u, ud, un, und})) {
        const int rows = rows_d2(n), nstrips = (int)(n / WS2), nwaves = nstrips * (int)(n / rows);
        STADE_TIMED("diffusion2d_d", stream, with_rows<32>(rows, [&](auto rc) {
                        diffusion_d_wave2<decltype(rc)::value, WD><<<(nwaves + 3) / 4, 256, 0, stream>>>(
                            u, ud, un, und, (int)n, nstrips, nwaves, ws->partials);
                    }));
        STADE_LAUNCHED("diffusion_d_wave2");
        nparts = (nwaves + 3) / 4;
    } else if (wave_path(n)) {
        const WaveGrid w = wave_grid_of(n, WCH);
        STADE_TIMED("diffusion2d_d", stream,
                    diffusion_d_wave<WCH, WD><<<w.blocks, 256, 0, stream>>>(u, ud, un, und, (int)n, w.nstrips, w.nwaves, ws->partials));
        STADE_LAUNCHED("diffusion_d_wave");
        nparts = w.nwaves;
    } else {
        const Grid g = grid_of(n);
        STADE_TIMED("diffusion2d_d", stream,
                    diffusion_d_kernel<<<g.blocks, NT, 0, stream>>>(u, ud, un, und, (int)n, g.strips, ws->partials));
        STADE_LAUNCHED("diffusion_d_kernel");
        nparts = g.blocks;
    }
    STADE_TIMED("finalize", stream, finalize_kernel<2, 1024><<<1, 1024, 0, stream>>>(ws->partials, nparts, SumOuts{{loss, lossd}}));
    STADE_LAUNCHED("finalize_kernel");
    return STADE_HIP_OK;
}

int32_t stade_hip_diffusion2d_b(double* loss, const double* lossb, const double* u, double* ub, double* un, double* unb,
                                int64_t n, hipStream_t stream) {
    if (int32_t rc = check_n(n, "stade_hip_diffusion2d_b")) return rc;
    if (n == 0) return STADE_HIP_OK;
    if (!loss || !lossb || !u || !ub || !un || !unb) return set_error(STADE_HIP_EINVAL, "stade_hip_diffusion2d_b: null pointer");
    WsCall call_(stream);
    Workspace* ws = call_.ws;
    if (!ws) return STADE_HIP_ENOMEM;
    return adjoint(loss, lossb, u, ub, un, unb, n, ws->partials, stream);
}

int32_t stade_hip_diffusion2d_hv(double* loss, const double* lossb, const double* u, double* ub, double* un, double* unb,
                                 int64_t n, double* lossd, const double* lossbd, const double* ud, double* ubd, double* und,
                                 double* unbd, hipStream_t stream) {
    if (int32_t rc = check_n(n, "stade_hip_diffusion2d_hv")) return rc;
    if (n == 0) return STADE_HIP_OK;
    if (!loss || !lossb || !u || !ub || !un || !unb || !lossd || !lossbd || !ud || !ubd || !und || !unbd)
        return set_error(STADE_HIP_EINVAL, "stade_hip_diffusion2d_hv: null pointer");
    WsCall call_(stream);
    Workspace* ws = call_.ws;
    if (!ws) return STADE_HIP_ENOMEM;
    int nparts;
    if (pairs_ok(n, {u, ud, un, und, unb, unbd, ub, ubd})) {
        const int rows = rows_hv2(n), nstrips = (int)(n / WS2), nwaves = nstrips * (int)(n / rows);
        STADE_TIMED("diffusion2d_hv", stream, with_rows<32>(rows, [&](auto rc) {
                        diffusion_b_wave2<true, decltype(rc)::value, WD2_HV><<<(nwaves + 3) / 4, 256, 0, stream>>>(
                            u, ud, un, und, unb, unbd, ub, ubd, lossb, lossbd, (int)n, nstrips, nwaves, ws->partials);
                    }));
        STADE_LAUNCHED("diffusion_b_wave2<hv>");
        nparts = (nwaves + 3) / 4;
    } else if (wave_path(n)) {
        const WaveGrid w = wave_grid_of(n, WCH_HV);
        STADE_TIMED("diffusion2d_hv", stream,
                    diffusion_b_wave<true, WCH_HV, WD_HV><<<w.blocks, 256, 0, stream>>>(u, ud, un, und, unb, unbd, ub, ubd, lossb, lossbd,
                                                                                (int)n, w.nstrips, w.nwaves, ws->partials));
        STADE_LAUNCHED("diffusion_b_wave<hv>");
        nparts = w.nwaves;
    } else {
        const Grid g = grid_of(n);
        STADE_TIMED("diffusion2d_hv", stream,
                    diffusion_b_kernel<true><<<g.blocks, NT, 0, stream>>>(u, ud, un, und, unb, unbd, ub, ubd, lossb, lossbd,
                                                                          (int)n, g.strips, ws->partials));
        STADE_LAUNCHED("diffusion_b_kernel<hv>");
        nparts = g.blocks;
    }
    STADE_TIMED("zero", stream,
                zero2_kernel<2><<<zero_blocks(n * n), NT, 0, stream>>>(unb, unbd, (size_t)(n * n), ws->partials, nparts,
                                                                       SumOuts{{loss, lossd}}));
    STADE_LAUNCHED("zero2_kernel");
    return STADE_HIP_OK;
}

}  // extern "C"
