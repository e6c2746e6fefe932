// affine_lsq: tangent, adjoint and HVP of loss += 0.5 * sum((w * x + b - t) .^ 2) with a
// column-major w of shape (m, n).
//
// Generated code this replaces: stade.jl_amd/corpus/affine_lsq_{b,d,hv}.jl (STADE's
// `agen_emit` /root/reference/src/STADE.jl:3390-3419, `tgen_emit` 3271-3278, `hvp_emit`
// 6729-6782).  Under `stade_amdgpu_file` the row loop runs one thread per row with the column
// sum sequential inside it, and the adjoint's `xb[j] += w[i,j] * sb` becomes a per-element
// atomic (`cgen_device_assign` 11941-11969): m atomics on each of the n entries of xb.
//
// Here: 64 x 64 tiles of w, one wave per 16 columns and one lane per row, so every wave
// load is a 512-byte contiguous column segment.
//   1. rows:    partial row sums  s_i = sum_j w[i,j] x[j]  per 64-column chunk (LDS tree);
//               the adjoint forms also stage rb and reset it
//   2. columns: every block recomputes its rows' r = (b - t) + sum of chunk partials and
//               sb, then wb[i,j] += x[j] sb_i (read-modify-write, the dominant traffic) and
//               the per-tile column sums of w[i,j] sb_i (DPP wave sums), no atomics; the
//               blocks of column chunk 0 write r, bb, tb and the row tiles' loss partials
//   3. xb:      xb[j] += sum over row tiles of the column partials, in tile order, and the
//               loss sum
// The tangent (no columns to scatter) runs rows, then a finish kernel for r, rd and the loss.
// Every reduction has a fixed order: results do not depend on scheduling.
#include "internal.hpp"
#include "../../include/stade_hip.h"

namespace stade {
namespace {

constexpr int RT = 64, CT = 64, CW = 16, NT = 256;  // rows per tile, columns per tile, columns per wave
enum Mode { ADJ = 0, TAN = 1, HVP = 2 };
constexpr int kMaxChunks = 16;                      // row-sum partials per row

template <int M>
__global__ __launch_bounds__(NT) void rows_kernel(const double* __restrict__ w, const double* __restrict__ wd,
                                                  const double* __restrict__ x, const double* __restrict__ xd,
                                                  double* __restrict__ P, double* __restrict__ Pd, int m, int n, int tpc,
                                                  double* __restrict__ rb, double* __restrict__ rbd, double* __restrict__ RBc,
                                                  double* __restrict__ RBdc) {
    __shared__ double part[2][4][RT];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int chunk = blockIdx.x, i = blockIdx.y * RT + lane;
    const int ic = min(i, m - 1);
    const int t_end = min((chunk + 1) * tpc, (n + CT - 1) / CT);
    double s = 0.0, sd = 0.0;
    // the chunk's column tiles in order; per tile, the wave's 16 columns: every load issued
    // (clamped, unconditional) before the first use; columns past n and rows past m
    // contribute nothing
    for (int tile = chunk * tpc; tile < t_end; ++tile) {
        const int j0 = tile * CT + wv * CW;
        double wv_[CW], xv_[CW], wdv_[CW], xdv_[CW];
#pragma unroll
        for (int jj = 0; jj < CW; ++jj) {
            const int jc = min(j0 + jj, n - 1);
            const size_t g = (size_t)jc * m + ic;
            wv_[jj] = w[g];
            xv_[jj] = x[jc];
            wdv_[jj] = M != ADJ ? wd[g] : 0.0;
            xdv_[jj] = M != ADJ ? xd[jc] : 0.0;
        }
        __builtin_amdgcn_sched_barrier(0);
        if (i < m) {
#pragma unroll
            for (int jj = 0; jj < CW; ++jj) {
                if (j0 + jj >= n) continue;  // columns past n (a guard, not an exit: the loop unrolls)
                const double wij = wv_[jj], xj = xv_[jj];
                if (M != ADJ) sd = sd + (xj * wdv_[jj] + wij * xdv_[jj]);
                s = s + wij * xj;
            }
        }
    }
    part[0][wv][lane] = s;
    part[1][wv][lane] = sd;
    __syncthreads();
    if (wv == 0 && i < m) {
        P[(size_t)chunk * m + i] = ((part[0][0][lane] + part[0][1][lane]) + part[0][2][lane]) + part[0][3][lane];
        if (M != ADJ) Pd[(size_t)chunk * m + i] = ((part[1][0][lane] + part[1][1][lane]) + part[1][2][lane]) + part[1][3][lane];
        // the adjoint forms: rb (rbd) staged for the column kernel and reset here, the only
        // reader of rb in this launch, so that every column block can read the staged value
        if (M != TAN && RBc && chunk == 0) {
            const double v = rb[i];
            const double vd = M == HVP ? rbd[i] : 0.0;
            RBc[i] = v;
            rb[i] = 0.0;
            if (M == HVP) {
                RBdc[i] = vd;
                rbd[i] = 0.0;
            }
        }
    }
}

struct FinishArgs {
    const double *b, *t, *bd, *td, *P, *Pd, *lossb, *lossbd;
    double *r, *rd, *rb, *rbd, *bb, *bbd, *tb, *tbd, *S, *Sd, *loss, *lossd;
    int m, nchunks;
};

// r_i = (b_i - t_i) + the chunk partials of row i in chunk order (and its tangent): chunk
// partials 16 at a time, all loads in flight
template <int M>
__device__ __forceinline__ void row_value(const FinishArgs& a, int i, double& s, double& sd) {
    s = a.b[i] - a.t[i];
    sd = M != ADJ ? a.bd[i] - a.td[i] : 0.0;
    for (int c0 = 0; c0 < a.nchunks; c0 += 16) {
        double pv[16], pdv[16];
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            const size_t q = (size_t)min(c0 + c, a.nchunks - 1) * a.m + i;
            pv[c] = a.P[q];
            pdv[c] = M != ADJ ? a.Pd[q] : 0.0;
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            if (c0 + c >= a.nchunks) continue;
            s = s + pv[c];
            if (M != ADJ) sd = sd + pdv[c];
        }
    }
}

// the tangent, and the adjoint forms with no columns (n = 0).  BT threads a block, RPB rows a
// thread (rows i, i + BT * grid, ...).  A single block (m <= BT * RPB) adds the loss terms into
// the outputs itself; otherwise each block writes partials for a second-stage sum.
template <int M, int BT, int RPB>
__global__ __launch_bounds__(BT) void finish_kernel(FinishArgs a, double* partials, SumOuts outs) {
    __shared__ double red[32];
    double acc[2] = {0.0, 0.0};
#pragma unroll
    for (int rr = 0; rr < RPB; ++rr) {
    const int i = blockIdx.x * BT + threadIdx.x + rr * BT * gridDim.x;
    if (i < a.m) {
        double s, sd;
        row_value<M>(a, i, s, sd);
        if (M != ADJ) {
            a.rd[i] = sd;
            acc[1] += 0.5 * ((2.0 * s) * sd);   // a thread's rows accumulate (RPB > 1)
        }
        a.r[i] = s;
        acc[0] += 0.5 * (s * s);
        if (M == ADJ) {
            double rbt = a.rb[i] + 0.5 * (2.0 * s) * a.lossb[0];
            a.rb[i] = 0.0;
            a.S[i] = rbt;
            a.bb[i] = a.bb[i] + rbt;
            a.tb[i] = a.tb[i] + -rbt;
        } else if (M == HVP) {
            double h3 = a.lossb[0], h4 = 0.5 * (2.0 * s);
            double rbdt = a.rbd[i] + (h3 * (0.5 * (2.0 * sd)) + h4 * a.lossbd[0]);
            double rbt = a.rb[i] + h4 * h3;
            a.rbd[i] = 0.0;
            a.rb[i] = 0.0;
            a.S[i] = rbt;
            a.Sd[i] = rbdt;
            a.bbd[i] = a.bbd[i] + rbdt;
            a.bb[i] = a.bb[i] + rbt;
            a.tbd[i] = a.tbd[i] + -rbdt;
            a.tb[i] = a.tb[i] + -rbt;
        }
    }
    }
    if (gridDim.x == 1) {
        // one block: the loss (and its tangent) straight into the outputs
        block_sum<2>(acc, red);
        if (threadIdx.x == 0) {
            const double l0 = outs.p[0][0];
            const double l1 = M != ADJ ? outs.p[1][0] : 0.0;
            outs.p[0][0] = l0 + acc[0];
            if (M != ADJ) outs.p[1][0] = l1 + acc[1];
        }
    } else if (M == ADJ) {
        double v[1] = {acc[0]};
        block_partials<1>(v, red, partials);
    } else {
        block_partials<2>(acc, red, partials);
    }
}

// The adjoint forms with n > 0.  Every block recomputes the row values of its 64 rows from
// the chunk partials (r, then sb = rb + (2 r / 2) lossb with rb as staged by rows_kernel),
// and the blocks of column chunk 0 also write r, bb, tb (and the tangents) and the row
// tile's loss partials.  A wave takes CWC columns (8 or 16; a block 4 CWC).  The HVP takes 8:
// its six streams of a column (w, wd, wb, wbd, x, xd) would otherwise hold 192 registers a
// lane (two blocks a CU instead of one: 12-17 % faster from 2048^2 up, the same at 1024^2).
// The adjoint takes 8 up to 2^21 matrix elements, where an evaluation is launch-bound and
// two blocks a CU overlap one's loads with the other's stores (+4.6 % at 1024^2 by graph
// replays), and 16 above (2-3 % faster there).
template <int M, int CWC>
__global__ __launch_bounds__(NT) void cols_kernel(const double* __restrict__ w, const double* __restrict__ wd,
                                                  double* __restrict__ wb, double* __restrict__ wbd,
                                                  const double* __restrict__ x, const double* __restrict__ xd, FinishArgs fa,
                                                  const double* __restrict__ RBc, const double* __restrict__ RBdc,
                                                  double* __restrict__ XP, double* __restrict__ XPd, int m, int n,
                                                  double* __restrict__ partials) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    // row tiles along x: blocks dispatched together stream consecutive segments of the same
    // columns (measured 6-20 % faster at 4096^2-8192^2 than column tiles along x)
    const int rtile = blockIdx.x, i = rtile * RT + lane;
    const int j0 = blockIdx.y * (4 * CWC) + wv * CWC;
    const bool live = i < m;
    const int ic = min(i, m - 1);
    // every read of the wave's 16 columns (w, wb, x and the tangents) issued before any use or
    // store: clamped and unconditional, with dead rows and columns masked afterwards
    double wv_[CWC], wbv_[CWC], xv_[CWC], wdv_[CWC], wbdv_[CWC], xdv_[CWC];
#pragma unroll
    for (int jj = 0; jj < CWC; ++jj) {
        const int jc = min(j0 + jj, n - 1);
        const size_t g = (size_t)jc * m + ic;
        wv_[jj] = w[g];
        wbv_[jj] = __builtin_nontemporal_load(&wb[g]);  // wb, wbd: streamed once
        xv_[jj] = x[jc];
        wdv_[jj] = M == HVP ? wd[g] : 0.0;
        wbdv_[jj] = M == HVP ? __builtin_nontemporal_load(&wbd[g]) : 0.0;
        xdv_[jj] = M == HVP ? xd[jc] : 0.0;
    }
    double rv, rvd;
    row_value<M>(fa, ic, rv, rvd);
    const double lb = fa.lossb[0];
    const double rbv = RBc[ic];
    double si, sid = 0.0;
    if (M == ADJ) {
        si = rbv + 0.5 * (2.0 * rv) * lb;
    } else {
        const double h4 = 0.5 * (2.0 * rv);
        sid = RBdc[ic] + (lb * (0.5 * (2.0 * rvd)) + h4 * fa.lossbd[0]);
        si = rbv + h4 * lb;
    }
    if (blockIdx.y == 0 && wv == 0) {
        // every destination read before any is written
        const double bb0 = fa.bb[ic], tb0 = fa.tb[ic];
        const double bbd0 = M == HVP ? fa.bbd[ic] : 0.0, tbd0 = M == HVP ? fa.tbd[ic] : 0.0;
        if (live) {
            fa.r[i] = rv;
            fa.bb[i] = bb0 + si;
            fa.tb[i] = tb0 + -si;
            if (M == HVP) {
                fa.rd[i] = rvd;
                fa.bbd[i] = bbd0 + sid;
                fa.tbd[i] = tbd0 + -sid;
            }
        }
        double l0 = wave_sum(live ? 0.5 * (rv * rv) : 0.0);
        double l1 = M == HVP ? wave_sum(live ? 0.5 * ((2.0 * rv) * rvd) : 0.0) : 0.0;
        if (lane == 0) {
            if (M == ADJ) {
                partials[rtile] = l0;
            } else {
                partials[2 * rtile] = l0;
                partials[2 * rtile + 1] = l1;
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    double cx[CWC], cxd[CWC];
#pragma unroll
    for (int jj = 0; jj < CWC; ++jj) {
        const bool ok = live && j0 + jj < n;
        const size_t g = (size_t)(j0 + jj) * m + i;
        const double xj = xv_[jj], wij = wv_[jj];
        cx[jj] = ok ? wij * si : 0.0;
        cxd[jj] = (M == HVP && ok) ? si * wdv_[jj] + wij * sid : 0.0;
        if (ok) {
            if (M == HVP) __builtin_nontemporal_store(wbdv_[jj] + (si * xdv_[jj] + xj * sid), &wbd[g]);
            __builtin_nontemporal_store(wbv_[jj] + xj * si, &wb[g]);
        }
    }
    // column sums over the tile's rows (DPP wave sums), all 16 columns at once
#pragma unroll
    for (int jj = 0; jj < CWC; ++jj) {
        cx[jj] = wave_sum(cx[jj]);
        if (M == HVP) cxd[jj] = wave_sum(cxd[jj]);
    }
    if (lane == 0) {
#pragma unroll
        for (int jj = 0; jj < CWC; ++jj) {
            if (j0 + jj >= n) continue;
            XP[(size_t)rtile * n + j0 + jj] = cx[jj];
            if (M == HVP) XPd[(size_t)rtile * n + j0 + jj] = cxd[jj];
        }
    }
}

// The tangent (and the adjoint forms with n = 0) for m <= kTicketRows: one wave a block, RPB
// rows a lane, at most kTicketBlocks blocks.  Each block writes its loss partials, makes them
// visible (one device-scope fence a block: with this few blocks the L2 write-backs it costs
// are a fraction of a launch) and takes a ticket; the last block adds the partials in block
// order into the loss and resets the ticket counter for the next call.  Spreading the rows
// over many CUs is what makes this faster than one 1024-thread block (one CU pulling every
// chunk partial).
constexpr int kTicketBlocks = 32, kTicketRows = 2 * 64 * kTicketBlocks;

template <int M, int RPB>
__global__ __launch_bounds__(64) void finish_ticket_kernel(FinishArgs a, double* partials, SumOuts outs,
                                                           uint32_t* ticket) {
    __shared__ uint32_t last;
    double acc[2] = {0.0, 0.0};
#pragma unroll
    for (int rr = 0; rr < RPB; ++rr) {
        const int i = (blockIdx.x * RPB + rr) * 64 + threadIdx.x;
        if (i < a.m) {
            double s, sd;
            row_value<M>(a, i, s, sd);
            if (M != ADJ) {
                a.rd[i] = sd;
                acc[1] += 0.5 * ((2.0 * s) * sd);
            }
            a.r[i] = s;
            acc[0] += 0.5 * (s * s);
            if (M == ADJ) {
                double rbt = a.rb[i] + 0.5 * (2.0 * s) * a.lossb[0];
                a.rb[i] = 0.0;
                a.bb[i] = a.bb[i] + rbt;
                a.tb[i] = a.tb[i] + -rbt;
            } else if (M == HVP) {
                double h3 = a.lossb[0], h4 = 0.5 * (2.0 * s);
                double rbdt = a.rbd[i] + (h3 * (0.5 * (2.0 * sd)) + h4 * a.lossbd[0]);
                double rbt = a.rb[i] + h4 * h3;
                a.rbd[i] = 0.0;
                a.rb[i] = 0.0;
                a.bbd[i] = a.bbd[i] + rbdt;
                a.bb[i] = a.bb[i] + rbt;
                a.tbd[i] = a.tbd[i] + -rbdt;
                a.tb[i] = a.tb[i] + -rbt;
            }
        }
    }
    acc[0] = wave_sum(acc[0]);
    acc[1] = wave_sum(acc[1]);
    if (threadIdx.x == 0) {
        partials[2 * blockIdx.x] = acc[0];
        partials[2 * blockIdx.x + 1] = acc[1];
    }
    __threadfence();
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();
    // the blocks' partials in block order (lane b holds block b's; gridDim.x <= 64)
    const int b = threadIdx.x;
    const double p0 = b < (int)gridDim.x ? __hip_atomic_load(&partials[2 * b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.0;
    const double p1 = b < (int)gridDim.x ? __hip_atomic_load(&partials[2 * b + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.0;
    double t0 = 0.0, t1 = 0.0;
    for (int k = 0; k < (int)gridDim.x; ++k) {
        t0 += lane_val(p0, k);
        t1 += lane_val(p1, k);
    }
    if (threadIdx.x == 0) {
        const double l0 = outs.p[0][0];
        const double l1 = M != ADJ ? outs.p[1][0] : 0.0;
        outs.p[0][0] = l0 + t0;
        if (M != ADJ) outs.p[1][0] = l1 + t1;
        __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// one-wave blocks (the column partials are latency-bound reads: spread over many CUs), the
// last block taking the loss's second stage on its own
template <int M>
__global__ __launch_bounds__(64) void xfinish_kernel(double* __restrict__ xb, double* __restrict__ xbd,
                                                     const double* __restrict__ XP, const double* __restrict__ XPd,
                                                     int n, int mtiles, const double* partials, SumOuts outs) {
    __shared__ double red[32];
    // second stage of the loss sums (the column kernel's row-tile partials)
    if (blockIdx.x == gridDim.x - 1) {
        if (M == ADJ)
            finalize_partials<1>(partials, mtiles, red, outs);
        else
            finalize_partials<2>(partials, mtiles, red, outs);
        return;
    }
    const int j = blockIdx.x * 64 + threadIdx.x;
    if (j >= n) return;
    // row-tile partials 16 at a time, all loads in flight, added in tile order; xb (xbd) read
    // before either is written
    const double xb0 = xb[j];
    const double xbd0 = M == HVP ? xbd[j] : 0.0;
    double s = 0.0, sd = 0.0;
    for (int r0 = 0; r0 < mtiles; r0 += 16) {
        double pv[16], pdv[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const size_t q = (size_t)min(r0 + r, mtiles - 1) * n + j;
            pv[r] = XP[q];
            pdv[r] = M == HVP ? XPd[q] : 0.0;
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            if (r0 + r >= mtiles) continue;
            s += pv[r];
            if (M == HVP) sd += pdv[r];
        }
    }
    if (M == HVP) xbd[j] = xbd0 + sd;
    xb[j] = xb0 + s;
}

int32_t check_sizes(int64_t m, int64_t n, const char* fn) {
    if (m < 0 || n < 0) return set_error(STADE_HIP_EINVAL, "%s: negative size (i_m = %lld, i_n = %lld)", fn, (long long)m, (long long)n);
    if (m > (1 << 26) || n > (1 << 26) || m * n > (int64_t)1 << 34)
        return set_error(STADE_HIP_ERANGE, "%s: size out of range (i_m = %lld, i_n = %lld)", fn, (long long)m, (long long)n);
    if ((m + RT - 1) / RT * 2 > kPartialSlots) return set_error(STADE_HIP_ERANGE, "%s: i_m too large for the workspace", fn);
    // row tiles are the rows kernel's grid y dimension, column tiles the column kernel's
    if ((m + RT - 1) / RT > 65535) return set_error(STADE_HIP_ERANGE, "%s: i_m = %lld exceeds 65535 row tiles of 64", fn, (long long)m);
    if ((n + CT - 1) / CT > 65535) return set_error(STADE_HIP_ERANGE, "%s: i_n = %lld exceeds 65535 column tiles of 64", fn, (long long)n);
    return STADE_HIP_OK;
}

template <int M>
int32_t run(FinishArgs fa, const double* w, const double* wd, double* wb, double* wbd, const double* x, const double* xd,
            double* xb, double* xbd, int64_t m, int64_t n, hipStream_t stream) {
    if (m == 0) return STADE_HIP_OK;
    // the column kernel's columns a wave (8 or 16, above) and its tiles along the grid's y
    // dimension (checked before any device work; the 64-column tiles with the other sizes)
    const bool narrow = M == HVP || (m * n <= ((int64_t)1 << 21) && (n + 31) / 32 <= 65535);
    const int ct = narrow ? 32 : 64;
    const int ctiles = (int)((n + ct - 1) / ct);
    if (M != TAN && ctiles > 65535)
        return set_error(STADE_HIP_ERANGE, "stade_hip_affine_lsq_%s: i_n = %lld exceeds 65535 column tiles of %d",
                         M == HVP ? "hv" : "b", (long long)n, ct);
    WsCall call_(stream);
    Workspace* ws = call_.ws;
    if (!ws) return STADE_HIP_ENOMEM;
    // column tiles of 64, grouped into at most kMaxChunks chunks of tpc tiles for the row sums,
    // so that each row's value is the sum of at most kMaxChunks partials (one round of loads
    // wherever it is recomputed)
    const int ntiles = (int)((n + CT - 1) / CT), mtiles = (int)((m + RT - 1) / RT);
    const int tpc = (ntiles + kMaxChunks - 1) / kMaxChunks, nchunks = ntiles > 0 ? (ntiles + tpc - 1) / tpc : 0;
    const int two = (M == ADJ) ? 1 : 2;
    size_t nP = (size_t)nchunks * m, nS = (size_t)m, nX = (size_t)mtiles * n;
    double* base = (double*)scratch(sizeof(double) * two * (nP + nS + nX) + 256);
    if (!base) return scratch_error();
    double *P = base, *Pd = P + nP, *S = P + two * nP, *Sd = S + nS, *XP = S + two * nS, *XPd = XP + nX;
    // the adjoint forms with columns: rows (+ rb staged in S), columns (row values recomputed
    // per block), xb; otherwise rows, finish, the loss sum
    const bool fused = M != TAN && n > 0;
    if (nchunks > 0) {
        STADE_TIMED("affine_rows", stream,
                    rows_kernel<M><<<dim3(nchunks, mtiles), NT, 0, stream>>>(w, wd, x, xd, P, Pd, (int)m, (int)n, tpc, fa.rb, fa.rbd,
                                                                              fused ? S : nullptr, Sd));
        STADE_LAUNCHED("affine rows_kernel");
    }
    fa.P = P;
    fa.Pd = Pd;
    fa.S = S;
    fa.Sd = Sd;
    fa.m = (int)m;
    fa.nchunks = nchunks;
    SumOuts outs{{fa.loss, fa.lossd}};
    if (!fused) {
        if (m <= kTicketRows) {
            // up to kTicketBlocks one-wave blocks, the last of which sums the loss
            if (m <= 64 * kTicketBlocks) {
                STADE_TIMED("affine_finish", stream,
                            finish_ticket_kernel<M, 1><<<(unsigned)((m + 63) / 64), 64, 0, stream>>>(fa, ws->partials, outs,
                                                                                                   ws->sync));
            } else {
                STADE_TIMED("affine_finish", stream,
                            finish_ticket_kernel<M, 2><<<(unsigned)((m + 127) / 128), 64, 0, stream>>>(fa, ws->partials, outs,
                                                                                                     ws->sync));
            }
            STADE_LAUNCHED("affine finish_ticket_kernel");
            return STADE_HIP_OK;
        }
        const int nfin = (int)((m + NT - 1) / NT);
        STADE_TIMED("affine_finish", stream, finish_kernel<M, NT, 1><<<(unsigned)nfin, NT, 0, stream>>>(fa, ws->partials, outs));
        STADE_LAUNCHED("affine finish_kernel");
        if (M == ADJ)
            finalize_kernel<1><<<1, NT, 0, stream>>>(ws->partials, nfin, outs);
        else
            finalize_kernel<2><<<1, NT, 0, stream>>>(ws->partials, nfin, outs);
        STADE_LAUNCHED("affine finalize_kernel");
        return STADE_HIP_OK;
    }
    if (narrow) {
        STADE_TIMED("affine_cols", stream,
                    (cols_kernel<M, 8><<<dim3(mtiles, ctiles), NT, 0, stream>>>(w, wd, wb, wbd, x, xd, fa, S, Sd, XP, XPd, (int)m,
                                                                              (int)n, ws->partials)));
    } else {
        STADE_TIMED("affine_cols", stream,
                    (cols_kernel<M, 16><<<dim3(mtiles, ctiles), NT, 0, stream>>>(w, wd, wb, wbd, x, xd, fa, S, Sd, XP, XPd, (int)m,
                                                                               (int)n, ws->partials)));
    }
    STADE_LAUNCHED("affine cols_kernel");
    STADE_TIMED("affine_xfinish", stream,
                xfinish_kernel<M><<<(unsigned)((n + 63) / 64 + 1), 64, 0, stream>>>(xb, xbd, XP, XPd, (int)n, mtiles, ws->partials,
                                                                                     outs));
    STADE_LAUNCHED("affine xfinish_kernel");
    return STADE_HIP_OK;
}

}  // namespace
}  // namespace stade

using namespace stade;

extern "C" {

int32_t stade_hip_affine_lsq_b(double* loss, const double* lossb, const double* w, double* wb, const double* x, double* xb,
                               const double* b, double* bb, const double* t, double* tb, double* r, double* rb,
                               int64_t i_m, int64_t i_n, hipStream_t stream) {
    if (int32_t rc = check_sizes(i_m, i_n, "stade_hip_affine_lsq_b")) return rc;
    // (arrays of no elements may be null: with i_n = 0 the matrix and x are never touched)
    if (i_m > 0 && (!loss || !lossb || !b || !bb || !t || !tb || !r || !rb || (i_n > 0 && (!w || !wb || !x || !xb))))
        return set_error(STADE_HIP_EINVAL, "stade_hip_affine_lsq_b: null pointer");
    FinishArgs fa{};
    fa.b = b; fa.t = t; fa.lossb = lossb; fa.r = r; fa.rb = rb; fa.bb = bb; fa.tb = tb; fa.loss = loss;
    return run<ADJ>(fa, w, nullptr, wb, nullptr, x, nullptr, xb, nullptr, i_m, i_n, stream);
}

int32_t stade_hip_affine_lsq_d(double* loss, double* lossd, const double* w, const double* wd, const double* x, const double* xd,
                               const double* b, const double* bd, const double* t, const double* td, double* r, double* rd,
                               int64_t i_m, int64_t i_n, hipStream_t stream) {
    if (int32_t rc = check_sizes(i_m, i_n, "stade_hip_affine_lsq_d")) return rc;
    if (i_m > 0 && (!loss || !lossd || !b || !bd || !t || !td || !r || !rd || (i_n > 0 && (!w || !wd || !x || !xd))))
        return set_error(STADE_HIP_EINVAL, "stade_hip_affine_lsq_d: null pointer");
    FinishArgs fa{};
    fa.b = b; fa.t = t; fa.bd = bd; fa.td = td; fa.r = r; fa.rd = rd; fa.loss = loss; fa.lossd = lossd;
    return run<TAN>(fa, w, wd, nullptr, nullptr, x, xd, nullptr, nullptr, i_m, i_n, stream);
}

int32_t stade_hip_affine_lsq_hv(double* loss, const double* lossb, const double* w, double* wb, const double* x, double* xb,
                                const double* b, double* bb, const double* t, double* tb, double* r, double* rb,
                                int64_t i_m, int64_t i_n, double* lossd, const double* lossbd, const double* wd, double* wbd,
                                const double* xd, double* xbd, const double* bd, double* bbd, const double* td, double* tbd,
                                double* rd, double* rbd, hipStream_t stream) {
    if (int32_t rc = check_sizes(i_m, i_n, "stade_hip_affine_lsq_hv")) return rc;
    if (i_m > 0 && (!loss || !lossb || !b || !bb || !t || !tb || !r || !rb || !lossd || !lossbd || !bd || !bbd || !td || !tbd ||
                    !rd || !rbd || (i_n > 0 && (!w || !wb || !x || !xb || !wd || !wbd || !xd || !xbd))))
        return set_error(STADE_HIP_EINVAL, "stade_hip_affine_lsq_hv: null pointer");
    FinishArgs fa{};
    fa.b = b; fa.t = t; fa.bd = bd; fa.td = td; fa.lossb = lossb; fa.lossbd = lossbd;
    fa.r = r; fa.rd = rd; fa.rb = rb; fa.rbd = rbd; fa.bb = bb; fa.bbd = bbd; fa.tb = tb; fa.tbd = tbd;
    fa.loss = loss; fa.lossd = lossd;
    return run<HVP>(fa, w, wd, wb, wbd, x, xd, xb, xbd, i_m, i_n, stream);
}

}  // extern "C"
