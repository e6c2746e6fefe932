// Config 4: conv3x3 -- 3 x 3 convolution (stride 1, zero padding held in the input) and
// half the squared norm of the output, Float32.  Executes the generated adjoint, tangent and
// HVP of corpus/conv3x3.jl (corpus/conv3x3_{b,d,hv}.jl), the functions `stade_amdgpu_file`
// would port (/root/reference/src/STADE.jl:18604-18605).
//
// Layouts (Julia column-major, 0-based below):
//   xp  (i_w+2, i_h+2, i_c, i_nb): xp[n][c][yp][xq] at ((n*C + c)*Hp + yp)*Wp + xq
//   w   (3, 3, i_c, i_k):          w[co][c][ky][kx] at ((co*C + c)*3 + ky)*3 + kx
//   out (i_w, i_h, i_k, i_nb):     out[n][co][y][x] at ((n*K + co)*H + y)*W + x
//
// The generated loops are three products over one index space (pixel, tap, c, co):
//   forward  out[n][co][y][x]   = sum_{c,ky,kx} w[co][c][ky][kx] xp[n][c][y+ky][x+kx]
//   adjoint  g = outb + (0.5 (2 out)) lossb  (the accumulated outb, then reset to 0)
//            wb[co][c][ky][kx] += sum_{n,y,x} g[n][co][y][x] xp[n][c][y+ky][x+kx]
//            xpb[n][c][yp][xq] += sum_{co,ky,kx} w[co][c][ky][kx] g[n][co][yp-ky][xq-kx]
// All three run on the fp32 matrix cores (v_mfma_f32_32x32x2_f32) as implicit GEMMs: no
// im2col buffer; each block stages an input patch and a weight slice in LDS and the MFMA
// operands are read from the patch at tap-shifted offsets.
//   tap_kernel    forward (and the tangent's two products) and the interior of xpb, which
//                 is the same shifted product on g with flipped, transposed weights
//   border_kernel the one-cell frame of xpb (taps that land on the zero padding): four 1-D
//                 3-tap line correlations
//   wgrad_kernel  split over pixel tiles, partial 9 x 64 x 64 weight gradients per block
//   wreduce_kernel sums the partials in a fixed order into wb
#include "internal.hpp"

#include <algorithm>

namespace stade {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int NT = 256;
constexpr int kBufWord3 = 0x00020000;  // gfx9-family buffer resource word 3 (raw, 32-bit data)

enum { FWD_B, FWD_D, FWD_HV, DG_B, DG_HV };

__device__ __forceinline__ floatx16 mfma(float a, float b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------------------------------
// weight layouts for the tap kernel: wt[cin][t][r] (rows padded to a multiple of 64 with
// zeros).  Forward: cin = c, r = co, t = 3 ky + kx.  Interior of xpb: cin = co, r = c, and
// the tap flipped (t' = 8 - t), so both products read their source at (y + ky' - 1 + ...).
// ------------------------------------------------------------------------------------------
__global__ __launch_bounds__(NT) void prep_kernel(const float* __restrict__ w, int C, int K, float* __restrict__ wf,
                                                  int Kpad, float* __restrict__ wg, int Cpad) {
    const long nf = (long)C * 9 * Kpad, ng = wg ? (long)K * 9 * Cpad : 0;
    const long q = (long)blockIdx.x * NT + threadIdx.x;
    if (q < nf) {
        const int r = (int)(q % Kpad);
        const long ct = q / Kpad;
        const int t = (int)(ct % 9), c = (int)(ct / 9);
        wf[q] = r < K ? w[((long)r * C + c) * 9 + t] : 0.f;
    } else if (q < nf + ng) {
        const long p = q - nf;
        const int r = (int)(p % Cpad);
        const long ct = p / Cpad;
        const int t = (int)(ct % 9), co = (int)(ct / 9);
        wg[p] = r < C ? w[((long)co * C + r) * 9 + (8 - t)] : 0.f;
    }
}

// ------------------------------------------------------------------------------------------
// tap kernel: o[r][y][x] = sum_{cin, ty, tx} wt[cin][3 ty + tx][r] * src[cin][y + ty + ofs][x + tx + ofs]
//
// Block: 256 threads, a 64-row (r) x (64 x 4 pixel) output tile.  Wave w owns pixel row
// y0 + w: 2 x 2 MFMA 32 x 32 tiles (r halves x pixel halves).  Input channels advance CC at a
// time (CC = 16 with one source, 8 with two); each step stages the (4+2) x (64+2) patch of
// every channel and the 9 x 64 weight rows in LDS.  The next step's global loads are issued
// into registers before the MFMAs of the current one.  The MFMA k pair (lane / 32) is a pair
// of channels at the same tap, so every LDS read has a lane base plus an immediate offset.
// ------------------------------------------------------------------------------------------
constexpr int TX = 64, TY = 4, RT = 64;
constexpr int PXW = TX + 2, PYH = TY + 2, PPL = PXW * PYH;  // patch row, rows, plane (floats)
constexpr int KW = 9 * RT;                                    // weight floats per channel

struct TapArgs {
    const float* src[2];  // sources (n, cin, SH, SW)
    const float* wt[2];   // weights [cin][9][Rpad]
    int Cin, R, Rpad, N;
    int SH, SW, ofs;      // source plane and patch origin offset
    int H, W;             // output domain
    float* o0;            // out / xpb
    float* o1;            // outd / xpbd
    int OH, OW, oofs;     // o[((n*R + r)*OH + y + oofs)*OW + x + oofs]
    float* g0;            // forward adjoint: g = accumulated outb, and its tangent
    float* g1;
    float* ob;            // outb, outbd (read, then reset to zero)
    float* obd;
    const float* lossb;
    const float* lossbd;
    double* partials;     // loss sums per block
};

template <int MODE>
__global__ __launch_bounds__(NT, (MODE == FWD_B || MODE == DG_B) ? 2 : 1) void tap_kernel(TapArgs a) {
    constexpr int NP = (MODE == FWD_B || MODE == DG_B) ? 1 : 2;  // sources = weight sets = outputs
    constexpr int CC = 16 / NP;
    constexpr int PSZ = CC * PPL, WSZ = CC * KW;
    constexpr int WLD = NP * WSZ / 4 / NT;
    static_assert(NP * WSZ % (4 * NT) == 0, "weight stage");
    constexpr bool FWD = MODE == FWD_B || MODE == FWD_D || MODE == FWD_HV;
    constexpr int NV = MODE == FWD_B ? 1 : 2;

    __shared__ float lds[NP * (PSZ + WSZ)];
    __shared__ double red[16 * NV];
    float* Ps = lds;
    float* Ws = lds + NP * PSZ;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = lane >> 5, l32 = lane & 31;
    const int x0 = blockIdx.x * TX, y0 = blockIdx.y * TY;
    const int rtiles = a.Rpad / RT;
    const int n = blockIdx.z / rtiles, rt = blockIdx.z - n * rtiles;

    // Patch staging by rows: the NP * CC * PYH = 96 patch rows of PXW = 66 floats; wave w
    // takes rows w, w + 4, ..., one column per lane (columns 0..63), so the channel, row and
    // row bounds are wave-uniform (scalar) and a lane's address is a row base plus its lane;
    // columns 64, 65 of every row go to threads 0..191, one element each.
    constexpr int PROWS = NP * CC * PYH, RPW = PROWS / 4;
    static_assert(PROWS % 4 == 0 && PXW == 66 && 2 * PROWS <= NT, "patch rows");
    float pr[RPW + 1];
    float4 wr[WLD];
    // Staging loads are buffer loads: a scalar resource per source image n (and per weight
    // set), the row part of a patch address as a scalar offset (patch rows are wave-uniform)
    // and the column as the lane's offset.  An element outside the source reads offset =
    // the resource's size, which returns 0.  Vector registers hold no 64-bit addresses, so the
    // staging fits two waves per SIMD without spilling.  (The host keeps one image of a
    // source and a weight set under 2^31 bytes.)
    const long plane = (long)a.SH * a.SW;
    const uint32_t sbytes = (uint32_t)((long)a.Cin * plane * 4);
    const uint32_t wbytes = (uint32_t)((long)a.Cin * 9 * a.Rpad * 4);
    __amdgpu_buffer_rsrc_t rs[NP], rw[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        rs[p] = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.src[p] + (long)n * a.Cin * plane), (short)0, sbytes,
                                                  kBufWord3);
        rw[p] = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.wt[p] + rt * RT), (short)0, wbytes, kBufWord3);
    }
    const int sx_l = x0 + lane + a.ofs;
    const uint32_t lane_col = (unsigned)sx_l < (unsigned)a.SW ? (uint32_t)sx_l * 4u : sbytes;
    auto load = [&](int c0) {
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const int rr = wave + 4 * i;  // wave-uniform patch row (p, cc, ty)
            const int p = NP == 1 ? 0 : rr / (CC * PYH);
            const int rem = rr - p * (CC * PYH);
            const int cc = rem / PYH, ty = rem - cc * PYH;
            const int c = c0 + cc, sy = y0 + ty + a.ofs;
            const bool ok = c < a.Cin && (unsigned)sy < (unsigned)a.SH;
            const uint32_t soff = ok ? (uint32_t)(((long)c * a.SH + sy) * a.SW * 4) : 0u;
            const uint32_t voff = ok ? lane_col : sbytes;
            pr[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(p ? rs[NP - 1] : rs[0], voff, soff, 0));
        }
        if (threadIdx.x < 2 * PROWS) {
            // columns 64, 65: the row varies across a wave, so the whole offset is the lane's
            const int rr = threadIdx.x >> 1, col = 64 + (threadIdx.x & 1);
            const int p = NP == 1 ? 0 : rr / (CC * PYH);
            const int rem = rr - p * (CC * PYH);
            const int cc = rem / PYH, ty = rem - cc * PYH;
            const int c = c0 + cc, sy = y0 + ty + a.ofs, sx = x0 + col + a.ofs;
            float v = 0.f;
            if (c < a.Cin && (unsigned)sy < (unsigned)a.SH && (unsigned)sx < (unsigned)a.SW)
                v = a.src[p][((long)(n * a.Cin + c) * a.SH + sy) * a.SW + sx];
            pr[RPW] = v;
        }
        const uint32_t wsoff = (uint32_t)((long)c0 * 9 * a.Rpad * 4);
#pragma unroll
        for (int q = 0; q < WLD; ++q) {
            const int f = threadIdx.x + q * NT;  // float4 slot of [w][cc][t][r]
            const int wi = NP == 1 ? 0 : __builtin_amdgcn_readfirstlane(f / (WSZ / 4));  // uniform per wave
            const int rem = f - wi * (WSZ / 4);
            const int row = rem / (RT / 4), r4 = (rem - row * (RT / 4)) * 4;
            const int cc = row / 9, t = row - cc * 9;
            const uint32_t voff = c0 + cc < a.Cin ? (uint32_t)(((cc * 9 + t) * a.Rpad + r4) * 4) : wbytes;
            const v4f x = __builtin_amdgcn_raw_buffer_load_b128(wi ? rw[NP - 1] : rw[0], voff, wsoff, 0);
            wr[q] = make_float4(x.x, x.y, x.z, x.w);
        }
    };
    auto store = [&]() {
        // patch row rr = (p, cc, ty) is at Ps + p * PSZ + cc * PPL + ty * PXW = Ps + rr * PXW
#pragma unroll
        for (int i = 0; i < RPW; ++i) Ps[(wave + 4 * i) * PXW + lane] = pr[i];
        if (threadIdx.x < 2 * PROWS) Ps[(threadIdx.x >> 1) * PXW + 64 + (threadIdx.x & 1)] = pr[RPW];
#pragma unroll
        for (int q = 0; q < WLD; ++q) {
            const int f = threadIdx.x + q * NT;
            *reinterpret_cast<float4*>(Ws + 4 * f) = wr[q];
        }
    };

    floatx16 acc[NP][2][2];
#pragma unroll
    for (int o = 0; o < NP; ++o)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 16; ++q) acc[o][i][j][q] = 0.f;

    // lane bases: patch channel (2 qq + h), row (wave + ky), column (32 j + l32 + kx);
    // weight row (2 qq + h, t), column 32 i + l32
    const int pbase = h * PPL + wave * PXW + l32;
    const int wbase = h * KW + l32;
    const int nchunks = (a.Cin + CC - 1) / CC;
    if (nchunks > 0) load(0);
    for (int ch = 0; ch < nchunks; ++ch) {
        __syncthreads();
        store();
        __syncthreads();
        if (ch + 1 < nchunks) load((ch + 1) * CC);
        // k steps st = (channel pair qq, tap t); the fragments of step st+1 are read from LDS
        // while the MFMAs of step st run (two register sets; the scheduling barriers keep
        // the compiler from sinking each read to its use)
        constexpr int NSTEP = CC / 2 * 9;
        float pf[2][NP][2], wf[2][NP][2];
        auto frag = [&](int st, int buf) {
            const int qq = st / 9, t = st % 9, ky = t / 3, kx = t % 3;
#pragma unroll
            for (int p = 0; p < NP; ++p)
#pragma unroll
                for (int j = 0; j < 2; ++j) pf[buf][p][j] = Ps[p * PSZ + pbase + 2 * qq * PPL + ky * PXW + kx + 32 * j];
#pragma unroll
            for (int p = 0; p < NP; ++p)
#pragma unroll
                for (int i = 0; i < 2; ++i) wf[buf][p][i] = Ws[p * WSZ + wbase + (2 * qq * 9 + t) * RT + 32 * i];
        };
        frag(0, 0);
#pragma unroll
        for (int st = 0; st < NSTEP; ++st) {
            const int b = st & 1;
            if (st + 1 < NSTEP) frag(st + 1, b ^ 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    acc[0][i][j] = mfma(wf[b][0][i], pf[b][0][j], acc[0][i][j]);
                    if constexpr (NP == 2) {
                        acc[1][i][j] = mfma(wf[b][1][i], pf[b][0][j], acc[1][i][j]);
                        acc[1][i][j] = mfma(wf[b][0][i], pf[b][1][j], acc[1][i][j]);
                    }
                }
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // epilogue: accumulator (i, j, q) is row r = rt*64 + 32 i + 8 (q / 4) + 4 h + q % 4,
    // pixel x = x0 + 32 j + l32 of row y = y0 + wave
    double ls[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) ls[k] = 0.0;
    float lb = 0.f, lbd = 0.f;
    if constexpr (MODE == FWD_B || MODE == FWD_HV) lb = a.lossb[0];
    if constexpr (MODE == FWD_HV) lbd = a.lossbd[0];
    const int y = y0 + wave;
    // The read-modify-write inputs (outb, outbd of the forward adjoint; xpb, xpbd of the
    // interior) are all loaded before any store: the output arrays may alias as far as the
    // compiler knows, so interleaving would serialise one HBM round trip per element.
    constexpr bool RMW = MODE != FWD_D;
    constexpr int NR = (MODE == FWD_HV || MODE == DG_HV) ? 2 : 1;
    float pre[NR][2][2][16];
    auto index = [&](int i, int j, int q, long& oi) {
        const int x = x0 + 32 * j + l32;
        const int r = rt * RT + 32 * i + 8 * (q >> 2) + 4 * h + (q & 3);
        oi = ((long)(n * a.R + r) * a.OH + y + a.oofs) * a.OW + x + a.oofs;
        return y < a.H && x < a.W && r < a.R;
    };
    if constexpr (RMW) {
        const float* s0 = FWD ? a.ob : a.o0;
        const float* s1 = FWD ? a.obd : a.o1;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    long oi;
                    const bool ok = index(i, j, q, oi);
                    pre[0][i][j][q] = ok ? s0[oi] : 0.f;
                    if constexpr (NR == 2) pre[NR - 1][i][j][q] = ok ? s1[oi] : 0.f;
                }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                long oi;
                if (!index(i, j, q, oi)) continue;
                const float v = acc[0][i][j][q];
                if constexpr (FWD) {
                    a.o0[oi] = v;
                    ls[0] += 0.5 * (double)v * (double)v;
                    if constexpr (MODE == FWD_B) {
                        a.g0[oi] = pre[0][i][j][q] + (0.5f * (2.0f * v)) * lb;
                        a.ob[oi] = 0.f;
                    } else {
                        const float vd = acc[1][i][j][q];
                        a.o1[oi] = vd;
                        ls[1] += 0.5 * ((double)(2.0f * v) * (double)vd);
                        if constexpr (MODE == FWD_HV) {
                            const float c8 = 0.5f * (2.0f * v);
                            a.g1[oi] = pre[NR - 1][i][j][q] + (lb * (0.5f * (2.0f * vd)) + c8 * lbd);
                            a.g0[oi] = pre[0][i][j][q] + c8 * lb;
                            a.ob[oi] = 0.f;
                            a.obd[oi] = 0.f;
                        }
                    }
                } else {
                    a.o0[oi] = pre[0][i][j][q] + v;
                    if constexpr (MODE == DG_HV) a.o1[oi] = pre[NR - 1][i][j][q] + acc[1][i][j][q];
                }
            }
    if constexpr (FWD) block_partials<NV>(ls, red, a.partials);
}

// loss (and lossd) += the sum of the tap kernel's block partials, rounded once to Float32
template <int NV>
__global__ __launch_bounds__(NT) void loss_kernel(const double* __restrict__ partials, int nparts, float* l0, float* l1) {
    __shared__ double red[16 * NV];
    double acc[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) acc[k] = 0.0;
    // unrolled so that several partials' loads are in flight (the sums keep their order)
#pragma unroll 8
    for (int b = threadIdx.x; b < nparts; b += NT)
#pragma unroll
        for (int k = 0; k < NV; ++k) acc[k] += partials[(long)b * NV + k];
    block_sum<NV>(acc, red);
    if (threadIdx.x == 0) {
        // both destinations read before either is written (they may alias as far as the
        // compiler knows)
        const float o0 = l0[0], o1 = NV == 2 ? l1[0] : 0.f;
        l0[0] = (float)((double)o0 + acc[0]);
        if (NV == 2) l1[0] = (float)((double)o1 + acc[NV - 1]);
    }
}

// ------------------------------------------------------------------------------------------
// frame of xpb: padded cells with yp in {0, Hp-1} or xq in {0, Wp-1}.  On each edge only one
// tap row (or column) lands inside the image, so an edge is a 1-D 3-tap full correlation
// along one line of g:
//   top    (yp = 0,    p = xq in 0..W+1):  sum_co sum_d w[co][c][0][d]  g[co][0][p - d]
//   bottom (yp = Hp-1, p = xq):            sum_co sum_d w[co][c][2][d]  g[co][H-1][p - d]
//   left   (xq = 0,    p = yp-1 in 0..H-1): sum_co sum_d w[co][c][d][0] g[co][p + 1 - d][0]
//   right  (xq = Wp-1, p = yp-1):          sum_co sum_d w[co][c][d][2]  g[co][p + 1 - d][W-1]
// (g zero outside the image).  Block: 64 cells of one edge x 16 channels c; output
// channels advance 16 at a time through LDS (the g line segment and the weight slice).
// ------------------------------------------------------------------------------------------
constexpr int BSEG = 64, BKC = 64, BCG = 16;  // cells, output channels per staging round, input channels

struct BorderArgs {
    const float* w;
    const float* wd;
    const float* g;
    const float* gd;
    float* xpb;
    float* xpbd;
    int N, C, K, H, W;
};

template <bool HV>
__global__ __launch_bounds__(NT) void border_kernel(BorderArgs a) {
    constexpr int NG = HV ? 2 : 1;
    __shared__ float gl[NG][BKC][BSEG + 2];
    __shared__ float4 wv[NG][BKC][3][BCG / 4];  // [kk][d][c]: a thread's 4 channels in one read
    const int e = blockIdx.y;
    const int L = e < 2 ? a.W + 2 : a.H;
    const int p0 = blockIdx.x * BSEG;
    if (p0 >= L) return;  // whole block
    const int ncg = (a.C + BCG - 1) / BCG;
    const int n = blockIdx.z / ncg, c0 = (blockIdx.z % ncg) * BCG;
    const int off = e < 2 ? 0 : 1;
    const int fixed = (e == 0 || e == 2) ? 0 : 2;
    const int lim = e < 2 ? a.W : a.H;
    const int cell = threadIdx.x & 63, cg = threadIdx.x >> 6;
    float acc[4] = {0.f, 0.f, 0.f, 0.f}, accd[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < a.K; k0 += BKC) {
        __syncthreads();
        // every staging load of the round issued before any LDS store (one memory round trip)
        constexpr int NGL = (BKC * (BSEG + 2) + NT - 1) / NT, NWL = BKC * BCG * 3 / NT;
        static_assert(BKC * BCG * 3 % NT == 0, "weight staging");
        float gv_[NGL], gvd_[NGL], wv_[NWL], wvd_[NWL];
#pragma unroll
        for (int u = 0; u < NGL; ++u) {
            const int f = threadIdx.x + u * NT;
            const int kk = f / (BSEG + 2), i = f - kk * (BSEG + 2);
            const int co = k0 + kk, q = p0 + off - 2 + i;
            float v = 0.f, vd = 0.f;
            if (f < BKC * (BSEG + 2) && co < a.K && q >= 0 && q < lim) {
                const long plane = (long)(n * a.K + co) * a.H;
                const long gi = e < 2 ? (plane + (e == 0 ? 0 : a.H - 1)) * a.W + q : (plane + q) * a.W + (e == 2 ? 0 : a.W - 1);
                v = a.g[gi];
                if (HV) vd = a.gd[gi];
            }
            gv_[u] = v;
            gvd_[u] = vd;
        }
#pragma unroll
        for (int u = 0; u < NWL; ++u) {
            const int f = threadIdx.x + u * NT;
            const int kk = f / (BCG * 3), r = f - kk * (BCG * 3);
            const int cc = r / 3, d = r - cc * 3;
            const int co = k0 + kk, c = c0 + cc;
            float v = 0.f, vd = 0.f;
            if (co < a.K && c < a.C) {
                const int ky = e < 2 ? fixed : d, kx = e < 2 ? d : fixed;
                const long wi = ((long)co * a.C + c) * 9 + 3 * ky + kx;
                v = a.w[wi];
                if (HV) vd = a.wd[wi];
            }
            wv_[u] = v;
            wvd_[u] = vd;
        }
#pragma unroll
        for (int u = 0; u < NGL; ++u) {
            const int f = threadIdx.x + u * NT;
            if (f < BKC * (BSEG + 2)) {
                const int kk = f / (BSEG + 2), i = f - kk * (BSEG + 2);
                gl[0][kk][i] = gv_[u];
                if (HV) gl[NG - 1][kk][i] = gvd_[u];
            }
        }
#pragma unroll
        for (int u = 0; u < NWL; ++u) {
            const int f = threadIdx.x + u * NT;
            const int kk = f / (BCG * 3), r = f - kk * (BCG * 3);
            const int cc = r / 3, d = r - cc * 3;
            reinterpret_cast<float*>(&wv[0][kk][d][0])[cc] = wv_[u];
            if (HV) reinterpret_cast<float*>(&wv[NG - 1][kk][d][0])[cc] = wvd_[u];
        }
        __syncthreads();
#pragma unroll 4
        for (int kk = 0; kk < BKC; ++kk)
#pragma unroll
            for (int d = 0; d < 3; ++d) {
                const float gv = gl[0][kk][cell + 2 - d];
                const float gvd = HV ? gl[NG - 1][kk][cell + 2 - d] : 0.f;
                const float4 w4 = wv[0][kk][d][cg];
                const float4 wd4 = HV ? wv[NG - 1][kk][d][cg] : make_float4(0.f, 0.f, 0.f, 0.f);
                const float wc_[4] = {w4.x, w4.y, w4.z, w4.w}, wdc_[4] = {wd4.x, wd4.y, wd4.z, wd4.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    acc[i] += wc_[i] * gv;
                    if (HV) accd[i] += wdc_[i] * gv + wc_[i] * gvd;
                }
            }
    }
    const int p = p0 + cell;
    if (p >= L) return;
    const int Hp = a.H + 2, Wp = a.W + 2;
    const int yp = e == 0 ? 0 : e == 1 ? Hp - 1 : p + 1;
    const int xq = e < 2 ? p : (e == 2 ? 0 : Wp - 1);
    // every xpb (xpbd) value read before any is written (the arrays may alias as far as the
    // compiler knows)
    float old[4], oldd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = c0 + 4 * cg + i;
        const long oi = ((long)(n * a.C + c) * Hp + yp) * Wp + xq;
        old[i] = c < a.C ? a.xpb[oi] : 0.f;
        oldd[i] = (HV && c < a.C) ? a.xpbd[oi] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = c0 + 4 * cg + i;
        if (c >= a.C) continue;
        const long oi = ((long)(n * a.C + c) * Hp + yp) * Wp + xq;
        a.xpb[oi] = old[i] + acc[i];
        if (HV) a.xpbd[oi] = oldd[i] + accd[i];
    }
}

// ------------------------------------------------------------------------------------------
// weight gradient: part[split][ct][kt][t][ci][co] = sum over the split's pixel tiles of
//   sum_p sum_{pixel} x_p[n][c][y+ky][x+kx] * g_p[n][co][y][x]
// Block: 256 threads, a 64 (c) x 64 (co) slab of all 9 taps; wave (wa, wb) owns the
// 32 x 32 quarter (c half wa, co half wb) of every tap: 9 accumulator tiles.  Pixel tiles of
// 32 x 2 pixels: the (2+2) x (32+2) patch of 64 channels and the 64 x 64 g tile are staged in
// LDS (next tile prefetched into registers); the MFMA k pair is a pair of adjacent pixels.
// ------------------------------------------------------------------------------------------
constexpr int WTX = 32, WTY = 2;
constexpr int XPX = WTX + 2;                   // 34
constexpr int XPL = XPX * (WTY + 2);           // 136 floats of one channel's patch
constexpr int XPP = XPL + 1;                   // LDS plane stride (odd)
constexpr int GPX = WTX * WTY, GPP = GPX + 1;  // 64 pixels, LDS row stride 65
constexpr int XSZ = 64 * XPP, GSZ = 64 * GPP;

struct WgArgs {
    const float* x[2];  // xp-shaped
    const float* g[2];  // out-shaped
    int N, C, K, H, W;
    int ntx, nty, ntiles;  // pixel tiles of one (x, g) pair
    int npairs;            // NPR = 1: tiles [p * ntiles, (p + 1) * ntiles) use pair p
    float* part;
};

template <int NPR>
__global__ __launch_bounds__(NT) void wgrad_kernel(WgArgs a) {
    constexpr int XLD = 64 * XPL / NT;  // 34
    constexpr int GLD = 64 * GPX / NT;  // 16
    static_assert(64 * XPL % NT == 0 && 64 * GPX % NT == 0, "wgrad stage");
    __shared__ float lds[NPR * (XSZ + GSZ)];
    float* Xs = lds;
    float* Gs = lds + NPR * XSZ;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = lane >> 5, l32 = lane & 31;
    const int ktn = (a.K + 63) / 64;
    const int ct = blockIdx.x / ktn, kt = blockIdx.x - ct * ktn;
    const int c0 = ct * 64, k0 = kt * 64;
    const int wa = wave & 1, wb = wave >> 1;
    const int Hp = a.H + 2, Wp = a.W + 2;

    float xr[NPR][XLD], gr[NPR][GLD];
    auto load = [&](int tile) {
        // NPR = 1 with two pairs: the pair is uniform over the block's tile
        const int pr = NPR == 1 && tile >= a.ntiles ? 1 : 0;
        tile -= pr * a.ntiles;
        const float* xs[2] = {a.x[pr], a.x[1]};
        const float* gs[2] = {a.g[pr], a.g[1]};
        const int xt = tile % a.ntx;
        const int rest = tile / a.ntx;
        const int yt = rest % a.nty, n = rest / a.nty;
        const int x0 = xt * WTX, y0 = yt * WTY;
#pragma unroll
        for (int p = 0; p < NPR; ++p) {
#pragma unroll
            for (int q = 0; q < XLD; ++q) {
                const int f = threadIdx.x + q * NT;
                const int ci = f / XPL, e = f - ci * XPL;
                const int ty = e / XPX, tx = e - ty * XPX;
                const int c = c0 + ci, yy = y0 + ty, xx = x0 + tx;
                xr[p][q] = (c < a.C && yy < Hp && xx < Wp) ? xs[p][((long)(n * a.C + c) * Hp + yy) * Wp + xx] : 0.f;
            }
#pragma unroll
            for (int q = 0; q < GLD; ++q) {
                const int f = threadIdx.x + q * NT;
                const int co = f / GPX, px = f - co * GPX;
                const int k = k0 + co, yy = y0 + px / WTX, xx = x0 + px % WTX;
                gr[p][q] = (k < a.K && yy < a.H && xx < a.W) ? gs[p][((long)(n * a.K + k) * a.H + yy) * a.W + xx] : 0.f;
            }
        }
    };
    auto store = [&]() {
#pragma unroll
        for (int p = 0; p < NPR; ++p) {
#pragma unroll
            for (int q = 0; q < XLD; ++q) {
                const int f = threadIdx.x + q * NT;
                const int ci = f / XPL;
                Xs[p * XSZ + ci * XPP + (f - ci * XPL)] = xr[p][q];
            }
#pragma unroll
            for (int q = 0; q < GLD; ++q) {
                const int f = threadIdx.x + q * NT;
                const int co = f / GPX;
                Gs[p * GSZ + co * GPP + (f - co * GPX)] = gr[p][q];
            }
        }
    };

    floatx16 acc[9];
#pragma unroll
    for (int t = 0; t < 9; ++t)
#pragma unroll
        for (int q = 0; q < 16; ++q) acc[t][q] = 0.f;

    // lane bases: patch channel 32 wa + l32, pixel + h;  g row 32 wb + l32, pixel + h
    const int xb = (32 * wa + l32) * XPP + h;
    const int gb = (32 * wb + l32) * GPP + h;
    const int ntot = a.ntiles * a.npairs;
    int tile = blockIdx.y;
    if (tile < ntot) load(tile);
    for (; tile < ntot; tile += gridDim.y) {
        __syncthreads();
        store();
        __syncthreads();
        if (tile + (int)gridDim.y < ntot) load(tile + gridDim.y);
        // k steps s (pixel pairs 2s, 2s+1); step s+1's fragments are read during step s's MFMAs
        constexpr int NSTEP = GPX / 2;
        float gf[2][NPR], xf[2][NPR][9];
        auto frag = [&](int st, int buf) {
            const int py = (2 * st) / WTX, px = (2 * st) % WTX;
#pragma unroll
            for (int p = 0; p < NPR; ++p) {
                gf[buf][p] = Gs[p * GSZ + gb + 2 * st];
#pragma unroll
                for (int t = 0; t < 9; ++t) xf[buf][p][t] = Xs[p * XSZ + xb + (py + t / 3) * XPX + px + t % 3];
            }
        };
        frag(0, 0);
#pragma unroll
        for (int st = 0; st < NSTEP; ++st) {
            const int b = st & 1;
            if (st + 1 < NSTEP) frag(st + 1, b ^ 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < 9; ++t)
#pragma unroll
                for (int p = 0; p < NPR; ++p) acc[t] = mfma(xf[b][p][t], gf[b][p], acc[t]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // accumulator (t, q): c = 32 wa + 8 (q / 4) + 4 h + q % 4, co = 32 wb + l32 (slab-local)
    float* dst = a.part + (long)(blockIdx.y * gridDim.x + blockIdx.x) * 9 * 4096;
#pragma unroll
    for (int t = 0; t < 9; ++t)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const int ci = 32 * wa + 8 * (q >> 2) + 4 * h + (q & 3), co = 32 * wb + l32;
            dst[t * 4096 + ci * 64 + co] = acc[t][q];
        }
}

// wb[co][c][t] += the sum of the partials over splits.  Block: 64 consecutive partial
// elements x 4 split lanes; lane l sums splits l, l+4, ... in order, then the 4 lane sums
// are added in lane order (a fixed order: the result does not depend on scheduling).
__global__ __launch_bounds__(NT) void wreduce_kernel(const float* __restrict__ part, int nsplit, int nslab, int ktn, int C,
                                                     int K, float* __restrict__ wb) {
    __shared__ double red[4][64];
    const long total = (long)nslab * 9 * 4096;
    const int el = threadIdx.x & 63, sl = threadIdx.x >> 6;
    const long q = (long)blockIdx.x * 64 + el;
    double s = 0.0;
    // unrolled so that several splits' loads are in flight (the sum keeps its order)
    if (q < total) {
#pragma unroll 8
        for (int sp = sl; sp < nsplit; sp += 4) s += part[(long)sp * total + q];
    }
    red[sl][el] = s;
    __syncthreads();
    if (sl != 0 || q >= total) return;
    s = ((red[0][el] + red[1][el]) + red[2][el]) + red[3][el];
    const int co_l = (int)(q & 63), ci_l = (int)((q >> 6) & 63);
    const long rest = q >> 12;
    const int t = (int)(rest % 9), slab = (int)(rest / 9);
    const int ct = slab / ktn, kt = slab - ct * ktn;
    const int c = ct * 64 + ci_l, k = kt * 64 + co_l;
    if (c >= C || k >= K) return;
    const long wi = ((long)k * C + c) * 9 + t;
    wb[wi] = (float)((double)wb[wi] + s);
}

// ------------------------------------------------------------------------------------------
// host
// ------------------------------------------------------------------------------------------
enum { ADJ, TAN, HVP };

struct Ptrs {
    float *loss, *lossb, *xp, *xpb, *w, *wb, *out, *outb;
    float *lossd, *lossbd, *xpd, *xpbd, *wd, *wbd, *outd, *outbd;
};

struct Dims {
    int N, C, K, H, W, Hp, Wp, Kpad, Cpad;
};

int32_t check(int64_t N, int64_t C, int64_t K, int64_t H, int64_t W, const char* fn, Dims& d) {
    if (N < 0 || C < 0 || K < 0 || H < 0 || W < 0) return set_error(STADE_HIP_EINVAL, "%s: negative size", fn);
    const double lim = 2147483647.0;
    // one image of a source and one weight set are read through buffer resources: < 2^31 bytes
    const double blim = 536870911.0;
    if ((double)C * (H + 2) * (W + 2) > blim || (double)K * H * W > blim || 9.0 * (C + 64) * (K + 64) > blim)
        return set_error(STADE_HIP_ERANGE, "%s: one image or the weights exceed 2^29 elements", fn);
    if ((double)N * C * (H + 2) * (W + 2) > lim || (double)N * K * H * W > lim || 9.0 * C * K > lim ||
        (double)N * ((K + 63) / 64) > 65535 || (double)N * ((C + 15) / 16) > 65535 || H > 200000 || W > 200000)
        return set_error(STADE_HIP_ERANGE, "%s: sizes out of range", fn);
    d.N = (int)N; d.C = (int)C; d.K = (int)K; d.H = (int)H; d.W = (int)W;
    d.Hp = d.H + 2; d.Wp = d.W + 2;
    d.Kpad = (d.K + 63) / 64 * 64;
    d.Cpad = (d.C + 63) / 64 * 64;
    const long tapblocks = (long)((d.W + TX - 1) / TX) * ((d.H + TY - 1) / TY) * d.N * (d.Kpad / 64);
    if (tapblocks * 2 > kPartialSlots) return set_error(STADE_HIP_ERANGE, "%s: sizes out of range", fn);
    return STADE_HIP_OK;
}

inline size_t up64(size_t n) { return (n + 63) / 64 * 64; }

template <int MODE>
hipError_t launch_tap(const TapArgs& a, const char* name, hipStream_t stream, unsigned& nblocks) {
    dim3 grid((a.W + TX - 1) / TX, (a.H + TY - 1) / TY, a.N * (a.Rpad / RT));
    nblocks = grid.x * grid.y * grid.z;
    STADE_TIMED(name, stream, (tap_kernel<MODE><<<grid, NT, 0, stream>>>(a)));
    return hipGetLastError();
}

template <int NPR>
int32_t weight_grad(const Dims& d, const float* x0, const float* g0, const float* x1, const float* g1, float* part,
                    int nsplit, float* wb, const char* name, hipStream_t stream) {
    WgArgs a{};
    a.x[0] = x0; a.g[0] = g0; a.x[1] = x1; a.g[1] = g1;
    a.N = d.N; a.C = d.C; a.K = d.K; a.H = d.H; a.W = d.W;
    a.ntx = (d.W + WTX - 1) / WTX;
    a.nty = (d.H + WTY - 1) / WTY;
    a.ntiles = a.ntx * a.nty * d.N;
    a.npairs = NPR == 1 && x1 ? 2 : 1;
    a.part = part;
    const int ctn = d.Cpad / 64, ktn = d.Kpad / 64;
    dim3 grid(ctn * ktn, nsplit);
    STADE_TIMED(name, stream, (wgrad_kernel<NPR><<<grid, NT, 0, stream>>>(a)));
    STADE_LAUNCHED("conv3x3 wgrad_kernel");
    const long nr = (long)ctn * ktn * 9 * 4096;
    STADE_TIMED("conv_wreduce", stream,
                (wreduce_kernel<<<(unsigned)((nr + 63) / 64), NT, 0, stream>>>(part, nsplit, ctn * ktn, ktn, d.C, d.K, wb)));
    STADE_LAUNCHED("conv3x3 wreduce_kernel");
    return STADE_HIP_OK;
}

template <int MODE>
int32_t run(const Ptrs& p, const Dims& d, hipStream_t stream) {
    if (d.N == 0 || d.K == 0 || d.H == 0 || d.W == 0) return STADE_HIP_OK;
    WsCall call_(stream);
    Workspace* ws = call_.ws;
    if (!ws) return STADE_HIP_ENOMEM;
    const size_t nwf = up64((size_t)d.C * 9 * d.Kpad), nwg = up64((size_t)d.K * 9 * d.Cpad);
    const size_t nout = up64((size_t)d.N * d.K * d.H * d.W);
    const int ctn = d.Cpad / 64, ktn = d.Kpad / 64;
    const long ntiles = (long)((d.W + WTX - 1) / WTX) * ((d.H + WTY - 1) / WTY) * d.N;
    // ctn is 0 when C = 0 (no weight gradient to form)
    const int nsplit = ctn == 0 ? 0 : (int)std::max(1L, std::min(ntiles, (long)std::max(1, 256 / (ctn * ktn))));
    const size_t npart = (MODE == TAN || d.C == 0) ? 0 : (size_t)nsplit * ctn * ktn * 9 * 4096;
    const int two = MODE == ADJ ? 1 : 2;
    const size_t total = two * nwf + (MODE == TAN ? 0 : two * nwg + two * nout) + npart;
    float* base = (float*)scratch(sizeof(float) * total + 256);
    if (!base) return scratch_error();
    float* wf0 = base;
    float* wf1 = wf0 + nwf;
    float* wg0 = wf0 + two * nwf;
    float* wg1 = wg0 + nwg;
    float* G = wg0 + (MODE == TAN ? 0 : two * nwg);
    float* GD = G + nout;
    float* part = G + (MODE == TAN ? 0 : two * nout);

    // weights in tap-kernel layouts
    {
        const long n = (long)d.C * 9 * d.Kpad + (MODE == TAN ? 0 : (long)d.K * 9 * d.Cpad);
        const unsigned nb = (unsigned)((n + NT - 1) / NT);
        if (n > 0) {
            STADE_TIMED("conv_prep", stream, (prep_kernel<<<nb, NT, 0, stream>>>(p.w, d.C, d.K, wf0, d.Kpad,
                                                                                 MODE == TAN ? nullptr : wg0, d.Cpad)));
            STADE_LAUNCHED("conv3x3 prep_kernel");
            if (MODE != ADJ) {
                STADE_TIMED("conv_prep", stream, (prep_kernel<<<nb, NT, 0, stream>>>(p.wd, d.C, d.K, wf1, d.Kpad,
                                                                                     MODE == TAN ? nullptr : wg1, d.Cpad)));
                STADE_LAUNCHED("conv3x3 prep_kernel");
            }
        }
    }
    // forward: out (and outd), loss (and lossd); adjoint seeds g (and gd), outb (and outbd) reset
    {
        TapArgs a{};
        a.src[0] = p.xp; a.src[1] = p.xpd;
        a.wt[0] = wf0; a.wt[1] = wf1;
        a.Cin = d.C; a.R = d.K; a.Rpad = d.Kpad; a.N = d.N;
        a.SH = d.Hp; a.SW = d.Wp; a.ofs = 0;
        a.H = d.H; a.W = d.W;
        a.o0 = p.out; a.o1 = p.outd;
        a.OH = d.H; a.OW = d.W; a.oofs = 0;
        a.g0 = G; a.g1 = GD; a.ob = p.outb; a.obd = p.outbd;
        a.lossb = p.lossb; a.lossbd = p.lossbd;
        a.partials = ws->partials;
        unsigned nblocks = 0;
        hipError_t e;
        if (MODE == ADJ) e = launch_tap<FWD_B>(a, "conv_fwd", stream, nblocks);
        else if (MODE == TAN) e = launch_tap<FWD_D>(a, "conv_fwd_d", stream, nblocks);
        else e = launch_tap<FWD_HV>(a, "conv_fwd_hv", stream, nblocks);
        if (e != hipSuccess) return check_hip(e, "conv3x3 tap_kernel (forward)");
        if (MODE == ADJ) {
            STADE_TIMED("conv_loss", stream, (loss_kernel<1><<<1, NT, 0, stream>>>(ws->partials, (int)nblocks, p.loss, nullptr)));
        } else {
            STADE_TIMED("conv_loss", stream, (loss_kernel<2><<<1, NT, 0, stream>>>(ws->partials, (int)nblocks, p.loss, p.lossd)));
        }
        STADE_LAUNCHED("conv3x3 loss_kernel");
    }
    if (MODE == TAN || d.C == 0) return STADE_HIP_OK;
    // wb += sum xp g;  HVP: wbd += sum (xpd g + xp gd)
    int32_t rc = weight_grad<1>(d, p.xp, G, nullptr, nullptr, part, nsplit, p.wb, "conv_wgrad", stream);
    if (rc) return rc;
    if (MODE == HVP) {
        // both products of wbd through the single-pair kernel, over twice the tiles (holding
        // two pairs' tiles at once spilled registers and ran at 64 TFLOP/s)
        rc = weight_grad<1>(d, p.xpd, G, p.xp, GD, part, nsplit, p.wbd, "conv_wgrad2", stream);
        if (rc) return rc;
    }
    // xpb interior += flipped taps over g;  HVP: xpbd += wd g + w gd
    {
        TapArgs a{};
        a.src[0] = G; a.src[1] = GD;
        a.wt[0] = wg0; a.wt[1] = wg1;
        a.Cin = d.K; a.R = d.C; a.Rpad = d.Cpad; a.N = d.N;
        a.SH = d.H; a.SW = d.W; a.ofs = -1;
        a.H = d.H; a.W = d.W;
        a.o0 = p.xpb; a.o1 = p.xpbd;
        a.OH = d.Hp; a.OW = d.Wp; a.oofs = 1;
        unsigned nblocks = 0;
        hipError_t e = MODE == ADJ ? launch_tap<DG_B>(a, "conv_dgrad", stream, nblocks)
                                   : launch_tap<DG_HV>(a, "conv_dgrad_hv", stream, nblocks);
        if (e != hipSuccess) return check_hip(e, "conv3x3 tap_kernel (xpb)");
    }
    // xpb frame
    {
        BorderArgs b{p.w, p.wd, G, GD, p.xpb, p.xpbd, d.N, d.C, d.K, d.H, d.W};
        const dim3 grid((std::max(d.W + 2, d.H) + BSEG - 1) / BSEG, 4, d.N * ((d.C + BCG - 1) / BCG));
        if (MODE == ADJ) {
            STADE_TIMED("conv_border", stream, (border_kernel<false><<<grid, NT, 0, stream>>>(b)));
        } else {
            STADE_TIMED("conv_border", stream, (border_kernel<true><<<grid, NT, 0, stream>>>(b)));
        }
        STADE_LAUNCHED("conv3x3 border_kernel");
    }
    return STADE_HIP_OK;
}

}  // namespace
}  // namespace stade

using namespace stade;

extern "C" {

int32_t stade_hip_conv3x3_b(float* loss, const float* lossb, const float* xp, float* xpb, const float* w, float* wb,
                            float* out, float* outb, int64_t i_nb, int64_t i_c, int64_t i_k, int64_t i_h, int64_t i_w,
                            hipStream_t stream) {
    Dims d;
    if (int32_t rc = check(i_nb, i_c, i_k, i_h, i_w, "stade_hip_conv3x3_b", d)) return rc;
    Ptrs p{};
    p.loss = loss; p.lossb = (float*)lossb; p.xp = (float*)xp; p.xpb = xpb; p.w = (float*)w; p.wb = wb; p.out = out; p.outb = outb;
    return run<ADJ>(p, d, stream);
}

int32_t stade_hip_conv3x3_d(float* loss, float* lossd, const float* xp, const float* xpd, const float* w, const float* wd,
                            float* out, float* outd, int64_t i_nb, int64_t i_c, int64_t i_k, int64_t i_h, int64_t i_w,
                            hipStream_t stream) {
    Dims d;
    if (int32_t rc = check(i_nb, i_c, i_k, i_h, i_w, "stade_hip_conv3x3_d", d)) return rc;
    Ptrs p{};
    p.loss = loss; p.lossd = lossd; p.xp = (float*)xp; p.xpd = (float*)xpd; p.w = (float*)w; p.wd = (float*)wd;
    p.out = out; p.outd = outd;
    return run<TAN>(p, d, stream);
}

int32_t stade_hip_conv3x3_hv(float* loss, const float* lossb, const float* xp, float* xpb, const float* w, float* wb,
                             float* out, float* outb, int64_t i_nb, int64_t i_c, int64_t i_k, int64_t i_h, int64_t i_w,
                             float* lossd, const float* lossbd, const float* xpd, float* xpbd, const float* wd, float* wbd,
                             float* outd, float* outbd, hipStream_t stream) {
    Dims d;
    if (int32_t rc = check(i_nb, i_c, i_k, i_h, i_w, "stade_hip_conv3x3_hv", d)) return rc;
    Ptrs p{};
    p.loss = loss; p.lossb = (float*)lossb; p.xp = (float*)xp; p.xpb = xpb; p.w = (float*)w; p.wb = wb; p.out = out; p.outb = outb;
    p.lossd = lossd; p.lossbd = (float*)lossbd; p.xpd = (float*)xpd; p.xpbd = xpbd; p.wd = (float*)wd; p.wbd = wbd;
    p.outd = outd; p.outbd = outbd;
    return run<HVP>(p, d, stream);
}

}  // extern "C"
