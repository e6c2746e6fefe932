// mlp2_ce: tangent, adjoint and HVP of a tanh perceptron with a softmax cross-entropy loss
// summed over a mini-batch held inside the launch (fp32).
//
// Generated code this replaces: stade.jl_amd/corpus/mlp2_ce_{b,d,hv}.jl.  Under
// `stade_amdgpu_file` (/root/reference/src/STADE.jl:18604) each (sample, unit) is one thread
// running its 784- or 1024-long dot product alone, and every weight-gradient update
// `w1b[j,k] += x[k,s] * s1b` is an atomic add (`cgen_device_assign` 11941-11969): 4096
// same-address fp32 atomics per weight; the reference's tiled contraction twins
// (`cgen_adjoint_contraction_` 14762) are CUDA-only.
//
// Here the three contractions run on the fp32 matrix cores (gemm_f32.hpp), each with its
// elementwise neighbours fused into the epilogue:
//   S1 = W1 X            epilogue h1 = tanh(S1 + b1)                 (H x B, K = I)
//   head (per sample)    z = W2 h1 + b2, CE, d2 = dloss/dz, zb reset,
//                        d1 = (1 - h1^2) (h1b + W2' d2), h1b reset    (one wave per sample)
//   colsum               W2b += d2 h1', b1b += sum_s d1, b2b         (deterministic partials)
//   W1b += d1 X'  and  Xb += W1' d1                                    (one paired launch:
//                        H x I with K = B, I x B with K = H; the final sums ride along)
// The adjoint (i_h <= 1024) forms head and column sums in one pass over h1 (headd1_kernel);
// the tangent adds S1d = W1d X + W1 Xd (one dual GEMM, epilogue h1d = (1 - h1^2)(S1d + b1d));
// the HVP adds the tangents of every backward product in dual launches.
#include "internal.hpp"

#include <algorithm>
#include "gemm_f32.hpp"
#include "../../include/stade_hip.h"

#include <math.h>

namespace stade {
namespace {

constexpr int NT = 256, OMAX = 16;
enum Mode { ADJ = 0, TAN = 1, HVP = 2 };

// tanh in fp32 from the hardware exp2 and reciprocal, branch-free (the forward epilogues
// apply it to every element of h1).  For |x| >= 0.625 it is 1 - 2 / (e^{2|x|} + 1), with
// e^{2|x|} = 2^{(2 / ln 2) |x|} (infinite above |x| ~ 44, where the result is 1); there the
// subtraction keeps the result at least 0.55, and with a 1-ulp exp2 and reciprocal the error
// stays under 2 ulp.  Below 0.625, where that form cancels, it is x + x^3 P(x^2): P is a
// degree-4 fit of (tanh(x) - x) / x^3 in s = x^2 on [0, 0.625^2], weighted for relative error
// (least squares on Chebyshev nodes with Lawson reweighting), whose fp32 evaluation by FMAs
// is within 0.7 ulp of tanh.  NaN stays NaN, and the sign of zero is kept.
__device__ __forceinline__ float tanh_f32(float x) {
    const float t = fabsf(x);
    const float e = __builtin_amdgcn_exp2f(t * 2.88539008f);
    const float big = 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
    const float s = t * t;
    float p = -0.005704978481f;
    p = fmaf(p, s, 0.02063907869f);
    p = fmaf(p, s, -0.05373971164f);
    p = fmaf(p, s, 0.1333144158f);
    p = fmaf(p, s, -0.3333328068f);
    const float small = fmaf(t * s, p, t);
    return copysignf(t < 0.625f ? small : big, x);
}

// ---------------------------------------------------------------------------------------
// GEMM epilogues (column-major outputs, leading dimension ld)
// ---------------------------------------------------------------------------------------
struct EpiTanh {  // h1 = tanh(s1), s1 = b1 + W1 x
    float* h1;
    const float* b1;
    long ld;
    static constexpr bool kRowLoad = true;
    __device__ float load(int m, int) const { return b1[m]; }
    __device__ void operator()(int m, int n, float v, float b) const { __builtin_nontemporal_store(tanh_f32(v + b), &h1[m + n * ld]); }
};
// dual forward (tangent and HVP): from P = W1 x and Q = W1 xd + W1d x in one launch,
// h1 = tanh(P + b1) and h1d = (1.0 - h1^2) * (Q + b1d)
struct EpiTanhPair {
    float *h1, *h1d;
    const float *b1, *b1d;
    long ld;
    static constexpr bool kRowLoad = true;
    __device__ float2 load(int m, int) const { return make_float2(b1[m], b1d[m]); }
    __device__ void operator()(int m, int n, float p, float q, float2 b) const {
        const float h = tanh_f32(p + b.x);
        __builtin_nontemporal_store(h, &h1[m + n * ld]);
        __builtin_nontemporal_store((1.0f - h * h) * (q + b.y), &h1d[m + n * ld]);
    }
};
// dual accumulation (HVP): C += P, Cd += Q
struct EpiAccPair {
    float *C, *Cd;
    long ld;
    __device__ float2 load(int m, int n) const {
        return make_float2(__builtin_nontemporal_load(&C[m + n * ld]), __builtin_nontemporal_load(&Cd[m + n * ld]));
    }
    __device__ void operator()(int m, int n, float p, float q, float2 c) const {
        __builtin_nontemporal_store(c.x + p, &C[m + n * ld]);
        __builtin_nontemporal_store(c.y + q, &Cd[m + n * ld]);
    }
    static constexpr bool kAtomic = true;
    __device__ void atomic(int m, int n, float p, float q) const {
        unsafeAtomicAdd(&C[m + n * ld], p);
        unsafeAtomicAdd(&Cd[m + n * ld], q);
    }
};
struct EpiAcc {  // C += v (a shadow accumulated, as the generated code does)
    float* C;
    long ld;
    __device__ float load(int m, int n) const { return __builtin_nontemporal_load(&C[m + n * ld]); }
    __device__ void operator()(int m, int n, float v, float c) const { __builtin_nontemporal_store(c + v, &C[m + n * ld]); }
    static constexpr bool kAtomic = true;
    __device__ void atomic(int m, int n, float v) const { unsafeAtomicAdd(&C[m + n * ld], v); }
};

// ---------------------------------------------------------------------------------------
// head: one wave per sample, 512-thread blocks.  With LDSW (the adjoint, i_h <= HLDS) the block first
// copies W2 (and W2d) into LDS as [j][o] rows padded to OP = 17 floats: a lane's reads of
// its columns j = lane + 64 q are one base register plus immediate offsets, and the odd row
// stride keeps the 64 lanes on distinct banks.  Without it the weights are read from global
// memory.
// ---------------------------------------------------------------------------------------
constexpr int HNT = 512, OP = OMAX + 1, HLDS = 1024;

struct HeadArgs {
    const float *h1, *w2, *b2, *lossb;
    float *z, *zb, *h1b, *D1, *D2;
    const float *h1d, *w2d, *b2d, *lossbd;
    float *zd, *zbd, *h1bd, *D1d, *D2d;
    const int64_t* lab;
    int B, H, O;
    double* partials;  // per block: loss, lossd
    int* err;          // set when a label is outside 1..O
};

template <int MODE, int HPL, bool LDSW>
__global__ __launch_bounds__(HNT) void head_kernel(HeadArgs a) {
    constexpr int NWS = LDSW ? (MODE == ADJ ? 1 : 2) : 0;
    __shared__ double red[16 * 2];
    __shared__ float w2s[NWS ? NWS * HLDS * OP : 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = a.H, O = a.O;
    if constexpr (LDSW) {
        // CB loads in flight per thread, then their LDS stores (a load-store loop would wait
        // out one global-memory round trip per element)
        constexpr int CB = 8;
        for (int q0 = 0; q0 < O * H; q0 += HNT * CB) {
            float v[CB], vd[CB];
#pragma unroll
            for (int c = 0; c < CB; ++c) {
                const int q = q0 + c * HNT + threadIdx.x;
                v[c] = q < O * H ? a.w2[q] : 0.f;
                vd[c] = (MODE != ADJ && q < O * H) ? a.w2d[q] : 0.f;
            }
#pragma unroll
            for (int c = 0; c < CB; ++c) {
                const int q = q0 + c * HNT + threadIdx.x;
                if (q < O * H) {
                    const int j = q / O, o = q - j * O;
                    w2s[j * OP + o] = v[c];
                    if (MODE != ADJ) w2s[HLDS * OP + j * OP + o] = vd[c];
                }
            }
        }
        __syncthreads();
    }
    // W2(o, j), W2d(o, j)
    auto W2 = [&](int o, int j) { return LDSW ? w2s[j * OP + o] : a.w2[(long)j * O + o]; };
    auto W2d = [&](int o, int j) { return LDSW ? w2s[(NWS - 1) * HLDS * OP + j * OP + o] : a.w2d[(long)j * O + o]; };
    double acc[2];  // loss, lossd
#pragma unroll
    for (int k = 0; k < 2; ++k) acc[k] = 0.0;
    const float lb = (MODE == TAN) ? 0.f : a.lossb[0];
    const float lbd = (MODE == HVP) ? a.lossbd[0] : 0.f;
    for (int s = blockIdx.x * (HNT / 64) + wave; s < a.B; s += gridDim.x * (HNT / 64)) {
        const long hs = (long)s * H, os = (long)s * O;
        // every global read of the sample first: h1 (+ h1d), then h1b (+ h1bd), zb (+ zbd) and
        // the label, so one memory round trip covers them
        float hj[HPL], hdj[HPL], hbj[HPL], hbdj[HPL];
#pragma unroll
        for (int q = 0; q < HPL; ++q) {
            const int j = lane + 64 * q;
            hj[q] = j < H ? a.h1[hs + j] : 0.f;
            hdj[q] = (MODE != ADJ && j < H) ? a.h1d[hs + j] : 0.f;
        }
#pragma unroll
        for (int q = 0; q < HPL; ++q) {
            const int j = lane + 64 * q;
            hbj[q] = (MODE != TAN && j < H) ? a.h1b[hs + j] : 0.f;
            hbdj[q] = (MODE == HVP && j < H) ? a.h1bd[hs + j] : 0.f;
        }
        const float zb_l = (MODE != TAN && lane < O) ? a.zb[os + lane] : 0.f;
        const float zbd_l = (MODE == HVP && lane < O) ? a.zbd[os + lane] : 0.f;
        const int64_t lab_s = a.lab[s];
        // z = b2 + W2 h1 (and zd = b2d + W2d h1 + W2 h1d)
        float z[OMAX], zd[OMAX];
#pragma unroll
        for (int o = 0; o < OMAX; ++o) z[o] = zd[o] = 0.f;
#pragma unroll
        for (int q = 0; q < HPL; ++q) {
            const int j = lane + 64 * q;
            if (j >= H) continue;
#pragma unroll
            for (int o = 0; o < OMAX; ++o) {
                if (o < O) {
                    const float w = W2(o, j);
                    z[o] += w * hj[q];
                    if (MODE != ADJ) zd[o] += hj[q] * W2d(o, j) + w * hdj[q];
                }
            }
            // one column block's weights live at a time (the scheduler would otherwise hoist
            // every LDS read of the loop and spill)
            if constexpr (LDSW) asm volatile("" ::: "memory");
        }
#pragma unroll
        for (int o = 0; o < OMAX; ++o) {
            if (o < O) {
                z[o] = a.b2[o] + wave_sum(z[o]);
                if (MODE != ADJ) zd[o] = a.b2d[o] + wave_sum(zd[o]);
            }
        }
        // softmax cross-entropy: loss += log(se) - z[l]
        float se = 0.f, sed = 0.f, e[OMAX];
#pragma unroll
        for (int o = 0; o < OMAX; ++o) {
            if (o < O) {
                e[o] = expf(z[o]);
                if (MODE != ADJ) sed = sed + e[o] * zd[o];
                se = se + e[o];
            }
        }
        int l = (int)lab_s - 1;
        if (l < 0 || l >= O) {
            if (lane == 0) atomicOr(a.err, kErrIndex);
            l = -1;
        }
        float zl = 0.f, zdl = 0.f;
#pragma unroll
        for (int o = 0; o < OMAX; ++o)
            if (o == l) {
                zl = z[o];
                zdl = zd[o];
            }
        if (lane == 0 && l >= 0) {
            acc[0] += (double)(logf(se) - zl);
            if (MODE != ADJ) acc[1] += (double)((1.0f / se) * sed + -zdl);
        }
        if (MODE != ADJ && lane < O) {
#pragma unroll
            for (int o = 0; o < OMAX; ++o)
                if (o == lane) a.zd[os + o] = zd[o];
        }
        if (lane < O) {
#pragma unroll
            for (int o = 0; o < OMAX; ++o)
                if (o == lane) a.z[os + o] = z[o];
        }
        if (MODE == TAN) continue;
        // reverse of the loss: d2 = zb + [o == l](-lb) + exp(z) seb, seb = (1 / se) lb
        const float seb = (1.0f / se) * lb;
        const float sebd = (MODE == HVP) ? (lb * (-(1.0f / (se * se)) * sed) + (1.0f / se) * lbd) : 0.f;
        float d2[OMAX], d2d[OMAX];
#pragma unroll
        for (int o = 0; o < OMAX; ++o) {
            d2[o] = d2d[o] = 0.f;
            if (o < O) {
                float t = __shfl(zb_l, o, 64);
                if (o == l) t = t + -lb;
                d2[o] = t + e[o] * seb;
                if (MODE == HVP) {
                    float td = __shfl(zbd_l, o, 64);
                    if (o == l) td = td + -lbd;
                    d2d[o] = td + (seb * (e[o] * zd[o]) + e[o] * sebd);
                }
            }
        }
        if (lane < O) {
#pragma unroll
            for (int o = 0; o < OMAX; ++o)
                if (o == lane) {
                    a.zb[os + o] = 0.f;
                    a.D2[os + o] = d2[o];
                    if (MODE == HVP) {
                        a.zbd[os + o] = 0.f;
                        a.D2d[os + o] = d2d[o];
                    }
                }
        }
        // d1 = (1 - h1^2) * (h1b + sum_o w2[o, j] d2[o]), o descending as the generated loop
#pragma unroll
        for (int q = 0; q < HPL; ++q) {
            const int j = lane + 64 * q;
            if (j >= H) continue;
            float t = hbj[q];
            float td = hbdj[q];
#pragma unroll
            for (int o = OMAX - 1; o >= 0; --o) {
                if (o < O) {
                    const float w = W2(o, j);
                    if (MODE == HVP) td = td + (d2[o] * W2d(o, j) + w * d2d[o]);
                    t = t + w * d2[o];
                }
            }
            if constexpr (LDSW) asm volatile("" ::: "memory");
            const float h = hj[q];
            const float g = 1.0f - h * h;
            a.h1b[hs + j] = 0.f;
            a.D1[hs + j] = g * t;
            if (MODE == HVP) {
                a.h1bd[hs + j] = 0.f;
                a.D1d[hs + j] = t * -((2.0f * h) * hdj[q]) + g * td;
            }
        }
    }
    // block partials: loss, lossd
    block_partials<2>(acc, red, a.partials);
}

// ---------------------------------------------------------------------------------------
// head, split form (i_h <= 1024, the form the launcher uses there), first half: z = W2 h1 + b2,
// the cross-entropy, d2 = dloss/dz and the zb reset, per sample; the second half (D1, h1b
// reset) is fused with the column sums in d1sum_kernel.  A 256-thread block stages W2 (+ W2d)
// in LDS once as [j][o] rows of OP floats, zero-padded to OMAX outputs and 64 * HPL columns;
// each wave takes SPW samples at a time with their reads of h1 (+ h1d) issued together, and
// one LDS read of a weight serves the SPW samples.  Padded outputs carry zeros, so the o loops
// have no branches.  Per sample the arithmetic is that of head_kernel, in the same order.
// ---------------------------------------------------------------------------------------
// threads of a head4 block: the adjoint's 4 waves (its per-wave LDS transpose arrays fill the
// rest of the LDS), the tangent's and HVP's 8 (two waves per SIMD beside the staged weights)
template <int MODE>
constexpr int h4nt() {
    return MODE == 0 ? 256 : 512;
}
constexpr int SC = 128;  // samples per chunk of the column sums

// sum over the 16 lanes of a DPP row (every lane of the row gets it)
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f32<kDppQuadSwap1>(v);
    v += dpp_f32<kDppQuadSwap2>(v);
    v += dpp_f32<kDppRowRor4>(v);
    v += dpp_f32<kDppRowRor8>(v);
    return v;
}

template <int MODE, int HPL, int SPW>
__global__ __launch_bounds__(h4nt<MODE>()) void head4_kernel(HeadArgs a) {
    constexpr int H4NT = h4nt<MODE>();
    constexpr int NW = MODE == ADJ ? 1 : 2;
    constexpr int JR = 64 * HPL;
    // the adjoint reduces its lane partial sums through LDS: per wave a [64][ZW] array
    constexpr int ZW = SPW * OMAX + 4;
    static_assert(MODE != ADJ || SPW * OMAX <= 64, "one lane per (sample, output) of a wave");
    __shared__ float w2s[NW * JR * OP];
    __shared__ float zt[MODE == ADJ ? (H4NT / 64) * 64 * ZW : 1];
    __shared__ double red[16 * 2];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = a.H, O = a.O, B = a.B;
    {
        // LDS row j, entry o: W2[o, j] for j < H and o < O, zero elsewhere; a thread takes whole
        // rows j = threadIdx.x + H4NT c with every load in flight at once (no index division,
        // and the padding is written with the data)
        constexpr int RPT = (JR + H4NT - 1) / H4NT;  // (threads past row JR - 1 load and store nothing new)
        float v[RPT][OMAX], vd[RPT][OMAX];
#pragma unroll
        for (int c = 0; c < RPT; ++c) {
            const int j = threadIdx.x + H4NT * c;
#pragma unroll
            for (int o = 0; o < OMAX; ++o) {
                // clamped, unconditional loads (a load under a branch makes the compiler wait
                // for every load in flight); the padding is applied after all are issued
                const long q = (long)min(j, H - 1) * O + min(o, O - 1);
                v[c][o] = a.w2[q];
                vd[c][o] = MODE != ADJ ? a.w2d[q] : 0.f;
            }
        }
        // keep every load above the first use (the scheduler would otherwise place each select
        // right after its load and wait for it)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < RPT; ++c) {
            const int j = threadIdx.x + H4NT * c;
            if (JR % H4NT != 0 && j >= JR) continue;
#pragma unroll
            for (int o = 0; o < OMAX; ++o) {
                const bool in = j < H && o < O;
                w2s[j * OP + o] = in ? v[c][o] : 0.f;
                if (MODE != ADJ) w2s[JR * OP + j * OP + o] = in ? vd[c][o] : 0.f;
            }
        }
    }
    const float lb = (MODE == TAN) ? 0.f : a.lossb[0];
    const float lbd = (MODE == HVP) ? a.lossbd[0] : 0.f;
    double acc[2] = {0.0, 0.0};  // loss, lossd
    __syncthreads();
    const float* W2s = w2s;
    const float* W2ds = w2s + (NW - 1) * JR * OP;
    const int nw = gridDim.x * (H4NT / 64);
    for (int s0 = (blockIdx.x * (H4NT / 64) + wave) * SPW; s0 < B; s0 += nw * SPW) {
        // every global read of the SPW samples first (a sample past B re-reads sample B-1)
        float h[SPW][HPL], hd[SPW][HPL];
        float zb_l[SPW], zbd_l[SPW];
        int64_t lab[SPW];
#pragma unroll
        for (int i = 0; i < SPW; ++i) {
            const int s = min(s0 + i, B - 1);
            const long hs = (long)s * H, os = (long)s * O;
#pragma unroll
            for (int q = 0; q < HPL; ++q) {
                const int jc = min(lane + 64 * q, H - 1);
                h[i][q] = a.h1[hs + jc];
                if (MODE != ADJ) hd[i][q] = a.h1d[hs + jc];
            }
            if (MODE != ADJ) {
                const int oc = min(lane, O - 1);
                zb_l[i] = (MODE != TAN) ? a.zb[os + oc] : 0.f;
                zbd_l[i] = (MODE == HVP) ? a.zbd[os + oc] : 0.f;
                lab[i] = a.lab[s];
            }
        }
        // the adjoint's lane L = 16 i + o: sample s0 + i, output o
        const int li = lane >> 4, lo = lane & (OMAX - 1);
        const int ls = min(s0 + li, B - 1);
        const float zb_lane = (MODE == ADJ) ? a.zb[(long)ls * O + min(lo, O - 1)] : 0.f;
        const float b2_lane = (MODE == ADJ) ? a.b2[min(lo, O - 1)] : 0.f;
        const int64_t lab_lane = (MODE == ADJ) ? a.lab[ls] : 0;
        // every read above stays ahead of the first use; columns past H then contribute zero
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < SPW; ++i)
#pragma unroll
            for (int q = 0; q < HPL; ++q) {
                const bool in = lane + 64 * q < H;
                h[i][q] = in ? h[i][q] : 0.f;
                if (MODE != ADJ) hd[i][q] = in ? hd[i][q] : 0.f;
            }
        // z = b2 + W2 h1 (zd = b2d + W2d h1 + W2 h1d): lane partial sums over its columns
        float z[SPW][OMAX], zd[SPW][OMAX];
#pragma unroll
        for (int i = 0; i < SPW; ++i)
#pragma unroll
            for (int o = 0; o < OMAX; ++o) z[i][o] = zd[i][o] = 0.f;
#pragma unroll
        for (int q = 0; q < HPL; ++q) {
            // the column's weights (and their tangents) read together, then used: one LDS
            // latency per column block (with one wave per SIMD nothing else hides it)
            const int row = (lane + 64 * q) * OP;
            float wq[OMAX], wdq[OMAX];
#pragma unroll
            for (int o = 0; o < OMAX; ++o) {
                wq[o] = W2s[row + o];
                wdq[o] = (MODE != ADJ) ? W2ds[row + o] : 0.f;
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int o = 0; o < OMAX; ++o) {
#pragma unroll
                for (int i = 0; i < SPW; ++i) {
                    z[i][o] = fmaf(wq[o], h[i][q], z[i][o]);
                    if (MODE != ADJ) zd[i][o] = fmaf(wq[o], hd[i][q], fmaf(h[i][q], wdq[o], zd[i][o]));
                }
            }
            // one column block's weights live at a time (the scheduler would otherwise hoist
            // every LDS read of the loop)
            asm volatile("" ::: "memory");
        }
        if constexpr (MODE == ADJ) {
            // lane l writes its partial sums as row l of the wave's array; lane L = 16 i + o then
            // adds column L over the 64 rows in lane order (a wave's LDS operations complete in
            // issue order, so no barrier is needed between the writes and the reads)
            float* zw = zt + (threadIdx.x >> 6) * 64 * ZW;
#pragma unroll
            for (int i = 0; i < SPW; ++i)
#pragma unroll
                for (int o = 0; o < OMAX; o += 4)
                    *reinterpret_cast<float4*>(zw + lane * ZW + i * OMAX + o) =
                        make_float4(z[i][o], z[i][o + 1], z[i][o + 2], z[i][o + 3]);
            float zs = 0.f;
            const int col = min(lane, SPW * OMAX - 1);
#pragma unroll 16
            for (int r = 0; r < 64; ++r) zs += zw[r * ZW + col];
            asm volatile("" ::: "memory");
            // softmax cross-entropy of sample s0 + li, output lo, over the lanes of its DPP row
            const bool live = li < SPW && s0 + li < B, vo = lo < O;
            const long os = (long)ls * O;
            const float zv = vo ? b2_lane + zs : 0.f;
            const float e = vo ? expf(zv) : 0.f;
            const float se = row16_sum(e);
            const int l = (int)lab_lane - 1;
            const bool lok = l >= 0 && l < O;
            if (live && lo == 0 && !lok) atomicOr(a.err, kErrIndex);
            if (live && lok && lo == l) acc[0] += (double)(logf(se) - zv);
            // reverse of the loss: d2 = zb + [o == l](-lb) + exp(z) seb, seb = (1 / se) lb
            const float seb = (1.0f / se) * lb;
            float t = zb_lane;
            if (lo == l) t = t + -lb;
            const float d2 = t + e * seb;
            if (live && vo) {
                a.z[os + lo] = zv;
                a.zb[os + lo] = 0.f;
                a.D2[os + lo] = d2;
            }
            continue;
        }
#pragma unroll
        for (int i = 0; i < SPW; ++i) {
            const int s = s0 + i;
            const bool live = s < B;  // uniform over the wave
            const long os = (long)min(s, B - 1) * O;
#pragma unroll
            for (int o = 0; o < OMAX; ++o) {
                if (o < O) {
                    z[i][o] = a.b2[o] + wave_sum(z[i][o]);
                    if (MODE != ADJ) zd[i][o] = a.b2d[o] + wave_sum(zd[i][o]);
                }
            }
            // softmax cross-entropy: loss += log(se) - z[l]
            float se = 0.f, sed = 0.f, e[OMAX];
#pragma unroll
            for (int o = 0; o < OMAX; ++o) {
                e[o] = 0.f;
                if (o < O) {
                    e[o] = expf(z[i][o]);
                    if (MODE != ADJ) sed = sed + e[o] * zd[i][o];
                    se = se + e[o];
                }
            }
            int l = (int)lab[i] - 1;
            if (l < 0 || l >= O) {
                if (live && lane == 0) atomicOr(a.err, kErrIndex);
                l = -1;
            }
            float zl = 0.f, zdl = 0.f, zo = 0.f, zdo = 0.f;
#pragma unroll
            for (int o = 0; o < OMAX; ++o) {
                if (o == l) {
                    zl = z[i][o];
                    zdl = zd[i][o];
                }
                if (o == lane) {
                    zo = z[i][o];
                    zdo = zd[i][o];
                }
            }
            if (live && lane == 0 && l >= 0) {
                acc[0] += (double)(logf(se) - zl);
                if (MODE != ADJ) acc[1] += (double)((1.0f / se) * sed + -zdl);
            }
            if (live && lane < O) {
                if (MODE != ADJ) a.zd[os + lane] = zdo;
                a.z[os + lane] = zo;
            }
            if (MODE == TAN) continue;
            // reverse of the loss: d2 = zb + [o == l](-lb) + exp(z) seb, seb = (1 / se) lb
            const float seb = (1.0f / se) * lb;
            const float sebd = (MODE == HVP) ? (lb * (-(1.0f / (se * se)) * sed) + (1.0f / se) * lbd) : 0.f;
            float d2o = 0.f, d2do = 0.f;
#pragma unroll
            for (int o = 0; o < OMAX; ++o) {
                if (o < O) {
                    float t = __shfl(zb_l[i], o, 64);
                    if (o == l) t = t + -lb;
                    const float d2 = t + e[o] * seb;
                    float d2d = 0.f;
                    if (MODE == HVP) {
                        float td = __shfl(zbd_l[i], o, 64);
                        if (o == l) td = td + -lbd;
                        d2d = td + (seb * (e[o] * zd[i][o]) + e[o] * sebd);
                    }
                    if (o == lane) {
                        d2o = d2;
                        d2do = d2d;
                    }
                }
            }
            if (live && lane < O) {
                a.zb[os + lane] = 0.f;
                a.D2[os + lane] = d2o;
                if (MODE == HVP) {
                    a.zbd[os + lane] = 0.f;
                    a.D2d[os + lane] = d2do;
                }
            }
        }
    }
    block_partials<2>(acc, red, a.partials);
}

// ---------------------------------------------------------------------------------------
// The adjoint's whole head in one pass over h1 (i_h <= 1024): a block of HDB = 16 waves
// takes 16 consecutive samples.
//  A. Wave w, sample s0 + w: lane l loads h1 of its columns j = l + 64 q; W2 is staged in LDS
//     as rows [j][opl] (opl = i_out rounded up to odd: conflict-free row reads; zero past i_out
//     and i_h).  z = b2 + W2 h1: the lane's 16 output partial sums are reduced across the
//     wave by a reduce-scatter butterfly (xor shuffles 8, 4, 2, 1 within each 16-lane row, each
//     halving the values a lane holds, then 16 and 32), after which lane l holds z of output
//     l & 15.  Softmax cross-entropy, d2 = dloss/dz and the zb reset as in head4_kernel.  d2
//     and the sample's h1 go to LDS.
//  B. Thread t owns column j = t: for the block's samples in order,
//     d1 = (1 - h1^2) (h1b + sum_o w2[o, j] d2[o]) (o descending, as the generated loop),
//     the h1b reset, and the column's sums of W2b += d2 h1' and b1b, written as the block's
//     partials in d1sum_kernel's layout (the block is the chunk); b2b and the loss likewise.
// h1 and h1b are read once, D1 and the h1b reset written once (the split form read h1 twice,
// in two launches), with four waves per SIMD.  Every sum has a fixed order.
// ---------------------------------------------------------------------------------------
// (the arguments of the column-sum kernels: d1sum_kernel, and headd1_kernel's step B)
struct D1Args {
    const float *h1, *h1b_in, *w2, *D2, *h1d, *w2d, *D2d;
    float *h1b, *D1, *h1bd, *D1d;
    float* part;   // [chunk][2 * (O + 1)][H]
    float* part2;  // [chunk][2 * OMAX]
    int B, H, O;
};

constexpr int HDB = 16, HDNT = 64 * HDB;

__host__ __device__ constexpr int hd_opl(int O) { return O | 1; }

// LDS of headd1_kernel, in floats: red (32 doubles), W2 rows [JR][opl], d2 [HDB][OMAX],
// h1 [HDB][JR]
__host__ __device__ constexpr int hd_lds_floats(int JR, int O) {
    return 64 + JR * hd_opl(O) + HDB * OMAX + HDB * JR;
}

// A block barrier that waits only for the wave's LDS operations: __syncthreads() also waits
// for every global load in flight, which would expose the step-B loads issued at the start.
#ifndef STADE_HD_RAW_BARRIER
#define STADE_HD_RAW_BARRIER 1
#endif
__device__ __forceinline__ void lds_barrier() {
#if STADE_HD_RAW_BARRIER
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt not waited for
    __builtin_amdgcn_s_barrier();
#else
    __syncthreads();
#endif
}

template <int HPL, int OM>
__global__ __launch_bounds__(HDNT) void headd1_kernel(HeadArgs a, D1Args c) {
    static_assert(OM <= OMAX, "output slots");
    constexpr int JR = 64 * HPL;
    static_assert(JR <= HDNT, "a column per thread in step B");
    // (static, sized for i_out = OMAX)
    __shared__ float hd_smem[hd_lds_floats(JR, OMAX)];
    const int H = a.H, O = a.O, B = a.B;
    constexpr int opl = hd_opl(OM);  // (i_out <= OM: rows of OM outputs, zero past i_out)
    double* red = reinterpret_cast<double*>(hd_smem);
    float* w2s = hd_smem + 64;
    float* d2s = w2s + JR * opl;
    float* hs = d2s + HDB * OMAX;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sb0 = blockIdx.x * HDB, s = sb0 + wave;
    const bool live = s < B;
    const int sc = min(s, B - 1);
    // every global read first, in the order of use (loads complete in order): W2 (row
    // j = threadIdx.x), the sample's h1 and the lane values (step A), then h1b of column j for
    // the block's samples (step B), still in flight through step A (the barriers wait for
    // LDS operations only)
    const int j = threadIdx.x;
    const int jc = min(j, H - 1);
    float w2v[opl];
#pragma unroll
    for (int o = 0; o < opl; ++o) w2v[o] = a.w2[(long)jc * O + min(o, O - 1)];
    // (row pointers are wave-uniform and column offsets 32-bit: scalar-base addressing)
    const float* hrow = a.h1 + (long)sc * H;
    float h[HPL];
#pragma unroll
    for (int q = 0; q < HPL; ++q) h[q] = hrow[min(lane + 64 * q, H - 1)];
    const int lo = lane & (OMAX - 1);
    const float zb_lane = a.zb[(long)sc * O + min(lo, O - 1)];
    const float b2_lane = a.b2[min(lo, O - 1)];
    const int64_t lab_s = a.lab[sc];
    const float lb = a.lossb[0];
    float hbv[HDB];
#pragma unroll
    for (int k = 0; k < HDB; ++k) hbv[k] = __builtin_nontemporal_load(&(a.h1b + (long)min(sb0 + k, B - 1) * H)[jc]);
    __builtin_amdgcn_sched_barrier(0);
    if (j < JR) {
#pragma unroll
        for (int o = 0; o < opl; ++o) w2s[j * opl + o] = (j < H && o < O) ? w2v[o] : 0.f;
    }
    lds_barrier();
    // columns past i_h contribute nothing (a dead sample's values are never stored or used)
#pragma unroll
    for (int q = 0; q < HPL; ++q) h[q] = lane + 64 * q < H ? h[q] : 0.f;
    float v[OMAX];
#pragma unroll
    for (int o = 0; o < OMAX; ++o) v[o] = 0.f;
#pragma unroll
    for (int q = 0; q < HPL; ++q) {
        const int row = (lane + 64 * q) * opl;
        float wq[OM];
#pragma unroll
        for (int o = 0; o < OM; ++o) wq[o] = w2s[row + o];
#pragma unroll
        for (int o = 0; o < OM; ++o) v[o] = fmaf(wq[o], h[q], v[o]);
    }
    // reduce-scatter within the 16-lane rows, then across them: lane l ends with output l & 15
#pragma unroll
    for (int half = 8; half >= 1; half >>= 1) {
        // keep / send by a bit select on the values (a select on the array index would make
        // the compiler index the register array dynamically: a compare and select chain)
        const int m = (lane & half) ? -1 : 0;
#pragma unroll
        for (int p = 0; p < half; ++p) {
            const int lo_ = __float_as_int(v[p]), hi_ = __float_as_int(v[p + half]);
            const float keep = __int_as_float((hi_ & m) | (lo_ & ~m));
            const float send = __int_as_float((lo_ & m) | (hi_ & ~m));
            v[p] = keep + __shfl_xor(send, half, 64);
        }
    }
    v[0] += __shfl_xor(v[0], 16, 64);
    v[0] += __shfl_xor(v[0], 32, 64);
    // softmax cross-entropy of the sample over the lanes of a DPP row (every row the same)
    double acc[2] = {0.0, 0.0};
    {
        const bool vo = lo < O;
        const long os = (long)sc * O;
        const float zv = vo ? b2_lane + v[0] : 0.f;
        const float e = vo ? expf(zv) : 0.f;
        const float se = row16_sum(e);
        const int l = (int)lab_s - 1;
        const bool lok = l >= 0 && l < O;
        if (live && lane == 0 && !lok) atomicOr(a.err, kErrIndex);
        if (live && lok && lane == l) acc[0] += (double)(logf(se) - zv);
        // reverse of the loss: d2 = zb + [o == l](-lb) + exp(z) seb, seb = (1 / se) lb
        const float seb = (1.0f / se) * lb;
        float t = zb_lane;
        if (lo == l) t = t + -lb;
        const float d2 = t + e * seb;
        if (live && lane < O) {
            a.z[os + lane] = zv;
            a.zb[os + lane] = 0.f;
        }
        if (lane < OMAX) d2s[wave * OMAX + lane] = (live && vo) ? d2 : 0.f;
    }
#pragma unroll
    for (int q = 0; q < HPL; ++q) hs[wave * JR + lane + 64 * q] = h[q];
    lds_barrier();
    // step B: column j over the block's samples
    const int ns = min(HDB, B - sb0);
    if (j < JR) {
        float wc[OM];
#pragma unroll
        for (int o = 0; o < OM; ++o) wc[o] = w2s[j * opl + o];
        float w2acc[OM];
#pragma unroll
        for (int o = 0; o < OM; ++o) w2acc[o] = 0.f;
        float b1acc = 0.f;
#pragma unroll
        for (int k = 0; k < HDB; ++k) {
            if (k >= ns) continue;  // a guard, not an exit: the loop unrolls
            const float hv = hs[k * JR + j];
            const float* d2 = d2s + k * OMAX;
            float t = hbv[k];
#pragma unroll
            for (int o = OM - 1; o >= 0; --o) t = t + wc[o] * d2[o];
            const float d1 = (1.0f - hv * hv) * t;
            if (j < H) {
                const long r0 = (long)(sb0 + k) * H;
                __builtin_nontemporal_store(0.f, &(a.h1b + r0)[j]);
                (a.D1 + r0)[j] = d1;
            }
            // (a sum over the block's samples, in a different order from the generated loop's
            // anyway: fused multiply-adds)
#pragma unroll
            for (int o = 0; o < OM; ++o) w2acc[o] = fmaf(hv, d2[o], w2acc[o]);
            b1acc += d1;
        }
        if (j < H) {
            float* p = c.part + (long)blockIdx.x * 2 * (O + 1) * H;
#pragma unroll
            for (int o = 0; o < OM; ++o)
                if (o < O) p[(long)o * H + j] = w2acc[o];
            p[(long)O * H + j] = b1acc;
        }
    }
    if (threadIdx.x < OMAX) {
        double t = 0.0;
        for (int k = 0; k < HDB; ++k) t += (double)d2s[k * OMAX + threadIdx.x];
        c.part2[(long)blockIdx.x * 2 * OMAX + threadIdx.x] = threadIdx.x < O ? (float)t : 0.f;
    }
    block_partials<2>(acc, red, a.partials);
}

// ---------------------------------------------------------------------------------------
// second half of the split head fused with the column sums (i_h <= 1024): per chunk of SC
// samples and 64 columns j,
//   d1 = (1 - h1^2) (h1b + sum_o w2[o, j] d2[o]) (o descending, as the generated loop), h1b = 0
//   (HVP: d1d, h1bd = 0), and the chunk partials of W2b += d2 h1', b1b += sum_s d1 (+ W2bd,
//   b1bd) and of b2b (+ b2bd), in colsum_kernel's layout and summation order.
// A thread owns column j (its W2 column in registers) and the samples s0 + sl + 4 k.
// ---------------------------------------------------------------------------------------
template <int MODE>
__global__ __launch_bounds__(NT) void d1sum_kernel(D1Args a) {
    constexpr int NR = 2 * (OMAX + 1);
    constexpr bool HV = MODE == HVP;
    __shared__ float d2s[SC * OMAX];               // [s][o], zero past O
    __shared__ float d2ds[HV ? SC * OMAX : 1];
    __shared__ float red[4][NR][64];
    const int jl = threadIdx.x & 63, sl = threadIdx.x >> 6;
    const int j = blockIdx.x * 64 + jl, c = blockIdx.y;
    const int s0 = c * SC, s1 = min(a.B, s0 + SC), O = a.O, H = a.H;
    const int jc = min(j, H - 1);
    {
        constexpr int CB = SC * OMAX / NT;
        float v[CB], vd[CB];
#pragma unroll
        for (int k = 0; k < CB; ++k) {
            // clamped, unconditional loads; the zero padding is applied after all are issued
            const int q = k * NT + threadIdx.x;
            const int ss = q / OMAX, o = q % OMAX;
            const long qi = (long)min(s0 + ss, s1 - 1) * O + min(o, O - 1);
            v[k] = a.D2[qi];
            vd[k] = HV ? a.D2d[qi] : 0.f;
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < CB; ++k) {
            const int q = k * NT + threadIdx.x;
            const bool in = s0 + q / OMAX < s1 && q % OMAX < O;
            d2s[k * NT + threadIdx.x] = in ? v[k] : 0.f;
            if (HV) d2ds[k * NT + threadIdx.x] = in ? vd[k] : 0.f;
        }
    }
    float w[OMAX], wd[OMAX];
#pragma unroll
    for (int o = 0; o < OMAX; ++o) {
        // clamped, unconditional loads (see head4_kernel); the padding is applied below
        const long q = (long)jc * O + min(o, O - 1);
        w[o] = a.w2[q];
        wd[o] = HV ? a.w2d[q] : 0.f;
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int o = 0; o < OMAX; ++o) {
        const bool in = j < H && o < O;
        w[o] = in ? w[o] : 0.f;
        wd[o] = in ? wd[o] : 0.f;
    }
    __syncthreads();
    // b2b (+ b2bd) partials of the chunk: the column-independent sums of d2 over samples
    if (blockIdx.x == 0 && threadIdx.x < 2 * OMAX) {
        const int o = threadIdx.x % OMAX;
        const bool dd = threadIdx.x >= OMAX;
        double t = 0.0;
        if (o < O && (!dd || HV))
            for (int q = 0; q < s1 - s0; ++q) t += (double)(dd ? d2ds[q * OMAX + o] : d2s[q * OMAX + o]);
        a.part2[(long)c * 2 * OMAX + threadIdx.x] = (float)t;
    }
    float wacc[OMAX], wdacc[OMAX], bsum = 0.f, bsumd = 0.f;
#pragma unroll
    for (int o = 0; o < OMAX; ++o) wacc[o] = wdacc[o] = 0.f;
    // the wave's samples s0 + sl, s0 + sl + 4, ... in batches of SB: every load of a batch
    // (clamped, unconditional) issued before the batch's first store, since h1b (h1bd) is
    // reset in place and the compiler must otherwise keep each load behind the previous store
    constexpr int SB = HV ? 8 : 16;
    for (int sb = s0 + sl; sb < s1; sb += 4 * SB) {
    float hv_[SB], hbv_[SB], hdv_[SB], hbdv_[SB];
#pragma unroll
    for (int u = 0; u < SB; ++u) {
        const long k = (long)min(sb + 4 * u, s1 - 1) * H + jc;
        hv_[u] = a.h1[k];
        hbv_[u] = __builtin_nontemporal_load(&a.h1b_in[k]);
        hdv_[u] = HV ? a.h1d[k] : 0.f;
        hbdv_[u] = HV ? __builtin_nontemporal_load(&a.h1bd[k]) : 0.f;
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < SB; ++u) {
        const int s = sb + 4 * u;
        if (s >= s1) continue;  // a guard, not an exit: the loop unrolls
        const long k = (long)s * H + jc;
        const float h = hv_[u];
        const float hb = hbv_[u];
        const float hd = hdv_[u];
        const float hbd = hbdv_[u];
        const float* d2 = d2s + (s - s0) * OMAX;
        const float* d2d = d2ds + (HV ? (s - s0) * OMAX : 0);
        float t = hb, td = hbd;
#pragma unroll
        for (int o = OMAX - 1; o >= 0; --o) {
            if (HV) td = td + (d2[o] * wd[o] + w[o] * d2d[o]);
            t = t + w[o] * d2[o];
        }
        const float g = 1.0f - h * h;
        const float d1 = g * t;
        const float d1d = HV ? t * -((2.0f * h) * hd) + g * td : 0.f;
        if (j < H) {
            __builtin_nontemporal_store(0.f, &a.h1b[k]);
            a.D1[k] = d1;
            if (HV) {
                __builtin_nontemporal_store(0.f, &a.h1bd[k]);
                a.D1d[k] = d1d;
            }
        }
#pragma unroll
        for (int o = 0; o < OMAX; ++o) {
            wacc[o] += h * d2[o];
            if (HV) wdacc[o] += d2[o] * hd + h * d2d[o];
        }
        bsum += d1;
        if (HV) bsumd += d1d;
    }
    }
#pragma unroll
    for (int o = 0; o < OMAX; ++o) {
        red[sl][o][jl] = wacc[o];
        red[sl][OMAX + 1 + o][jl] = wdacc[o];
    }
    red[sl][OMAX][jl] = bsum;
    red[sl][2 * OMAX + 1][jl] = bsumd;
    __syncthreads();
    if (j >= H) return;
    float* p = a.part + (long)c * 2 * (O + 1) * H;
    for (int r = sl; r < 2 * (O + 1); r += 4) {
        if (!HV && r > O) break;
        const int src = r < O ? r : (r == O ? OMAX : (r < 2 * O + 1 ? OMAX + 1 + (r - O - 1) : 2 * OMAX + 1));
        const float v = ((red[0][src][jl] + red[1][src][jl]) + red[2][src][jl]) + red[3][src][jl];
        p[(long)r * H + j] = v;
    }
}

// ---------------------------------------------------------------------------------------
// colsum: per chunk of samples, W2b[o, j] += sum_s d2[o, s] h1[j, s], b1b[j] += sum_s d1[j, s]
// (HVP: W2bd += d2 h1d + h1 d2d, b1bd += d1d); chunk partials reduced in order by final_kernel
// ---------------------------------------------------------------------------------------
struct ColArgs {
    const float *h1, *D1, *D2, *h1d, *D1d, *D2d;
    float* part;   // [chunk][2 * (O + 1)][H]
    float* part2;  // [chunk][2 * OMAX]: sum over the chunk's samples of d2 (and d2d)
    int B, H, O;
};

template <int MODE>
__global__ __launch_bounds__(NT) void colsum_kernel(ColArgs a) {
    // block: 64 columns j x 4 sample lanes; lane sl takes samples s0 + sl, s0 + sl + 4, ...
    // and the 4 lane sums are added in lane order
    constexpr int NR = 2 * (OMAX + 1);
    __shared__ float d2s[SC * OMAX], d2ds[SC * OMAX];
    __shared__ float red[4][NR][64];
    const int jl = threadIdx.x & 63, sl = threadIdx.x >> 6;
    const int j = blockIdx.x * 64 + jl, c = blockIdx.y;
    const int s0 = c * SC, s1 = min(a.B, s0 + SC), O = a.O, H = a.H;
    {
        constexpr int CB = (SC * OMAX + NT - 1) / NT;  // every element of the chunk in one round trip
        float v[CB], vd[CB];
#pragma unroll
        for (int c = 0; c < CB; ++c) {
            const int q = c * NT + threadIdx.x;
            v[c] = q < (s1 - s0) * O ? a.D2[(long)s0 * O + q] : 0.f;
            vd[c] = (MODE == HVP && q < (s1 - s0) * O) ? a.D2d[(long)s0 * O + q] : 0.f;
        }
#pragma unroll
        for (int c = 0; c < CB; ++c) {
            const int q = c * NT + threadIdx.x;
            if (q < (s1 - s0) * O) {
                d2s[q] = v[c];
                if (MODE == HVP) d2ds[q] = vd[c];
            }
        }
    }
    __syncthreads();
    // b2b (+ b2bd) partials of the chunk: the column-independent sums of d2 over samples
    if (blockIdx.x == 0 && threadIdx.x < 2 * OMAX) {
        const int o = threadIdx.x % OMAX;
        const bool dd = threadIdx.x >= OMAX;
        double t = 0.0;
        if (o < O && (!dd || MODE == HVP))
            for (int q = 0; q < s1 - s0; ++q) t += (double)(dd ? d2ds[q * O + o] : d2s[q * O + o]);
        a.part2[(long)c * 2 * OMAX + threadIdx.x] = (float)t;
    }
    float w[OMAX], wd[OMAX], bsum = 0.f, bsumd = 0.f;
#pragma unroll
    for (int o = 0; o < OMAX; ++o) w[o] = wd[o] = 0.f;
    if (j < H) {
        // 8 samples' loads in flight (the per-sample sums keep their order)
#pragma unroll 8
        for (int s = s0 + sl; s < s1; s += 4) {
            const long k = (long)s * H + j;
            const float h = a.h1[k];
            const float hd = (MODE == HVP) ? a.h1d[k] : 0.f;
            const float* d2 = d2s + (s - s0) * O;
            const float* d2d = d2ds + (s - s0) * O;
#pragma unroll
            for (int o = 0; o < OMAX; ++o) {
                if (o < O) {
                    w[o] += h * d2[o];
                    if (MODE == HVP) wd[o] += d2[o] * hd + h * d2d[o];
                }
            }
            bsum += a.D1[k];
            if (MODE == HVP) bsumd += a.D1d[k];
        }
    }
#pragma unroll
    for (int o = 0; o < OMAX; ++o) {
        red[sl][o][jl] = w[o];
        red[sl][OMAX + 1 + o][jl] = wd[o];
    }
    red[sl][OMAX][jl] = bsum;
    red[sl][2 * OMAX + 1][jl] = bsumd;
    __syncthreads();
    if (j >= H) return;
    float* p = a.part + (long)c * 2 * (O + 1) * H;
    // rows of this thread's column: r = sl, sl + 4, ... of the 2 (O + 1) partial rows
    for (int r = sl; r < 2 * (O + 1); r += 4) {
        if (MODE != HVP && r > O) break;
        const int src = r < O ? r : (r == O ? OMAX : (r < 2 * O + 1 ? OMAX + 1 + (r - O - 1) : 2 * OMAX + 1));
        const float v = ((red[0][src][jl] + red[1][src][jl]) + red[2][src][jl]) + red[3][src][jl];
        p[(long)r * H + j] = v;
    }
}

// block 0: loss (+ lossd) from the head partials and b2b (+ b2bd) from the colsum chunk sums;
// the other blocks: W2b, b1b (+ W2bd, b1bd) from the colsum chunk partials, chunks in order
struct FinalArgs {
    const double* hpart;
    int nhead;
    const float* cpart;
    const float* c2part;
    int nchunks;
    float *loss, *lossd, *b2b, *b2bd, *w2b, *w2bd, *b1b, *b1bd;
    int H, O;
};

constexpr int kFinalNV = 2 + 2 * OMAX;  // loss, lossd, b2b[OMAX], b2bd[OMAX]

// block `bid` of the final sums, with `red` a block-shared array of 16 + kFinalNV doubles
template <int MODE>
__device__ __forceinline__ void final_block(const FinalArgs& f, int bid, double* red) {
    constexpr int NV = kFinalNV;
    const int O = f.O, H = f.H;
    if (bid == 0) {
        // one value at a time (few registers: this block may ride along in a launch of
        // matrix-core tiles): a thread-strided sum in index order, then a block reduction.
        // Values: 0 loss, 1 lossd, 2 + o b2b[o], 2 + OMAX + o b2bd[o]
        double* tot = red + 16;  // red[0..15]: the block reduction's wave slots
#pragma unroll 1
        for (int k = 0; k < NV; ++k) {
            const bool need = k == 0 || (k == 1 && MODE != ADJ) || (k >= 2 && k < 2 + OMAX && MODE != TAN && k - 2 < O) ||
                              (k >= 2 + OMAX && MODE == HVP && k - 2 - OMAX < O);
            if (!need) continue;
            double v[1] = {0.0};
            if (k < 2) {
                for (int b = threadIdx.x; b < f.nhead; b += NT) v[0] += f.hpart[(size_t)b * 2 + k];
            } else {
                for (int c = threadIdx.x; c < f.nchunks; c += NT) v[0] += (double)f.c2part[(size_t)c * 2 * OMAX + (k - 2)];
            }
            block_sum<1>(v, red);
            if (threadIdx.x == 0) tot[k] = v[0];
        }
        __syncthreads();
        // every output read before any is written: the stores may alias the later reads as far
        // as the compiler knows, and interleaving would cost a memory round trip per output
        if (threadIdx.x == 0) {
            float old[NV];
            old[0] = f.loss[0];
            old[1] = MODE != ADJ ? f.lossd[0] : 0.f;
#pragma unroll
            for (int o = 0; o < OMAX; ++o) {
                old[2 + o] = (MODE != TAN && o < O) ? f.b2b[o] : 0.f;
                old[2 + OMAX + o] = (MODE == HVP && o < O) ? f.b2bd[o] : 0.f;
            }
            f.loss[0] = old[0] + (float)tot[0];
            if (MODE != ADJ) f.lossd[0] = old[1] + (float)tot[1];
#pragma unroll
            for (int o = 0; o < OMAX; ++o) {
                if (MODE != TAN && o < O) f.b2b[o] = old[2 + o] + (float)tot[2 + o];
                if (MODE == HVP && o < O) f.b2bd[o] = old[2 + OMAX + o] + (float)tot[2 + OMAX + o];
            }
        }
        return;
    }
    if (MODE == TAN) return;
    const int rows = (MODE == HVP ? 2 : 1) * (O + 1);
    const long q = (long)(bid - 1) * NT + threadIdx.x;
    if (q >= (long)rows * H) return;
    const int r = (int)(q / H), j = (int)(q % H);
    // the destination: W2b / b1b (HVP: W2bd / b1bd), read before the partial loads go out
    float* dst;
    if (r < O) dst = f.w2b + (long)j * O + r;
    else if (r == O) dst = f.b1b + j;
    else if (r < 2 * O + 1) dst = f.w2bd + (long)j * O + (r - O - 1);
    else dst = f.b1bd + j;
    const float old = *dst;
    // 32 chunk partials in flight at a time (indices past the last chunk clamped to it and never
    // added), added in chunk order
    float s = 0.f;
    const long cstride = 2L * (O + 1) * H;
    for (int c0 = 0; c0 < f.nchunks; c0 += 32) {
        float v[32];
#pragma unroll
        for (int c = 0; c < 32; ++c) v[c] = f.cpart[(long)min(c0 + c, f.nchunks - 1) * cstride + (long)r * H + j];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < 32; ++c)
            if (c0 + c < f.nchunks) s += v[c];
    }
    *dst = old + s;
}

template <int MODE>
__global__ __launch_bounds__(NT) void final_kernel(FinalArgs f) {
    __shared__ double red[16 + kFinalNV];
    final_block<MODE>(f, blockIdx.x, red);
}

// resident blocks per CU of the adjoint's paired backward launch (its registers would allow
// four; three measured faster)
#ifndef STADE_MLP_BWD_BLOCKS
#define STADE_MLP_BWD_BLOCKS 3
#endif
constexpr int kBwdBlocksPerCu = STADE_MLP_BWD_BLOCKS;

// the final sums as extra blocks of the backward products' launch (they read only the head
// and column-sum partials, so they run beside the product tiles)
template <int MODE>
struct FinalBlocks {
    FinalArgs f;
    int count;
    __device__ __forceinline__ void operator()(int b, float* smem) const {
        final_block<MODE>(f, b, reinterpret_cast<double*>(smem));
    }
};

struct Ptrs {
    float *loss, *x, *w1, *b1, *w2, *b2, *h1, *z;       // primal (loss, h1, z written)
    float *lossb, *xb, *w1b, *b1b, *w2b, *b2b, *h1b, *zb;  // adjoint shadows
    float *lossd, *xd, *w1d, *b1d, *w2d, *b2d, *h1d, *zd;  // tangents
    float *lossbd, *xbd, *w1bd, *b1bd, *w2bd, *b2bd, *h1bd, *zbd;
    const int64_t* lab;
};

int32_t check(int64_t B, int64_t I, int64_t H, int64_t O, const char* fn) {
    if (B < 0 || I < 0 || H < 0 || O < 0) return set_error(STADE_HIP_EINVAL, "%s: negative size", fn);
    if (O > OMAX) return set_error(STADE_HIP_ERANGE, "%s: i_out = %lld exceeds %d", fn, (long long)O, OMAX);
    if (H > 2048) return set_error(STADE_HIP_ERANGE, "%s: i_h = %lld exceeds 2048", fn, (long long)H);
    if (B > (1 << 24) || I > (1 << 24) || (double)B * (double)(H > I ? H : I) > 2e9)
        return set_error(STADE_HIP_ERANGE, "%s: sizes out of range", fn);
    // with samples, an empty output layer leaves every label out of range (the generated code
    // throws a BoundsError), and an empty hidden layer is not supported by the head kernels
    if (B > 0 && O == 0) return set_error(STADE_HIP_ERANGE, "%s: i_out = 0 with i_b = %lld samples: every label is out of range", fn, (long long)B);
    if (B > 0 && H == 0) return set_error(STADE_HIP_ERANGE, "%s: i_h = 0 is not supported", fn);
    return STADE_HIP_OK;
}

template <int MODE, int HPL>
void launch_head(const HeadArgs& h, unsigned blocks, hipStream_t stream) {
    // (the tangent and HVP forms keep W2, W2d in global memory: with both in LDS their
    // register demand exceeds the 256 VGPRs a 512-thread block allows)
    if constexpr (MODE == ADJ) {
        if (h.H <= HLDS) {
            head_kernel<MODE, HPL, true><<<blocks, HNT, 0, stream>>>(h);
            return;
        }
    }
    head_kernel<MODE, HPL, false><<<blocks, HNT, 0, stream>>>(h);
}

template <int MODE>
int32_t run(const Ptrs& p, int64_t B_, int64_t I_, int64_t H_, int64_t O_, hipStream_t stream) {
    const int B = (int)B_, I = (int)I_, H = (int)H_, O = (int)O_;
    if (B == 0) return STADE_HIP_OK;  // (i_h = 0 and i_out = 0 with samples are refused by check)
    WsCall call_(stream);
    Workspace* ws = call_.ws;
    if (!ws) return STADE_HIP_ENOMEM;
    // the adjoint with i_h <= 1024 runs its head in one pass (headd1_kernel), a chunk of the
    // column sums per block of HDB samples; the other forms split it (head4 / head, then
    // d1sum / colsum over chunks of SC samples)
    const bool fused_head = MODE == ADJ && H > 0 && H <= 1024;
    const int nchunks = fused_head ? (B + HDB - 1) / HDB : (B + SC - 1) / SC;
    const size_t nD1 = (size_t)H * B, nD2 = (size_t)O * B, nC = (size_t)nchunks * 2 * (O + 1) * H;
    const int hv = MODE == HVP ? 2 : 1;
    using namespace gemm;
    // tile and K-split plans of the matrix-core products
    const int cus = device_cus();
    // (the tangent and the HVP form s1 with s1d, the HVP W1b with W1bd and xb with xbd, as dual
    // products: one launch each, operand tiles shared)
    const Plan p_s1 = plan(H, B, I, cus), p_s1d = plan(H, B, I, cus, 2);
    // (the backward products only accumulate into shadows: their K splits may add by atomics)
    const Plan p_w1b = plan(H, I, B, cus, 1, true), p_w1bd = plan(H, I, B, cus, 2, true);
    const Plan p_xb = plan(I, B, H, cus, 1, true), p_xbd = plan(I, B, H, cus, 2, true);
    size_t npart = 0;
    auto need = [&](const Plan& q, long M, long N) {
        if (q.ksplit > 1) npart = std::max(npart, (size_t)q.ksplit * M * N);
    };
    if (MODE == ADJ) {
        need(p_s1, H, B);
        need(p_w1b, H, I);
        need(p_xb, I, B);
    } else {
        need(p_s1d, 2L * H, B);  // dual products keep two partial planes per slice
    }
    if (MODE == HVP) {
        need(p_w1bd, 2L * H, I);
        need(p_xbd, 2L * I, B);
    }
    npart = (npart + 63) / 64 * 64;
    const size_t nlocal = hv * (nD1 + nD2) + nC + (size_t)nchunks * 2 * OMAX;
    float* D1 = (float*)scratch(sizeof(float) * ((nlocal + 63) / 64 * 64 + npart) + 256);
    if (!D1) return scratch_error();
    float *D2 = D1 + nD1, *D1d = D2 + nD2, *D2d = D1d + (MODE == HVP ? nD1 : 0), *cpart = D2d + (MODE == HVP ? nD2 : 0);
    float* c2part = cpart + nC;
    float* kpart = D1 + (nlocal + 63) / 64 * 64;
    int* err = (int*)(ws->dscalars + kErrFlagSlot);
    // forward: h1 = tanh(W1 x + b1); the tangent and HVP also h1d = (1 - h1^2)(W1 xd + W1d x + b1d),
    // as one dual product
    if (MODE == ADJ) {
        Args g{};
        g.part = kpart;
        g.seg[0] = Seg{p.w1, p.x, H, I, I};
        g.nseg = 1;
        g.M = H;
        g.N = B;
        hipError_t e;
        STADE_TIMED("mlp_gemm_s1", stream, e = (launch<false, true>(g, EpiTanh{p.h1, p.b1, H}, stream, p_s1)));
        if (e != hipSuccess) return check_hip(e, "mlp gemm s1");
    } else {
        Args g{};
        g.part = kpart;
        g.seg[0] = Seg{p.w1, p.x, H, I, I};    // A0 = W1, B0 = x
        g.seg[1] = Seg{p.w1d, p.xd, H, I, I};  // A1 = W1d, B1 = xd
        g.nseg = 2;
        g.M = H;
        g.N = B;
        hipError_t e;
        STADE_TIMED("mlp_gemm_s1d", stream,
                    e = (launch<false, true, EpiTanhPair, true>(g, EpiTanhPair{p.h1, p.h1d, p.b1, p.b1d, H}, stream, p_s1d)));
        if (e != hipSuccess) return check_hip(e, "mlp gemm s1 + s1d");
    }
    HeadArgs h{};
    h.h1 = p.h1; h.w2 = p.w2; h.b2 = p.b2; h.lossb = p.lossb; h.z = p.z; h.zb = p.zb; h.h1b = p.h1b; h.D1 = D1; h.D2 = D2;
    h.h1d = p.h1d; h.w2d = p.w2d; h.b2d = p.b2d; h.lossbd = p.lossbd; h.zd = p.zd; h.zbd = p.zbd; h.h1bd = p.h1bd;
    h.D1d = D1d; h.D2d = D2d; h.lab = p.lab; h.B = B; h.H = H; h.O = O; h.partials = ws->partials; h.err = err;
    // i_h <= 1024: the batched head, SPW samples per wave, at most one block per CU (each
    // block stages W2 once); wider layers: one wave per sample, 8 waves and 16 samples a block
    constexpr int SPW = MODE == ADJ ? 4 : 1, H4W = h4nt<MODE>() / 64;
    const unsigned hb = fused_head ? (unsigned)nchunks
                        : H <= 1024 ? (unsigned)std::min<long>(((long)B + SPW * H4W - 1) / (SPW * H4W), cus)
                                    : (unsigned)((B + 16 - 1) / 16);
    if (fused_head) {
        D1Args c{p.h1, p.h1b, p.w2, D2, p.h1d, p.w2d, D2d, p.h1b, D1, p.h1bd, D1d, cpart, c2part, B, H, O};
        STADE_TIMED("mlp_head", stream, {
            // (output rows of 10 slots for i_out <= 10, else 16)
            if (H <= 256 && O <= 10) headd1_kernel<4, 10><<<hb, HDNT, 0, stream>>>(h, c);
            else if (H <= 256) headd1_kernel<4, OMAX><<<hb, HDNT, 0, stream>>>(h, c);
            else if (O <= 10) headd1_kernel<16, 10><<<hb, HDNT, 0, stream>>>(h, c);
            else headd1_kernel<16, OMAX><<<hb, HDNT, 0, stream>>>(h, c);
        });
        STADE_LAUNCHED("mlp headd1_kernel");
    } else {
        STADE_TIMED("mlp_head", stream, {
            if (H <= 256) head4_kernel<MODE, 4, SPW><<<hb, h4nt<MODE>(), 0, stream>>>(h);
            else if (H <= 1024) head4_kernel<MODE, 16, SPW><<<hb, h4nt<MODE>(), 0, stream>>>(h);
            else launch_head<MODE, 32>(h, hb, stream);
        });
        STADE_LAUNCHED("mlp head_kernel");
    }
    if (fused_head) {
        // (the column sums were formed by headd1_kernel)
    } else if (MODE != TAN && H <= 1024 && H > 0) {
        D1Args c{p.h1, p.h1b, p.w2, D2, p.h1d, p.w2d, D2d, p.h1b, D1, p.h1bd, D1d, cpart, c2part, B, H, O};
        STADE_TIMED("mlp_colsum", stream, d1sum_kernel<MODE><<<dim3((H + 63) / 64, nchunks), NT, 0, stream>>>(c));
        STADE_LAUNCHED("mlp d1sum_kernel");
    } else if (MODE != TAN) {
        // (one column block even when i_h = 0: its first block forms the b2b chunk sums)
        ColArgs c{p.h1, D1, D2, p.h1d, D1d, D2d, cpart, c2part, B, H, O};
        STADE_TIMED("mlp_colsum", stream,
                    colsum_kernel<MODE><<<dim3(std::max(1, (H + 63) / 64), nchunks), NT, 0, stream>>>(c));
        STADE_LAUNCHED("mlp colsum_kernel");
    }
    FinalArgs f{ws->partials, (int)hb, cpart, c2part, nchunks, p.loss, p.lossd, p.b2b, p.b2bd, p.w2b, p.w2bd, p.b1b, p.b1bd, H, O};
    const long rows = (long)(MODE == HVP ? 2 : 1) * (O + 1) * H;
    const unsigned fb = 1 + (MODE == TAN ? 0 : (unsigned)((rows + NT - 1) / NT));
    if (MODE == TAN || H == 0 || I == 0) {
        STADE_TIMED("mlp_final", stream, final_kernel<MODE><<<fb, NT, 0, stream>>>(f));
        STADE_LAUNCHED("mlp final_kernel");
        return STADE_HIP_OK;
    }
    const FinalBlocks<MODE> fin{f, (int)fb};
    // W1b += d1 x'   (M = H, N = I, K = B) and Xb += W1' d1   (M = I, N = B, K = H): two products
    // that both read d1, run as one launch whose blocks share the CUs; the HVP's dual forms
    // add W1bd += d1 xd' + d1d x' and Xbd += W1' d1d + W1d' d1
    {
        Args gw{}, gx{};
        gw.part = kpart;
        gw.seg[0] = Seg{D1, p.x, H, I, B};  // A0 = d1, B0 = x'
        gw.M = H;
        gw.N = I;
        gx.part = kpart;
        gx.seg[0] = Seg{p.w1, D1, H, H, H};  // A0 = W1', B0 = d1
        gx.M = I;
        gx.N = B;
        hipError_t e;
        if (MODE == ADJ) {
            gw.nseg = gx.nseg = 1;
            STADE_TIMED("mlp_gemm_bwd", stream,
                        e = (launch_pair<false, false, EpiAcc, true, true, EpiAcc>(gw, EpiAcc{p.w1b, H}, p_w1b, gx, EpiAcc{p.xb, I},
                                                                                   p_xb, stream, fin, kBwdBlocksPerCu)));
        } else {
            gw.seg[1] = Seg{D1d, p.xd, H, I, B};     // A1 = d1d, B1 = xd'
            gx.seg[1] = Seg{p.w1d, D1d, H, H, H};    // A1 = W1d', B1 = d1d
            gw.nseg = gx.nseg = 2;
            STADE_TIMED("mlp_gemm_bwd2", stream,
                        e = (launch_pair<false, false, EpiAccPair, true, true, EpiAccPair, true>(
                            gw, EpiAccPair{p.w1b, p.w1bd, H}, p_w1bd, gx, EpiAccPair{p.xb, p.xbd, I}, p_xbd, stream, fin)));
        }
        if (e != hipSuccess) return check_hip(e, "mlp gemm w1b + xb");
    }
    return STADE_HIP_OK;
}

}  // namespace
}  // namespace stade

using namespace stade;

extern "C" {

int32_t stade_hip_mlp2_ce_b(float* loss, const float* lossb, const float* x, float* xb, const int64_t* lab, const float* w1,
                            float* w1b, const float* b1, float* b1b, const float* w2, float* w2b, const float* b2, float* b2b,
                            float* h1, float* h1b, float* z, float* zb, int64_t i_b, int64_t i_in, int64_t i_h, int64_t i_out,
                            hipStream_t stream) {
    if (int32_t rc = check(i_b, i_in, i_h, i_out, "stade_hip_mlp2_ce_b")) return rc;
    // (with i_in = 0, x and W1 have no elements and may be null)
    if (i_b > 0 && (!loss || !lossb || !lab || !b1 || !b1b || !w2 || !w2b || !b2 || !b2b || !h1 || !h1b || !z || !zb ||
                    (i_in > 0 && (!x || !xb || !w1 || !w1b))))
        return set_error(STADE_HIP_EINVAL, "stade_hip_mlp2_ce_b: null pointer");
    Ptrs p{};
    p.loss = loss; p.x = (float*)x; p.w1 = (float*)w1; p.b1 = (float*)b1; p.w2 = (float*)w2; p.b2 = (float*)b2; p.h1 = h1; p.z = z;
    p.lossb = (float*)lossb; p.xb = xb; p.w1b = w1b; p.b1b = b1b; p.w2b = w2b; p.b2b = b2b; p.h1b = h1b; p.zb = zb; p.lab = lab;
    return run<ADJ>(p, i_b, i_in, i_h, i_out, stream);
}

int32_t stade_hip_mlp2_ce_d(float* loss, float* lossd, const float* x, const float* xd, const int64_t* lab, const float* w1,
                            const float* w1d, const float* b1, const float* b1d, const float* w2, const float* w2d,
                            const float* b2, const float* b2d, float* h1, float* h1d, float* z, float* zd, int64_t i_b,
                            int64_t i_in, int64_t i_h, int64_t i_out, hipStream_t stream) {
    if (int32_t rc = check(i_b, i_in, i_h, i_out, "stade_hip_mlp2_ce_d")) return rc;
    if (i_b > 0 && (!loss || !lossd || !lab || !b1 || !b1d || !w2 || !w2d || !b2 || !b2d || !h1 || !h1d || !z || !zd ||
                    (i_in > 0 && (!x || !xd || !w1 || !w1d))))
        return set_error(STADE_HIP_EINVAL, "stade_hip_mlp2_ce_d: null pointer");
    Ptrs p{};
    p.loss = loss; p.x = (float*)x; p.w1 = (float*)w1; p.b1 = (float*)b1; p.w2 = (float*)w2; p.b2 = (float*)b2; p.h1 = h1; p.z = z;
    p.lossd = lossd; p.xd = (float*)xd; p.w1d = (float*)w1d; p.b1d = (float*)b1d; p.w2d = (float*)w2d; p.b2d = (float*)b2d;
    p.h1d = h1d; p.zd = zd; p.lab = lab;
    return run<TAN>(p, i_b, i_in, i_h, i_out, stream);
}

int32_t stade_hip_mlp2_ce_hv(float* loss, const float* lossb, const float* x, float* xb, const int64_t* lab, const float* w1,
                             float* w1b, const float* b1, float* b1b, const float* w2, float* w2b, const float* b2, float* b2b,
                             float* h1, float* h1b, float* z, float* zb, int64_t i_b, int64_t i_in, int64_t i_h, int64_t i_out,
                             float* lossd, const float* lossbd, const float* xd, float* xbd, const float* w1d, float* w1bd,
                             const float* b1d, float* b1bd, const float* w2d, float* w2bd, const float* b2d, float* b2bd,
                             float* h1d, float* h1bd, float* zd, float* zbd, hipStream_t stream) {
    if (int32_t rc = check(i_b, i_in, i_h, i_out, "stade_hip_mlp2_ce_hv")) return rc;
    if (i_b > 0 && (!loss || !lossb || !lab || !b1 || !b1b || !w2 || !w2b || !b2 || !b2b || !h1 || !h1b || !z || !zb || !lossd ||
                    !lossbd || !b1d || !b1bd || !w2d || !w2bd || !b2d || !b2bd || !h1d || !h1bd || !zd || !zbd ||
                    (i_in > 0 && (!x || !xb || !w1 || !w1b || !xd || !xbd || !w1d || !w1bd))))
        return set_error(STADE_HIP_EINVAL, "stade_hip_mlp2_ce_hv: null pointer");
    Ptrs p{};
    p.loss = loss; p.x = (float*)x; p.w1 = (float*)w1; p.b1 = (float*)b1; p.w2 = (float*)w2; p.b2 = (float*)b2; p.h1 = h1; p.z = z;
    p.lossb = (float*)lossb; p.xb = xb; p.w1b = w1b; p.b1b = b1b; p.w2b = w2b; p.b2b = b2b; p.h1b = h1b; p.zb = zb; p.lab = lab;
    p.lossd = lossd; p.xd = (float*)xd; p.w1d = (float*)w1d; p.b1d = (float*)b1d; p.w2d = (float*)w2d; p.b2d = (float*)b2d;
    p.h1d = h1d; p.zd = zd;
    p.lossbd = (float*)lossbd; p.xbd = xbd; p.w1bd = w1bd; p.b1bd = b1bd; p.w2bd = w2bd; p.b2bd = b2bd; p.h1bd = h1bd; p.zbd = zbd;
    return run<HVP>(p, i_b, i_in, i_h, i_out, stream);
}

}  // extern "C"
