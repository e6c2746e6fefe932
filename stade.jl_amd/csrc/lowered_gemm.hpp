// The general lowering's matrix products (stade_hip/lower/contract.py): a contraction of the
// generated code run by the fp32 matrix-core GEMM (gemm_f32.hpp), whose output is any strided
// array element C[m * sm + n * sn] (the pointer already at the product's first element).
#pragma once

#include <algorithm>

#include "gemm_f32.hpp"

namespace stade_lowered {

// ACC: the product is added to the element (a shadow accumulated, as the generated adjoint
// code does: a K split may then add its slices by atomics); else it is stored (a scratch
// array of sums the loop reads).
template <bool ACC>
struct GemmOut {
    float* C;
    long sm, sn;
    __device__ float load(int m, int n) const { return ACC ? C[(long)m * sm + (long)n * sn] : 0.0f; }
    __device__ void operator()(int m, int n, float v, float c) const { C[(long)m * sm + (long)n * sn] = ACC ? c + v : v; }
    static constexpr bool kAtomic = ACC;
    __device__ void atomic(int m, int n, float v) const { unsafeAtomicAdd(&C[(long)m * sm + (long)n * sn], v); }
};

}  // namespace stade_lowered

namespace stade_lowered {

// ------------------------------------------------------------------------------------------
// Table-addressed product (a contraction whose factors are gathers, such as a convolution's
// taps; contract.py's table form):
//
//   C[c0 + ro(m) + co(n)] (+)= sum_k A[a0 + ar(m) + ak(k)] * B[b0 + bk(k) + bc(n)]
//
// every offset a TabDim: a table of 0-based element offsets (Int64) or, without one, i x stride.
// Block: 256 threads as 2 x 2 waves, a (64 TM) x (64 TN) tile; each wave a (32 TM) x (32 TN)
// part as TM x TN v_mfma_f32_32x32x2_f32 accumulators, so that each operand value read from
// LDS feeds TN (or TM) MFMAs.  K advances 16 a step: a step's operand tiles are gathered into
// registers during the step before, stored to LDS between two barriers, and read back as the
// MFMA operands (B first, so that the accumulator's lane index runs along m).  The rows' and
// columns' table offsets are read once per block (the columns' output offsets through LDS).
// blockIdx.x runs over n tiles, blockIdx.y over m tiles, blockIdx.z over K slices (which then
// add by atomics: MODE 2).  MODE: 0 store, 1 add (one writer per element), 2 atomic add.
// ------------------------------------------------------------------------------------------
struct TabDim {
    const int64_t* t;
    long s;
    __device__ __forceinline__ long at(long i) const { return t ? (long)t[i] : i * s; }
};

struct GemmTabArgs {
    const float* A;
    TabDim ar, ak;
    const float* B;
    TabDim bk, bc;
    float* C;
    TabDim ro, co;
    int M, N, K;
    int ksplit;
};

constexpr int GT_NT = 256, GT_KT = 16;

// AKM / BKM: which way a thread's gathered values of an operand run.  Without it a thread
// keeps one row (column) of the tile and takes every 256 / BM-th k, so a wave's loads run
// along the rows: for operands whose rows are adjacent in memory.  With it 16 consecutive
// threads take the 16 k of one row: for operands whose k are adjacent in memory.
template <int MODE, int TM, int TN, bool AKM, bool BKM>
__global__ __launch_bounds__(GT_NT) void gemm_tab_kernel(const GemmTabArgs g) {
    typedef float floatx16 __attribute__((ext_vector_type(16)));
    constexpr int BM = 64 * TM, BN = 64 * TN;
    constexpr int AR = BM * GT_KT / GT_NT, BR = BN * GT_KT / GT_NT;  // gathered values a thread
    constexpr int LA = BM + 1, LB = BN + 1;  // LDS row pitch: the k-major stores do not conflict
    __shared__ float As[GT_KT * LA];
    __shared__ float Bs[GT_KT * LB];
    __shared__ long cof[BN];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int wm = (wave & 1) * 32 * TM, wn = (wave >> 1) * 32 * TN;
    const int steps = (g.K + GT_KT - 1) / GT_KT;
    const int per = (steps + g.ksplit - 1) / g.ksplit;
    const int s_begin = blockIdx.z * per, s_end = min(steps, s_begin + per);
    // value q of this thread: A row ar_(q), k ak_(q); B k bk_(q), column bc_(q)
    auto ar_ = [&](int q) { return AKM ? tid / GT_KT + (GT_NT / GT_KT) * q : tid % BM; };
    auto ak_ = [&](int q) { return AKM ? tid % GT_KT : tid / BM + (GT_NT / BM) * q; };
    auto bc_ = [&](int q) { return BKM ? tid / GT_KT + (GT_NT / GT_KT) * q : tid % BN; };
    auto bk_ = [&](int q) { return BKM ? tid % GT_KT : tid / BN + (GT_NT / BN) * q; };
    long aoff[AKM ? AR : 1], boff[BKM ? BR : 1];
    bool aok[AKM ? AR : 1], bok[BKM ? BR : 1];
#pragma unroll
    for (int q = 0; q < (AKM ? AR : 1); ++q) {
        aok[q] = m0 + ar_(q) < g.M;
        aoff[q] = aok[q] ? g.ar.at(m0 + ar_(q)) : 0;
    }
#pragma unroll
    for (int q = 0; q < (BKM ? BR : 1); ++q) {
        bok[q] = n0 + bc_(q) < g.N;
        boff[q] = bok[q] ? g.bc.at(n0 + bc_(q)) : 0;
    }
    if (tid < BN) cof[tid] = n0 + tid < g.N ? g.co.at(n0 + tid) : 0;
    float va[AR], vb[BR];
    auto gather = [&](int st) {
        const int k0 = st * GT_KT;
        const long akv = AKM && k0 + ak_(0) < g.K ? g.ak.at(k0 + ak_(0)) : 0;
        const long bkv = BKM && k0 + bk_(0) < g.K ? g.bk.at(k0 + bk_(0)) : 0;
#pragma unroll
        for (int q = 0; q < AR; ++q) {
            const int k = k0 + ak_(q);
            const int qa = AKM ? q : 0;
            va[q] = (aok[qa] && k < g.K) ? g.A[aoff[qa] + (AKM ? akv : g.ak.at(k))] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < BR; ++q) {
            const int k = k0 + bk_(q);
            const int qb = BKM ? q : 0;
            vb[q] = (bok[qb] && k < g.K) ? g.B[(BKM ? bkv : g.bk.at(k)) + boff[qb]] : 0.0f;
        }
    };
    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    if (s_begin < s_end) gather(s_begin);
    for (int st = s_begin; st < s_end; ++st) {
        __syncthreads();  // the step before has read the tiles
#pragma unroll
        for (int q = 0; q < AR; ++q) As[ak_(q) * LA + ar_(q)] = va[q];
#pragma unroll
        for (int q = 0; q < BR; ++q) Bs[bk_(q) * LB + bc_(q)] = vb[q];
        __syncthreads();
        if (st + 1 < s_end) gather(st + 1);  // in flight during this step's MFMAs
#pragma unroll
        for (int h = 0; h < GT_KT / 2; ++h) {
            const int k = 2 * h + (lane >> 5);
            float a[TM], b[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) a[i] = As[k * LA + wm + 32 * i + (lane & 31)];
#pragma unroll
            for (int j = 0; j < TN; ++j) b[j] = Bs[k * LB + wn + 32 * j + (lane & 31)];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(b[j], a[i], acc[i][j], 0, 0, 0);
        }
    }
    __syncthreads();  // cof written (a block with no steps has had no barrier)
    // accumulator (i, j, r): m = m0 + wm + 32 i + lane % 32, n = n0 + wn + 32 j + 8 (r / 4) + 4 (lane / 32) + r % 4
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int m = m0 + wm + 32 * i + (lane & 31);
        if (m >= g.M) continue;
        float* const cm = g.C + g.ro.at(m);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int nl = wn + 32 * j + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                if (n0 + nl < g.N) {
                    float* p = cm + cof[nl];
                    if (MODE == 0)
                        *p = acc[i][j][r];
                    else if (MODE == 1)
                        *p += acc[i][j][r];
                    else
                        unsafeAtomicAdd(p, acc[i][j][r]);
                }
            }
        }
    }
}

// Tile shape: 128 x 64 when M is at least twice N, 64 x 128 when N is at least twice M,
// else 128 x 128 (64 x 64 when both are small).  K slices (atomic mode only): enough blocks to
// fill the CUs about twice when the tile grid alone does not, each slice at least 8 steps.
inline void gemm_tab_shape(int M, int N, int& tm, int& tn) {
    if (M <= 64 && N <= 64) {
        tm = tn = 1;
    } else if ((long)M >= 2L * N) {
        tm = 2;
        tn = 1;
    } else if ((long)N >= 2L * M) {
        tm = 1;
        tn = 2;
    } else {
        tm = tn = 2;
    }
}

inline int gemm_tab_split(int M, int N, int K, int tm, int tn, int cus) {
    const long tiles = (long)((M + 64 * tm - 1) / (64 * tm)) * ((N + 64 * tn - 1) / (64 * tn));
    const long steps = (K + GT_KT - 1) / GT_KT;
    long ks = (2L * cus + tiles - 1) / tiles;
    ks = std::min<long>(ks, std::max<long>(1, steps / 8));
    return (int)std::max<long>(1, std::min<long>(ks, 65535));
}

// MODE 0 / 1 / 2 as the kernel's; a K split only with MODE 2
template <int MODE, bool AKM, bool BKM>
hipError_t gemm_tab(GemmTabArgs g, hipStream_t stream) {
    if (g.M <= 0 || g.N <= 0) return hipSuccess;
    int tm, tn;
    gemm_tab_shape(g.M, g.N, tm, tn);
    g.ksplit = MODE == 2 ? gemm_tab_split(g.M, g.N, g.K, tm, tn, stade::gemm::device_cus()) : 1;
    const long nt = (g.N + 64L * tn - 1) / (64L * tn), mt = (g.M + 64L * tm - 1) / (64L * tm);
    if (nt > 0x7fffffffL || mt > 65535) return hipErrorInvalidValue;
    const dim3 grid((unsigned)nt, (unsigned)mt, (unsigned)g.ksplit);
    if (tm == 2 && tn == 1)
        gemm_tab_kernel<MODE, 2, 1, AKM, BKM><<<grid, GT_NT, 0, stream>>>(g);
    else if (tm == 1 && tn == 2)
        gemm_tab_kernel<MODE, 1, 2, AKM, BKM><<<grid, GT_NT, 0, stream>>>(g);
    else if (tm == 2 && tn == 2)
        gemm_tab_kernel<MODE, 2, 2, AKM, BKM><<<grid, GT_NT, 0, stream>>>(g);
    else
        gemm_tab_kernel<MODE, 1, 1, AKM, BKM><<<grid, GT_NT, 0, stream>>>(g);
    return hipGetLastError();
}

}  // namespace stade_lowered
