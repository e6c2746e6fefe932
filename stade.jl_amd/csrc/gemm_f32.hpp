// fp32 GEMM on CDNA4 matrix cores (v_mfma_f32_32x32x2_f32), with a fused per-element epilogue.
//
//   C(m, n) = sum over segments s of  sum_k A_s(m, k) * B_s(k, n),   epi(m, n, C(m, n), epi.load(m, n))
//
// An epilogue functor reads what it needs of the old output in load(m, n) (gathered for the
// whole tile before any store) and writes in operator()(m, n, v, loaded).
//
// A_s is M x K_s and B_s is K_s x N, column-major (Julia) with either storage order:
//   A_KM = false: A(m, k) at A[m + k * lda] (m contiguous);  A_KM = true: at A[k + m * lda]
//   B_KM = true:  B(k, n) at B[k + n * ldb] (k contiguous);  B_KM = false: at B[n + k * ldb]
// Up to two segments accumulate into one tile, so a tangent product such as
// W1d * X + W1 * Xd is one launch.
//
// Tiling: a 256-thread block (4 waves) computes a 128 x BNT tile of C (BNT = 128 or 64);
// each wave a 64 x BNT/2 part as 2 x BNT/64 MFMA 32 x 32 tiles.  K advances 16 at a time
// through two LDS buffers (one barrier per step: the next tile's global loads are issued
// before the MFMAs of the current one and stored to the other buffer after them).  LDS rows
// are padded by 4 floats.  The MFMA operands are swapped (B tile as the matrix-core A
// operand) so that the accumulator's lane index runs along m: each epilogue store of a wave
// covers 32 consecutive rows of a column-major C, a 128-byte segment.
//
// Split K: with `ksplit` > 1 the K steps (of all segments, in order) are cut into ksplit
// contiguous ranges, one per blockIdx.z; each writes its partial tile to a scratch slice
// and a second kernel adds the slices in slice order and applies the epilogue.  The host
// picks the narrow tile and the split so that small-M*N products still give every CU about
// two blocks.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

namespace stade {
namespace gemm {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = 128, KT = 16, NT = 256, PAD = 4;
constexpr int LDA_S = BM + PAD;

struct Seg {
    const float* A;
    const float* B;
    long lda, ldb;
    int K;
};

struct Args {
    Seg seg[2];
    int nseg;
    int M, N;
    int ksplit;     // blockIdx.z ranges over ksplit slices of the K steps
    float* part;    // ksplit > 1: partial tiles, slice z at part + z * M * N, column-major
    bool bufok;     // set by launch(): every operand's byte extent fits 31 bits and the two
                    // segments share lda and ldb, so whole tiles may use buffer loads
};

// Registers holding one ROWS x 16 operand tile between its global load and its LDS store.
template <int ROWS>
struct Stage {
    float4 v[ROWS * KT / 4 / NT];
};

// A tile (r 0..ROWS-1, k 0..15) at (r0, k0) into registers; zero outside rows x K.
template <bool KMAJ, int ROWS>
__device__ __forceinline__ void load_tile(Stage<ROWS>& st, const float* __restrict__ P, long ld, int rows, int K, int r0,
                                          int k0, bool vec) {
    constexpr int R4 = ROWS / 4;  // float4 per k row (KMAJ = false)
#pragma unroll
    for (int q = 0; q < ROWS * KT / 4 / NT; ++q) {
        const int f = threadIdx.x + NT * q;
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        if (!KMAJ) {
            // rows contiguous: f -> (k = f / R4, r4 = (f % R4) * 4)
            const int kk = f / R4, r4 = (f % R4) * 4;
            const int k = k0 + kk, r = r0 + r4;
            if (k < K) {
                const float* p = P + (long)r + (long)k * ld;
                if (vec && r + 3 < rows) {
                    x = *reinterpret_cast<const float4*>(p);
                } else {
                    if (r + 0 < rows) x.x = p[0];
                    if (r + 1 < rows) x.y = p[1];
                    if (r + 2 < rows) x.z = p[2];
                    if (r + 3 < rows) x.w = p[3];
                }
            }
        } else {
            // k contiguous: f -> (r = f / 4, k4 = (f % 4) * 4)
            const int rr = f >> 2, k4 = (f & 3) * 4;
            const int r = r0 + rr, k = k0 + k4;
            if (r < rows) {
                const float* p = P + (long)k + (long)r * ld;
                if (vec && k + 3 < K) {
                    x = *reinterpret_cast<const float4*>(p);
                } else {
                    if (k + 0 < K) x.x = p[0];
                    if (k + 1 < K) x.y = p[1];
                    if (k + 2 < K) x.z = p[2];
                    if (k + 3 < K) x.w = p[3];
                }
            }
        }
        st.v[q] = x;
    }
}

// The same for a tile known to lie inside the operand, with 16-byte aligned rows, as buffer
// loads: a scalar resource over the operand, this thread's constant byte offsets (tile_offsets)
// and a scalar byte offset for the K step.  No per-step address arithmetic in vector
// registers, so the loads' destination registers are not reused as address temporaries
// while the loads are in flight.
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kBufWord3 = 0x00020000;  // gfx9-family buffer resource word 3 (raw, 32-bit data)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t operand_rsrc(const float* P) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(P), (short)0, 0x7fffffff, kBufWord3);
}

template <bool KMAJ, int ROWS>
struct TileOffsets {
    uint32_t o[ROWS * KT / 4 / NT];
};

// byte offsets of this thread's float4s of the tile at rows r0.., k step 0
template <bool KMAJ, int ROWS>
__device__ __forceinline__ TileOffsets<KMAJ, ROWS> tile_offsets(long ld, int r0) {
    constexpr int R4 = ROWS / 4;
    TileOffsets<KMAJ, ROWS> t;
#pragma unroll
    for (int q = 0; q < ROWS * KT / 4 / NT; ++q) {
        const int f = threadIdx.x + NT * q;
        const long e = !KMAJ ? (long)(r0 + (f % R4) * 4) + (long)(f / R4) * ld : (long)((f & 3) * 4) + (long)(r0 + (f >> 2)) * ld;
        t.o[q] = (uint32_t)(e * 4);
    }
    return t;
}

// soff: byte offset of K step k0 (k0 * ld * 4 for KMAJ = false, k0 * 4 for KMAJ = true)
template <bool KMAJ, int ROWS>
__device__ __forceinline__ void load_tile_full(Stage<ROWS>& st, __amdgpu_buffer_rsrc_t r, const TileOffsets<KMAJ, ROWS>& to,
                                               uint32_t soff) {
#pragma unroll
    for (int q = 0; q < ROWS * KT / 4 / NT; ++q) {
        const v4f x = __builtin_amdgcn_raw_buffer_load_b128(r, to.o[q], soff, 0);
        st.v[q] = make_float4(x.x, x.y, x.z, x.w);
    }
}

// Registers -> LDS tile S[k][r] (row stride LD)
template <bool KMAJ, int ROWS, int LD>
__device__ __forceinline__ void store_tile(const Stage<ROWS>& st, float* __restrict__ S) {
    constexpr int R4 = ROWS / 4;
#pragma unroll
    for (int q = 0; q < ROWS * KT / 4 / NT; ++q) {
        const int f = threadIdx.x + NT * q;
        const float4 x = st.v[q];
        if (!KMAJ) {
            const int kk = f / R4, r4 = (f % R4) * 4;
            *reinterpret_cast<float4*>(S + kk * LD + r4) = x;
        } else {
            const int rr = f >> 2, k4 = (f & 3) * 4;
            S[(k4 + 0) * LD + rr] = x.x;
            S[(k4 + 1) * LD + rr] = x.y;
            S[(k4 + 2) * LD + rr] = x.z;
            S[(k4 + 3) * LD + rr] = x.w;
        }
    }
}

template <bool A_KM, bool B_KM, int BNT, class Epi>
__global__ __launch_bounds__(NT) void gemm_kernel(Args g, bool vec, Epi epi) {
    constexpr int LDB_S = BNT + PAD, NJ = BNT / 64;
    __shared__ float As[2][KT * LDA_S];
    __shared__ float Bs[2][KT * LDB_S];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m0 = blockIdx.x * BM, n0 = blockIdx.y * BNT;
    const int wm = (wave & 1) * 64, wn = (wave >> 1) * (BNT / 2);

    // Both segments' operands in registers (indexing g.seg[s] with a runtime s would reload
    // them from the kernel-argument segment at every step).
    const float* const A0 = g.seg[0].A;
    const float* const B0 = g.seg[0].B;
    const long lda0 = g.seg[0].lda, ldb0 = g.seg[0].ldb;
    const int K0 = g.seg[0].K;
    const bool two = g.nseg > 1;
    const float* const A1 = two ? g.seg[1].A : A0;
    const float* const B1 = two ? g.seg[1].B : B0;
    const long lda1 = two ? g.seg[1].lda : lda0, ldb1 = two ? g.seg[1].ldb : ldb0;
    const int K1 = two ? g.seg[1].K : 0;

    // the K steps of all segments, in order; this block's slice of them
    const int steps0 = (K0 + KT - 1) / KT;
    const int total = steps0 + (K1 + KT - 1) / KT;
    const int t_begin = (int)((long)total * blockIdx.z / g.ksplit);
    const int t_end = (int)((long)total * (blockIdx.z + 1) / g.ksplit);
    // a block whose tiles all lie inside the operands (M, N and every K step) loads with no
    // per-element tests
    const bool full = vec && g.bufok && m0 + BM <= g.M && n0 + BNT <= g.N && K0 % KT == 0 && K1 % KT == 0;
    // buffer resources of both segments' operands and this thread's offsets (the segments
    // share lda and ldb when bufok is set)
    const __amdgpu_buffer_rsrc_t rA0 = operand_rsrc(A0), rA1 = operand_rsrc(A1);
    const __amdgpu_buffer_rsrc_t rB0 = operand_rsrc(B0), rB1 = operand_rsrc(B1);
    const TileOffsets<A_KM, BM> offA = tile_offsets<A_KM, BM>(lda0, m0);
    const TileOffsets<B_KM, BNT> offB = tile_offsets<B_KM, BNT>(ldb0, n0);

    floatx16 acc[2][NJ];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // two register stages: the global loads of step t+2 are issued at step t, and the stage
    // holding step t+1 (loaded at step t-1) goes to LDS at the end of step t, so a load has
    // two steps of matrix-core work to arrive.  Loads and stores are unconditional (a step
    // past the slice reloads its last step, whose data is never read) so that the compiler
    // waits only for the older stage.
    Stage<BM> sa[2];
    Stage<BNT> sb[2];
    auto load = [&](int p, int t, bool fast) {
        t = t < t_end ? t : t_end - 1;
        const bool s1 = t >= steps0;
        const float* A = s1 ? A1 : A0;
        const float* B = s1 ? B1 : B0;
        const long lda = s1 ? lda1 : lda0, ldb = s1 ? ldb1 : ldb0;
        const int K = s1 ? K1 : K0;
        const int k0 = (s1 ? t - steps0 : t) * KT;
        if (fast) {
            const uint32_t sa_off = (uint32_t)((A_KM ? (long)k0 : (long)k0 * lda0) * 4);
            const uint32_t sb_off = (uint32_t)((B_KM ? (long)k0 : (long)k0 * ldb0) * 4);
            load_tile_full<A_KM, BM>(sa[p], s1 ? rA1 : rA0, offA, sa_off);
            load_tile_full<B_KM, BNT>(sb[p], s1 ? rB1 : rB0, offB, sb_off);
        } else {
            load_tile<A_KM, BM>(sa[p], A, lda, g.M, K, m0, k0, vec);
            load_tile<B_KM, BNT>(sb[p], B, ldb, g.N, K, n0, k0, vec);
        }
    };
    auto mainloop = [&](auto fast_tag) {
        constexpr bool FAST = decltype(fast_tag)::value;
        if (t_begin >= t_end) return;
        load(0, t_begin, FAST);
        load(1, t_begin + 1, FAST);
        store_tile<A_KM, BM, LDA_S>(sa[0], As[0]);
        store_tile<B_KM, BNT, LDB_S>(sb[0], Bs[0]);
        __syncthreads();
        // step t with p = (t - t_begin) % 2: LDS buffer p and register stage p
        auto step = [&](int t, auto p_tag) {
            constexpr int cur = decltype(p_tag)::value;
            load(cur, t + 2, FAST);
            const float* A_ = As[cur];
            const float* B_ = Bs[cur];
            // every fragment of the stage first (the LDS reads overlap each other), then the MFMAs
            float a[KT / 2][2], b[KT / 2][NJ];
#pragma unroll
            for (int ks = 0; ks < KT / 2; ++ks) {
                const int kk = ks * 2 + (lane >> 5);
#pragma unroll
                for (int i = 0; i < 2; ++i) a[ks][i] = A_[kk * LDA_S + wm + i * 32 + (lane & 31)];
#pragma unroll
                for (int j = 0; j < NJ; ++j) b[ks][j] = B_[kk * LDB_S + wn + j * 32 + (lane & 31)];
            }
            // keep the reads ahead of the MFMAs (the scheduler would sink each read to its use
            // and expose the LDS latency at every k step)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int ks = 0; ks < KT / 2; ++ks)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(b[ks][j], a[ks][i], acc[i][j], 0, 0, 0);
            store_tile<A_KM, BM, LDA_S>(sa[cur ^ 1], As[cur ^ 1]);
            store_tile<B_KM, BNT, LDB_S>(sb[cur ^ 1], Bs[cur ^ 1]);
            __syncthreads();
        };
        for (int t = t_begin; t < t_end; t += 2) {
            step(t, std::integral_constant<int, 0>{});
            if (t + 1 < t_end) step(t + 1, std::integral_constant<int, 1>{});
        }
    };
    if (full) mainloop(std::true_type{});
    else mainloop(std::false_type{});
    // accumulator (i, j, r): m = m0 + wm + 32 i + lane % 32,  n = n0 + wn + 32 j + 8 (r / 4) + 4 (lane / 32) + r % 4
    if (g.ksplit > 1) {
        float* part = g.part + (long)blockIdx.z * g.M * g.N;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int m = m0 + wm + i * 32 + (lane & 31);
            if (m >= g.M) continue;
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int n = n0 + wn + j * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                    if (n < g.N) part[m + (long)n * g.M] = acc[i][j][r];
                }
        }
        return;
    }
    // the epilogue's inputs (e.g. C of C += v) for the whole tile first, then the stores: the
    // output may alias them as far as the compiler knows, and interleaving would serialise one
    // memory round trip per element
    float pre[2][NJ][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm + i * 32 + (lane & 31);
                const int n = n0 + wn + j * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                pre[i][j][r] = (m < g.M && n < g.N) ? epi.load(m, n) : 0.f;
            }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int m = m0 + wm + i * 32 + (lane & 31);
        if (m >= g.M) continue;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int n = n0 + wn + j * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                if (n < g.N) epi(m, n, acc[i][j][r], pre[i][j][r]);
            }
    }
}

// second stage of a split-K product: C(m, n) = sum over slices in order, then the epilogue
template <class Epi>
__global__ __launch_bounds__(NT) void splitk_reduce_kernel(const float* __restrict__ part, int ksplit, int M, int N, Epi epi) {
    const long q = (long)blockIdx.x * NT + threadIdx.x;
    const long mn = (long)M * N;
    if (q >= mn) return;
    // every slice's value in flight at once (ksplit <= 16; indices past the last slice clamped
    // to it and never added), added in slice order
    const int m = (int)(q % M), n = (int)(q / M);
    float v[16];
#pragma unroll
    for (int z = 0; z < 16; ++z) v[z] = part[q + min(z, ksplit - 1) * mn];
    const auto old = epi.load(m, n);
    __builtin_amdgcn_sched_barrier(0);
    float s = v[0];
#pragma unroll
    for (int z = 1; z < 16; ++z)
        if (z < ksplit) s += v[z];
    epi(m, n, s, old);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Tile width and K split for an M x N x K product on `cus` compute units: the wide tile
// when it gives at least two blocks per CU, else the narrow one, split along K (slices of at
// least 256) until there are about two blocks per CU.
struct Plan {
    int bnt, ksplit;
};
#ifndef STADE_GEMM_BPC
#define STADE_GEMM_BPC 2
#endif
inline Plan plan(int M, int N, int Ktot, int cus) {
    constexpr long bpc = STADE_GEMM_BPC;  // blocks per CU the plan aims for
    const long wide = (long)((M + BM - 1) / BM) * ((N + 127) / 128);
    if (wide >= bpc * cus) return Plan{128, 1};
    const long narrow = (long)((M + BM - 1) / BM) * ((N + 63) / 64);
    int ks = 1;
    while (narrow * ks < bpc * cus && Ktot / (ks * 2) >= 256 && ks < 16) ks *= 2;
    return Plan{64, ks};
}

// Number of compute units of the current device (cached per process for device 0..15).
inline int device_cus() {
    static int cached[16] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) return 256;
    if (!cached[dev]) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}

// Launch; returns the hipError of the launch.  `part` must hold ksplit * M * N floats when
// the plan splits K (ask with plan() first); it may be null otherwise.
template <bool A_KM, bool B_KM, class Epi>
hipError_t launch(Args g, Epi epi, hipStream_t stream, const Plan& p) {
    if (g.M <= 0 || g.N <= 0) return hipSuccess;
    bool vec = true;
    for (int s = 0; s < g.nseg; ++s) {
        vec = vec && aligned16(g.seg[s].A) && aligned16(g.seg[s].B) && g.seg[s].lda % 4 == 0 && g.seg[s].ldb % 4 == 0;
    }
    g.ksplit = p.ksplit;
    if (p.ksplit > 1 && !g.part) return hipErrorInvalidValue;
    // byte extent of each operand: A spans K columns of lda (A_KM = false) or M columns,
    // B spans N columns of ldb (B_KM = true) or K columns
    g.bufok = g.nseg == 1 || (g.seg[0].lda == g.seg[1].lda && g.seg[0].ldb == g.seg[1].ldb);
    for (int s = 0; s < g.nseg; ++s) {
        const double ea = (double)g.seg[s].lda * (A_KM ? g.M : g.seg[s].K) * 4.0;
        const double eb = (double)g.seg[s].ldb * (B_KM ? g.N : g.seg[s].K) * 4.0;
        g.bufok = g.bufok && ea < 2147483648.0 && eb < 2147483648.0;
    }
    if (p.bnt == 128) {
        dim3 grid((g.M + BM - 1) / BM, (g.N + 127) / 128, p.ksplit);
        gemm_kernel<A_KM, B_KM, 128, Epi><<<grid, NT, 0, stream>>>(g, vec, epi);
    } else {
        dim3 grid((g.M + BM - 1) / BM, (g.N + 63) / 64, p.ksplit);
        gemm_kernel<A_KM, B_KM, 64, Epi><<<grid, NT, 0, stream>>>(g, vec, epi);
    }
    if (p.ksplit > 1) {
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const long mn = (long)g.M * g.N;
        splitk_reduce_kernel<Epi><<<(unsigned)((mn + NT - 1) / NT), NT, 0, stream>>>(g.part, p.ksplit, g.M, g.N, epi);
    }
    return hipGetLastError();
}

}  // namespace gemm
}  // namespace stade
