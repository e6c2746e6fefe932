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
// W1d * X + W1 * Xd is one launch.  A dual launch instead reads both segments in the same K
// steps and writes two outputs, P = A0 B0 and Q = A0 B1 + A1 B0 (a product with its tangent).
//
// Tiling: a 256-thread block (4 waves) computes a 128 x BNT tile of C (BNT = 128 or 64);
// each wave a 64 x BNT/2 part as 2 x BNT/64 MFMA 32 x 32 tiles.  K advances 16 at a time
// through two LDS buffers (one barrier per step: a later step's global loads are issued as a
// step starts, the next step's stage goes to the other buffer between the two halves of the
// step's MFMAs, and the next step's fragments are read right after the barrier).  Operand
// tiles sit in LDS in a k-quad layout (below), read as one 128-bit fragment per 4 MFMAs.
// The MFMA operands are swapped (B tile as the matrix-core A operand) so that the
// accumulator's lane index runs along m: each epilogue store of a wave covers 32 consecutive
// rows of a column-major C, a 128-byte segment.
//
// Split K: with `ksplit` > 1 the K steps (of all segments, in order) are cut into ksplit
// contiguous ranges, one per blockIdx.z; each writes its partial tile to a scratch slice
// and a second kernel adds the slices in slice order and applies the epilogue.  An epilogue
// that only accumulates (C += v: a shadow, as the generated adjoint code accumulates it)
// can instead take the slices by atomic addition straight into C (`Epi::kAtomic`): no
// partial tiles and no second kernel, with the slices' order left to the hardware.  The host
// picks the tile width and the split from a cost model (plan()).
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>
#include <utility>

namespace stade {
namespace gemm {

typedef float floatx16 __attribute__((ext_vector_type(16)));

#ifndef STADE_GEMM_KT
#define STADE_GEMM_KT 16
#endif
constexpr int BM = 128, KT = STADE_GEMM_KT, NT = 256;
constexpr int KQ = KT / 4;  // k-planes per step
static_assert(KT == 16 || KT == 32, "K step of 16 or 32");

// LDS operand tiles use a "quad" layout: element (k, r) of a ROWS x KT tile sits at
// S[(k / 4) * ldq(ROWS) + r * 4 + k % 4], i.e. KT / 4 k-planes each holding, per row, that
// row's four consecutive k values as one 16-byte cell.  A matrix-core fragment is then one
// 128-bit LDS read per 32 rows and 4 k values.  The plane stride ROWS * 4 + 128 / KT floats
// spreads the KT / 4 planes of a row over distinct 16-byte bank groups, so the 128-bit
// stores of k-contiguous operands (eight lanes: 32 / KT rows x KT / 4 planes) do not conflict.
template <int ROWS>
constexpr int ldq() {
    return ROWS * 4 + 128 / KT;
}

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
    bool atomic;    // ksplit > 1: slices added into the output by atomics (Epi::kAtomic)
    float* part;    // ksplit > 1, !atomic: partial tiles, slice z at part + z * M * N, column-major
    bool bufok;     // set by launch(): every operand's byte extent fits 31 bits and the two
                    // segments share lda and ldb, so whole tiles may use buffer loads
};

// The cells (row, k-plane) of a ROWS x KT tile are shared out over the block: cell
// e = threadIdx.x + NT * q of this thread is
//   KMAJ (k contiguous in memory):    row e / KQ,   plane e % KQ   (one 16-byte load per cell;
//                                     KQ threads read a row's 4 KT contiguous bytes)
//   !KMAJ (rows contiguous in memory): row e % ROWS, plane e / ROWS (four 4-byte loads per
//                                     cell, one per k; a wave reads 64 consecutive rows of a k)
template <int ROWS>
struct Stage {
    float4 v[ROWS * KQ / NT];
};

template <bool KMAJ, int ROWS>
__device__ __forceinline__ void cell_of(int e, int& r, int& kq) {
    if (KMAJ) {
        r = e / KQ;
        kq = e % KQ;
    } else {
        r = e % ROWS;
        kq = e / ROWS;
    }
}

// A tile (r 0..ROWS-1, k 0..KT-1) at (r0, k0) into registers; zero outside rows x K.
template <bool KMAJ, int ROWS>
__device__ __forceinline__ void load_tile(Stage<ROWS>& st, const float* __restrict__ P, long ld, int rows, int K, int r0,
                                          int k0, bool vec) {
#pragma unroll
    for (int q = 0; q < ROWS * KQ / NT; ++q) {
        int rr, kq;
        cell_of<KMAJ, ROWS>(threadIdx.x + NT * q, rr, kq);
        const int r = r0 + rr, k = k0 + 4 * kq;
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < rows) {
            if (KMAJ) {
                const float* p = P + (long)k + (long)r * ld;
                if (vec && k + 3 < K) {
                    x = *reinterpret_cast<const float4*>(p);
                } else {
                    if (k + 0 < K) x.x = p[0];
                    if (k + 1 < K) x.y = p[1];
                    if (k + 2 < K) x.z = p[2];
                    if (k + 3 < K) x.w = p[3];
                }
            } else {
                const float* p = P + (long)r + (long)k * ld;
                if (k + 0 < K) x.x = p[0];
                if (k + 1 < K) x.y = p[ld];
                if (k + 2 < K) x.z = p[2 * ld];
                if (k + 3 < K) x.w = p[3 * ld];
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
    uint32_t o[ROWS * KQ / NT];
};

// byte offsets of this thread's cells of the tile at rows r0.., k step 0
template <bool KMAJ, int ROWS>
__device__ __forceinline__ TileOffsets<KMAJ, ROWS> tile_offsets(long ld, int r0) {
    TileOffsets<KMAJ, ROWS> t;
#pragma unroll
    for (int q = 0; q < ROWS * KQ / NT; ++q) {
        int rr, kq;
        cell_of<KMAJ, ROWS>(threadIdx.x + NT * q, rr, kq);
        const long e = KMAJ ? (long)(4 * kq) + (long)(r0 + rr) * ld : (long)(r0 + rr) + (long)(4 * kq) * ld;
        t.o[q] = (uint32_t)(e * 4);
    }
    return t;
}

// soff: byte offset of K step k0 (k0 * ld * 4 for KMAJ = false, k0 * 4 for KMAJ = true);
// ld4 = ld * 4 (the byte stride between consecutive k of a rows-contiguous operand)
template <bool KMAJ, int ROWS>
__device__ __forceinline__ void load_tile_full(Stage<ROWS>& st, __amdgpu_buffer_rsrc_t r, const TileOffsets<KMAJ, ROWS>& to,
                                               uint32_t soff, uint32_t ld4) {
#pragma unroll
    for (int q = 0; q < ROWS * KQ / NT; ++q) {
        if (KMAJ) {
            const v4f x = __builtin_amdgcn_raw_buffer_load_b128(r, to.o[q], soff, 0);
            st.v[q] = make_float4(x.x, x.y, x.z, x.w);
        } else {
            st.v[q].x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, to.o[q], soff, 0));
            st.v[q].y = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, to.o[q], soff + ld4, 0));
            st.v[q].z = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, to.o[q], soff + 2 * ld4, 0));
            st.v[q].w = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, to.o[q], soff + 3 * ld4, 0));
        }
    }
}

// Registers -> LDS tile in the quad layout (one 16-byte store per cell)
template <bool KMAJ, int ROWS>
__device__ __forceinline__ void store_tile(const Stage<ROWS>& st, float* __restrict__ S) {
#pragma unroll
    for (int q = 0; q < ROWS * KQ / NT; ++q) {
        int rr, kq;
        cell_of<KMAJ, ROWS>(threadIdx.x + NT * q, rr, kq);
        *reinterpret_cast<float4*>(S + kq * ldq<ROWS>() + rr * 4) = st.v[q];
    }
}

// an epilogue that only accumulates declares `static constexpr bool kAtomic = true` and an
// atomic(m, n, v) (dual: atomic(m, n, p, q)) adding into its output
template <class E, class = void>
struct has_atomic : std::false_type {};
template <class E>
struct has_atomic<E, std::void_t<decltype(E::kAtomic)>> : std::integral_constant<bool, E::kAtomic> {};
// an epilogue whose load(m, n) depends on m only (a bias per row) declares
// `static constexpr bool kRowLoad = true`: the block reads its rows' values before the main
// loop, so that their latency is hidden under the products
template <class E, class = void>
struct has_row_load : std::false_type {};
template <class E>
struct has_row_load<E, std::void_t<decltype(E::kRowLoad)>> : std::integral_constant<bool, E::kRowLoad> {};

template <int... U, class F>
__device__ __forceinline__ void unroll_seq(std::integer_sequence<int, U...>, F&& f) {
    (f(std::integral_constant<int, U>{}), ...);
}

#ifndef STADE_GEMM_PF
#define STADE_GEMM_PF 2
#endif

// DUAL: the two segments share K and their operands are read in the same K steps, giving two
// outputs from three products,
//   P = A0 B0,   Q = A0 B1 + A1 B0,
// (a tangent pair such as s1 = W1 x, s1d = W1 xd + W1d x) with each operand tile loaded once.
// The epilogue then takes both: load(m, n) returns a float2 of old values and
// operator()(m, n, p, q, old) writes.
// LDS floats of one block: two buffers of the A and B operand tiles (DUAL: two of each)
template <int BNT, bool DUAL>
constexpr int smem_floats() {
    return 2 * (DUAL ? 2 : 1) * KQ * (ldq<BM>() + ldq<BNT>());
}

// One block of the product: the tile at (bx, by) of slice bz, with its LDS at smem.
template <bool A_KM, bool B_KM, int BNT, class Epi, bool DUAL>
__device__ __forceinline__ void gemm_block(const Args& g, bool vec, const Epi& epi, int bx, int by, int bz, float* smem) {
    constexpr int NJ = BNT / 64, LQA = ldq<BM>(), LQB = ldq<BNT>();
    constexpr int NOP = DUAL ? 2 : 1;  // operand pairs staged per step
    auto As = reinterpret_cast<float(*)[NOP][KQ * LQA]>(smem);
    auto Bs = reinterpret_cast<float(*)[NOP][KQ * LQB]>(smem + 2 * NOP * KQ * LQA);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m0 = bx * BM, n0 = by * BNT;
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

    // the K steps of all segments, in order (DUAL: of the shared K); this block's slice of them
    const int steps0 = (K0 + KT - 1) / KT;
    const int total = DUAL ? steps0 : steps0 + (K1 + KT - 1) / KT;
    const int t_begin = (int)((long)total * bz / g.ksplit);
    const int t_end = (int)((long)total * (bz + 1) / g.ksplit);
    // a block whose tiles all lie inside the operands (M, N and every K step) loads with no
    // per-element tests
    const bool full = vec && g.bufok && m0 + BM <= g.M && n0 + BNT <= g.N && K0 % KT == 0 && K1 % KT == 0;
    // buffer resources of both segments' operands and this thread's offsets (the segments
    // share lda and ldb when bufok is set)
    const __amdgpu_buffer_rsrc_t rA0 = operand_rsrc(A0), rA1 = operand_rsrc(A1);
    const __amdgpu_buffer_rsrc_t rB0 = operand_rsrc(B0), rB1 = operand_rsrc(B1);
    const TileOffsets<A_KM, BM> offA = tile_offsets<A_KM, BM>(lda0, m0);
    const TileOffsets<B_KM, BNT> offB = tile_offsets<B_KM, BNT>(ldb0, n0);

    floatx16 acc[NOP][2][NJ];  // DUAL: [0] P, [1] Q
#pragma unroll
    for (int o = 0; o < NOP; ++o)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[o][i][j][r] = 0.f;

    // PF register stages: the global loads of step t+PF are issued at step t, and the stage
    // holding step t+1 (loaded at step t+1-PF) goes to LDS in the middle of step t, so a load
    // has PF - 1 steps of matrix-core work to arrive.  Loads and stores are unconditional (a
    // step past the slice reloads its last step, whose data is never read) so that the
    // compiler waits only for the oldest stage.
    constexpr int PF = STADE_GEMM_PF;
    Stage<BM> sa[PF][NOP];
    Stage<BNT> sb[PF][NOP];
    auto load = [&](int p, int t, bool fast) {
        t = t < t_end ? t : t_end - 1;
        if constexpr (DUAL) {
            const int k0 = t * KT;
            if (fast) {
                const uint32_t sa_off = (uint32_t)((A_KM ? (long)k0 : (long)k0 * lda0) * 4);
                const uint32_t sb_off = (uint32_t)((B_KM ? (long)k0 : (long)k0 * ldb0) * 4);
                load_tile_full<A_KM, BM>(sa[p][0], rA0, offA, sa_off, (uint32_t)(lda0 * 4));
                load_tile_full<A_KM, BM>(sa[p][1], rA1, offA, sa_off, (uint32_t)(lda0 * 4));
                load_tile_full<B_KM, BNT>(sb[p][0], rB0, offB, sb_off, (uint32_t)(ldb0 * 4));
                load_tile_full<B_KM, BNT>(sb[p][1], rB1, offB, sb_off, (uint32_t)(ldb0 * 4));
            } else {
                load_tile<A_KM, BM>(sa[p][0], A0, lda0, g.M, K0, m0, k0, vec);
                load_tile<A_KM, BM>(sa[p][1], A1, lda1, g.M, K0, m0, k0, vec);
                load_tile<B_KM, BNT>(sb[p][0], B0, ldb0, g.N, K0, n0, k0, vec);
                load_tile<B_KM, BNT>(sb[p][1], B1, ldb1, g.N, K0, n0, k0, vec);
            }
        } else {
            const bool s1 = t >= steps0;
            const float* A = s1 ? A1 : A0;
            const float* B = s1 ? B1 : B0;
            const long lda = s1 ? lda1 : lda0, ldb = s1 ? ldb1 : ldb0;
            const int K = s1 ? K1 : K0;
            const int k0 = (s1 ? t - steps0 : t) * KT;
            if (fast) {
                const uint32_t sa_off = (uint32_t)((A_KM ? (long)k0 : (long)k0 * lda0) * 4);
                const uint32_t sb_off = (uint32_t)((B_KM ? (long)k0 : (long)k0 * ldb0) * 4);
                load_tile_full<A_KM, BM>(sa[p][0], s1 ? rA1 : rA0, offA, sa_off, (uint32_t)(lda0 * 4));
                load_tile_full<B_KM, BNT>(sb[p][0], s1 ? rB1 : rB0, offB, sb_off, (uint32_t)(ldb0 * 4));
            } else {
                load_tile<A_KM, BM>(sa[p][0], A, lda, g.M, K, m0, k0, vec);
                load_tile<B_KM, BNT>(sb[p][0], B, ldb, g.N, K, n0, k0, vec);
            }
        }
    };
    auto store = [&](int rs, int buf) {
#pragma unroll
        for (int o = 0; o < NOP; ++o) {
            store_tile<A_KM, BM>(sa[rs][o], As[buf][o]);
            store_tile<B_KM, BNT>(sb[rs][o], Bs[buf][o]);
        }
    };
    // the epilogue's per-row values, read now when they depend on the row only (kRowLoad)
    using Pre = decltype(epi.load(0, 0));
    Pre prow[2] = {};
    if constexpr (has_row_load<Epi>::value) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int m = m0 + wm + i * 32 + (lane & 31);
            if (m < g.M) prow[i] = epi.load(m, 0);
        }
    }
    auto mainloop = [&](auto fast_tag) {
        constexpr bool FAST = decltype(fast_tag)::value;
        if (t_begin >= t_end) return;
#pragma unroll
        for (int q = 0; q < PF; ++q) load(q, t_begin + q, FAST);
        store(0, 0);
        __syncthreads();
        // fragments of a step in registers: F[p] is read from LDS buffer p during the step
        // before (after its barrier), so the LDS latency hides behind half a step of MFMAs.
        // The MFMA's k index (lane / 32) selects the k-plane: MFMA 4 h + c of the step takes
        // k = 4 (2 h + lane / 32) + c, the same for both operands, so the KT / 2 MFMAs cover
        // the KT k of the step once each.
        constexpr int NH = KT / 8;
        v4f fa[2][NH][NOP][2], fb[2][NH][NOP][NJ];  // [buffer][plane pair][operand][tile]
        auto read_frags = [&](auto p_tag) {
            constexpr int p = decltype(p_tag)::value;
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const int kq = 2 * h + (lane >> 5);
#pragma unroll
                for (int o = 0; o < NOP; ++o) {
#pragma unroll
                    for (int i = 0; i < 2; ++i)
                        fa[p][h][o][i] = *reinterpret_cast<const v4f*>(As[p][o] + kq * LQA + (wm + i * 32 + (lane & 31)) * 4);
#pragma unroll
                    for (int j = 0; j < NJ; ++j)
                        fb[p][h][o][j] = *reinterpret_cast<const v4f*>(Bs[p][o] + kq * LQB + (wn + j * 32 + (lane & 31)) * 4);
                }
            }
        };
        // the MFMAs of plane pairs [h0, h1) of fragments F[p] (DUAL: P += A0 B0,
        // Q += A0 B1 + A1 B0; the operands are swapped, B first)
        // (a tile edge block skips the MFMAs of its 32 x 32 tiles that lie wholly past M or N:
        // wave-uniform tests, compile-time true in whole blocks; those accumulators stay zero
        // and are never stored)
        bool live_i[2], live_j[NJ];
#pragma unroll
        for (int i = 0; i < 2; ++i) live_i[i] = FAST || m0 + wm + 32 * i < g.M;
#pragma unroll
        for (int j = 0; j < NJ; ++j) live_j[j] = FAST || n0 + wn + 32 * j < g.N;
        auto mma = [&](auto p_tag, int h0, int h1) {
            constexpr int p = decltype(p_tag)::value;
#pragma unroll
            for (int h = h0; h < h1; ++h)
#pragma unroll
                for (int c = 0; c < 4; ++c)
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < NJ; ++j) {
                            if (!(live_i[i] && live_j[j])) continue;
                            acc[0][i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[p][h][0][j][c], fa[p][h][0][i][c], acc[0][i][j], 0, 0, 0);
                            if constexpr (DUAL) {
                                acc[1][i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[p][h][1][j][c], fa[p][h][0][i][c], acc[1][i][j], 0, 0, 0);
                                acc[1][i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[p][h][0][j][c], fa[p][h][1][i][c], acc[1][i][j], 0, 0, 0);
                            }
                        }
        };
        read_frags(std::integral_constant<int, 0>{});
        // step t with register stage rs = (t - t_begin) % PF and LDS buffer / fragments
        // p = (t - t_begin) % 2: first half of the MFMAs, the next stage to LDS and the
        // barrier, the next step's fragments, second half.
        auto step = [&](int t, auto rs_tag, auto p_tag) {
            constexpr int rs = decltype(rs_tag)::value, cur = decltype(p_tag)::value;
            constexpr std::integral_constant<int, cur ^ 1> nxt{};
            load(rs, t + PF, FAST);
            mma(p_tag, 0, NH / 2);
            __builtin_amdgcn_sched_barrier(0);
            store((rs + 1) % PF, cur ^ 1);
            __syncthreads();
            // a step past the slice reads its clamped reload, never used
            read_frags(nxt);
            __builtin_amdgcn_sched_barrier(0);
            mma(p_tag, NH / 2, NH);
            __builtin_amdgcn_sched_barrier(0);
        };
        // unrolled over a whole cycle of both rings, so every index is a compile-time constant
        constexpr int UL = PF % 2 == 0 ? PF : 2 * PF;
        for (int t = t_begin; t < t_end; t += UL) {
            unroll_seq(std::make_integer_sequence<int, UL>{}, [&](auto u) {
                constexpr int U = decltype(u)::value;
                if (U == 0 || t + U < t_end)
                    step(t + U, std::integral_constant<int, U % PF>{}, std::integral_constant<int, U % 2>{});
            });
        }
    };
    if (full) mainloop(std::true_type{});
    else mainloop(std::false_type{});
    // accumulator (i, j, r): m = m0 + wm + 32 i + lane % 32,  n = n0 + wn + 32 j + 8 (r / 4) + 4 (lane / 32) + r % 4
    if constexpr (has_atomic<Epi>::value) {
        if (g.ksplit > 1 && g.atomic) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int m = m0 + wm + i * 32 + (lane & 31);
                if (m >= g.M) continue;
#pragma unroll
                for (int j = 0; j < NJ; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int n = n0 + wn + j * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                        if (n < g.N) {
                            if constexpr (DUAL)
                                epi.atomic(m, n, acc[0][i][j][r], acc[NOP - 1][i][j][r]);
                            else
                                epi.atomic(m, n, acc[0][i][j][r]);
                        }
                    }
            }
            return;
        }
    }
    if (g.ksplit > 1) {
        // slice z at part + z * NOP * M * N (DUAL: P then Q)
        const long mn = (long)g.M * g.N;
        float* part = g.part + (long)bz * NOP * mn;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int m = m0 + wm + i * 32 + (lane & 31);
            if (m >= g.M) continue;
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int n = n0 + wn + j * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                    if (n < g.N) {
#pragma unroll
                        for (int o = 0; o < NOP; ++o) part[o * mn + m + (long)n * g.M] = acc[o][i][j][r];
                    }
                }
        }
        return;
    }
    // the epilogue's inputs (e.g. C of C += v) for the whole tile first, then the stores: the
    // output may alias them as far as the compiler knows, and interleaving would serialise one
    // memory round trip per element
    Pre pre[2][NJ][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm + i * 32 + (lane & 31);
                const int n = n0 + wn + j * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                if constexpr (has_row_load<Epi>::value)
                    pre[i][j][r] = prow[i];
                else
                    pre[i][j][r] = (m < g.M && n < g.N) ? epi.load(m, n) : Pre{};
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
                if (n < g.N) {
                    if constexpr (DUAL)
                        epi(m, n, acc[0][i][j][r], acc[NOP - 1][i][j][r], pre[i][j][r]);
                    else
                        epi(m, n, acc[0][i][j][r], pre[i][j][r]);
                }
            }
    }
}

template <bool A_KM, bool B_KM, int BNT, class Epi, bool DUAL = false>
__global__ __launch_bounds__(NT) void gemm_kernel(Args g, bool vec, Epi epi) {
    __shared__ __attribute__((aligned(16))) float smem[smem_floats<BNT, DUAL>()];
    gemm_block<A_KM, B_KM, BNT, Epi, DUAL>(g, vec, epi, blockIdx.x, blockIdx.y, blockIdx.z, smem);
}

// Two products in one launch, each block one tile of one of them: blocks [0, nblocks(P0))
// are P0's (m tiles fastest, then n tiles, then K slices), the rest P1's.  Neither may need a
// second kernel (a K split adds by atomics).  The two share the CUs, so the tail of one is
// filled by blocks of the other.
template <bool A_KM, bool B_KM, class Epi>
struct Part {
    Args g;
    bool vec;
    Epi epi;
    int gx, gy;  // tile grid: m tiles, n tiles (slices: g.ksplit)
};
//
// X: independent work that rides along as x.count extra blocks at the front of the grid, each
// calling x(block, smem) with NT threads and at least 1088 floats of LDS (NoExtra: none).
struct NoExtra {
    int count = 0;
    __device__ __forceinline__ void operator()(int, float*) const {}
};
template <class X>
__global__ __launch_bounds__(NT) void extra_kernel(X x) {
    __shared__ __attribute__((aligned(16))) float smem[1088];
    x(blockIdx.x, smem);
}
template <int BNT, bool DUAL, bool A0, bool B0, class E0, bool A1, bool B1, class E1, class X>
__global__ __launch_bounds__(NT) void gemm_pair_kernel(Part<A0, B0, E0> p0, Part<A1, B1, E1> p1, X x) {
    static_assert(smem_floats<BNT, DUAL>() >= 1088, "the extra blocks' LDS");
    __shared__ __attribute__((aligned(16))) float smem[smem_floats<BNT, DUAL>()];
    const int n0 = p0.gx * p0.gy * p0.g.ksplit;
    int b = blockIdx.x;
    if (b < x.count) {
        x(b, smem);
        return;
    }
    b -= x.count;
    if (b < n0) {
        const int per = p0.gx * p0.gy, r = b % per;
        gemm_block<A0, B0, BNT, E0, DUAL>(p0.g, p0.vec, p0.epi, r % p0.gx, r / p0.gx, b / per, smem);
    } else {
        b -= n0;
        const int per = p1.gx * p1.gy, r = b % per;
        gemm_block<A1, B1, BNT, E1, DUAL>(p1.g, p1.vec, p1.epi, r % p1.gx, r / p1.gx, b / per, smem);
    }
}

// second stage of a split-K product: C(m, n) = sum over slices in order, then the epilogue
// (DUAL: P and Q, each summed in slice order)
template <class Epi, bool DUAL = false>
__global__ __launch_bounds__(NT) void splitk_reduce_kernel(const float* __restrict__ part, int ksplit, int M, int N, Epi epi) {
    constexpr int NOP = DUAL ? 2 : 1;
    const long q = (long)blockIdx.x * NT + threadIdx.x;
    const long mn = (long)M * N;
    if (q >= mn) return;
    // every slice's value in flight at once (ksplit <= 16; indices past the last slice clamped
    // to it and never added), added in slice order
    const int m = (int)(q % M), n = (int)(q / M);
    float v[NOP][16];
#pragma unroll
    for (int o = 0; o < NOP; ++o)
#pragma unroll
        for (int z = 0; z < 16; ++z) v[o][z] = part[(long)min(z, ksplit - 1) * NOP * mn + o * mn + q];
    const auto old = epi.load(m, n);
    __builtin_amdgcn_sched_barrier(0);
    float s[NOP];
#pragma unroll
    for (int o = 0; o < NOP; ++o) {
        s[o] = v[o][0];
#pragma unroll
        for (int z = 1; z < 16; ++z)
            if (z < ksplit) s[o] += v[o][z];
    }
    if constexpr (DUAL)
        epi(m, n, s[0], s[NOP - 1], old);
    else
        epi(m, n, s[0], old);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Tile width and K split for an M x N x K product on `cus` compute units, from a cost model
// in microseconds: the CU with the most blocks sets the time (blocks per CU x K steps per
// block x the time of one block step, about 0.7 us for a 128 x 64 x 16 step measured on
// MI355X at two resident blocks per CU), scaled by the rate at the CU's residency (one
// block: 3/4, one wave per SIMD hides no latency; three: 1.08; four or more: 1.13, measured
// on the MLP's products), and a K split costs its partial tiles' round trip through memory
// (8 bytes per element and slice at about 5 TB/s) plus the reduction launch, or, by atomics,
// their atomic traffic (4 bytes per element and slice, overlapped with the other blocks'
// work: about 10 TB/s of issue).  Every K slice keeps at least 8 steps.  Ties go to the
// narrow tile and the smaller split.
struct Plan {
    int bnt, ksplit;
    bool atomic;  // the slices are added into the output by atomics (an accumulate epilogue)
};
#ifndef STADE_GEMM_STEP_US
#define STADE_GEMM_STEP_US 0.7
#endif
// nout = 2 plans a dual product (three products per step over shared loads, two outputs).
// atomic_ok: the epilogue only accumulates, so a split may add its slices by atomics (no
// partial tiles, no reduction launch).
#ifndef STADE_GEMM_ATOMIC_GBS
#define STADE_GEMM_ATOMIC_GBS 10000.0
#endif
inline Plan plan(int M, int N, int Ktot, int cus, int nout = 1, bool atomic_ok = false) {
    const double work = nout == 2 ? 2.5 : 1.0;  // block-step time relative to a single product
    const long mt = (M + BM - 1) / BM;
    const long steps = (Ktot + KT - 1) / KT;
    Plan best{64, 1, false};
    double best_cost = 0.0;
    // (a dual product keeps the narrow tile: with the wide one its registers allow one wave per SIMD)
    for (int bnt = 64; bnt <= (nout == 2 ? 64 : 128); bnt *= 2) {
        const long tiles = mt * ((N + bnt - 1) / bnt);
        for (int ks = 1; ks <= 16; ++ks) {
            if (ks > 1 && steps / ks < 8) break;
            const long per_cu = (tiles * ks + cus - 1) / cus;
            const long st = (steps + ks - 1) / ks;
            // an atomic split is kept to one round of resident blocks (four per CU)
            if (atomic_ok && ks > 1 && per_cu > 4) break;
            double cost = (double)per_cu * st * STADE_GEMM_STEP_US * (KT / 16.0) * (bnt / 64) * work;
            cost /= per_cu < 2 ? 0.75 : per_cu == 2 ? 1.0 : per_cu == 3 ? 1.08 : 1.13;
            if (ks > 1) cost += atomic_ok ? 4.0 * ks * nout * (double)M * N / (STADE_GEMM_ATOMIC_GBS * 1e3)
                                          : 8.0 * ks * nout * (double)M * N / 5e6 + 3.0;
            if (cost < best_cost || best_cost == 0.0) {
                best_cost = cost;
                best = Plan{bnt, ks, atomic_ok && ks > 1};
            }
        }
    }
    return best;
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

// Launch; returns the hipError of the launch.  `part` must hold ksplit * M * N floats (DUAL:
// twice that) when the plan splits K (ask with plan() first); it may be null otherwise.  A
// dual product takes two segments of the same K.
// the launch-time fields of g (split, atomic, buffer-load eligibility); vec: every operand
// 16-byte aligned with leading dimensions a multiple of 4
template <bool A_KM, bool B_KM, class Epi, bool DUAL>
hipError_t prepare(Args& g, bool& vec, const Plan& p) {
    if (DUAL && (g.nseg != 2 || g.seg[0].K != g.seg[1].K)) return hipErrorInvalidValue;
    vec = true;
    for (int s = 0; s < g.nseg; ++s) {
        vec = vec && aligned16(g.seg[s].A) && aligned16(g.seg[s].B) && g.seg[s].lda % 4 == 0 && g.seg[s].ldb % 4 == 0;
    }
    g.ksplit = p.ksplit;
    g.atomic = p.atomic && has_atomic<Epi>::value;
    if (p.ksplit > 1 && !g.atomic && !g.part) return hipErrorInvalidValue;
    // byte extent of each operand: A spans K columns of lda (A_KM = false) or M columns,
    // B spans N columns of ldb (B_KM = true) or K columns
    g.bufok = g.nseg == 1 || (g.seg[0].lda == g.seg[1].lda && g.seg[0].ldb == g.seg[1].ldb);
    for (int s = 0; s < g.nseg; ++s) {
        const double ea = (double)g.seg[s].lda * (A_KM ? g.M : g.seg[s].K) * 4.0;
        const double eb = (double)g.seg[s].ldb * (B_KM ? g.N : g.seg[s].K) * 4.0;
        g.bufok = g.bufok && ea < 2147483648.0 && eb < 2147483648.0;
    }
    return hipSuccess;
}

template <bool A_KM, bool B_KM, class Epi, bool DUAL = false>
hipError_t launch(Args g, Epi epi, hipStream_t stream, const Plan& p) {
    if (g.M <= 0 || g.N <= 0) return hipSuccess;
    bool vec = true;
    if (hipError_t e = prepare<A_KM, B_KM, Epi, DUAL>(g, vec, p)) return e;
    if (p.bnt == 128) {
        dim3 grid((g.M + BM - 1) / BM, (g.N + 127) / 128, p.ksplit);
        gemm_kernel<A_KM, B_KM, 128, Epi, DUAL><<<grid, NT, 0, stream>>>(g, vec, epi);
    } else {
        dim3 grid((g.M + BM - 1) / BM, (g.N + 63) / 64, p.ksplit);
        gemm_kernel<A_KM, B_KM, 64, Epi, DUAL><<<grid, NT, 0, stream>>>(g, vec, epi);
    }
    if (p.ksplit > 1 && !g.atomic) {
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        const long mn = (long)g.M * g.N;
        splitk_reduce_kernel<Epi, DUAL><<<(unsigned)((mn + NT - 1) / NT), NT, 0, stream>>>(g.part, p.ksplit, g.M, g.N, epi);
    }
    return hipGetLastError();
}

// Dynamic LDS that caps a kernel using `static_bytes` of LDS per block at `blocks` resident
// blocks per CU (160 KiB of LDS per CU on gfx950); 0 when blocks <= 0.
inline size_t lds_cap_bytes(size_t static_bytes, int blocks) {
    constexpr size_t kLdsPerCu = 160 * 1024;
    if (blocks <= 0) return 0;
    size_t per = kLdsPerCu / (size_t)(blocks + 1) + 1;  // more than a (blocks + 1)-th of the CU's LDS
    per = (per + 255) / 256 * 256;
    return per > static_bytes ? per - static_bytes : 0;
}

// Two products as one launch (gemm_pair_kernel) when both plans use the narrow tile and
// neither needs a second kernel; otherwise one launch each.  Both are enqueued on `stream`.
// max_blocks > 0 caps the paired launch at that many resident blocks per CU (by LDS).
template <bool A0, bool B0, class E0, bool A1, bool B1, class E1, bool DUAL = false, class X = NoExtra>
hipError_t launch_pair(Args g0, E0 e0, const Plan& p0, Args g1, E1 e1, const Plan& p1, hipStream_t stream, X x = X{},
                       int max_blocks = 0) {
    const bool one0 = p0.ksplit == 1 || (p0.atomic && has_atomic<E0>::value);
    const bool one1 = p1.ksplit == 1 || (p1.atomic && has_atomic<E1>::value);
    if (g0.M <= 0 || g0.N <= 0 || g1.M <= 0 || g1.N <= 0 || p0.bnt != 64 || p1.bnt != 64 || !one0 || !one1) {
        if (x.count > 0) {
            extra_kernel<X><<<(unsigned)x.count, NT, 0, stream>>>(x);
            if (hipError_t e = hipGetLastError()) return e;
        }
        if (hipError_t e = launch<A0, B0, E0, DUAL>(g0, e0, stream, p0)) return e;
        return launch<A1, B1, E1, DUAL>(g1, e1, stream, p1);
    }
    Part<A0, B0, E0> q0{g0, true, e0, (g0.M + BM - 1) / BM, (g0.N + 63) / 64};
    Part<A1, B1, E1> q1{g1, true, e1, (g1.M + BM - 1) / BM, (g1.N + 63) / 64};
    if (hipError_t e = prepare<A0, B0, E0, DUAL>(q0.g, q0.vec, p0)) return e;
    if (hipError_t e = prepare<A1, B1, E1, DUAL>(q1.g, q1.vec, p1)) return e;
    const long nb = (long)x.count + (long)q0.gx * q0.gy * p0.ksplit + (long)q1.gx * q1.gy * p1.ksplit;
    const size_t dyn = lds_cap_bytes(sizeof(float) * smem_floats<64, DUAL>(), max_blocks);
    gemm_pair_kernel<64, DUAL, A0, B0, E0, A1, B1, E1, X><<<(unsigned)nb, NT, dyn, stream>>>(q0, q1, x);
    return hipGetLastError();
}

}  // namespace gemm
}  // namespace stade
