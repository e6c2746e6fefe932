// The general lowering's matrix products (stade_hip/lower/contract.py): a contraction of the
// generated code run by the fp32 matrix-core GEMM (gemm_f32.hpp), whose output is any strided
// array element C[m * sm + n * sn] (the pointer already at the product's first element).
#pragma once

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
