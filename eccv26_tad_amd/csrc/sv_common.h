// Shared device helpers for the SparseConv2D HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/svtad_sparse.h"

namespace svtad {

typedef _Float16 f16;
typedef __bf16 bf16;

// Accumulator type: fp64 for fp64 data, fp32 otherwise.
template <typename T> struct Acc { typedef float type; };
template <> struct Acc<double> { typedef double type; };

template <typename A, typename T> __device__ __forceinline__ A to_acc(T v) { return (A)v; }
template <> __device__ __forceinline__ float to_acc<float, bf16>(bf16 v) { return (float)v; }

// Round-to-nearest-even conversion from the accumulator to the storage type.
template <typename T, typename A> __device__ __forceinline__ T from_acc(A v) { return (T)v; }

// Source row of neighbor entry (i, k): -1 when missing, out of range, or
// negative. tpb > 0 adds the per-row batch offset (i / tpb) * tpb.
__device__ __forceinline__ int64_t src_row(const int32_t* __restrict__ nbr, int64_t i, int k,
                                           int64_t n, int64_t tpb) {
    int32_t v = nbr[i * 9 + k];
    if (v < 0) return -1;
    int64_t r = (int64_t)v + (tpb > 0 ? (i / tpb) * tpb : 0);
    return r < n ? r : -1;
}

// Row j's source for offset k of the transposed table, taken from the
// symmetric partner: i = src(j, 8-k), accepted only if src(i, k) == j. Every
// table entry (i, k) -> j is thereby claimed exactly once, either here (when
// its transpose is present) or by the orphan pass.
__device__ __forceinline__ int64_t src_row_t(const int32_t* __restrict__ nbr, int64_t j, int k,
                                             int64_t n, int64_t tpb) {
    int64_t i = src_row(nbr, j, 8 - k, n, tpb);
    if (i < 0) return -1;
    return src_row(nbr, i, k, n, tpb) == j ? i : -1;
}

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace svtad
