// Matrix-core (MFMA) and buffer-load helpers shared by the gfx950 kernel
// files (conv_mfma.hip, adapter.hip).
//
// MFMA lane layout of v_mfma_f32_16x16x32_{f16,bf16} (16x16 output tile,
// 64 lanes): lane l supplies row l%16 of A and column l%16 of B with 8
// reduction values at slot l/16; it receives C[(l/16)*4 + j][l%16], j = 0..3.
#pragma once

#include "sv_common.h"

namespace svtad {

typedef unsigned short u16;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <typename T> struct MfmaOp;
template <> struct MfmaOp<f16> {
    static __device__ __forceinline__ f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
    }
};
template <> struct MfmaOp<bf16> {
    static __device__ __forceinline__ f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    }
};

constexpr int KS = 32;     // reduction values per step
constexpr int PITCH = 40;  // LDS row pitch in 16-bit elements

// Buffer loads: a raw buffer resource over [base, base + bytes); a load whose
// offset is at or beyond `bytes` returns zeros without touching memory, so
// missing neighbors and tile edges need neither branches nor a zero row.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kOOB = 0x80000000u;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Workgroup -> tile mapping that keeps consecutive tiles on one XCD.
// Workgroups are dispatched round-robin over the 8 XCDs (wg b runs on XCD
// b % 8); tile t = (XCD-major rank of b) so XCD x owns a contiguous range of
// tiles and the rows those tiles gather stay in its L2.
__device__ __forceinline__ int64_t xcd_tile(int64_t b, int64_t g) {
    const int64_t q = g >> 3, r = g & 7, x = b & 7, j = b >> 3;
    return x * q + (x < r ? x : r) + j;
}

}  // namespace svtad
