// Dense GEMMs of the sparse-conv adapter with fused epilogues (gfx950 MFMA).
//
// The adapter around SparseConv2D (reference
// opentad/models/backbones/vit_sparse_adapter_poguise.py:305-362,652-653) is
//   u = x W_d^T + b_d,  g = GELU(u)      (down_proj, act)
//   split g into special tokens and patch tokens; patches -> SparseConv2D
//   c = cat(special, conv(patches))
//   y = (c W_u^T + b_u) * gamma + x      (up_proj, gamma, residual)
// Both GEMMs read their operands with the reduction index contiguous (token
// rows and nn.Linear's (out, in) weight rows), so the LDS tiles need no
// transposes. The epilogues remove the activation round trips of the
// unfused chain:
//  * down: bias, the rounding of the Linear output, GELU, and the split: u is
//    written (autograd keeps it for the GELU backward) and GELU(u) goes
//    straight into a special-token buffer and a contiguous patch buffer (the
//    SparseConv2D input), so there is no GELU pass and no slice copy;
//  * up: the A rows come from the special-token buffer and the SparseConv2D
//    output in place of the concatenation, and bias, gamma and the residual
//    are applied before the single store (no cat, no scale pass, no add pass).
// Roundings follow the unfused chain in the same dtype: the Linear output is
// rounded to T, GELU is evaluated in fp32 on the rounded value, z * gamma is
// rounded to T before the residual add.
#include "sv_common.h"
#include "sv_conv.h"
#include "sv_internal.h"
#include "sv_mfma.h"

namespace svtad {

enum { EPI_DOWN_GELU = 0, EPI_UP_SCALE_RES = 1 };

// Row m of a [batch, n_tokens, *] token tensor as a special-token row
// (b * n_special + r) or a patch row (b * n_patch + r - n_special).
// Rows are below 2^31 (checked on the host), so the division is 32-bit.
struct RowMap {
    int64_t n_tokens, n_special, n_patch;
    __device__ __forceinline__ int64_t split(int64_t m, bool& special) const {
        const uint32_t b = (uint32_t)m / (uint32_t)n_tokens;
        const int64_t r = m - (int64_t)b * n_tokens;
        special = r < n_special;
        return special ? (int64_t)b * n_special + r : (int64_t)b * n_patch + (r - n_special);
    }
};

constexpr int cmax_i(int a, int b) { return a > b ? a : b; }

__device__ __forceinline__ float gelu_erf(float u) { return 0.5f * u * (1.0f + erff(u * 0.70710678118654752f)); }

// out = epilogue(A W^T + bias): A [m_rows, k_red], W [n_out, k_red]. Four waves
// as 2 x 2, each with FM x FN fragments: a BM = 32 FM by BN = 32 FN tile,
// BK reduction values per stage (BK / 32 MFMA steps between barriers). The
// weight fragment is the MFMA's A operand, so a lane accumulates 4
// consecutive output columns of one row.
// LDS rows are BK + 8 elements: for BK = 64 (144 bytes) and BK = 32 (80
// bytes) the 16 rows one fragment read touches fall on distinct bank groups.
// Global rows of the output and residual are moved as 16-byte pieces.
//
// MIX (up epilogue only) takes gamma, the residual and the output each in T
// or in fp32, as `mix` says (MIX_GAMMA_F32, MIX_RES_F32, MIX_OUT_F32): the
// dtypes of the reference chain under autocast, where gamma is an fp32
// parameter, so z * gamma is an fp32 product of the rounded z (no rounding
// to T), and the residual add is in fp32; the sum is stored as fp32 or
// rounded once to T.
enum { MIX_GAMMA_F32 = 1, MIX_RES_F32 = 2, MIX_OUT_F32 = 4 };
template <typename T, int EPI, int FM, int FN, int BK, bool MIX = false>
__global__ __launch_bounds__(256) void k_adapter_gemm(
    const T* __restrict__ a0, const T* __restrict__ a1, const T* __restrict__ w,
    const T* __restrict__ bias, const void* __restrict__ gamma, const void* __restrict__ res,
    T* __restrict__ out0, T* __restrict__ out1, T* __restrict__ out2, int64_t m_rows, int k_red,
    int n_out, RowMap rm, int n_col_tiles, int64_t n_tiles, int mix) {
    constexpr int BM = 2 * FM * 16, BN = 2 * FN * 16;
    constexpr int CPR = BK / 8;                                  // 16-byte chunks per row and stage
    constexpr int LP = BK + 8;                                   // LDS pitch in elements
    constexpr int A_PER = BM * CPR / 256, B_PER = BN * CPR / 256;  // chunks per thread
    static_assert(A_PER * 256 == BM * CPR && B_PER * 256 == BN * CPR, "tile / thread count");
    constexpr int OP = BN + 8;  // pitch (elements) of the output tiles of the epilogue
    constexpr int OPF = BN + 4;  // pitch (floats) of the fp32 tile of the mixed epilogue
    constexpr int SMEM = cmax_i(cmax_i(2 * (BM + BN) * LP, 2 * BM * OP), MIX ? 2 * BM * OPF : 0);
    // one array: the stage buffers, reused by the epilogue's two output tiles
    __shared__ __align__(16) u16 smem[SMEM];
    u16(*const As)[BM][LP] = (u16(*)[BM][LP])smem;
    u16(*const Bs)[BN][LP] = (u16(*)[BN][LP])(smem + 2 * BM * LP);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t tile = xcd_tile(blockIdx.x, n_tiles);
    const int64_t row0 = (tile / n_col_tiles) * BM;
    const int col0 = (int)(tile % n_col_tiles) * BN;

    // the thread's A rows and weight rows. Rows past the end read the last row
    // instead (their outputs are not stored, and an output row depends on its
    // own A row only), so every load is unconditional: a load under a
    // condition becomes a branch, and the branch merge a wait for all loads
    // in flight.
    const T* arow[A_PER];
#pragma unroll
    for (int q = 0; q < A_PER; ++q) {
        const int e = tid + q * 256;
        const int64_t m = min<int64_t>(row0 + e / CPR, m_rows - 1);
        const T* p;
        if constexpr (EPI == EPI_UP_SCALE_RES) {
            bool sp;
            const int64_t r = rm.split(m, sp);
            p = (sp ? a0 : a1) + r * k_red;
        } else {
            p = a0 + m * k_red;
        }
        arow[q] = p + (e % CPR) * 8;
    }
    const T* wrow[B_PER];
#pragma unroll
    for (int q = 0; q < B_PER; ++q) {
        const int e = tid + q * 256;
        wrow[q] = w + (int64_t)(col0 + e / CPR) * k_red + (e % CPR) * 8;
    }

    const int steps = k_red / BK;
    u32x4 ra0[A_PER], rb0[B_PER], ra1[A_PER], rb1[B_PER];
    auto load = [&](int t, u32x4* ra, u32x4* rb) {
#pragma unroll
        for (int q = 0; q < A_PER; ++q) ra[q] = *(const u32x4*)(arow[q] + t * BK);
#pragma unroll
        for (int q = 0; q < B_PER; ++q) rb[q] = *(const u32x4*)(wrow[q] + t * BK);
    };
    auto store = [&](int buf, const u32x4* ra, const u32x4* rb) {
#pragma unroll
        for (int q = 0; q < A_PER; ++q) {
            const int e = tid + q * 256;
            *(u32x4*)&As[buf][e / CPR][(e % CPR) * 8] = ra[q];
        }
#pragma unroll
        for (int q = 0; q < B_PER; ++q) {
            const int e = tid + q * 256;
            *(u32x4*)&Bs[buf][e / CPR][(e % CPR) * 8] = rb[q];
        }
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int wm = wave >> 1, wn = wave & 1;
    const int arw = wm * FM * 16 + (lane & 15), brw = wn * FN * 16 + (lane & 15);
    const int kof = (lane >> 4) * 8;

    auto compute = [&](int buf) {
#pragma unroll
        for (int h = 0; h < BK / KS; ++h) {
            u32x4 fa[FM], fb[FN];
#pragma unroll
            for (int a = 0; a < FM; ++a) fa[a] = *(const u32x4*)&As[buf][arw + a * 16][h * KS + kof];
#pragma unroll
            for (int b = 0; b < FN; ++b) fb[b] = *(const u32x4*)&Bs[buf][brw + b * 16][h * KS + kof];
#pragma unroll
            for (int a = 0; a < FM; ++a)
#pragma unroll
                for (int b = 0; b < FN; ++b) acc[a][b] = MfmaOp<T>::run(fb[b], fa[a], acc[a][b]);
        }
    };
    // Two register sets: the loads of stage t+2 are issued before the MFMAs
    // of stage t, so each load has two stages to arrive. Past the last stage
    // the loads re-read it (clamped index: no conditional loads) and the
    // stores fill a buffer nobody reads.
    const int last = steps - 1;
    load(0, ra0, rb0);
    store(0, ra0, rb0);
    load(min(1, last), ra1, rb1);
    __syncthreads();
    for (int t = 0; t < steps; t += 2) {
        load(min(t + 2, last), ra0, rb0);
        compute(0);
        store(1, ra1, rb1);
        __syncthreads();
        load(min(t + 3, last), ra1, rb1);
        if (t + 1 < steps) compute(1);  // uniform
        store(0, ra0, rb0);
        __syncthreads();
    }

    // epilogue: acc[a][b][j] = C[m][n0 + j] (m = ... + lane % 16, n0 = ... +
    // (lane / 16) * 4). The rounded tile goes through LDS (the stage buffers
    // are free after the last barrier) so that global rows are read and
    // written as 16-byte pieces of 8 consecutive lanes (whole 128-byte lines)
    // rather than 8-byte pieces of 16 rows.
    u16* const tile0 = smem;             // z (down: the Linear output) or T(z * gamma)
    u16* const tile1 = smem + BM * OP;   // down: GELU(z)
    float* const tilef = (float*)smem;   // mixed up epilogue: z * gamma in fp32
    const bool g32 = MIX && (mix & MIX_GAMMA_F32);
    const float gm = EPI != EPI_UP_SCALE_RES ? 0.f
                     : g32 ? *(const float*)gamma : (float)*(const T*)gamma;
#pragma unroll
    for (int b = 0; b < FN; ++b) {
        const int nl = wn * FN * 16 + b * 16 + (lane >> 4) * 4;
        float bv[4] = {0.f, 0.f, 0.f, 0.f};
        if (bias) {
#pragma unroll
            for (int j = 0; j < 4; ++j) bv[j] = (float)bias[col0 + nl + j];
        }
#pragma unroll
        for (int a = 0; a < FM; ++a) {
            const int ml = wm * FM * 16 + a * 16 + (lane & 15);
            u16 z[4], gz[4];
            float zf[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const T zt = (T)(acc[a][b][j] + bv[j]);
                if constexpr (EPI == EPI_DOWN_GELU) {
                    z[j] = __builtin_bit_cast(u16, zt);
                    gz[j] = __builtin_bit_cast(u16, (T)gelu_erf((float)zt));
                } else if constexpr (MIX) {
                    // fp32 product of the rounded z; rounded to T only when gamma is T
                    const float p = f32_rounded((float)zt * gm);
                    zf[j] = g32 ? p : (float)(T)p;
                } else {
                    z[j] = __builtin_bit_cast(u16, (T)((float)zt * gm));
                }
            }
            if constexpr (MIX) {
                *(f32x4*)&tilef[ml * OPF + nl] = f32x4{zf[0], zf[1], zf[2], zf[3]};
                continue;
            }
            *(uint2*)&tile0[ml * OP + nl] = uint2{(unsigned)z[0] | ((unsigned)z[1] << 16),
                                                 (unsigned)z[2] | ((unsigned)z[3] << 16)};
            if constexpr (EPI == EPI_DOWN_GELU)
                *(uint2*)&tile1[ml * OP + nl] = uint2{(unsigned)gz[0] | ((unsigned)gz[1] << 16),
                                                     (unsigned)gz[2] | ((unsigned)gz[3] << 16)};
        }
    }
    __syncthreads();
    constexpr int RC = BN / 8;  // 16-byte chunks per tile row
#pragma unroll
    for (int c = tid; c < BM * RC; c += 256) {
        const int ml = c / RC, nc = (c % RC) * 8;
        const int64_t m = row0 + ml;
        if (m >= m_rows) continue;
        if constexpr (MIX) {
            // y = z * gamma + residual in fp32, stored as fp32 or rounded once
            // (the fp32 sum, then the cast)
            float y[8];
            const f32x4 p0 = *(const f32x4*)&tilef[ml * OPF + nc], p1 = *(const f32x4*)&tilef[ml * OPF + nc + 4];
            const int64_t off = m * n_out + col0 + nc;
            if (mix & MIX_RES_F32) {
                const f32x4 r0 = *(const f32x4*)((const float*)res + off);
                const f32x4 r1 = *(const f32x4*)((const float*)res + off + 4);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    y[j] = p0[j] + r0[j];
                    y[4 + j] = p1[j] + r1[j];
                }
            } else {
                const u32x4 rr = *(const u32x4*)((const T*)res + off);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const f32x4& pp = q < 2 ? p0 : p1;
                    y[2 * q] = pp[(2 * q) & 3] + (float)__builtin_bit_cast(T, (u16)(rr[q] & 0xffffu));
                    y[2 * q + 1] = pp[(2 * q + 1) & 3] + (float)__builtin_bit_cast(T, (u16)(rr[q] >> 16));
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) y[j] = f32_rounded(y[j]);
            if (mix & MIX_OUT_F32) {
                *(f32x4*)((float*)out0 + off) = f32x4{y[0], y[1], y[2], y[3]};
                *(f32x4*)((float*)out0 + off + 4) = f32x4{y[4], y[5], y[6], y[7]};
            } else {
                u32x4 o;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    o[q] = (unsigned)__builtin_bit_cast(u16, (T)y[2 * q]) |
                           ((unsigned)__builtin_bit_cast(u16, (T)y[2 * q + 1]) << 16);
                *(u32x4*)(out0 + off) = o;
            }
            continue;
        }
        const u32x4 v0 = *(const u32x4*)&tile0[ml * OP + nc];
        if constexpr (EPI == EPI_DOWN_GELU) {
            *(u32x4*)(out0 + m * n_out + col0 + nc) = v0;
            bool sp;
            const int64_t r = rm.split(m, sp);
            *(u32x4*)((sp ? out1 : out2) + r * n_out + col0 + nc) = *(const u32x4*)&tile1[ml * OP + nc];
        } else {
            const u32x4 rr = *(const u32x4*)((const T*)res + m * n_out + col0 + nc);
            u32x4 y;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float lo = (float)__builtin_bit_cast(T, (u16)(v0[q] & 0xffffu)) +
                                 (float)__builtin_bit_cast(T, (u16)(rr[q] & 0xffffu));
                const float hi = (float)__builtin_bit_cast(T, (u16)(v0[q] >> 16)) +
                                 (float)__builtin_bit_cast(T, (u16)(rr[q] >> 16));
                y[q] = (unsigned)__builtin_bit_cast(u16, (T)lo) | ((unsigned)__builtin_bit_cast(u16, (T)hi) << 16);
            }
            *(u32x4*)(out0 + m * n_out + col0 + nc) = y;
        }
    }
}

static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// shape checks shared by both entry points; 0 when the launch may proceed
static int adapter_check(const char* what, int64_t batch, int64_t n_tokens, int64_t n_special, int k,
                         int n, int dtype) {
    if (dtype != SVTAD_F16 && dtype != SVTAD_BF16)
        return set_error(SVTAD_ERR_UNSUPPORTED, what);
    if (batch < 0 || n_tokens < 0 || n_special < 0 || n_special > n_tokens || k <= 0 || n <= 0)
        return set_error(SVTAD_ERR_INVALID, what);
    if (k % KS != 0 || n % 64 != 0) return set_error(SVTAD_ERR_UNSUPPORTED, what);
    if (batch * n_tokens >= (int64_t)INT32_MAX) return set_error(SVTAD_ERR_UNSUPPORTED, what);
    return SVTAD_OK;
}

template <typename T, int EPI, int FN, int BK, int FM = 4, bool MIX = false>
static void launch_tiles(const void* a0, const void* a1, const void* w, const void* bias,
                         const void* gamma, const void* res, void* o0, void* o1, void* o2,
                         int64_t rows, int k, int n, RowMap rm, int mix, hipStream_t s) {
    constexpr int BM = 32 * FM, BN = 32 * FN;
    const int nct = n / BN;
    const int64_t tiles = cdiv(rows, BM) * nct;
    hipLaunchKernelGGL((k_adapter_gemm<T, EPI, FM, FN, BK, MIX>), dim3((unsigned)tiles), dim3(256), 0, s,
                       (const T*)a0, (const T*)a1, (const T*)w, (const T*)bias, gamma, res, (T*)o0, (T*)o1,
                       (T*)o2, rows, k, n, rm, nct, tiles, mix);
}

// 64 x 64 tiles (enough workgroups per CU to cover the load latency), 64-deep
// stages when k allows; `mix` != 0 selects the mixed-dtype up epilogue
template <typename T, int EPI>
static void launch_adapter(const void* a0, const void* a1, const void* w, const void* bias,
                           const void* gamma, const void* res, void* o0, void* o1, void* o2,
                           int64_t rows, int k, int n, RowMap rm, hipStream_t s, int mix = 0) {
    if constexpr (EPI == EPI_UP_SCALE_RES) {
        if (mix) {
            if (k % 64 == 0)
                launch_tiles<T, EPI, 2, 64, 2, true>(a0, a1, w, bias, gamma, res, o0, o1, o2, rows, k, n, rm, mix, s);
            else
                launch_tiles<T, EPI, 2, 32, 2, true>(a0, a1, w, bias, gamma, res, o0, o1, o2, rows, k, n, rm, mix, s);
            return;
        }
    }
    if (k % 64 == 0) launch_tiles<T, EPI, 2, 64, 2>(a0, a1, w, bias, gamma, res, o0, o1, o2, rows, k, n, rm, 0, s);
    else launch_tiles<T, EPI, 2, 32, 2>(a0, a1, w, bias, gamma, res, o0, o1, o2, rows, k, n, rm, 0, s);
}

// Column sums out[c] = sum_r a[r][c] (the bias gradients of the adapter's
// Linear layers), deterministic: a workgroup owns 64 columns (8 per thread,
// 16-byte loads) of one row split; 32 row lanes walk the split's rows and
// are added in order through LDS into part[split][c]; split_reduce adds the
// splits in order.
constexpr int kColRowsPerSplit = 512;
template <typename T>
__global__ __launch_bounds__(256) void k_colsum_part(const T* __restrict__ a, float* __restrict__ part,
                                                     int64_t rows, int cols, int n_col_blocks) {
    __shared__ float red[32][64 + 4];
    const int tid = threadIdx.x, cl = tid & 7, rl = tid >> 3;
    const int cb = blockIdx.x % n_col_blocks, sp = blockIdx.x / n_col_blocks;
    const int c0 = cb * 64 + cl * 8;
    const int64_t r0 = (int64_t)sp * kColRowsPerSplit, r1 = min(rows, r0 + kColRowsPerSplit);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (c0 < cols) {
        for (int64_t r = r0 + rl; r < r1; r += 32) {
            const u32x4 v = *(const u32x4*)(a + r * cols + c0);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc[2 * q] += (float)__builtin_bit_cast(T, (u16)(v[q] & 0xffffu));
                acc[2 * q + 1] += (float)__builtin_bit_cast(T, (u16)(v[q] >> 16));
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) red[rl][cl * 8 + j] = acc[j];
    __syncthreads();
    if (tid < 64 && cb * 64 + tid < cols) {
        float v = 0.f;
#pragma unroll 8
        for (int q = 0; q < 32; ++q) v += red[q][tid];
        part[(int64_t)sp * cols + cb * 64 + tid] = v;
    }
}

// GELU backward (erf form) of the down projection, with the incoming gradient
// read from the special-token and patch-token gradient buffers in place of
// their concatenation (the dg assembly of the unfused chain):
//   grad_pre[m][c] = g(m, c) * (Phi(u) + u * phi(u)),  u = pre[m][c],
// evaluated in fp32 and rounded once, the derivative of x * Phi(x) that the
// reference's nn.GELU backward takes (vit_sparse_adapter_poguise.py:305-306). A
// missing gradient buffer counts as zeros. One thread per 8 elements.
template <typename T>
__global__ __launch_bounds__(256) void k_gelu_bwd_split(const T* __restrict__ g_sp, const T* __restrict__ g_pa,
                                                        const T* __restrict__ pre, T* __restrict__ out,
                                                        int total_chunks, int cpr, int n, RowMap rm) {
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= total_chunks) return;
    const int m = e / cpr, q = e - m * cpr;
    bool special;
    const int64_t r = rm.split(m, special);
    const T* const gsrc = special ? g_sp : g_pa;
    const u32x4 u = *(const u32x4*)(pre + (int64_t)m * n + q * 8);
    const u32x4 gv = gsrc ? *(const u32x4*)(gsrc + r * n + q * 8) : u32x4{0u, 0u, 0u, 0u};
    u32x4 o;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        unsigned packed = 0;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const float x = (float)__builtin_bit_cast(T, (u16)(u[h] >> (16 * j)));
            const float dy = (float)__builtin_bit_cast(T, (u16)(gv[h] >> (16 * j)));
            const float cdf = 0.5f * (1.0f + erff(x * 0.70710678118654752f));
            const float pdf = expf(-0.5f * x * x) * 0.39894228040143268f;  // 1 / sqrt(2 pi)
            packed |= (unsigned)__builtin_bit_cast(u16, (T)(dy * (cdf + x * pdf))) << (16 * j);
        }
        o[h] = packed;
    }
    *(u32x4*)(out + (int64_t)m * n + q * 8) = o;
}

// part[p] = sum over the p-th slice of the 8-element chunks of
// w[i] g[i] (then b[j] gs[j]) in fp32: the gradient of gamma in
// (c W^T + b) * gamma (vit_sparse_adapter_poguise.py:652-653), which is
// sum(go * z) = <W, go^T c> + <b, column sums of go>. kGammaParts
// workgroups of 256 threads; the weight chunks and the bias chunks form one
// index range, split into equal slices; each thread's strided sum and the
// workgroup's fixed tree keep the order fixed, and split_reduce adds the
// slices in order.
constexpr int kGammaParts = 64;
// With gamma, the pass also writes the scaled copies the backward needs
// (NULL outputs are skipped): w_sc = T(w * gamma), g_sc = T(g * gamma),
// gs_sc = T(gs * gamma), each product in fp32 and rounded once, as PyTorch's
// elementwise multiply rounds it.
// With G = float (g32) g is fp32 (the unrounded weight-gradient sums): the
// dot products use it as is and g_sc = T(g * gamma) is its only rounding.
template <typename T, typename G = T>
__global__ __launch_bounds__(256) void k_gamma_part(const T* __restrict__ w, const G* __restrict__ g,
                                                    int64_t chunks, const T* __restrict__ b,
                                                    const T* __restrict__ gs, int64_t chunks_b,
                                                    float* __restrict__ part, const void* __restrict__ gamma,
                                                    bool gamma32, T* __restrict__ w_sc, T* __restrict__ g_sc,
                                                    T* __restrict__ gs_sc) {
    __shared__ float red[256];
    const int tid = threadIdx.x;
    const float gm = !gamma ? 0.f : gamma32 ? *(const float*)gamma : (float)*(const T*)gamma;
    auto scale8 = [&](const u32x4 a) {
        u32x4 o;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            // fp32 product, then the cast (PyTorch's multiply and .to())
            const T lo = (T)f32_rounded((float)__builtin_bit_cast(T, (u16)(a[h] & 0xffffu)) * gm);
            const T hi = (T)f32_rounded((float)__builtin_bit_cast(T, (u16)(a[h] >> 16)) * gm);
            o[h] = (unsigned)__builtin_bit_cast(u16, lo) | ((unsigned)__builtin_bit_cast(u16, hi) << 16);
        }
        return o;
    };
    const int64_t total = chunks + chunks_b;
    const int64_t per = (total + kGammaParts - 1) / kGammaParts;
    const int64_t c0 = (int64_t)blockIdx.x * per, c1 = min(total, c0 + per);
    float acc = 0.f;
    auto dot8 = [&](const u32x4 a, const u32x4 c) {
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            acc += (float)__builtin_bit_cast(T, (u16)(a[h] & 0xffffu)) * (float)__builtin_bit_cast(T, (u16)(c[h] & 0xffffu));
            acc += (float)__builtin_bit_cast(T, (u16)(a[h] >> 16)) * (float)__builtin_bit_cast(T, (u16)(c[h] >> 16));
        }
    };
    for (int64_t c = c0 + tid; c < c1; c += 256) {
        if (c < chunks) {
            const u32x4 wv = *(const u32x4*)(w + c * 8);
            if constexpr (sizeof(G) == 4) {
                const f32x4 g0 = *(const f32x4*)(g + c * 8), g1 = *(const f32x4*)(g + c * 8 + 4);
                u32x4 gs8;
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const float glo = h < 2 ? g0[2 * h] : g1[2 * h - 4];
                    const float ghi = h < 2 ? g0[2 * h + 1] : g1[2 * h - 3];
                    acc += (float)__builtin_bit_cast(T, (u16)(wv[h] & 0xffffu)) * glo;
                    acc += (float)__builtin_bit_cast(T, (u16)(wv[h] >> 16)) * ghi;
                    gs8[h] = (unsigned)__builtin_bit_cast(u16, (T)f32_rounded(glo * gm)) |
                             ((unsigned)__builtin_bit_cast(u16, (T)f32_rounded(ghi * gm)) << 16);
                }
                if (w_sc) *(u32x4*)(w_sc + c * 8) = scale8(wv);
                if (g_sc) *(u32x4*)(g_sc + c * 8) = gs8;
            } else {
                const u32x4 gv = *(const u32x4*)(g + c * 8);
                dot8(wv, gv);
                if (w_sc) *(u32x4*)(w_sc + c * 8) = scale8(wv);
                if (g_sc) *(u32x4*)(g_sc + c * 8) = scale8(gv);
            }
        } else {
            const u32x4 bv = *(const u32x4*)(b + (c - chunks) * 8), sv = *(const u32x4*)(gs + (c - chunks) * 8);
            dot8(bv, sv);
            if (gs_sc) *(u32x4*)(gs_sc + (c - chunks) * 8) = scale8(sv);
        }
    }
    red[tid] = acc;
    __syncthreads();
    for (int h = 128; h > 0; h >>= 1) {
        if (tid < h) red[tid] += red[tid + h];
        __syncthreads();
    }
    if (tid == 0) part[blockIdx.x] = red[0];
}

}  // namespace svtad

using namespace svtad;

extern "C" int svtad_adapter_down(const void* x, const void* weight, const void* bias, void* pre_act,
                                  void* act_special, void* act_patch, int64_t batch, int64_t n_tokens,
                                  int64_t n_special, int k, int n, int dtype, void* stream) {
    int st = adapter_check("adapter_down: needs f16/bf16, k % 32 == 0, n % 64 == 0, 0 <= n_special <= n_tokens",
                           batch, n_tokens, n_special, k, n, dtype);
    if (st) return st;
    const int64_t rows = batch * n_tokens;
    if (rows == 0) return SVTAD_OK;
    if (!x || !weight || !pre_act || (n_special > 0 && !act_special) || (n_tokens > n_special && !act_patch))
        return set_error(SVTAD_ERR_INVALID, "adapter_down: null pointer");
    if (!al16(x) || !al16(weight) || !al16(pre_act) || (act_special && !al16(act_special)) ||
        (act_patch && !al16(act_patch)))
        return set_error(SVTAD_ERR_INVALID, "adapter_down: x, weight and outputs need 16-byte alignment");
    const RowMap rm{n_tokens, n_special, n_tokens - n_special};
    hipStream_t s = (hipStream_t)stream;
    if (dtype == SVTAD_F16)
        launch_adapter<f16, EPI_DOWN_GELU>(x, nullptr, weight, bias, nullptr, nullptr, pre_act, act_special,
                                           act_patch, rows, k, n, rm, s);
    else
        launch_adapter<bf16, EPI_DOWN_GELU>(x, nullptr, weight, bias, nullptr, nullptr, pre_act, act_special,
                                            act_patch, rows, k, n, rm, s);
    return launch_status();
}

extern "C" int svtad_adapter_up(const void* a_special, const void* a_patch, const void* weight,
                                const void* bias, const void* gamma, const void* residual, void* out,
                                int64_t batch, int64_t n_tokens, int64_t n_special, int k, int n,
                                int dtype, void* stream) {
    return svtad_adapter_up_mixed(a_special, a_patch, weight, bias, gamma, residual, out, batch, n_tokens,
                                  n_special, k, n, dtype, dtype, dtype, dtype, stream);
}

extern "C" int svtad_adapter_up_mixed(const void* a_special, const void* a_patch, const void* weight,
                                      const void* bias, const void* gamma, const void* residual, void* out,
                                      int64_t batch, int64_t n_tokens, int64_t n_special, int k, int n,
                                      int dtype, int gamma_dtype, int residual_dtype, int out_dtype,
                                      void* stream) {
    int st = adapter_check("adapter_up: needs f16/bf16, k % 32 == 0, n % 64 == 0, 0 <= n_special <= n_tokens",
                           batch, n_tokens, n_special, k, n, dtype);
    if (st) return st;
    auto is_t_or_f32 = [&](int d) { return d == dtype || d == SVTAD_F32; };
    if (!is_t_or_f32(gamma_dtype) || !is_t_or_f32(residual_dtype) || !is_t_or_f32(out_dtype))
        return set_error(SVTAD_ERR_UNSUPPORTED, "adapter_up: gamma, residual and out take dtype or f32");
    if (gamma_dtype == dtype && (residual_dtype != dtype || out_dtype != dtype))
        return set_error(SVTAD_ERR_UNSUPPORTED,
                         "adapter_up: an f32 residual or output needs an f32 gamma (the reference's dtype promotion)");
    const int mix = (gamma_dtype == SVTAD_F32 ? MIX_GAMMA_F32 : 0) | (residual_dtype == SVTAD_F32 ? MIX_RES_F32 : 0) |
                    (out_dtype == SVTAD_F32 ? MIX_OUT_F32 : 0);
    const int64_t rows = batch * n_tokens;
    if (rows == 0) return SVTAD_OK;
    if (!weight || !gamma || !residual || !out || (n_special > 0 && !a_special) ||
        (n_tokens > n_special && !a_patch))
        return set_error(SVTAD_ERR_INVALID, "adapter_up: null pointer");
    if (!al16(weight) || (a_special && !al16(a_special)) || (a_patch && !al16(a_patch)) || !al16(residual) ||
        !al16(out))
        return set_error(SVTAD_ERR_INVALID, "adapter_up: inputs, weight, residual and out need 16-byte alignment");
    const RowMap rm{n_tokens, n_special, n_tokens - n_special};
    hipStream_t s = (hipStream_t)stream;
    if (dtype == SVTAD_F16)
        launch_adapter<f16, EPI_UP_SCALE_RES>(a_special, a_patch, weight, bias, gamma, residual, out, nullptr,
                                              nullptr, rows, k, n, rm, s, mix);
    else
        launch_adapter<bf16, EPI_UP_SCALE_RES>(a_special, a_patch, weight, bias, gamma, residual, out, nullptr,
                                               nullptr, rows, k, n, rm, s, mix);
    return launch_status();
}

extern "C" size_t svtad_linear_wgrad_workspace_bytes(int64_t n, int c_g, int c_x, int dtype) {
    (void)dtype;
    if (n < 0 || c_g <= 0 || c_x <= 0) return 0;
    return plan_wgrad(n, c_g, c_x).ws_bytes;
}

extern "C" int svtad_linear_wgrad(const void* g, const int32_t* rows, const void* x, void* out, void* workspace,
                                  size_t workspace_bytes, int64_t n, int64_t n_g_rows, int c_g, int c_x,
                                  int dtype, void* stream) {
    return svtad_linear_wgrad_mixed(g, rows, x, out, workspace, workspace_bytes, n, n_g_rows, c_g, c_x, dtype,
                                    dtype, stream);
}

extern "C" int svtad_linear_wgrad_mixed(const void* g, const int32_t* rows, const void* x, void* out,
                                        void* workspace, size_t workspace_bytes, int64_t n, int64_t n_g_rows,
                                        int c_g, int c_x, int dtype, int out_dtype, void* stream) {
    if (dtype != SVTAD_F16 && dtype != SVTAD_BF16)
        return set_error(SVTAD_ERR_UNSUPPORTED, "linear_wgrad: needs f16/bf16");
    if (out_dtype != dtype && out_dtype != SVTAD_F32)
        return set_error(SVTAD_ERR_UNSUPPORTED, "linear_wgrad: out takes dtype or f32");
    if (n < 0 || n_g_rows < 0 || c_g <= 0 || c_x <= 0 || (!rows && n_g_rows < n))
        return set_error(SVTAD_ERR_INVALID, "linear_wgrad: bad sizes");
    const BwPlan p = plan_wgrad(n, c_g, c_x);
    if (!p.path) return set_error(SVTAD_ERR_UNSUPPORTED, "linear_wgrad: no tile configuration for these widths");
    if (std::max(n, n_g_rows) * (int64_t)std::max(c_g, c_x) * 2 >= (int64_t)INT32_MAX)
        return set_error(SVTAD_ERR_UNSUPPORTED, "linear_wgrad: more than 2^31 bytes per operand");
    if (!out || !workspace || (n > 0 && (!g || !x)))
        return set_error(SVTAD_ERR_INVALID, "linear_wgrad: null pointer");
    if ((g && !al16(g)) || (x && !al16(x)))
        return set_error(SVTAD_ERR_INVALID, "linear_wgrad: g and x need 16-byte alignment");
    if (workspace_bytes < p.ws_bytes)
        return set_error(SVTAD_ERR_WORKSPACE, "linear_wgrad: workspace smaller than svtad_linear_wgrad_workspace_bytes()");
    const int st = wgrad_mfma(dtype, p, g, rows, x, out, workspace, workspace_bytes, n, rows ? n_g_rows : n, c_g,
                              c_x, out_dtype == SVTAD_F32, (hipStream_t)stream);
    if (st) return st;
    return launch_status();
}

extern "C" size_t svtad_column_sums_workspace_bytes(int64_t rows, int cols, int dtype) {
    (void)dtype;
    if (rows < 0 || cols <= 0) return 0;
    return (size_t)std::max<int64_t>(1, cdiv(rows, kColRowsPerSplit)) * cols * sizeof(float);
}

extern "C" int svtad_column_sums(const void* a, void* out, void* workspace, size_t workspace_bytes, int64_t rows,
                                 int cols, int dtype, void* stream) {
    if (dtype != SVTAD_F16 && dtype != SVTAD_BF16)
        return set_error(SVTAD_ERR_UNSUPPORTED, "column_sums: needs f16/bf16");
    if (rows < 0 || cols <= 0 || cols % 8 != 0)
        return set_error(SVTAD_ERR_INVALID, "column_sums: needs rows >= 0 and cols a positive multiple of 8");
    if (!out || !workspace || (rows > 0 && !a))
        return set_error(SVTAD_ERR_INVALID, "column_sums: null pointer");
    if (a && !al16(a)) return set_error(SVTAD_ERR_INVALID, "column_sums: a needs 16-byte alignment");
    const int64_t splits = std::max<int64_t>(1, cdiv(rows, kColRowsPerSplit));
    if (workspace_bytes < (size_t)splits * cols * sizeof(float))
        return set_error(SVTAD_ERR_WORKSPACE, "column_sums: workspace smaller than svtad_column_sums_workspace_bytes()");
    hipStream_t s = (hipStream_t)stream;
    const int ncb = (cols + 63) / 64;
    if (dtype == SVTAD_F16)
        hipLaunchKernelGGL((k_colsum_part<f16>), dim3((unsigned)(ncb * splits)), dim3(256), 0, s, (const f16*)a,
                           (float*)workspace, rows, cols, ncb);
    else
        hipLaunchKernelGGL((k_colsum_part<bf16>), dim3((unsigned)(ncb * splits)), dim3(256), 0, s, (const bf16*)a,
                           (float*)workspace, rows, cols, ncb);
    split_reduce(dtype, workspace, cols, (int)splits, out, s);
    return launch_status();
}

extern "C" int svtad_gelu_backward_split(const void* grad_special, const void* grad_patch, const void* pre_act,
                                         void* grad_pre, int64_t batch, int64_t n_tokens, int64_t n_special,
                                         int n, int dtype, void* stream) {
    if (dtype != SVTAD_F16 && dtype != SVTAD_BF16)
        return set_error(SVTAD_ERR_UNSUPPORTED, "gelu_backward_split: needs f16/bf16");
    if (batch < 0 || n_tokens < 0 || n_special < 0 || n_special > n_tokens || n <= 0 || n % 8 != 0)
        return set_error(SVTAD_ERR_INVALID, "gelu_backward_split: needs 0 <= n_special <= n_tokens and n % 8 == 0");
    const int64_t rows = batch * n_tokens;
    if (rows == 0) return SVTAD_OK;
    if (rows * (int64_t)n >= (int64_t)INT32_MAX)
        return set_error(SVTAD_ERR_UNSUPPORTED, "gelu_backward_split: 2^31 elements or more");
    if (!pre_act || !grad_pre) return set_error(SVTAD_ERR_INVALID, "gelu_backward_split: null pointer");
    if (!al16(pre_act) || !al16(grad_pre) || (grad_special && !al16(grad_special)) ||
        (grad_patch && !al16(grad_patch)))
        return set_error(SVTAD_ERR_INVALID, "gelu_backward_split: buffers need 16-byte alignment");
    const RowMap rm{n_tokens, n_special, n_tokens - n_special};
    const int cpr = n / 8;
    const int total = (int)(rows * cpr);
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid((unsigned)cdiv(total, 256));
    if (dtype == SVTAD_F16)
        hipLaunchKernelGGL((k_gelu_bwd_split<f16>), grid, dim3(256), 0, s, (const f16*)grad_special,
                           (const f16*)grad_patch, (const f16*)pre_act, (f16*)grad_pre, total, cpr, n, rm);
    else
        hipLaunchKernelGGL((k_gelu_bwd_split<bf16>), grid, dim3(256), 0, s, (const bf16*)grad_special,
                           (const bf16*)grad_patch, (const bf16*)pre_act, (bf16*)grad_pre, total, cpr, n, rm);
    return launch_status();
}

// Heatmap injection of the adapter (vit_sparse_adapter_poguise.py:311-355):
// patch[i] = T(patch[i] + T(special[src[i]] * gate)), in place, with src[i]
// the flattened special-token row (b * S + 1 + heatmap cell) patch row i
// samples. A thread owns 8 channels (16 bytes) of one row; rows whose source
// is outside [0, n_special_rows) are left unchanged. The patch rows gather
// special rows that other workgroups of the down GEMM produce, so the add
// is a launch of its own after that GEMM.
namespace svtad {

//
// With an fp32 gate (`gate32`, the reference chain under autocast, where the
// gate is an fp32 parameter) the product and the sum are fp32 and the sum is
// rounded to T once, which is the cast SparseConv2d applies to its fp32 input
// there: patch[i] = T(float(patch[i]) + float(special[src[i]]) * gate).
template <typename T>
__global__ __launch_bounds__(256) void k_heatmap_add(T* __restrict__ patch, const T* __restrict__ special,
                                                     const int32_t* __restrict__ src, const void* __restrict__ gate,
                                                     int64_t rows, int64_t n_special_rows, int cols, bool gate32) {
    // products and sums rounded as the unfused chain: no fused multiply-add
#pragma clang fp contract(off)
    const int cpr = cols / 8;
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= rows * cpr) return;
    const int64_t i = e / cpr;
    const int c = (int)(e - i * cpr) * 8;
    const int32_t r = src[i];
    if (r < 0 || r >= n_special_rows) return;
    const float g = gate32 ? *(const float*)gate : (float)*(const T*)gate;
    u32x4* const pp = (u32x4*)(patch + i * cols + c);
    const u32x4 pv = *pp;
    const u32x4 hv = *(const u32x4*)(special + (int64_t)r * cols + c);
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        unsigned w = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const T pt = __builtin_bit_cast(T, (u16)(pv[q] >> (16 * h)));
            const T ht = __builtin_bit_cast(T, (u16)(hv[q] >> (16 * h)));
            const float prod32 = f32_rounded((float)ht * g);
            const float prod = gate32 ? prod32 : (float)(T)prod32;
            w |= (unsigned)__builtin_bit_cast(u16, (T)f32_rounded((float)pt + prod)) << (16 * h);
        }
        o[q] = w;
    }
    *pp = o;
}

}  // namespace svtad

extern "C" int svtad_heatmap_add(void* patch, const void* special, const int32_t* src_rows, const void* gate,
                                 int64_t rows, int64_t n_special_rows, int cols, int dtype, void* stream) {
    return svtad_heatmap_add_mixed(patch, special, src_rows, gate, rows, n_special_rows, cols, dtype, dtype,
                                   stream);
}

extern "C" int svtad_heatmap_add_mixed(void* patch, const void* special, const int32_t* src_rows,
                                       const void* gate, int64_t rows, int64_t n_special_rows, int cols,
                                       int dtype, int gate_dtype, void* stream) {
    if (dtype != SVTAD_F16 && dtype != SVTAD_BF16)
        return set_error(SVTAD_ERR_UNSUPPORTED, "heatmap_add: needs f16/bf16");
    if (gate_dtype != dtype && gate_dtype != SVTAD_F32)
        return set_error(SVTAD_ERR_UNSUPPORTED, "heatmap_add: the gate takes dtype or f32");
    const bool gate32 = gate_dtype == SVTAD_F32;
    if (rows < 0 || n_special_rows < 0 || cols <= 0 || cols % 8 != 0)
        return set_error(SVTAD_ERR_INVALID, "heatmap_add: needs rows >= 0 and cols a positive multiple of 8");
    if (rows == 0) return SVTAD_OK;
    if (!patch || !src_rows || !gate || (n_special_rows > 0 && !special))
        return set_error(SVTAD_ERR_INVALID, "heatmap_add: null pointer");
    if (!al16(patch) || (special && !al16(special)))
        return set_error(SVTAD_ERR_INVALID, "heatmap_add: patch and special need 16-byte alignment");
    const int64_t threads = rows * (cols / 8);
    const dim3 grid((unsigned)cdiv(threads, 256));
    if (dtype == SVTAD_F16)
        hipLaunchKernelGGL(k_heatmap_add<f16>, grid, dim3(256), 0, (hipStream_t)stream, (f16*)patch,
                           (const f16*)special, src_rows, gate, rows, n_special_rows, cols, gate32);
    else
        hipLaunchKernelGGL(k_heatmap_add<bf16>, grid, dim3(256), 0, (hipStream_t)stream, (bf16*)patch,
                           (const bf16*)special, src_rows, gate, rows, n_special_rows, cols, gate32);
    return launch_status();
}

extern "C" size_t svtad_gamma_grad_workspace_bytes(void) { return (size_t)kGammaParts * sizeof(float); }

extern "C" int svtad_gamma_grad(const void* w, const void* g, int64_t count, const void* b, const void* gs,
                                int64_t count_b, void* out, const void* gamma, void* w_scaled, void* g_scaled,
                                void* gs_scaled, void* workspace, size_t workspace_bytes, int dtype, void* stream) {
    return svtad_gamma_grad_mixed(w, g, count, b, gs, count_b, out, gamma, w_scaled, g_scaled, gs_scaled, workspace,
                                  workspace_bytes, dtype, dtype, dtype, stream);
}

extern "C" int svtad_gamma_grad_mixed(const void* w, const void* g, int64_t count, const void* b, const void* gs,
                                      int64_t count_b, void* out, const void* gamma, void* w_scaled,
                                      void* g_scaled, void* gs_scaled, void* workspace, size_t workspace_bytes,
                                      int dtype, int g_dtype, int gamma_dtype, void* stream) {
    if (dtype != SVTAD_F16 && dtype != SVTAD_BF16)
        return set_error(SVTAD_ERR_UNSUPPORTED, "gamma_grad: needs f16/bf16");
    if ((gamma_dtype != dtype && gamma_dtype != SVTAD_F32) || (g_dtype != dtype && g_dtype != SVTAD_F32))
        return set_error(SVTAD_ERR_UNSUPPORTED, "gamma_grad: g and gamma take dtype or f32");
    const bool gamma32 = gamma_dtype == SVTAD_F32;
    if (count < 0 || count_b < 0 || count % 8 != 0 || count_b % 8 != 0 || (!b != !gs))
        return set_error(SVTAD_ERR_INVALID, "gamma_grad: counts must be multiples of 8; b and gs go together");
    if (!out || !workspace || (count > 0 && (!w || !g)) || (count_b > 0 && !b))
        return set_error(SVTAD_ERR_INVALID, "gamma_grad: null pointer");
    if ((w && !al16(w)) || (g && !al16(g)) || (b && !al16(b)) || (gs && !al16(gs)) ||
        (w_scaled && !al16(w_scaled)) || (g_scaled && !al16(g_scaled)) || (gs_scaled && !al16(gs_scaled)))
        return set_error(SVTAD_ERR_INVALID, "gamma_grad: buffers need 16-byte alignment");
    if (!gamma && (w_scaled || g_scaled || gs_scaled))
        return set_error(SVTAD_ERR_INVALID, "gamma_grad: scaled outputs need gamma");
    if (gs_scaled && !b) return set_error(SVTAD_ERR_INVALID, "gamma_grad: gs_scaled needs b and gs");
    if (workspace_bytes < svtad_gamma_grad_workspace_bytes())
        return set_error(SVTAD_ERR_WORKSPACE, "gamma_grad: workspace smaller than svtad_gamma_grad_workspace_bytes()");
    hipStream_t s = (hipStream_t)stream;
    const int64_t nb = b ? count_b / 8 : 0;
    const bool g32 = g_dtype == SVTAD_F32;
#define SVTAD_GAMMA_LAUNCH(T, G)                                                                              \
    hipLaunchKernelGGL((k_gamma_part<T, G>), dim3(kGammaParts), dim3(256), 0, s, (const T*)w, (const G*)g,     \
                       count / 8, (const T*)b, (const T*)gs, nb, (float*)workspace, gamma, gamma32, (T*)w_scaled, \
                       (T*)g_scaled, (T*)gs_scaled)
    if (dtype == SVTAD_F16) {
        if (g32) SVTAD_GAMMA_LAUNCH(f16, float);
        else SVTAD_GAMMA_LAUNCH(f16, f16);
    } else {
        if (g32) SVTAD_GAMMA_LAUNCH(bf16, float);
        else SVTAD_GAMMA_LAUNCH(bf16, bf16);
    }
#undef SVTAD_GAMMA_LAUNCH
    // the gradient takes gamma's dtype (an fp32 parameter's gradient is fp32)
    split_reduce(gamma_dtype, workspace, 1, kGammaParts, out, s);
    return launch_status();
}
