// MFMA (matrix core) SparseConv2D kernels for f16 / bf16 on gfx950.
//
// All three GEMM shapes of the op run on v_mfma_f32_16x16x32_{f16,bf16}
// (fp32 accumulate):
//   forward      out[m, n]    = sum_k sum_c x[src(m,k), c]   * w[k][c][n]
//   bwd-input    gi[m, n]     = sum_k sum_c go[src_t(m,k), c] * w[k][n][c]
//   bwd-weight   gw[k][ci][co] = sum_i x[src(i,k), ci] * go[i, co]
// Operand tiles are staged through LDS with the reduction index contiguous
// ([row][32 k-values], pitch 40 elements = 80 bytes, so the 16 lanes that
// read one fragment column hit 16 distinct 16-byte slots), which makes every
// MFMA fragment a single 16-byte LDS read. Operands whose reduction index is
// strided in HBM (w in the forward, both operands of bwd-weight) are
// transposed while being written into LDS. Two LDS buffers alternate so the
// global loads of step t+1 are in flight while step t runs on the matrix
// cores.
//
// MFMA lane layout used (16x16 output tile, 64 lanes): lane l supplies row
// l%16 of A and column l%16 of B with 8 reduction values at slot l/16; it
// receives C[(l/16)*4 + j][l%16], j = 0..3. A and B use the same slot
// mapping, so the pairing of reduction values matches by construction.
#include <type_traits>

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "sv_common.h"
#include "sv_conv.h"
#include "sv_internal.h"
#include "sv_mfma.h"

namespace svtad {

__device__ __forceinline__ u16 half_of(const u32x4& v, int j) {
    const unsigned w = v[j >> 1];
    return (u16)((j & 1) ? (w >> 16) : (w & 0xffffu));
}

// ---------------------------------------------------------------------------
// Gathered GEMM (forward / backward-input)
// ---------------------------------------------------------------------------
template <typename T, int MODE, int WGM, int WGN, int FM, int FN>
__global__ __launch_bounds__(WGM* WGN * 64) void k_gg_mfma(
    const T* __restrict__ src, const int32_t* __restrict__ nbr, const T* __restrict__ w,
    const void* __restrict__ bias, int bias_mode, T* __restrict__ out, int64_t n, int c_red,
    int n_out, int64_t tpb, int n_col_tiles, int64_t n_tiles) {
    constexpr int NT = WGM * WGN * 64;
    constexpr int BM = WGM * FM * 16;
    constexpr int BN = WGN * FN * 16;
    constexpr int A_CHUNKS = BM * 4;                  // 16-byte chunks of an A tile
    constexpr int A_PER = (A_CHUNKS + NT - 1) / NT;
    constexpr int B_ITEMS = MODE == MODE_FWD ? 2 * BN : BN * 4;
    constexpr int B_PER = (B_ITEMS + NT - 1) / NT;

    __shared__ __align__(16) u16 As[2][BM][PITCH];
    __shared__ __align__(16) u16 Bs[2][BN][PITCH];
    __shared__ int32_t sidx[9][BM];
    __shared__ int kvalid[9];
    __shared__ int klist[9];
    __shared__ int nk_s;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int64_t tile = xcd_tile(blockIdx.x, n_tiles);
    const int64_t row0 = (tile / n_col_tiles) * BM;
    const int col0 = (int)(tile % n_col_tiles) * BN;

    if (tid < 9) kvalid[tid] = 0;
    __syncthreads();
    for (int e = tid; e < 9 * BM; e += NT) {
        const int k = e / BM, m = e - k * BM;
        const int64_t i = row0 + m;
        int64_t r = -1;
        if (i < n) r = MODE == MODE_FWD ? src_row(nbr, i, k, n, tpb) : src_row_t(nbr, i, k, n, tpb);
        sidx[k][m] = (int32_t)r;
        if (r >= 0) kvalid[k] = 1;
    }
    __syncthreads();
    if (tid == 0) {
        int c = 0;
        for (int k = 0; k < 9; ++k)
            if (kvalid[k]) klist[c++] = k;
        nk_s = c;
    }
    __syncthreads();
    const int nc = (c_red + KS - 1) / KS;
    const int steps = nk_s * nc;

    u32x4 ra[A_PER];
    u32x4 rb[B_PER][MODE == MODE_FWD ? 2 : 1];
    const u32x4 zero = {0u, 0u, 0u, 0u};

    auto load = [&](int t) {
        const int k = klist[t / nc];
        const int c0 = (t % nc) * KS;
#pragma unroll
        for (int q = 0; q < A_PER; ++q) {
            const int e = tid + q * NT;
            u32x4 v = zero;
            if (e < A_CHUNKS) {
                const int m = e >> 2, part = e & 3;
                const int32_t r = sidx[k][m];
                const int c = c0 + part * 8;
                if (r >= 0 && c < c_red) v = *(const u32x4*)(src + (int64_t)r * c_red + c);
            }
            ra[q] = v;
        }
        const T* wk = w + (int64_t)k * c_red * n_out;
#pragma unroll
        for (int q = 0; q < B_PER; ++q) {
            const int e = tid + q * NT;
            if constexpr (MODE == MODE_FWD) {
                // w[k][c][n]: rows c (reduction), n contiguous; two rows per item
                u32x4 v0 = zero, v1 = zero;
                if (e < B_ITEMS) {
                    const int cp = e & 15, g = e >> 4;
                    const int c = c0 + 2 * cp, nn = col0 + g * 8;
                    if (c < c_red && nn < n_out) {
                        v0 = *(const u32x4*)(wk + (int64_t)c * n_out + nn);
                        v1 = *(const u32x4*)(wk + (int64_t)(c + 1) * n_out + nn);
                    }
                }
                rb[q][0] = v0;
                if constexpr (MODE == MODE_FWD) rb[q][1] = v1;
            } else {
                // w[k][n][c] seen as B[c][n]: rows n with c contiguous
                u32x4 v = zero;
                if (e < B_ITEMS) {
                    const int nl = e >> 2, part = e & 3;
                    const int nn = col0 + nl, c = c0 + part * 8;
                    if (nn < n_out && c < c_red) v = *(const u32x4*)(wk + (int64_t)nn * c_red + c);
                }
                rb[q][0] = v;
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int q = 0; q < A_PER; ++q) {
            const int e = tid + q * NT;
            if (e < A_CHUNKS) *(u32x4*)&As[buf][e >> 2][(e & 3) * 8] = ra[q];
        }
#pragma unroll
        for (int q = 0; q < B_PER; ++q) {
            const int e = tid + q * NT;
            if (e >= B_ITEMS) continue;
            if constexpr (MODE == MODE_FWD) {
                const int cp = e & 15, g = e >> 4;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const unsigned lo = half_of(rb[q][0], j);
                    const unsigned hi = half_of(rb[q][1], j);
                    *(unsigned*)&Bs[buf][g * 8 + j][2 * cp] = lo | (hi << 16);
                }
            } else {
                *(u32x4*)&Bs[buf][e >> 2][(e & 3) * 8] = rb[q][0];
            }
        }
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int wm = wave / WGN, wn = wave % WGN;
    const int arow = wm * FM * 16 + (lane & 15);
    const int brow = wn * FN * 16 + (lane & 15);
    const int kof = (lane >> 4) * 8;

    if (steps > 0) {
        load(0);
        store(0);
    }
    __syncthreads();
    for (int t = 0; t < steps; ++t) {
        const int buf = t & 1;
        if (t + 1 < steps) load(t + 1);
        u32x4 fa[FM], fb[FN];
#pragma unroll
        for (int a = 0; a < FM; ++a) fa[a] = *(const u32x4*)&As[buf][arow + a * 16][kof];
#pragma unroll
        for (int b = 0; b < FN; ++b) fb[b] = *(const u32x4*)&Bs[buf][brow + b * 16][kof];
#pragma unroll
        for (int a = 0; a < FM; ++a)
#pragma unroll
            for (int b = 0; b < FN; ++b) acc[a][b] = MfmaOp<T>::run(fa[a], fb[b], acc[a][b]);
        if (t + 1 < steps) store(buf ^ 1);
        __syncthreads();
    }

    // epilogue: lane holds C[(lane/16)*4 + j][lane%16] of each 16x16 tile
#pragma unroll
    for (int b = 0; b < FN; ++b) {
        const int col = col0 + wn * FN * 16 + b * 16 + (lane & 15);
        if (col >= n_out) continue;
        float bv = 0.f;
        if (bias_mode == SVTAD_BIAS_FP32) bv = ((const float*)bias)[col];
        else if (bias_mode != SVTAD_BIAS_NONE) bv = (float)((const T*)bias)[col];
#pragma unroll
        for (int a = 0; a < FM; ++a) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t i = row0 + wm * FM * 16 + a * 16 + (lane >> 4) * 4 + j;
                if (i >= n) continue;
                const float v = acc[a][b][j];
                T o;
                if (bias_mode == SVTAD_BIAS_PRE || bias_mode == SVTAD_BIAS_FP32) o = (T)(v + bv);
                else if (bias_mode == SVTAD_BIAS_AFTER) o = (T)((float)(T)v + bv);
                else o = (T)v;
                out[i * n_out + col] = o;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Wide gathered GEMM (forward / backward-input) for reduction widths CR in
// {64, 128, 192, 256, 512}: a workgroup owns BM = FM*16 rows and BN = 4*FN*16
// output columns; each of its 4 waves owns FN*16 of the columns and all BM
// rows; WS wave sets of 4 waves split the neighbor offsets (set h takes
// klist[h], klist[h + WS], ...) and sum their accumulators through LDS.
//
// The gathered rows come from LDS in one of two modes, chosen per tile:
//  * window: the rows a tile gathers lie in a short range [lo, hi] of
//    source rows (for the tables built from masks, neighbors stay within a
//    frame, about BM + 30 rows). That range is loaded once, contiguously,
//    with a zero row for missing neighbors; every offset's fragments are then
//    read through the table from LDS, and the main loop has no A loads and no
//    barriers.
//  * slices (any table): per offset, the BM gathered rows are staged in LDS
//    (two slices alternate; the next slice's loads are in flight while the
//    current one is consumed).
// Weight fragments come straight from global memory (L2-resident), D steps
// ahead in a register ring (the fragment-ordered layout of k_pack_frag).
// The MFMA takes the weight fragment as its A operand and the gathered rows
// as B, so each lane accumulates 4 consecutive output columns of one row
// (acc[a][f][j] = out[a*16 + lane%16][f*16 + (lane/16)*4 + j] in the wave's
// columns), which the epilogue packs into 8-byte stores.
// ---------------------------------------------------------------------------
// LDS rows (of CR 16-bit elements) of k_gg_wide: the per-set slices, a
// window of at least BM + 64 rows, and the set reduction / output tile that
// reuse them at the end.
constexpr int cmax(int a, int b) { return a > b ? a : b; }
constexpr int gg_lds_rows(int CR, int FM, int FN, int WS) {
    return cmax(cmax(WS * FM * 16, FM * 16 + 64),
                cmax(WS > 1 ? (FM * 16 * (4 * FN * 16 + 4) * 4 + CR * 2 - 1) / (CR * 2) : 0,
                     (FM * 16 * (4 * FN * 16 + 8) * 2 + CR * 2 - 1) / (CR * 2)));
}

// Rows loaded on either side of a tile before its table is read: tables built
// from masks of frames up to 19 tokens wide stay within them at any keep rate.
constexpr int kSpecMargin = 20;

template <int CR, int FM, int FN, int WS>
struct GgWideLds {
    __align__(16) u16 Ab[gg_lds_rows(CR, FM, FN, WS)][CR];
    int srow[9][FM * 16];  // gathered source row, -1 if missing
    int kvalid[9];
    int klist[10];
    int nk_s, lo_s, hi_s;
    __align__(16) float bias[CR >= 512 ? 4 * FN * 16 : 4];  // the forward's bias (512 channels)
};

// One tile of the wide gathered GEMM, run by threads [0, 256 * WS) of a
// workgroup (k_gg_wide, or the backward-input role of k_bwd_fused) in the
// LDS block L.
template <typename T, int MODE, int CR, int FM, int FN, int D, int WS>
__device__ __forceinline__ void gg_wide_tile(
    GgWideLds<CR, FM, FN, WS>& L, int64_t tile, const T* __restrict__ src, const int32_t* __restrict__ nbr,
    const T* __restrict__ wb, const void* __restrict__ bias, int bias_mode, T* __restrict__ out, int64_t n,
    int n_out, int64_t tpb, int n_col_tiles, uint32_t* __restrict__ orphan_flag, bool sym) {
    constexpr int BM = FM * 16;
    constexpr int BN = 4 * FN * 16;
    constexpr int NC = CR / KS;
    // LDS rows are CR elements with no padding; 16-byte chunk q of row m is
    // stored at position q ^ (m & 7) (CR / 8 is a multiple of 8, so the swizzle
    // stays inside the row). Fragment reads (16 rows x 4 chunks) and the row
    // stores then both run at the full LDS rate; a 16-byte pad does not.
    constexpr int RP = CR;
    constexpr int CPR = CR / 8;  // 16-byte chunks per row
    static_assert(CPR % 8 == 0, "the chunk swizzle needs a multiple of 8 chunks per row");
    constexpr int A_CHUNKS = BM * CPR;
    constexpr int LROWS = gg_lds_rows(CR, FM, FN, WS);
    static_assert(NC % D == 0, "ring depth must divide the steps of a slice");

    static_assert(sizeof(L.Ab) == (size_t)LROWS * RP * 2, "LDS rows");
    auto& Ab = L.Ab;
    auto& srow = L.srow;
    auto& kvalid = L.kvalid;
    auto& klist = L.klist;
    int& nk_s = L.nk_s;
    int& lo_s = L.lo_s;
    int& hi_s = L.hi_s;

    const int tid = threadIdx.x;
    const int set = tid >> 8, ltid = tid & 255;
    const int lane = tid & 63, wave = ltid >> 6;
    const int64_t row0 = (tile / n_col_tiles) * BM;
    const int col0 = (int)(tile % n_col_tiles) * BN;
    const rsrc_t rs_src = make_rsrc(src, (uint32_t)(n * CR * 2));

    constexpr int NT = 256 * WS;
    // The tile's table rows are contiguous (entry e = m*9 + kk). All table
    // loads are issued before the speculative window's (below), so waiting for
    // them leaves the window loads in flight: load waits count loads in issue
    // order. Backward-input also gathers each entry's partner first.
    constexpr int TPER = (9 * BM + NT - 1) / NT;
    const int64_t tile_ents = min<int64_t>(BM, n - row0) * 9;
    const rsrc_t rs_tab = make_rsrc(nbr, (uint32_t)(n * 9 * 4));
    auto src_of = [&](int v, int64_t i) -> int64_t {  // table value of row i -> source row or -1
        if (v < 0) return -1;
        const int64_t r = (int64_t)v + (tpb > 0 ? (i / tpb) * tpb : 0);
        return r < n ? r : -1;
    };
    int tv[TPER], pv[TPER];
#pragma unroll
    for (int q = 0; q < TPER; ++q) {
        const int e = tid + q * NT;
        tv[q] = (int)__builtin_amdgcn_raw_buffer_load_b32(rs_tab, e < tile_ents ? (uint32_t)(row0 * 9 + e) * 4u : kOOB, 0, 0);
        pv[q] = -1;
    }
    // sym: the caller's promise that every entry has its partner (as in every
    // table built from a keep mask), so no partner loads, and the row offsets
    // wait for one round trip to memory instead of two
    if (MODE != MODE_FWD && !sym) {
#pragma unroll
        for (int q = 0; q < TPER; ++q) {
            const int e = tid + q * NT;
            const int m = e / 9, kk = e - m * 9;
            const int64_t p = e < tile_ents ? src_of(tv[q], row0 + m) : -1;
            pv[q] = (int)__builtin_amdgcn_raw_buffer_load_b32(rs_tab, p >= 0 ? (uint32_t)(p * 9 + (8 - kk)) * 4u : kOOB, 0, 0);
        }
    }

    // Speculative window: the rows a table built from a mask gathers lie within
    // W + 1 rows of the row (W the frame width), so rows [spec_lo, spec_lo +
    // SPECL), the tile and kSpecMargin rows on either side, are loaded now,
    // while the table is processed; LDS row SPEC is the zero row. Every tile
    // loads its window at the same time, so the window's bytes bound this
    // part of the prologue: a margin as wide as the LDS allows (31-41 rows)
    // cost 0.3-0.5 us per launch at 192 channels (55 % keep) and 0.8 us at
    // 512. A tile whose window is wider loads the exact window after the table.
    constexpr int SPEC = LROWS - 1;
    constexpr int SPECL = SPEC < BM + 2 * kSpecMargin ? SPEC : BM + 2 * kSpecMargin;
    constexpr int SPEC_CHUNKS = SPECL * CPR;
    constexpr int SPEC_PER = (SPEC_CHUNKS + NT - 1) / NT;
    const int64_t spec_lo = row0 - (SPECL - BM) / 2;
    u32x4 sp[SPEC_PER];
#pragma unroll
    for (int q = 0; q < SPEC_PER; ++q) {
        const int e = tid + q * NT;
        const int r = e / CPR;
        const int64_t gr = spec_lo + r;
        sp[q] = bload16(rs_src, e < SPEC_CHUNKS && gr >= 0 && gr < n
                                    ? (uint32_t)gr * (uint32_t)(CR * 2) + (uint32_t)(e - r * CPR) * 16u
                                    : kOOB);
    }
    // At 512 channels the forward's bias goes through LDS: one column per
    // thread, one 32-bit load with no branch issued behind the window's loads,
    // stored to LDS after the main loop. In registers (the other widths) each
    // lane holds FN * 4 values through the main loop, and at 512 channels the
    // kernel then spilled 10 registers (config 5 forward 70.4 -> 68.5 us).
    // At 192 channels the LDS form measured 2 us slower per training step
    // (c2 at 55 % keep) with no cause found, so the other widths keep the
    // registers.
    constexpr bool BIAS_LDS = CR >= 512;
    const bool has_bias = MODE == MODE_FWD && bias_mode != SVTAD_BIAS_NONE;  // uniform
    const bool bias32 = bias_mode == SVTAD_BIAS_FP32;
    uint32_t bias_raw = 0u;
    if constexpr (BIAS_LDS) {
        if (has_bias) {
            const rsrc_t rs_bias = make_rsrc(bias, (uint32_t)n_out * (bias32 ? 4u : 2u));
            const uint32_t col = (uint32_t)(col0 + tid);
            const uint32_t off = bias32 ? col * 4u : (col * 2u) & ~3u;  // n_out is even
            bias_raw = __builtin_amdgcn_raw_buffer_load_b32(rs_bias, tid < BN && col < (uint32_t)n_out ? off : kOOB, 0, 0);
        }
    }

    if (tid < 9) kvalid[tid] = 0;
    if (tid == 0) {
        lo_s = INT32_MAX;
        hi_s = -1;
    }
    __syncthreads();
    int lo = INT32_MAX, hi = -1;
#pragma unroll
    for (int q = 0; q < TPER; ++q) {
        const int e = tid + q * NT;
        if (e < 9 * BM) {
            const int m = e / 9, kk = e - m * 9;
            const int64_t i = row0 + m;
            const int k = MODE == MODE_FWD ? kk : 8 - kk;
            int64_t r = -1;
            if (e < tile_ents) {
                const int64_t p = src_of(tv[q], i);
                if (MODE == MODE_FWD) {
                    r = p;
                } else if (p >= 0) {
                    // transposed source of offset k (see src_row_t): entry
                    // (i, 8-k) -> p, accepted when its partner (p, k) -> i
                    // exists; one without a partner is left to the orphan
                    // pass, which the flag arms
                    if (sym || src_of(pv[q], p) == i) r = p;
                    else if (orphan_flag) *orphan_flag = 1u;
                }
            }
            srow[k][m] = (int)r;
            if (r >= 0) {
                kvalid[k] = 1;
                lo = min(lo, (int)r);
                hi = max(hi, (int)r);
            }
        }
    }
    // window bounds: reduce within the wave, then one LDS atomic pair per wave
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        lo = min(lo, __shfl_xor(lo, o));
        hi = max(hi, __shfl_xor(hi, o));
    }
    if (lane == 0 && hi >= 0) {
        atomicMin(&lo_s, lo);
        atomicMax(&hi_s, hi);
    }
    __syncthreads();
    if (tid == 0) {
        int c = 0;
        for (int k = 0; k < 9; ++k)
            if (kvalid[k]) klist[c++] = k;
        for (int q = c; q < 10; ++q) klist[q] = c > 0 ? klist[c - 1] : 0;  // always a valid offset
        nk_s = c;
    }
    __syncthreads();
    const int nk = nk_s;
    const int nk_set = nk > set ? (nk - set + WS - 1) / WS : 0;  // slices of this set
    const int iters = (nk + WS - 1) / WS;
    const int lo_t = lo_s, hi_t = hi_s;
    const int wrows = hi_t >= 0 ? hi_t - lo_t + 1 : 0;
    // uniform: the speculative rows hold the window / the exact window fits
    const bool spec_ok = hi_t < 0 || (lo_t >= spec_lo && hi_t < spec_lo + SPECL);
    const bool window = spec_ok || wrows + 1 <= LROWS;
    const int64_t wlo = spec_ok ? spec_lo : lo_t;  // LDS row r holds source row wlo + r
    const int zrow = spec_ok ? SPEC : wrows;       // the zero row
    if (spec_ok) {  // the speculative rows into LDS (before the ring takes registers)
        u16* const l = &Ab[0][0];
#pragma unroll
        for (int q = 0; q < SPEC_PER; ++q) {
            const int e = tid + q * 256 * WS;
            const int r = e / CPR;
            if (e < SPEC_CHUNKS) *(u32x4*)&l[r * RP + (((e - r * CPR) ^ (r & 7)) * 8)] = sp[q];
        }
        if (tid < CPR) *(u32x4*)&l[SPEC * RP + ((tid ^ (SPEC & 7)) * 8)] = u32x4{0u, 0u, 0u, 0u};
    }

    const int nf = (n_out + 15) / 16;
    const uint32_t step_bytes = (uint32_t)nf * 1024u;  // one reduction step, all column blocks
    const rsrc_t rs_w = make_rsrc(wb, 9u * NC * step_bytes);

    // Weight fragments (k_pack_frag layout): the 64 lanes of fragment (k,
    // step, column block) are 1 KB contiguous, so a fragment load is fully
    // coalesced. The per-lane part of the offset is fixed (kOOB for column
    // blocks past n_out, which then load zeros); the wave-uniform part (the
    // slab of the iteration's offset plus the step) goes in the scalar offset,
    // computed once per slice. Past the set's end the slab is offset 0's
    // (valid data, never used).
    uint32_t boff[FN];
#pragma unroll
    for (int f = 0; f < FN; ++f) {
        const int blk = (col0 + wave * FN * 16) / 16 + f;
        boff[f] = blk < nf ? (uint32_t)(blk * 64 + lane) * 16u : kOOB;
    }
    auto slab_of = [&](int it) -> uint32_t {
        const int k = it < nk_set ? klist[min(it * WS + set, 9)] : 0;
        return __builtin_amdgcn_readfirstlane((uint32_t)k * (uint32_t)NC * step_bytes);
    };
    u32x4 ring[D][FN];
    auto load_b = [&](uint32_t so, u32x4* rb) {
#pragma unroll
        for (int f = 0; f < FN; ++f)
            rb[f] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs_w, boff[f], so, 0));
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int arow = lane & 15;
    const int g = lane >> 4;  // reduction chunk of the lane within a step
    u16* const lds = &Ab[0][0];

    // the bias of this lane's output columns in registers (below 512
    // channels), loaded now so the epilogue does not wait for it
    float bv[BIAS_LDS ? 1 : FN][4];
    if constexpr (!BIAS_LDS) {
#pragma unroll
        for (int f = 0; f < FN; ++f)
#pragma unroll
            for (int j = 0; j < 4; ++j) bv[f][j] = 0.f;
        if (MODE == MODE_FWD && set == 0 && bias_mode != SVTAD_BIAS_NONE) {  // uniform
            // one straight-line loop per bias dtype
            const int c0 = col0 + wave * FN * 16 + g * 4;
            if (bias_mode == SVTAD_BIAS_FP32) {
#pragma unroll
                for (int f = 0; f < FN; ++f)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int col = c0 + f * 16 + j;
                        bv[f][j] = col < n_out ? ((const float*)bias)[col] : 0.f;
                    }
            } else {
#pragma unroll
                for (int f = 0; f < FN; ++f)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int col = c0 + f * 16 + j;
                        bv[f][j] = col < n_out ? (float)((const T*)bias)[col] : 0.f;
                    }
            }
        }
    }

    // One offset's slice: this lane's fragment rows start at element offsets
    // off0[a] (even steps) / off1[a] (odd steps) of the LDS rows; the ring
    // holds the slice's first D steps and is refilled D steps ahead, into the
    // next slice (slab_next) at the end.
    auto compute = [&](const int* off0, const int* off1, uint32_t slab, uint32_t slab_next) {
        // the row fragments of step c + 1 are read while step c's MFMAs run
        u32x4 fa[2][FM];
#pragma unroll
        for (int a = 0; a < FM; ++a) fa[0][a] = *(const u32x4*)&lds[off0[a]];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int d = c % D;
            if (c + 1 < NC) {
#pragma unroll
                for (int a = 0; a < FM; ++a)
                    fa[(c + 1) & 1][a] = *(const u32x4*)&lds[(((c + 1) & 1) ? off1[a] : off0[a]) + ((c + 1) & ~1) * KS];
            }
#pragma unroll
            for (int a = 0; a < FM; ++a)
#pragma unroll
                for (int f = 0; f < FN; ++f) acc[a][f] = MfmaOp<T>::run(ring[d][f], fa[c & 1][a], acc[a][f]);
            const int cn = c + D;
            load_b(cn < NC ? slab + (uint32_t)cn * step_bytes : slab_next + (uint32_t)(cn - NC) * step_bytes, ring[d]);
        }
    };
    // LDS row r, chunk position for reduction chunk q: (q ^ (r & 7)); the
    // element offsets of a lane's even / odd steps in row r:
    auto row_offs = [&](int r, int& o0, int& o1) {
        const int sw = (g ^ (r & 7)) * 8;
        o0 = r * RP + sw;
        o1 = r * RP + (sw ^ 32);
    };

    uint32_t slab = slab_of(0);
#pragma unroll
    for (int d = 0; d < D; ++d) load_b(slab + (uint32_t)d * step_bytes, ring[d]);

    if (window) {
        if (!spec_ok) {
            // rows wlo .. wlo + wrows - 1 into LDS rows 0 .., zeros in row wrows
            for (int e = tid; e < (wrows + 1) * CPR; e += 256 * WS) {
                const int r = e / CPR, q = e - r * CPR;
                const u32x4 v = bload16(rs_src, r < wrows ? (uint32_t)(wlo + r) * (uint32_t)(CR * 2) + (uint32_t)q * 16u : kOOB);
                *(u32x4*)&lds[r * RP + ((q ^ (r & 7)) * 8)] = v;
            }
        }
        __syncthreads();
        // no barrier from here on: the sets walk their slices independently
        for (int it = 0; it < nk_set; ++it) {
            const int k = klist[it * WS + set];
            const uint32_t slab_next = slab_of(it + 1);
            int off0[FM], off1[FM];
#pragma unroll
            for (int a = 0; a < FM; ++a) {
                const int r = srow[k][a * 16 + arow];
                row_offs(r >= 0 ? (int)(r - wlo) : zrow, off0[a], off1[a]);
            }
            compute(off0, off1, slab, slab_next);
            slab = slab_next;
        }
    } else {
        // any table: per iteration each set stages its offset's BM gathered
        // rows in its rows [set * BM, +BM) of LDS
        int off0[FM], off1[FM];
#pragma unroll
        for (int a = 0; a < FM; ++a) row_offs(set * BM + a * 16 + arow, off0[a], off1[a]);
        for (int it = 0; it < iters; ++it) {
            const bool live = it < nk_set;
            const int k = klist[live ? it * WS + set : 0];
            for (int e = ltid; e < A_CHUNKS; e += 256) {
                const int m = e / CPR, q = e - m * CPR;
                const int r = live ? srow[k][m] : -1;
                const u32x4 v = bload16(rs_src, r >= 0 ? (uint32_t)r * (uint32_t)(CR * 2) + (uint32_t)q * 16u : kOOB);
                *(u32x4*)&lds[(set * BM + m) * RP + ((q ^ (m & 7)) * 8)] = v;
            }
            __syncthreads();
            const uint32_t slab_next = slab_of(it + 1);
            if (live) compute(off0, off1, slab, slab_next);
            slab = slab_next;
            __syncthreads();
        }
    }
    // the bias into LDS for the epilogue (its load arrived long ago)
    if constexpr (BIAS_LDS) {
        if (has_bias && tid < BN)
            L.bias[tid] = bias32 ? __builtin_bit_cast(float, bias_raw)
                                 : (float)__builtin_bit_cast(T, (u16)(bias_raw >> (((col0 + tid) & 1) * 16)));
    }
    __syncthreads();  // all waves are done reading the LDS rows

    if constexpr (WS > 1) {
        // sets 1.. add their partial sums into set 0's through LDS (fixed
        // order); 16-byte rows of 4 columns, the pitch padded by 4 floats so
        // the 16 rows of an instruction fall on different banks
        constexpr int RED = BN + 4;
        static_assert((size_t)BM * RED * 4 <= sizeof(L.Ab), "the partial accumulators must fit in LDS");
        float* red = (float*)&Ab[0][0];
        for (int h = 1; h < WS; ++h) {
            if (set == h) {
#pragma unroll
                for (int f = 0; f < FN; ++f)
#pragma unroll
                    for (int a = 0; a < FM; ++a)
                        *(f32x4*)&red[(a * 16 + arow) * RED + wave * FN * 16 + f * 16 + g * 4] = acc[a][f];
            }
            __syncthreads();
            if (set == 0) {
#pragma unroll
                for (int f = 0; f < FN; ++f)
#pragma unroll
                    for (int a = 0; a < FM; ++a)
                        acc[a][f] += *(const f32x4*)&red[(a * 16 + arow) * RED + wave * FN * 16 + f * 16 + g * 4];
            }
            __syncthreads();
        }
    }

    // epilogue: round (with the bias) into an LDS copy of the output tile, 4
    // columns per 8-byte store, then write whole 16-byte chunks so each
    // output row goes out as one run
    constexpr int OP = BN + 8;
    static_assert((size_t)BM * OP * 2 <= sizeof(L.Ab), "output tile must fit in LDS");
    u16* ot = &Ab[0][0];
    // one straight-line copy per bias mode (a mode test per element compiles
    // to a branch per element, which cost more than the rest of the epilogue)
    auto epilogue = [&](auto mode) {
        constexpr int M = decltype(mode)::value;
#pragma unroll
        for (int f = 0; f < FN; ++f) {
            const int lc = wave * FN * 16 + f * 16 + g * 4;
            f32x4 bl = {0.f, 0.f, 0.f, 0.f};
            if constexpr (BIAS_LDS && M != 0) bl = *(const f32x4*)&L.bias[lc];
#pragma unroll
            for (int a = 0; a < FM; ++a) {
                unsigned h[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float v = acc[a][f][j];
                    float bj = 0.f;
                    if constexpr (BIAS_LDS) bj = bl[j];
                    else bj = bv[f][j];
                    T o;
                    if constexpr (M == 1) o = (T)(v + bj);
                    else if constexpr (M == 2) o = (T)((float)(T)v + bj);
                    else o = (T)v;
                    h[j] = (unsigned)__builtin_bit_cast(u16, o);
                }
                typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
                *(u32x2*)&ot[(a * 16 + arow) * OP + lc] = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
            }
        }
    };
    if (set == 0) {
        if (bias_mode == SVTAD_BIAS_PRE || bias_mode == SVTAD_BIAS_FP32)
            epilogue(std::integral_constant<int, 1>{});
        else if (bias_mode == SVTAD_BIAS_AFTER)
            epilogue(std::integral_constant<int, 2>{});
        else
            epilogue(std::integral_constant<int, 0>{});
    }
    __syncthreads();
    // 16-byte row pieces out, non-temporal: the output is not read by this
    // launch, and streaming it out saves the L2 write-back at the kernel's end
    // (c2 at 55 % keep: 1.1-1.3 µs per launch)
    constexpr int CH = BN / 8;
    for (int e = tid; e < BM * CH; e += 256 * WS) {
        const int r = e / CH, c8 = e - (e / CH) * CH;
        const int64_t i = row0 + r;
        const int col = col0 + c8 * 8;
        if (i < n && col < n_out) __builtin_nontemporal_store(*(const u32x4*)&ot[r * OP + c8 * 8], (u32x4*)(out + i * n_out + col));
    }
}

template <typename T, int MODE, int CR, int FM, int FN, int D, int WS>
__global__ __launch_bounds__(256 * WS) void k_gg_wide(
    const T* __restrict__ src, const int32_t* __restrict__ nbr, const T* __restrict__ wb,
    const void* __restrict__ bias, int bias_mode, T* __restrict__ out, int64_t n, int n_out,
    int64_t tpb, int n_col_tiles, int64_t n_tiles, uint32_t* __restrict__ orphan_flag, bool sym) {
    __shared__ GgWideLds<CR, FM, FN, WS> lds;
    gg_wide_tile<T, MODE, CR, FM, FN, D, WS>(lds, xcd_tile(blockIdx.x, n_tiles), src, nbr, wb, bias, bias_mode,
                                             out, n, n_out, tpb, n_col_tiles, orphan_flag, sym);
}

// Weight in MFMA fragment order for the gathered GEMMs. For reduction step cs
// (32 values) and column block nb (16 columns), the 64 lanes' B fragments are
// stored contiguously: wf[((k*NCS + cs)*NB + nb)*64 + lane][e] =
//   B(k, c = cs*32 + (lane/16)*8 + e, n = nb*16 + lane%16), 0 past n_out,
// with B(k,c,n) = w[k][c][n] for the forward (c over c_in, n over c_out) and
// w[k][n][c] for backward-input (c over c_out, n over c_in). One thread per
// 16-byte fragment slot; grid cdiv(9*NCS*NB*64, 256).
//
// The 8 values of a slot come from buffer loads (zeros past n_out), issued
// together: forward B(k, c + e, n) = w[k][c + e][n] are 8 strided 2-byte
// loads, backward-input B(k, c + e, n) = w[k][n][c + e] one 16-byte load when
// w is 16-byte aligned. (Plain loads under an n < n_out test compiled to a
// branch and a wait per pair of values, four dependent rounds per slot.) kb
// is offset k's first element; every offset fits 32 bits (host check).
template <bool FWD>
__device__ __forceinline__ u32x4 pack_slot(rsrc_t rw, uint32_t kb, int c, int n, int c_red, int n_out, bool al16) {
    if (!FWD && al16) return bload16(rw, n < n_out ? (kb + (uint32_t)n * c_red + c) * 2u : kOOB);
    uint32_t v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t idx = FWD ? kb + (uint32_t)(c + e) * n_out + n : kb + (uint32_t)n * c_red + c + e;
        v[e] = __builtin_amdgcn_raw_buffer_load_b16(rw, n < n_out ? idx * 2u : kOOB, 0, 0);
    }
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = v[2 * j] | (v[2 * j + 1] << 16);
    return o;
}

template <int MODE>
__global__ __launch_bounds__(256) void k_pack_frag(const u16* __restrict__ w, u16* __restrict__ wf,
                                                   int c_red, int n_out, uint32_t* __restrict__ flag) {
    const int ncs = c_red / KS, nb = (n_out + 15) / 16;
    const int64_t slot = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (flag && slot == 0) *flag = 0u;  // orphan flag after a backward-input layout
    if (slot >= (int64_t)9 * ncs * nb * 64) return;
    // slot counts stay below 2^31 (the weight is under 2 GiB): 32-bit index math
    const int lane = (int)(slot & 63);
    uint32_t q = (uint32_t)(slot >> 6);
    const int b = (int)(q % (uint32_t)nb);
    q /= (uint32_t)nb;
    const int cs = (int)(q % (uint32_t)ncs);
    const int k = (int)(q / (uint32_t)ncs);
    const int n = b * 16 + (lane & 15);
    const int c = cs * KS + (lane >> 4) * 8;
    const rsrc_t rw = make_rsrc(w, 9u * (uint32_t)c_red * (uint32_t)n_out * 2u);
    *(u32x4*)(wf + slot * 8) = pack_slot<MODE == MODE_FWD>(rw, (uint32_t)k * c_red * n_out, c, n, c_red, n_out,
                                                          ((uintptr_t)w & 15) == 0);
}

// Both fragment-ordered layouts in one launch: slots [0, sf) write the
// forward layout (if wf_fwd), slots [sf, sf + sb) the backward-input layout
// (if wf_bwd). Same slot formula as k_pack_frag.
__global__ __launch_bounds__(256) void k_pack_both(const u16* __restrict__ w, u16* __restrict__ wf_fwd,
                                                   u16* __restrict__ wf_bwd, int c_in, int c_out,
                                                   int64_t sf, int64_t sb) {
    int64_t slot = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (wf_bwd && slot == 0) *(uint32_t*)(wf_bwd + sb * 8) = 0u;  // orphan flag after the layout
    const bool fwd = slot < sf;
    if (!fwd) slot -= sf;
    if (slot >= (fwd ? sf : sb)) return;
    const int c_red = fwd ? c_in : c_out, n_out = fwd ? c_out : c_in;
    const int ncs = c_red / KS, nb = (n_out + 15) / 16;
    const int lane = (int)(slot & 63);
    uint32_t q = (uint32_t)(slot >> 6);  // below 2^31 (host check on the weight size)
    const int b = (int)(q % (uint32_t)nb);
    q /= (uint32_t)nb;
    const int cs = (int)(q % (uint32_t)ncs);
    const int k = (int)(q / (uint32_t)ncs);
    const int n = b * 16 + (lane & 15);
    const int c = cs * KS + (lane >> 4) * 8;
    const rsrc_t rw = make_rsrc(w, 9u * (uint32_t)c_in * (uint32_t)c_out * 2u);
    const uint32_t kb = (uint32_t)k * c_in * c_out;
    const bool al16 = ((uintptr_t)w & 15) == 0;
    // sf is a multiple of 64: fwd is uniform in a wave
    const u32x4 o = fwd ? pack_slot<true>(rw, kb, c, n, c_red, n_out, al16)
                        : pack_slot<false>(rw, kb, c, n, c_red, n_out, al16);
    *(u32x4*)((fwd ? wf_fwd : wf_bwd) + slot * 8) = o;
}

// ---------------------------------------------------------------------------
// Backward-weight partials: ws[s][k][ci][co] = sum over rows i of split s of
// x[src(i,k), ci] * go[i, co]; ws_bias[s][co] = sum of go[i, co] (written by
// the k == 4, ci-tile 0 workgroups). Grid: 1-D over (tiles x splits), the
// tiles of one split consecutive (they read the same rows).
// Per stage the workgroup takes KR = 64 rows: x rows gathered through the
// split's source-row list (staged in LDS once) and go rows, both written
// transposed into LDS ([channel][row], rows contiguous) so each MFMA operand
// fragment is one 16-byte read. Loads of stage t+1 are in flight while stage
// t runs; a split holds at most kMaxSplitRows rows.
// ---------------------------------------------------------------------------
constexpr int KR = 64;
constexpr int RPK = KR + 8;  // LDS pitch of a transposed stage: 144 bytes

template <typename T, int FM, int FN>
__global__ __launch_bounds__(256) void k_bw_mfma(
    const T* __restrict__ go, const T* __restrict__ x, const int32_t* __restrict__ nbr,
    float* __restrict__ ws, float* __restrict__ ws_bias, int64_t n, int c_in, int c_out,
    int64_t tpb, int64_t rows_per_split, int n_ci_tiles, int n_co_tiles, int64_t n_blocks) {
    constexpr int BM = 2 * FM * 16;  // ci
    constexpr int BN = 2 * FN * 16;  // co
    constexpr int A_ITEMS = (KR / 2) * (BM / 8);
    constexpr int B_ITEMS = (KR / 2) * (BN / 8);
    constexpr int A_PER = (A_ITEMS + 255) / 256;
    constexpr int B_PER = (B_ITEMS + 255) / 256;

    __shared__ __align__(16) u16 As[2][BM][RPK];
    __shared__ __align__(16) u16 Bs[2][BN][RPK];
    __shared__ uint32_t srow[kMaxSplitRows];  // byte offset of x[src(i,k)], kOOB if missing

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int64_t lin = xcd_tile(blockIdx.x, n_blocks);
    const int tiles = 9 * n_ci_tiles * n_co_tiles;
    const int s = (int)(lin / tiles);
    int rem = (int)(lin - (int64_t)s * tiles);
    const int k = rem / (n_ci_tiles * n_co_tiles);
    rem -= k * n_ci_tiles * n_co_tiles;
    const int ci0 = (rem / n_co_tiles) * BM;
    const int co0 = (rem % n_co_tiles) * BN;
    const int64_t r_begin = (int64_t)s * rows_per_split;
    const int rows = (int)max<int64_t>(0, min(n, r_begin + rows_per_split) - r_begin);
    const int steps = (rows + KR - 1) / KR;
    const bool do_bias = ws_bias != nullptr && k == 4 && ci0 == 0;

    for (int r = tid; r < steps * KR; r += 256) {
        const int64_t sr = r < rows ? src_row(nbr, r_begin + r, k, n, tpb) : -1;
        srow[r] = sr >= 0 ? (uint32_t)sr * (uint32_t)(c_in * 2) : kOOB;
    }
    __syncthreads();

    const rsrc_t rs_x = make_rsrc(x, (uint32_t)(n * c_in * 2));
    const rsrc_t rs_g = make_rsrc(go + r_begin * c_out, (uint32_t)((int64_t)rows * c_out * 2));

    // per-thread constants: channel byte offsets (x) and row-pair byte offsets (go)
    bool a_ok[A_PER];
    uint32_t a_c[A_PER];
    uint32_t b_off[B_PER];
#pragma unroll
    for (int q = 0; q < A_PER; ++q) {
        const int e = tid + q * 256;
        const int c = ci0 + (e >> 5) * 8;
        a_ok[q] = e < A_ITEMS && c < c_in;
        a_c[q] = (uint32_t)c * 2u;
    }
#pragma unroll
    for (int q = 0; q < B_PER; ++q) {
        const int e = tid + q * 256;
        const int c = co0 + (e >> 5) * 8;
        b_off[q] = (e < B_ITEMS && c < c_out) ? (uint32_t)(2 * (e & 31) * c_out + c) * 2u : kOOB;
    }

    u32x4 ra[A_PER][2], rb[B_PER][2];
    auto load = [&](int t) {
        const int r0 = t * KR;
#pragma unroll
        for (int q = 0; q < A_PER; ++q) {
            const int rp = (tid + q * 256) & 31;
            const uint32_t s0 = srow[r0 + 2 * rp], s1 = srow[r0 + 2 * rp + 1];
            ra[q][0] = bload16(rs_x, a_ok[q] ? s0 + a_c[q] : kOOB);
            ra[q][1] = bload16(rs_x, a_ok[q] ? s1 + a_c[q] : kOOB);
        }
        // rows past the split read out of range -> 0
        const uint32_t g0 = (uint32_t)(r0 * c_out) * 2u;
#pragma unroll
        for (int q = 0; q < B_PER; ++q) {
            rb[q][0] = bload16(rs_g, b_off[q] + g0);
            rb[q][1] = bload16(rs_g, b_off[q] + g0 + (uint32_t)c_out * 2u);
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int q = 0; q < A_PER; ++q) {
            const int e = tid + q * 256;
            if (e >= A_ITEMS) continue;
            const int rp = e & 31, g = e >> 5;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                *(unsigned*)&As[buf][g * 8 + j][2 * rp] =
                    (unsigned)half_of(ra[q][0], j) | ((unsigned)half_of(ra[q][1], j) << 16);
        }
#pragma unroll
        for (int q = 0; q < B_PER; ++q) {
            const int e = tid + q * 256;
            if (e >= B_ITEMS) continue;
            const int rp = e & 31, g = e >> 5;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                *(unsigned*)&Bs[buf][g * 8 + j][2 * rp] =
                    (unsigned)half_of(rb[q][0], j) | ((unsigned)half_of(rb[q][1], j) << 16);
        }
    };

    f32x4 acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    float bsum = 0.f;

    const int wm = wave >> 1, wn = wave & 1;
    const int arow = wm * FM * 16 + (lane & 15);
    const int brow = wn * FN * 16 + (lane & 15);
    const int kof = (lane >> 4) * 8;

    if (steps > 0) {
        load(0);
        store(0);
    }
    __syncthreads();
    for (int t = 0; t < steps; ++t) {
        const int buf = t & 1;
        if (t + 1 < steps) load(t + 1);
#pragma unroll
        for (int h = 0; h < KR / KS; ++h) {
            u32x4 fa[FM], fb[FN];
#pragma unroll
            for (int a = 0; a < FM; ++a) fa[a] = *(const u32x4*)&As[buf][arow + a * 16][h * KS + kof];
#pragma unroll
            for (int b = 0; b < FN; ++b) fb[b] = *(const u32x4*)&Bs[buf][brow + b * 16][h * KS + kof];
#pragma unroll
            for (int a = 0; a < FM; ++a)
#pragma unroll
                for (int b = 0; b < FN; ++b) acc[a][b] = MfmaOp<T>::run(fa[a], fb[b], acc[a][b]);
        }
        if (do_bias && tid < BN) {
#pragma unroll
            for (int r = 0; r < KR; r += 2) {
                const unsigned pr = *(const unsigned*)&Bs[buf][tid][r];
                bsum += (float)__builtin_bit_cast(T, (u16)(pr & 0xffffu));
                bsum += (float)__builtin_bit_cast(T, (u16)(pr >> 16));
            }
        }
        if (t + 1 < steps) store(buf ^ 1);
        __syncthreads();
    }

    float* dst = ws + ((int64_t)s * 9 + k) * c_in * c_out;
#pragma unroll
    for (int b = 0; b < FN; ++b) {
        const int co = co0 + wn * FN * 16 + b * 16 + (lane & 15);
        if (co >= c_out) continue;
#pragma unroll
        for (int a = 0; a < FM; ++a)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int ci = ci0 + wm * FM * 16 + a * 16 + (lane >> 4) * 4 + j;
                if (ci < c_in) dst[(int64_t)ci * c_out + co] = acc[a][b][j];
            }
    }
    if (do_bias && tid < BN && co0 + tid < c_out) ws_bias[(int64_t)s * c_out + co0 + tid] = bsum;
}

// ---------------------------------------------------------------------------
// Backward-weight partials, large tiles (the shapes of the adapter convs).
// A workgroup owns one work unit of a row split and a BM x BN (ci x co) tile
// of gw. A split has 10 units: each off-center offset k over the split's
// rows, visiting only the rows whose neighbor k exists (compacted in row
// order; a missing neighbor's x row is zero and adds nothing), and the center
// offset over each half of the split (all rows: the center units also sum
// the bias). At moderate keep rates about half of an off-center offset's
// neighbors exist, so all units take about as many stages. The workgroup has
// two kinds of waves:
//  * WGM x WGN matrix waves, each owning FM x FN 16x16 fragments of the tile;
//    per 64-row stage they read their fragments from LDS and run the MFMAs.
//  * WA + WB staging waves: per stage each thread loads an 8-row x 8-channel
//    block of the gathered x rows (waves [0, WA)) or of the go rows (the
//    next WB) with 16-byte loads (consecutive lanes on consecutive channel
//    chunks of a row), transposes it in registers (v_perm_b32) and writes
//    eight 16-byte rows of a [channel][row] LDS tile (swizzled by bw_swz), so
//    that an MFMA fragment (8 consecutive rows of one channel) is one 16-byte
//    LDS read.
// Between two barriers the matrix waves consume stage t from one LDS buffer
// while the staging waves fill the other with stage t+1 and have the loads of
// stage t+2 in flight: the MFMAs, the transposes and LDS writes, and the
// global loads run at the same time on different waves. (With one kind of
// wave doing both, every wave of a SIMD is in its transpose phase at the same
// time and the matrix core idles.) Partials are stored in fragment order
// (each lane's 4 values contiguous); k_bw_reduce sums the splits in a fixed
// order. In the center units of ci-tile 0 the go staging threads also sum
// their transposed go blocks per column (bias; fp32, v_dot2 against ones),
// and the row groups' sums are added in order through LDS at the end.
// ---------------------------------------------------------------------------
// A transposed stage row (one channel, KR = 64 source rows) is 128 bytes with
// no padding; its eight 16-byte chunks (8 rows each) are stored at position
// chunk ^ (channel & 7) ^ rot3((channel >> 3) & 7), rot3 a 3-bit rotate left.
// On gfx950 (measured with bank-conflict counters) a 16-byte LDS read serves
// lanes {0-7, 24-31}, {8-15, 16-23} (and the same in the upper half) together,
// and a 16-byte LDS write serves 8 consecutive lanes together; the 16 lanes
// served together must touch distinct 16-byte bank groups (64 banks of 4
// bytes). The fragment reads (16 consecutive channels x 4 chunks) then have
// no conflicts because rot3 changes between the two 8-channel halves of a
// fragment by an even amount, while (channel >> 3) alone changes by 1 and
// makes lanes i and 24+i collide; the transposed stores (8 lanes on 8
// consecutive channel chunks) have none because rot3 is a bijection. A padded
// 144-byte pitch halves the read rate. Returns the element offset in the row.
__device__ __forceinline__ int bw_swz(int channel, int chunk) {
    const int hi = (channel >> 3) & 7;
    return (chunk ^ (channel & 7) ^ (((hi << 1) | (hi >> 2)) & 7)) * 8;
}

// 8x8 transpose of 16-bit values: in[r] holds channels 0..7 of row r; out[c]
// gets rows 0..7 of channel c.
__device__ __forceinline__ void transpose8(const u32x4* in, u32x4* out) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int d = c >> 1;
        const unsigned sel = (c & 1) ? 0x07060302u : 0x05040100u;
        u32x4 o;
#pragma unroll
        for (int q = 0; q < 4; ++q) o[q] = __builtin_amdgcn_perm(in[2 * q + 1][d], in[2 * q][d], sel);
        out[c] = o;
    }
}

// gw[k][ci][co] = T(sum_s part[s]...) for the fragment-ordered partials of
// k_bw_big (quadruple e: 4 consecutive floats of one lane). Four threads
// (one per wave of the workgroup) share a quadruple: thread g sums its
// quarter of the splits with all its loads in flight, and the quarters are
// added in order g = 0..3 through LDS, so the order of the sum is fixed.
// The partials are read once: non-temporal loads.
template <typename T>
__device__ __forceinline__ void bw_store_quad(int64_t e, f32x4 acc, int c_in, int c_out, int fm, int fn,
                                              int wgm, int wgn, int n_ci_tiles, int n_co_tiles,
                                              T* __restrict__ gw);

template <typename T, int CP>
__device__ __forceinline__ void bw_reduce_quads(int64_t blk, const float* __restrict__ part,
                                                int splits, int n_off, int c_in, int c_out, int fm, int fn,
                                                int wgm, int wgn, int n_ci_tiles, int n_co_tiles,
                                                T* __restrict__ gw) {
    __shared__ f32x4 qsum[4][64];
    const int lane = threadIdx.x & 63, g = threadIdx.x >> 6;
    // a split's partials: one block of c_in * c_out per work unit (with the
    // 9 offsets: offsets 0-3, the center's CP parts, offsets 5-8)
    static_assert(CP == 2 || CP == 4, "center parts");
    const int units = n_off == 9 ? 8 + CP : n_off;
    const int64_t per_off = (int64_t)c_in * c_out;
    const int64_t per_split = units * per_off;
    const int64_t quads = (int64_t)n_off * per_off / 4;
    const int64_t e = blk * 64 + lane;
    const int spt = (splits + 3) / 4;
    const int s0 = g * spt, s1 = min(splits, s0 + spt);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (e < quads) {
        const int ko = (int)(e * 4 / per_off);
        const int64_t within = e * 4 - ko * per_off;
        const int unit = n_off == 9 && ko > 4 ? ko + CP - 1 : ko;
        const float* pe = part + unit * per_off + within;
        if (n_off == 9 && ko == 4) {
            // the center's parts, added in order per split (split-major):
            // 8 loads in flight, 8 / CP splits of CP parts
            for (int q = s0; q < s1; q += 8 / CP) {
                f32x4 v[8];
#pragma unroll
                for (int u = 0; u < 8 / CP; ++u) {
                    const bool ok = q + u < s1;
#pragma unroll
                    for (int pt = 0; pt < CP; ++pt)
                        v[u * CP + pt] = ok ? __builtin_nontemporal_load((const f32x4*)(pe + pt * per_off + (int64_t)(q + u) * per_split))
                                            : f32x4{0.f, 0.f, 0.f, 0.f};
                }
#pragma unroll
                for (int u = 0; u < 8; ++u) acc += v[u];
            }
        } else {
            for (int q = s0; q < s1; q += 8) {
                f32x4 v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u)
                    v[u] = q + u < s1 ? __builtin_nontemporal_load((const f32x4*)(pe + (int64_t)(q + u) * per_split)) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int u = 0; u < 8; ++u) acc += v[u];
            }
        }
    }
    qsum[g][lane] = acc;
    __syncthreads();
    if (g != 0 || e >= quads) return;
    acc = qsum[0][lane] + qsum[1][lane];
    acc += qsum[2][lane];
    acc += qsum[3][lane];
    bw_store_quad<T>(e, acc, c_in, c_out, fm, fn, wgm, wgn, n_ci_tiles, n_co_tiles, gw);
}

// The store of quadruple e's sum into gw (its fragment-order position decoded).
template <typename T>
__device__ __forceinline__ void bw_store_quad(int64_t e, f32x4 acc, int c_in, int c_out, int fm, int fn,
                                              int wgm, int wgn, int n_ci_tiles, int n_co_tiles,
                                              T* __restrict__ gw) {
    const int bm = wgm * fm * 16, bn = wgn * fn * 16;
    int64_t rest = e * 4;
    const int64_t tile_sz = (int64_t)bm * bn;
    const int64_t tile = rest / tile_sz;
    rest -= tile * tile_sz;
    const int k = (int)(tile / (n_ci_tiles * n_co_tiles));
    const int tr = (int)(tile - (int64_t)k * n_ci_tiles * n_co_tiles);
    const int ci0 = (tr / n_co_tiles) * bm, co0 = (tr % n_co_tiles) * bn;
    const int ln = (int)((rest >> 2) & 63);
    int fr = (int)(rest >> 8);  // (wave * fm + a) * fn + b
    const int b = fr % fn;
    fr /= fn;
    const int a = fr % fm;
    const int wave = fr / fm;
    const int ci = ci0 + (wave / wgn) * fm * 16 + a * 16 + (ln >> 4) * 4;
    const int co = co0 + (wave % wgn) * fn * 16 + b * 16 + (ln & 15);
    T* gp = gw + ((int64_t)k * c_in + ci) * c_out + co;
#pragma unroll
    for (int j = 0; j < 4; ++j) gp[(int64_t)j * c_out] = (T)acc[j];
}

// bw_reduce_quads with at most two splits (up to four work): one thread per
// quadruple sums each split (its center parts in order) and then the splits
// in order, with every load in flight and no LDS. These are the same
// additions in the same order as the four-thread form (a sum that starts at
// +0 is never -0, so the zero terms that form adds change nothing): the
// results are bit-identical. Config 4 at 10 % keep (2 splits): step 41.3 ->
// 40.3 us; with 4 splits (c2 at 10 %, 16 loads per thread on the center
// quadruples) the step was 1.4 us slower, so those keep the four threads.
template <typename T, int CP>
__device__ __forceinline__ void bw_reduce_quads_direct(int64_t e, const float* __restrict__ part,
                                                       int splits, int n_off, int c_in, int c_out, int fm,
                                                       int fn, int wgm, int wgn, int n_ci_tiles,
                                                       int n_co_tiles, T* __restrict__ gw) {
    const int units = n_off == 9 ? 8 + CP : n_off;
    const int64_t per_off = (int64_t)c_in * c_out;
    const int64_t per_split = units * per_off;
    if (e >= (int64_t)n_off * per_off / 4) return;
    const int ko = (int)(e * 4 / per_off);
    const int64_t within = e * 4 - ko * per_off;
    const int unit = n_off == 9 && ko > 4 ? ko + CP - 1 : ko;
    const float* pe = part + unit * per_off + within;
    const int np = n_off == 9 && ko == 4 ? CP : 1;  // the center's parts
    f32x4 v[4][CP];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int pt = 0; pt < CP; ++pt)
            v[q][pt] = q < splits && pt < np
                           ? __builtin_nontemporal_load((const f32x4*)(pe + pt * per_off + (int64_t)q * per_split))
                           : f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 sq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        sq[q] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int pt = 0; pt < CP; ++pt) sq[q] += v[q][pt];
    }
    f32x4 acc = sq[0] + sq[1];
    acc += sq[2];
    acc += sq[3];
    bw_store_quad<T>(e, acc, c_in, c_out, fm, fn, wgm, wgn, n_ci_tiles, n_co_tiles, gw);
}

// Workgroups of k_bw_reduce for the gw quadruples: 256 quadruples each with at
// most two splits (bw_reduce_quads_direct), else 64.
__host__ __device__ inline int64_t bw_quad_blocks(int64_t quads, int splits) {
    const int64_t per = splits <= 2 ? 256 : 64;
    return (quads + per - 1) / per;
}

// gb[c] = T(sum_s part_b[s][c]), splits summed in order.
template <typename T>
__device__ __forceinline__ void bw_reduce_bias(int64_t c, const float* __restrict__ part_b,
                                               int splits, int c_out, T* __restrict__ gb) {
    if (c >= c_out) return;
    float v = 0.f;
    int q = 0;
    for (; q + 8 <= splits; q += 8) {
        float t[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) t[u] = part_b[(int64_t)(q + u) * c_out + c];
#pragma unroll
        for (int u = 0; u < 8; ++u) v += t[u];
    }
    for (; q < splits; ++q) v += part_b[(int64_t)q * c_out + c];
    gb[c] = (T)v;
}

// acc + lo + hi of a pair of 16-bit values (v_dot2 against (1, 1): the
// products are exact, the sum is fp32)
template <typename T>
__device__ __forceinline__ float dot2_ones(uint32_t v, float acc);
template <>
__device__ __forceinline__ float dot2_ones<f16>(uint32_t v, float acc) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, v), h2{(_Float16)1, (_Float16)1}, acc, false);
}
template <>
__device__ __forceinline__ float dot2_ones<bf16>(uint32_t v, float acc) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, v), b2{(__bf16)1.0f, (__bf16)1.0f}, acc, false);
}

// staging waves of k_bw_big: one 8-row x 8-channel block of x rows or of go
// rows per thread and stage.
// With n_off = 9, nbr is the [n, 9] neighbor table and the partials cover the
// 9 offsets. With n_off = 1, nbr is a list of n source rows of x (NULL: row i
// itself) and the kernel computes the plain reduction gw[ci][co] = sum_i
// x[nbr[i]][ci] go[i][co] (a linear layer's weight gradient); x then has
// n_src rows.
constexpr int BW_IROWS = 8;
constexpr int bw_stage_waves(int fm, int fn, int wgm, int wgn) {
    return ((KR / BW_IROWS) * (wgm * fm * 2) + 63) / 64 + ((KR / BW_IROWS) * (wgn * fn * 2) + 63) / 64;
}
constexpr int bw_big_threads(int fm, int fn, int wgm, int wgn) {
    return 64 * (wgm * wgn + bw_stage_waves(fm, fn, wgm, wgn));
}

template <int FM, int FN, int WGM, int WGN>
struct BwBigLds {
    static constexpr int NT = bw_big_threads(FM, FN, WGM, WGN);
    // [buf][channel][row] tiles: the x operand's two buffers, then go's
    __align__(16) u16 stage[2 * (WGM * FM * 16 + WGN * FN * 16) * KR];
    // byte offsets of the split's rows in x (gathered) and in go (linear),
    // kOOB for missing neighbors and for rows past the split; two stages
    // past the last one so that the prefetch needs no bounds test
    __align__(16) uint32_t srow[2][kMaxSplitRows + 2 * KR];
    int wcnt[(kMaxSplitRows + NT - 1) / NT][NT / 64];  // per-wave counts of the row-list compaction
};

// One work unit (split s, unit u, ci tile, co tile = lin) of the
// backward-weight partials, run by all bw_big_threads threads of a workgroup
// (k_bw_big, or the backward-weight role of k_bwd_fused) in the LDS block L.
// With the 9 offsets the center offset's rows are split into CP (2 or 4)
// units: a split holds 8 + CP units.
template <typename T, int FM, int FN, int WGM, int WGN, int CP>
__device__ __forceinline__ void bw_big_unit(
    BwBigLds<FM, FN, WGM, WGN>& L, int64_t lin, const T* __restrict__ go, const T* __restrict__ x,
    const int32_t* __restrict__ nbr, float* __restrict__ ws, float* __restrict__ ws_bias, int64_t n,
    int c_in, int c_out, int64_t tpb, int64_t rows_per_split, int n_ci_tiles, int n_co_tiles, int n_off,
    int64_t n_src) {
    static_assert(CP == 2 || CP == 4, "center parts");
    constexpr int NT = bw_big_threads(FM, FN, WGM, WGN);
    constexpr int NMW = WGM * WGN;     // matrix waves
    constexpr int BM = WGM * FM * 16;  // ci
    constexpr int BN = WGN * FN * 16;  // co
    constexpr int A_ITEMS = (KR / BW_IROWS) * (BM / 8);  // 8x8 blocks per stage
    constexpr int B_ITEMS = (KR / BW_IROWS) * (BN / 8);
    // Consecutive items walk the 8-channel chunks of one row group, so eight
    // consecutive lanes load 128 contiguous bytes of a row (lanes walking the
    // row groups instead load 16 bytes from each of 8 rows per 8 lanes, which
    // costs more address-unit cycles than the LDS conflicts it avoids; the
    // bw_swz swizzle keeps the chunk-major stores conflict-free).
    constexpr int CPT_A = BM / 8, CPT_B = BN / 8;  // channel chunks per row group
    constexpr int WA = (A_ITEMS + 63) / 64, WB = (B_ITEMS + 63) / 64;
    static_assert(NMW + WA + WB == NT / 64, "wave roles");

    static_assert(sizeof(L.stage) == (size_t)2 * (BM + BN) * KR * 2, "stage tiles");
    u16* const stage_lds = L.stage;
    u16(*const As)[BM][KR] = (u16(*)[BM][KR])stage_lds;
    u16(*const Bs)[BN][KR] = (u16(*)[BN][KR])(stage_lds + 2 * BM * KR);
    auto& srow = L.srow;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    // work units of a split: with the 9 offsets, units 0-3 and 4+CP .. 7+CP
    // are the offsets 0-3 and 5-8 over the split's rows, and units 4 ..
    // 3+CP the center offset over consecutive parts of the split
    // (rows_per_split is a multiple of 256, so each part is whole stages)
    const int units = n_off == 9 ? 8 + CP : 1;
    const int tiles = units * n_ci_tiles * n_co_tiles;
    const int s = (int)(lin / tiles);
    int rem = (int)(lin - (int64_t)s * tiles);
    const int u = rem / (n_ci_tiles * n_co_tiles);
    rem -= u * n_ci_tiles * n_co_tiles;
    const int k = n_off == 9 ? (u < 4 ? u : (u < 4 + CP ? 4 : u - CP + 1)) : 0;
    const bool center = n_off == 9 && k == 4;
    const bool compact = n_off == 9 && !center;  // uniform
    const int cit = rem / n_co_tiles, cot = rem % n_co_tiles;
    const int ci0 = cit * BM, co0 = cot * BN;
    const int64_t part_len = rows_per_split / CP;
    const int64_t r_begin = (int64_t)s * rows_per_split + (center ? (u - 4) * part_len : 0);
    const int64_t r_len = center ? part_len : rows_per_split;
    const int rows_raw = (int)max<int64_t>(0, min(n, r_begin + r_len) - r_begin);
    const bool do_bias = ws_bias != nullptr && (n_off == 9 ? center : true) && ci0 == 0;  // uniform

    // An off-center offset's list holds only the rows whose neighbor exists,
    // in row order (a missing neighbor's x row is zero and adds nothing):
    // order-preserving compaction over chunks of NT rows. The table entries of
    // every chunk are loaded first (one memory round trip for the split), the
    // per-wave counts of all chunks meet in LDS behind one barrier, and each
    // thread then places its rows after the rows of earlier chunks and waves.
    constexpr int MAXCH = (kMaxSplitRows + NT - 1) / NT;
    auto& wcnt = L.wcnt;
    int rows = rows_raw;
    if (compact) {
        int sv[MAXCH];
#pragma unroll
        for (int c = 0; c < MAXCH; ++c) {
            const int r = c * NT + tid;
            sv[c] = r < rows_raw ? (int)src_row(nbr, r_begin + r, k, n, tpb) : -1;
        }
#pragma unroll
        for (int c = 0; c < MAXCH; ++c) {
            if (c * NT < rows_raw) {  // uniform
                const uint64_t bal = __ballot(sv[c] >= 0);
                if (lane == 0) wcnt[c][wave] = __popcll(bal);
            }
        }
        __syncthreads();
        int total = 0;
#pragma unroll
        for (int c = 0; c < MAXCH; ++c) {
            if (c * NT < rows_raw) {  // uniform
                const bool v = sv[c] >= 0;
                const uint64_t bal = __ballot(v);
                const int before = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                             __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
                int off = 0, all = 0;
#pragma unroll
                for (int w = 0; w < NT / 64; ++w) {
                    const int cnt = wcnt[c][w];
                    off += w < wave ? cnt : 0;
                    all += cnt;
                }
                if (v) {
                    srow[0][total + off + before] = (uint32_t)sv[c] * (uint32_t)(c_in * 2);
                    srow[1][total + off + before] = (uint32_t)(c * NT + tid) * (uint32_t)(c_out * 2);
                }
                total += all;
            }
        }
        rows = total;
    }
    const int steps = (rows + KR - 1) / KR;

    // The staging waves read the list two stages at a time up to stage
    // steps_even + 1 (steps rounded up to even), so it is filled that far;
    // with rows_per_split <= kMaxSplitRows (checked on the host) that is at
    // most kMaxSplitRows + 2 * KR entries (L.srow). A compacted list is only
    // padded.
    const int steps_even = (steps + 1) & ~1;
    for (int r = (compact ? rows : 0) + tid; r < (steps_even + 2) * KR; r += NT) {
        const bool live = !compact && r < rows;
        int64_t sr = -1;
        if (live) {
            if (n_off == 9) {
                sr = src_row(nbr, r_begin + r, k, n, tpb);
            } else {  // row list (NULL: identity)
                sr = nbr ? (int64_t)nbr[r_begin + r] : r_begin + r;
                if (sr >= n_src) sr = -1;
            }
        }
        srow[0][r] = sr >= 0 ? (uint32_t)sr * (uint32_t)(c_in * 2) : kOOB;
        srow[1][r] = live ? (uint32_t)r * (uint32_t)(c_out * 2) : kOOB;
    }
    __syncthreads();

    const int wv = __builtin_amdgcn_readfirstlane(wave);
    if (wv < NMW) {
        // ---------------- matrix waves ----------------
        f32x4 acc[FM][FN];
#pragma unroll
        for (int a = 0; a < FM; ++a)
#pragma unroll
            for (int b = 0; b < FN; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int wm = wv / WGN, wn = wv % WGN;
        const int arow = wm * FM * 16 + (lane & 15), brow = wn * FN * 16 + (lane & 15);
        // fragment chunk of k-step h is h*4 + lane/16 (bw_swz gives its position)
        const int kq = lane >> 4;
        auto compute = [&](int buf) {
#pragma unroll
            for (int h = 0; h < KR / KS; ++h) {
                u32x4 fb[FN];
#pragma unroll
                for (int b = 0; b < FN; ++b)
                    fb[b] = *(const u32x4*)&Bs[buf][brow + b * 16][bw_swz(brow + b * 16, h * 4 + kq)];
#pragma unroll
                for (int a = 0; a < FM; ++a) {
                    const u32x4 fa = *(const u32x4*)&As[buf][arow + a * 16][bw_swz(arow + a * 16, h * 4 + kq)];
#pragma unroll
                    for (int b = 0; b < FN; ++b) acc[a][b] = MfmaOp<T>::run(fa, fb[b], acc[a][b]);
                }
            }
        };
        __syncthreads();  // stage 0 staged
        for (int t = 0; t < steps; ++t) {
            compute(t & 1);  // stage t
            __syncthreads();
        }
        // partial tile in fragment order: [wave][a][b][lane][4]; non-temporal
        // stores (read once, by the reduction): they stream out while the
        // other workgroups finish instead of waiting in the L2 for the write-
        // back at the kernel's end
        float* dst = ws + (((int64_t)s * units + u) * n_ci_tiles * n_co_tiles + cit * n_co_tiles + cot) * BM * BN;
#pragma unroll
        for (int a = 0; a < FM; ++a)
#pragma unroll
            for (int b = 0; b < FN; ++b)
                __builtin_nontemporal_store(acc[a][b], (f32x4*)(dst + (((wv * FM + a) * FN + b) * 64 + lane) * 4));
        if (do_bias) __syncthreads();  // the staging waves' bias reduction
    } else {
        // ---------------- staging waves ----------------
        // item e of the wave's operand: rows 8*(e / cpt) .. +7 of the
        // stage, channels 8*(e % cpt) .. +7 of the tile. Stages at or past
        // `steps`, and threads without an item, load zeros (out-of-range
        // offsets). Everything that depends on the wave's operand is fixed
        // here, so the loop's loads and stores are one code path for both
        // operands (a select on a wave-uniform value inside the loop becomes
        // a branch around each load, and every branch makes the compiler wait
        // for the loads in flight).
        const int sw = wv - NMW;  // staging wave index
        const int st = tid - NMW * 64;
        const bool role_a = sw < WA;
        const int e = role_a ? st : st - WA * 64;
        const int n_items = role_a ? A_ITEMS : B_ITEMS;
        const bool has_item = e < n_items;
        const int cpt = role_a ? CPT_A : CPT_B;
        const int rgp = has_item ? e / cpt : 0, cl = has_item ? (e % cpt) * 8 : 0;
        const int chan = (role_a ? ci0 : co0) + cl;
        const bool chan_ok = has_item && chan < (role_a ? c_in : c_out);
        const rsrc_t rs = make_rsrc(role_a ? (const void*)x : (const void*)(go + r_begin * c_out),
                                    role_a ? (uint32_t)(n_src * c_in * 2) : (uint32_t)((int64_t)rows_raw * c_out * 2));
        // offsets stay below 2^31 + 2^16 (kOOB plus a channel offset): no wrap
        const uint32_t chan_b = chan_ok ? (uint32_t)chan * 2u : kOOB;
        const uint32_t* const tab = srow[role_a ? 0 : 1] + rgp * BW_IROWS;
        // this thread's 8 LDS rows (channels cl .. cl+7) of buffer 0; buffer
        // 1 is buf_step elements further
        u16* const dst0 = role_a ? &As[0][cl][0] : &Bs[0][cl][0];
        const int buf_step = role_a ? BM * KR : BN * KR;

        // two register sets: the loads of stage t+2 are in flight while stage
        // t+1 is transposed and stored
        u32x4 r0s[8], r1s[8];
        auto load = [&](int t, u32x4* rg) {
            const u32x4 s0 = *(const u32x4*)&tab[t * KR];
            const u32x4 s1 = *(const u32x4*)&tab[t * KR + 4];
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const uint32_t so = r < 4 ? s0[r] : s1[r - 4];
                rg[r] = bload16(rs, chan_ok ? so + chan_b : kOOB);
            }
        };
        // column sums of the staged go rows (the bias gradient; the center
        // units of column tile 0): each thread adds its 8-row x 8-channel
        // blocks per channel in fp32, two rows per dot2 instruction on the
        // transposed registers, and stores one partial per row group
        const bool bias_thr = do_bias && !role_a;  // wave-uniform
        float bacc[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) bacc[c] = 0.f;
        auto store = [&](int buf, const u32x4* rg) {
            u32x4 o[8];
            transpose8(rg, o);
            if (has_item) {
                u16* const d = dst0 + buf * buf_step;
#pragma unroll
                for (int c = 0; c < 8; ++c) *(u32x4*)&d[c * KR + bw_swz(cl + c, rgp)] = o[c];
            }
            if (bias_thr) {
#pragma unroll
                for (int c = 0; c < 8; ++c)
#pragma unroll
                    for (int q = 0; q < 4; ++q) bacc[c] = dot2_ones<T>(o[c][q], bacc[c]);
            }
        };
        load(0, r0s);
        load(1, r1s);
        store(0, r0s);
        __syncthreads();  // stage 0 staged
        int t = 0;
        for (; t + 1 < steps; t += 2) {
            load(t + 2, r0s);  // registers of set 0 are free again
            store(1, r1s);     // stage t+1
            __syncthreads();
            load(t + 3, r1s);
            store(0, r0s);     // stage t+2 (zeros past the end)
            __syncthreads();
        }
        if (t < steps) __syncthreads();  // the matrix waves' last single stage
        if (do_bias) {
            // the row groups' sums added in order through LDS (the stage
            // buffers are free: every wave is past its last stage)
            float* const red = (float*)stage_lds;  // [row group][column]
            if (bias_thr && has_item) {
#pragma unroll
                for (int c = 0; c < 8; ++c) red[rgp * BN + cl + c] = bacc[c];
            }
            __syncthreads();
            for (int col = tid - NMW * 64; col < BN; col += NT - NMW * 64) {
                float v = 0.f;
#pragma unroll
                for (int g = 0; g < BW_IROWS; ++g) v += red[g * BN + col];
                if (co0 + col < c_out) ws_bias[((int64_t)s * CP + (u - 4)) * c_out + co0 + col] = v;
            }
        }
    }
}

template <typename T, int FM, int FN, int WGM, int WGN>
__global__ __launch_bounds__(bw_big_threads(FM, FN, WGM, WGN)) void k_bw_big(
    const T* __restrict__ go, const T* __restrict__ x, const int32_t* __restrict__ nbr,
    float* __restrict__ ws, float* __restrict__ ws_bias, int64_t n, int c_in, int c_out,
    int64_t tpb, int64_t rows_per_split, int n_ci_tiles, int n_co_tiles, int64_t n_blocks, int n_off,
    int64_t n_src) {
    __shared__ BwBigLds<FM, FN, WGM, WGN> lds;
    bw_big_unit<T, FM, FN, WGM, WGN, 2>(lds, xcd_tile(blockIdx.x, n_blocks), go, x, nbr, ws, ws_bias, n, c_in,
                                        c_out, tpb, rows_per_split, n_ci_tiles, n_co_tiles, n_off, n_src);
}

// Backward-input and the backward-weight partials in one launch, for shapes
// where neither grid fills the chip (low keep rates): workgroups [0, n_bw)
// of the XCD-major order run the backward-weight units (all
// bw_big_threads threads), the rest the gathered-GEMM tiles of
// backward-input (threads [0, 256 * GWS); the other waves end at once, and
// a workgroup barrier waits only for waves that have not ended). The two
// roles share one LDS block. The host launches it only when the grid fits
// one workgroup per CU and the tile kernel's registers fit this launch's.
template <typename T, int CR, int GFM, int GFN, int GD, int GWS, int FM, int FN, int WGM, int WGN, int CP>
__global__ __launch_bounds__(bw_big_threads(FM, FN, WGM, WGN)) void k_bwd_fused(
    const T* __restrict__ go, const int32_t* __restrict__ nbr, const T* __restrict__ wb, T* __restrict__ gi,
    int n_in, int n_col_tiles, uint32_t* __restrict__ orphan_flag, const T* __restrict__ x,
    float* __restrict__ ws, float* __restrict__ ws_bias, int64_t n, int64_t tpb, int64_t rows_per_split,
    int n_ci_tiles, int n_co_tiles, int64_t n_bw, int64_t n_blocks, bool sym) {
    typedef GgWideLds<CR, GFM, GFN, GWS> GL;
    typedef BwBigLds<FM, FN, WGM, WGN> BL;
    static_assert(256 * GWS <= bw_big_threads(FM, FN, WGM, WGN), "tile role threads");
    __shared__ __align__(16) char lds[sizeof(GL) > sizeof(BL) ? sizeof(GL) : sizeof(BL)];
    const int64_t lin = xcd_tile(blockIdx.x, n_blocks);
    if (lin < n_bw) {
        bw_big_unit<T, FM, FN, WGM, WGN, CP>(*(BL*)lds, lin, go, x, nbr, ws, ws_bias, n, n_in, CR, tpb,
                                             rows_per_split, n_ci_tiles, n_co_tiles, 9, n);
    } else {
        if (threadIdx.x >= 256 * GWS) return;
        gg_wide_tile<T, MODE_BWDIN, CR, GFM, GFN, GD, GWS>(*(GL*)lds, lin - n_bw, go, nbr, wb, nullptr, 0, gi, n,
                                                         n_in, tpb, n_col_tiles, orphan_flag, sym);
    }
}

// The reduction of the partials; with a job (oj.gi != NULL) its first
// workgroup also runs the pass for entries without a symmetric partner of a
// backward-input computed before it (flag-gated as in k_orphans,
// orphan_exact), which saves that pass a launch of its own.
template <typename T, int CP>
__global__ __launch_bounds__(256) void k_bw_reduce(const float* __restrict__ part,
                                                   const float* __restrict__ part_b, int splits,
                                                   int n_off, int c_in, int c_out, int fm, int fn, int wgm,
                                                   int wgn, int n_ci_tiles, int n_co_tiles,
                                                   T* __restrict__ gw, T* __restrict__ gb,
                                                   OrphanJob oj) {
    // workgroups [0, quad_blocks) reduce gw, the rest the bias
    const int64_t quad_blocks = bw_quad_blocks((int64_t)n_off * c_in * c_out / 4, splits);
    if ((int64_t)blockIdx.x < quad_blocks) {
        if (splits <= 2)  // uniform
            bw_reduce_quads_direct<T, CP>((int64_t)blockIdx.x * 256 + threadIdx.x, part, splits, n_off, c_in,
                                          c_out, fm, fn, wgm, wgn, n_ci_tiles, n_co_tiles, gw);
        else
            bw_reduce_quads<T, CP>(blockIdx.x, part, splits, n_off, c_in, c_out, fm, fn, wgm, wgn,
                                   n_ci_tiles, n_co_tiles, gw);
    } else if (gb)
        bw_reduce_bias<T>(((int64_t)blockIdx.x - quad_blocks) * 256 + threadIdx.x, part_b,
                          n_off == 9 ? CP * splits : splits, c_out, gb);
    if (!oj.gi || (oj.flag && *oj.flag == 0u) || blockIdx.x != 0) return;
    // the exact pass for entries without a symmetric partner: one workgroup
    orphan_exact<T, false, 256>((const T*)oj.go, oj.nbr, (const T*)oj.w, (T*)oj.gi, oj.n, oj.c_in, oj.c_out,
                                oj.tpb);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

static bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

bool gg_mfma_supported(int dtype, int c_red, int n_out) {
    return (dtype == SVTAD_F16 || dtype == SVTAD_BF16) && c_red % 8 == 0 && n_out % 8 == 0 &&
           c_red >= 16 && n_out >= 16;
}

// Reduction widths with a wide-kernel instantiation and its (FM, FN, D).
struct WideCfg { int cr, fm, fn, d; };
// A two-step weight ring measured faster than deeper ones (fewer registers),
// except at CR = 512, where a step's 1 KB weight fragments are used by only
// 4 row fragments: four steps there (config 5, 13117 rows: forward 76.1 ->
// 72.3 us, backward-input 71.9 -> 68.9 us; eight steps leave registers for
// one wave set only, 108 us).
static const WideCfg kWide[] = {{64, 8, 1, 2}, {128, 8, 2, 2}, {192, 8, 3, 2},
                                {256, 8, 4, 2}, {512, 4, 4, 4}};

static const WideCfg* wide_cfg(int c_red, int n_out) {
    for (const WideCfg& c : kWide)
        if (c.cr == c_red && n_out >= (4 * c.fn * 16) / 2) return &c;
    return nullptr;
}

size_t gg_mfma_workspace(int dtype, int c_red, int n_out) {
    if (!gg_mfma_supported(dtype, c_red, n_out) || !wide_cfg(c_red, n_out)) return 0;
    return (size_t)9 * c_red * cdiv(n_out, 16) * 16 * 2;
}

template <typename T, int MODE, int WGM, int WGN, int FM, int FN>
static void launch_gg(const void* src, const int32_t* nbr, const void* w, const void* bias,
                      int bias_mode, void* out, int64_t n, int c_red, int n_out, int64_t tpb,
                      hipStream_t s) {
    constexpr int BM = WGM * FM * 16, BN = WGN * FN * 16;
    const int n_col = (int)cdiv(n_out, BN);
    const int64_t tiles = cdiv(n, BM) * n_col;
    hipLaunchKernelGGL((k_gg_mfma<T, MODE, WGM, WGN, FM, FN>), dim3((unsigned)tiles),
                       dim3(WGM * WGN * 64), 0, s, (const T*)src, nbr, (const T*)w, bias,
                       bias_mode, (T*)out, n, c_red, n_out, tpb, n_col, tiles);
}

// Compute units of the current device (cached per device).
int cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int c = 0;
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
            c = 256;
        cached[dev] = c;
    }
    return cached[dev];
}

template <typename T, int MODE, int CR, int FM, int FN, int D>
static void launch_wide(const void* src, const int32_t* nbr, const void* wb, const void* bias,
                        int bias_mode, void* out, int64_t n, int n_out, int64_t tpb, uint32_t* flag,
                        bool sym, hipStream_t s) {
    constexpr int BN = 4 * FN * 16;
    // two wave sets (two waves per SIMD, at most 256 registers each) when
    // their LDS fits and the accumulators, weight ring and row fragments
    // leave room for the rest; else one set
    constexpr int WS = (size_t)gg_lds_rows(CR, FM, FN, 2) * CR * 2 <= 150 * 1024 &&
                               4 * (FM * FN + D * FN + FM + (MODE == MODE_FWD ? FN : 0)) <= 176
                           ? 2
                           : 1;
    const int n_col = (int)cdiv(n_out, BN);
    const int64_t tiles = cdiv(n, 16 * FM) * n_col;
    hipLaunchKernelGGL((k_gg_wide<T, MODE, CR, FM, FN, D, WS>), dim3((unsigned)tiles), dim3(256 * WS),
                       0, s, (const T*)src, nbr, (const T*)wb, bias, bias_mode, (T*)out, n, n_out,
                       tpb, n_col, tiles, flag, sym);
}

// Row fragments per workgroup. The kernels hold one workgroup per CU
// (registers), so the time is about (rounds of workgroups) x (one
// workgroup's time), and the latter grows with FM. The largest instantiated
// FM gives the fewest rounds; take the smallest FM that needs no more rounds
// than that. With one round this is the smallest FM whose grid fits the CUs;
// when none fits (C = 256 at 27k rows: 282 workgroups at FM 6, 423 at FM 4,
// two rounds either way) it evens the rounds out instead of leaving a second
// round of a few workgroups (measured 50.1 -> 39.8 us there).
static int pick_fm(int64_t n, int n_col, const int* have, int count) {
    const int64_t cu = cu_count();
    auto rounds = [&](int fm) { return cdiv(cdiv(n, 16 * fm) * n_col, cu); };
    const int64_t r_min = rounds(have[count - 1]);
    for (int q = 0; q < count; ++q)
        if (rounds(have[q]) <= r_min) return have[q];
    return have[count - 1];
}

template <typename T, int MODE, int CR, int FN, int D>
static void launch_wide_fm(const void* src, const int32_t* nbr, const void* wb, const void* bias,
                           int bias_mode, void* out, int64_t n, int n_out, int64_t tpb,
                           uint32_t* flag, bool sym, hipStream_t s) {
    const int n_col = (int)cdiv(n_out, 4 * FN * 16);
    if constexpr (CR == 192 || CR == 256) {
        // at CR = 256, FM = 8 leaves room for one wave set only (one wave per
        // SIMD); FM = 6 with two sets is faster even with a partial second
        // round of workgroups
        static const int have[] = {1, 2, 3, 4, 5, 6, 8};
        const int fm = pick_fm(n, n_col, have, CR == 256 ? 6 : 7);
        if constexpr (CR == 192 && FN == 3) {
            // Few rows (one or two row fragments per full-width tile): 64-column
            // tiles of three row fragments instead. Each workgroup then streams
            // a third of the weight and the grid holds about as many tiles
            // (measured 10.8 -> 8.2 us at 3136 rows, 14.4 -> 11.5 us at 7840).
            // The weight ring holds a whole slice (six steps, 24 registers
            // with one column fragment): in a training step the packed weight
            // is new, not yet in the XCD's L2, and two steps of lookahead left
            // its fetches exposed (c2 step at 10 % keep 29.0 -> 27.5 us; the
            // forward timed alone on a weight already in L2 does not change).
            if (fm <= 2) {
                launch_wide<T, MODE, CR, 3, 1, 6>(src, nbr, wb, bias, bias_mode, out, n, n_out, tpb, flag, sym, s);
                return;
            }
        }
        if constexpr (CR == 256 && FN == 4) {
            // the same at C = 256: 128-column tiles of three row fragments
            // (measured 14.4 -> 11.7 us at 4916 rows), with a four-step weight
            // ring for the packed weight fresh from the pack (config 4 step at
            // 10 % keep 43.2 -> 40.9 us)
            if (fm <= 2) {
                launch_wide<T, MODE, CR, 3, 2, 4>(src, nbr, wb, bias, bias_mode, out, n, n_out, tpb, flag, sym, s);
                return;
            }
        }
        switch (fm) {
            case 1: launch_wide<T, MODE, CR, 1, FN, D>(src, nbr, wb, bias, bias_mode, out, n, n_out, tpb, flag, sym, s); return;
            case 2: launch_wide<T, MODE, CR, 2, FN, D>(src, nbr, wb, bias, bias_mode, out, n, n_out, tpb, flag, sym, s); return;
            case 3: launch_wide<T, MODE, CR, 3, FN, D>(src, nbr, wb, bias, bias_mode, out, n, n_out, tpb, flag, sym, s); return;
            case 4: launch_wide<T, MODE, CR, 4, FN, D>(src, nbr, wb, bias, bias_mode, out, n, n_out, tpb, flag, sym, s); return;
            case 5: launch_wide<T, MODE, CR, 5, FN, D>(src, nbr, wb, bias, bias_mode, out, n, n_out, tpb, flag, sym, s); return;
            case 6: launch_wide<T, MODE, CR, 6, FN, D>(src, nbr, wb, bias, bias_mode, out, n, n_out, tpb, flag, sym, s); return;
            default: launch_wide<T, MODE, CR, 8, FN, D>(src, nbr, wb, bias, bias_mode, out, n, n_out, tpb, flag, sym, s); return;
        }
    } else {
        static const int have[] = {2, 4};
        if (pick_fm(n, n_col, have, 2) == 2)
            launch_wide<T, MODE, CR, 2, FN, D>(src, nbr, wb, bias, bias_mode, out, n, n_out, tpb, flag, sym, s);
        else
            launch_wide<T, MODE, CR, 4, FN, D>(src, nbr, wb, bias, bias_mode, out, n, n_out, tpb, flag, sym, s);
    }
}

// Returns whether the orphan flag is maintained (the wide kernel ran with it).
template <typename T, int MODE>
static bool gg_dispatch(const void* src, const int32_t* nbr, const void* w, const void* bias,
                        int bias_mode, void* out, int64_t n, int c_red, int n_out, int64_t tpb,
                        void* ws, bool prepacked, uint32_t* flag, bool sym, hipStream_t s) {
    const WideCfg* wc = wide_cfg(c_red, n_out);
    // buffer loads address operands with 32-bit byte offsets
    const bool fits = n * c_red * 2 < (int64_t)INT32_MAX && 9LL * c_red * n_out * 2 < (int64_t)INT32_MAX;
    if (MODE == MODE_FWD) flag = nullptr;
    if (wc && fits && (ws || prepacked)) {
        const void* wb = prepacked ? w : ws;
        if (!prepacked) {
            const int64_t slots = (int64_t)9 * (c_red / KS) * cdiv(n_out, 16) * 64;
            hipLaunchKernelGGL((k_pack_frag<MODE>), dim3((unsigned)cdiv(slots, 256)), dim3(256), 0, s,
                               (const u16*)w, (u16*)ws, c_red, n_out, flag);
        }
#define SVTAD_WIDE_CASE(CR, FM, FN, D)                                                           \
    if (wc->cr == CR) {                                                                          \
        launch_wide_fm<T, MODE, CR, FN, D>(src, nbr, wb, bias, bias_mode, out, n, n_out, tpb, flag, sym, s); \
        return flag != nullptr;                                                                  \
    }
        SVTAD_WIDE_CASE(64, 8, 1, 2)
        SVTAD_WIDE_CASE(128, 8, 2, 2)
        SVTAD_WIDE_CASE(192, 8, 3, 2)
        SVTAD_WIDE_CASE(256, 8, 4, 2)
        SVTAD_WIDE_CASE(512, 4, 4, 4)
#undef SVTAD_WIDE_CASE
    }
    if (n_out % 96 == 0)
        launch_gg<T, MODE, 2, 2, 2, 3>(src, nbr, w, bias, bias_mode, out, n, c_red, n_out, tpb, s);
    else if (n_out % 64 == 0)
        launch_gg<T, MODE, 2, 2, 2, 2>(src, nbr, w, bias, bias_mode, out, n, c_red, n_out, tpb, s);
    else if (n_out % 48 == 0)
        launch_gg<T, MODE, 4, 1, 1, 3>(src, nbr, w, bias, bias_mode, out, n, c_red, n_out, tpb, s);
    else
        launch_gg<T, MODE, 4, 1, 1, 1>(src, nbr, w, bias, bias_mode, out, n, c_red, n_out, tpb, s);
    return false;
}

bool gg_mfma(int dtype, int mode, const void* src, const int32_t* nbr, const void* w,
             const void* bias, int bias_mode, void* out, int64_t n, int c_red, int n_out,
             int64_t tpb, void* ws, bool prepacked, uint32_t* orphan_flag, hipStream_t s, bool sym) {
    if (dtype == SVTAD_F16) {
        if (mode == MODE_FWD) return gg_dispatch<f16, MODE_FWD>(src, nbr, w, bias, bias_mode, out, n, c_red, n_out, tpb, ws, prepacked, nullptr, false, s);
        return gg_dispatch<f16, MODE_BWDIN>(src, nbr, w, nullptr, 0, out, n, c_red, n_out, tpb, ws, prepacked, orphan_flag, sym, s);
    }
    if (mode == MODE_FWD) return gg_dispatch<bf16, MODE_FWD>(src, nbr, w, bias, bias_mode, out, n, c_red, n_out, tpb, ws, prepacked, nullptr, false, s);
    return gg_dispatch<bf16, MODE_BWDIN>(src, nbr, w, nullptr, 0, out, n, c_red, n_out, tpb, ws, prepacked, orphan_flag, sym, s);
}

bool gg_mfma_packed_ok(int dtype, int64_t n, int c_red, int n_out) {
    return gg_mfma_workspace(dtype, c_red, n_out) > 0 && n * c_red * 2 < (int64_t)INT32_MAX &&
           9LL * c_red * n_out * 2 < (int64_t)INT32_MAX;
}

void pack_weight(const void* w, void* wf_fwd, void* wf_bwd, int c_in, int c_out, hipStream_t s) {
    const int64_t sf = wf_fwd ? (int64_t)9 * (c_in / KS) * cdiv(c_out, 16) * 64 : 0;
    const int64_t sb = wf_bwd ? (int64_t)9 * (c_out / KS) * cdiv(c_in, 16) * 64 : 0;
    if (sf + sb == 0) return;
    hipLaunchKernelGGL(k_pack_both, dim3((unsigned)cdiv(sf + sb, 256)), dim3(256), 0, s, (const u16*)w,
                       (u16*)wf_fwd, (u16*)wf_bwd, c_in, c_out, sf, sb);
}

bool bw_mfma_supported(int dtype, int64_t n, int c_in, int c_out) {
    // buffer loads address x and go with 32-bit byte offsets
    return (dtype == SVTAD_F16 || dtype == SVTAD_BF16) && c_in % 8 == 0 && c_out % 8 == 0 &&
           c_in >= 16 && c_out >= 16 && n * std::max(c_in, c_out) * 2 < (int64_t)INT32_MAX;
}

// Tile edge for a bwd-weight dimension: 96 when it divides, else 64, else 32.
int bw_mfma_tile(int c) { return c % 96 == 0 ? 96 : (c % 64 == 0 ? 64 : 32); }

// Host checks of a row-split plan against what the backward-weight partial
// kernels assume before any launch: splits of whole pairs of 64-row stages,
// each within the split's LDS row list (kMaxSplitRows), every row in some
// split, and a workspace that holds every workgroup's partial tile (part_bytes).
static int check_split_plan(const char* who, const BwPlan& p, int64_t n, size_t part_bytes,
                            size_t ws_bytes) {
    static thread_local char buf[256];
    if (p.splits < 1 || p.rows_per_split <= 0 || p.rows_per_split % (2 * KR) != 0 ||
        p.rows_per_split > kMaxSplitRows || (int64_t)p.splits * p.rows_per_split < n) {
        snprintf(buf, sizeof(buf), "%s: bad row-split plan (splits=%d rows_per_split=%lld n=%lld)", who,
                 p.splits, (long long)p.rows_per_split, (long long)n);
        return set_error(SVTAD_ERR_INVALID, buf);
    }
    if (part_bytes > ws_bytes) {
        snprintf(buf, sizeof(buf), "%s: %zu partial bytes exceed the %zu-byte workspace", who, part_bytes,
                 ws_bytes);
        return set_error(SVTAD_ERR_WORKSPACE, buf);
    }
    return SVTAD_OK;
}

template <typename T, int FM, int FN>
static int launch_bw(const BwPlan& p, const void* go, const void* x, const int32_t* nbr,
                     float* part, float* part_b, int64_t n, int c_in, int c_out, int64_t tpb,
                     size_t ws_bytes, hipStream_t s) {
    constexpr int BM = 2 * FM * 16, BN = 2 * FN * 16;
    const int nci = (int)cdiv(c_in, BM), nco = (int)cdiv(c_out, BN);
    const int64_t blocks = (int64_t)9 * nci * nco * p.splits;
    // ws[s][k][ci][co] for ci < c_in, co < c_out, then the bias partials
    const size_t need = (size_t)p.splits * 9 * c_in * c_out * 4 + (part_b ? (size_t)p.splits * c_out * 4 : 0);
    const int st = check_split_plan("bwd_w", p, n, need, ws_bytes);
    if (st) return st;
    hipLaunchKernelGGL((k_bw_mfma<T, FM, FN>), dim3((unsigned)blocks), dim3(256), 0, s,
                       (const T*)go, (const T*)x, nbr, part, part_b, n, c_in, c_out, tpb,
                       p.rows_per_split, nci, nco, blocks);
    return SVTAD_OK;
}

// Large-tile backward-weight configurations: WGM x WGN waves, each with
// FM x FN fragments, so (ci tile, co tile) = (16*WGM*FM, 16*WGN*FN). Eight
// waves put two on every SIMD (one wave alone cannot keep the matrix core
// busy).
struct BigCfg { int fm, fn, wgm, wgn; };
static bool big_cfg(int c_in, int c_out, BigCfg* out) {
    static const BigCfg cands[] = {{6, 3, 2, 4}, {4, 4, 2, 4}, {4, 2, 2, 4}, {3, 3, 2, 2}, {2, 2, 2, 2}};
    for (const BigCfg& c : cands) {
        const int bm = 16 * c.wgm * c.fm, bn = 16 * c.wgn * c.fn;
        if (c_in % bm == 0 && c_out % bn == 0) {
            *out = c;
            return true;
        }
    }
    return false;
}

bool bw_mfma_tiles(int c_in, int c_out, int* tm, int* tn) {
    BigCfg c;
    if (big_cfg(c_in, c_out, &c)) {
        *tm = 16 * c.wgm * c.fm;
        *tn = 16 * c.wgn * c.fn;
        return true;
    }
    *tm = bw_mfma_tile(c_in);
    *tn = bw_mfma_tile(c_out);
    return false;
}

template <typename T, int FM, int FN, int WGM, int WGN>
static int launch_big(const BwPlan& p, const void* go, const void* x, const int32_t* nbr,
                      float* part, float* part_b, int64_t n, int c_in, int c_out, int64_t tpb,
                      size_t ws_bytes, hipStream_t s) {
    constexpr int BM = WGM * FM * 16, BN = WGN * FN * 16;
    if (c_in % BM != 0 || c_out % BN != 0) return set_error(SVTAD_ERR_INVALID, "bwd_w: widths are not whole tiles");
    const int nci = c_in / BM, nco = c_out / BN;
    const int64_t blocks = (int64_t)10 * nci * nco * p.splits;
    // one BM x BN tile per workgroup (splits x 10 work units x nci x nco of
    // them), then the bias partials (two per split: the center's halves)
    const size_t need = (size_t)blocks * BM * BN * 4 + (part_b ? (size_t)2 * p.splits * c_out * 4 : 0);
    int st = check_split_plan("bwd_w", p, n, need, ws_bytes);
    if (st) return st;
    if (p.rows_per_split % (4 * KR) != 0)  // the center's halves are whole pairs of stages
        return set_error(SVTAD_ERR_INVALID, "bwd_w: rows_per_split is not a multiple of 256");
    hipLaunchKernelGGL((k_bw_big<T, FM, FN, WGM, WGN>), dim3((unsigned)blocks),
                       dim3(bw_big_threads(FM, FN, WGM, WGN)),
                       0, s, (const T*)go, (const T*)x, nbr, part, part_b, n, c_in, c_out, tpb,
                       p.rows_per_split, nci, nco, blocks, 9, n);
    return SVTAD_OK;
}

template <typename T>
static int bw_dispatch(const BwPlan& p, const void* go, const void* x, const int32_t* nbr,
                       float* part, float* part_b, int64_t n, int c_in, int c_out, int64_t tpb,
                       size_t ws_bytes, hipStream_t s) {
    BigCfg bc;
    if (big_cfg(c_in, c_out, &bc)) {
#define SVTAD_BIG_CASE(M, N, WM, WN)                                                                   \
    if (bc.fm == M && bc.fn == N && bc.wgm == WM && bc.wgn == WN)                                      \
        return launch_big<T, M, N, WM, WN>(p, go, x, nbr, part, part_b, n, c_in, c_out, tpb, ws_bytes, s);
        SVTAD_BIG_CASE(6, 3, 2, 4)
        SVTAD_BIG_CASE(4, 4, 2, 4)
        SVTAD_BIG_CASE(4, 2, 2, 4)
        SVTAD_BIG_CASE(3, 3, 2, 2)
        SVTAD_BIG_CASE(2, 2, 2, 2)
#undef SVTAD_BIG_CASE
    }
    const int tm = bw_mfma_tile(c_in), tn = bw_mfma_tile(c_out);
#define SVTAD_BW_CASE(M, N)                                                                              \
    if (tm == M && tn == N)                                                                              \
        return launch_bw<T, M / 32, N / 32>(p, go, x, nbr, part, part_b, n, c_in, c_out, tpb, ws_bytes, s);
    SVTAD_BW_CASE(96, 96)
    SVTAD_BW_CASE(96, 64)
    SVTAD_BW_CASE(64, 96)
    SVTAD_BW_CASE(64, 64)
    SVTAD_BW_CASE(96, 32)
    SVTAD_BW_CASE(32, 96)
    SVTAD_BW_CASE(64, 32)
    SVTAD_BW_CASE(32, 64)
    SVTAD_BW_CASE(32, 32)
#undef SVTAD_BW_CASE
    return set_error(SVTAD_ERR_UNSUPPORTED, "bwd_w: no tile configuration for these widths");
}

// Ordered reduction of the large-tile partials into gw / gb (k_bw_reduce),
// which also runs the orphan job oj (may be NULL); cparts is the units'
// center split.
static void bw_big_reduce(int dtype, const BigCfg& bc, int splits, const float* part, const float* part_b,
                          void* gw, void* gb, int c_in, int c_out, const OrphanJob* oj, int cparts, hipStream_t s) {
    const int nci = c_in / (16 * bc.wgm * bc.fm), nco = c_out / (16 * bc.wgn * bc.fn);
    const int64_t blocks = bw_quad_blocks((int64_t)9 * c_in * c_out / 4, splits) + (gb ? cdiv(c_out, 256) : 0);
    const dim3 grid((unsigned)blocks);
    const OrphanJob job = oj ? *oj : OrphanJob{nullptr, nullptr, nullptr, nullptr, 0, 0, 0, 0, nullptr};
#define SVTAD_REDUCE(T, CP)                                                                                  \
    hipLaunchKernelGGL((k_bw_reduce<T, CP>), grid, dim3(256), 0, s, part, gb ? part_b : nullptr, splits, 9, c_in, \
                       c_out, bc.fm, bc.fn, bc.wgm, bc.wgn, nci, nco, (T*)gw, (T*)gb, job)
    if (dtype == SVTAD_F16) {
        if (cparts == 4) SVTAD_REDUCE(f16, 4);
        else SVTAD_REDUCE(f16, 2);
    } else {
        if (cparts == 4) SVTAD_REDUCE(bf16, 4);
        else SVTAD_REDUCE(bf16, 2);
    }
#undef SVTAD_REDUCE
}

int bw_mfma(int dtype, const BwPlan& p, const void* go, const void* x, const int32_t* nbr,
            void* gw, void* gb, void* ws, size_t ws_bytes, int64_t n, int c_in, int c_out, int64_t tpb,
            const OrphanJob* oj, bool* oj_taken, hipStream_t s) {
    *oj_taken = false;
    float* part = (float*)ws;
    BigCfg bc0;
    // the large-tile kernel keeps 10 work units per split (the center offset in two halves)
    const int units = big_cfg(c_in, c_out, &bc0) ? 10 : 9;
    float* part_b = gb ? part + (int64_t)p.splits * units * c_in * c_out : nullptr;
    const int st = dtype == SVTAD_F16
                       ? bw_dispatch<f16>(p, go, x, nbr, part, part_b, n, c_in, c_out, tpb, ws_bytes, s)
                       : bw_dispatch<bf16>(p, go, x, nbr, part, part_b, n, c_in, c_out, tpb, ws_bytes, s);
    if (st) return st;
    if (!gw) return SVTAD_OK;  // partials only
    BigCfg bc;
    if (big_cfg(c_in, c_out, &bc)) {
        bw_big_reduce(dtype, bc, p.splits, part, part_b, gw, gb, c_in, c_out, oj, 2, s);
        *oj_taken = oj != nullptr;
        return SVTAD_OK;
    }
    split_reduce(dtype, part, 9LL * c_in * c_out, p.splits, gw, s);
    if (gb) split_reduce(dtype, part_b, (int64_t)c_out, p.splits, gb, s);
    return SVTAD_OK;
}

// The fused backward's choice: the backward-input tile shape (row fragments
// gfm, column fragments per wave gfn) and the backward-weight split count.
// SVTAD_BWD_FUSED in the environment overrides it: "off" never fuses,
// "<gfm>x<gfn>" or "<gfm>x<gfn>:<splits>" forces a shape (one of 3x1, 3x3,
// 4x3) for measurements; the launch checks still apply.
struct FusedChoice { int gfm, gfn, splits; };
// -1 off, 0 automatic, 1 forced, -2 unreadable (read on every call)
static int fused_env(FusedChoice* c) {
    const char* e = getenv("SVTAD_BWD_FUSED");
    if (!e || !*e) return 0;
    if (!strcmp(e, "off")) return -1;
    FusedChoice f{0, 0, 0};
    if (sscanf(e, "%dx%d:%d", &f.gfm, &f.gfn, &f.splits) < 2) return -2;
    *c = f;
    return 1;
}

// Center-offset units per split of the one-launch backward (two in the
// separate backward-weight launch). Its grid must fit one round, so it runs
// few, long splits, and at low keep the off-center units visit few rows:
// the center's halves were a split's longest units (config 4 at 10 % keep,
// 2 splits of 2560 rows: 20 stages against about 4). Four parts: config 4
// at 10 % keep 49.1 -> 40.8 us per step, c2 at 10 / 25 / 40 % keep 26.6 ->
// 26.1, 34.0 -> 34.2, 49.7 -> 47.6 us.
constexpr int kFusedCenterParts = 4;

// C_in = C_out = C: backward-input tiles of GFM row fragments and GFN column
// fragments per wave, backward-weight units on the large-tile configuration
// (BFM, BFN, BWM, BWN) of that width.
template <typename T, int C, int GFM, int GFN, int BFM, int BFN, int BWM, int BWN>
static void launch_fused(const void* go, const int32_t* nbr, const void* wb, void* gi, uint32_t* flag,
                         const void* x, float* part, float* part_b, int64_t n, int64_t tpb, int64_t rps,
                         int64_t n_gg, int64_t n_bw, bool sym, hipStream_t s) {
    constexpr int NCI = C / (16 * BWM * BFM), NCO = C / (16 * BWN * BFN);
    static_assert(NCI * 16 * BWM * BFM == C && NCO * 16 * BWN * BFN == C, "whole tiles");
    hipLaunchKernelGGL((k_bwd_fused<T, C, GFM, GFN, 2, 2, BFM, BFN, BWM, BWN, kFusedCenterParts>),
                       dim3((unsigned)(n_gg + n_bw)), dim3(bw_big_threads(BFM, BFN, BWM, BWN)), 0, s, (const T*)go, nbr, (const T*)wb, (T*)gi, C,
                       C / (64 * GFN), flag, (const T*)x, part, part_b, n, tpb, rps, NCI, NCO, n_bw, n_gg + n_bw, sym);
}

// Workgroups per split of the one-launch backward's large-tile configuration
// at width c (8 + kFusedCenterParts work units per ci x co tile): c = 192
// takes one 192 x 192 tile, c = 256 two 128 x 256 tiles.
static int fused_units(int c) { return (8 + kFusedCenterParts) * (c == 192 ? 1 : (c == 256 ? 2 : 0)); }
// Workspace bytes of the one-launch backward's partials for `splits` splits:
// a c_in x c_out fp32 tile per work unit, then one bias row per center unit.
static size_t fused_ws_bytes(int64_t splits, int c_in, int c_out) {
    constexpr int p = kFusedCenterParts;
    return (size_t)splits * ((size_t)(8 + p) * c_in * c_out + (size_t)p * c_out) * 4;
}

int bwd_fused_plan(int dtype, const BwPlan& p0, int64_t n, int c_in, int c_out, int* gfm, int* gfn,
                   BwPlan* p_out) {
    const int C = c_in, U = fused_units(C);
    if ((dtype != SVTAD_F16 && dtype != SVTAD_BF16) || c_in != c_out || U == 0 || n <= 0 || p0.path != 1 ||
        !gg_mfma_packed_ok(dtype, n, c_out, c_in) || !bw_mfma_supported(dtype, n, c_in, c_out))
        return 0;
    FusedChoice ch{0, 0, p0.splits};
    const int env = fused_env(&ch);
    if (env == -2)
        return set_error(SVTAD_ERR_INVALID, "bwd_packed: SVTAD_BWD_FUSED is neither off nor <rows>x<cols>[:<splits>]");
    if (env < 0) return 0;
    const int64_t cu = cu_count();
    auto n_gg = [&](int fm, int fn) { return cdiv(n, 16 * fm) * (C / (64 * fn)); };
    // the most splits whose partials fit the workspace plan_bw sized (p0)
    int64_t fit = p0.splits;
    while (fit > 0 && fused_ws_bytes(fit, c_in, c_out) > p0.ws_bytes) --fit;
    if (env == 0) {
        // C = 192: the tile shape the backward-input launch would take
        // (pick_fm), or a full-width tile of three row fragments in place of
        // the 64-column one; only shapes whose registers fit 128 per wave
        // (FM <= 4). C = 256: the 128-column tiles of three row fragments
        // that the backward-input launch takes for few rows (its full-width
        // tiles need more registers).
        static const int have[] = {1, 2, 3, 4, 5, 6, 8};
        const int fm = pick_fm(n, 1, have, C == 256 ? 6 : 7);
        static const FusedChoice narrow[] = {{3, 1, 0}, {3, 3, 0}};
        static const FusedChoice narrow256[] = {{3, 2, 0}};
        FusedChoice wide{fm, 3, 0};
        const FusedChoice* cands = C == 256 ? narrow256 : (fm <= 2 ? narrow : &wide);
        const int nc = C == 256 ? (fm <= 2 ? 1 : 0) : (fm <= 2 ? 2 : (fm <= 4 ? 1 : 0));
        // The split count drops below the plan's so that the grid fits, while
        // splits stay within 2560 rows: the tile role takes as long as the
        // longer splits, and fewer partials shorten the reduction.
        // Measured (step medians, the center offset then in two units per
        // split, so the workspace held the plan's count): c2 10 % keep 41.0
        // us two-launch, 36.8 fused with full-width tiles and 7 splits, 32.5
        // with 64-column tiles and 5; c2 40 % keep 62.3 two-launch, 53.4
        // fused with 6 splits (55.1 with 5, 61.1 with 4); c4 10 % keep
        // (C = 256) 55.4 two-launch, 49.9 fused with 2 splits (50.2 with 3,
        // 50.4 with 4, 52.4 with the plan's 5 over more than one round). A
        // grid over one round at c2 55 % was slower.
        bool found = false;
        for (int q = 0; q < nc && !found; ++q) {
            const int64_t room = (cu - n_gg(cands[q].gfm, cands[q].gfn)) / U;
            const int64_t sp = std::min<int64_t>(fit, room);
            if (sp >= 1 && sp * 2560 >= n) {
                ch = FusedChoice{cands[q].gfm, cands[q].gfn, (int)sp};
                found = true;
            }
        }
        if (!found) return 0;
    } else {
        // a forced split count is clamped to what the launch accepts: at most
        // the count whose partials the workspace holds, and enough splits
        // that none exceeds the LDS row list (kMaxSplitRows)
        const int64_t lo = cdiv(n, (int64_t)kMaxSplitRows);
        if (lo > fit)
            return set_error(SVTAD_ERR_INVALID, "bwd_packed: SVTAD_BWD_FUSED has no split count the workspace holds");
        if (ch.splits <= 0) ch.splits = (int)fit;
        ch.splits = (int)std::min<int64_t>(std::max<int64_t>(ch.splits, lo), fit);
        const bool ok192 = C == 192 && ((ch.gfm == 3 && ch.gfn == 1) || (ch.gfm == 3 && ch.gfn == 3) ||
                                        (ch.gfm == 4 && ch.gfn == 3));
        const bool ok256 = C == 256 && ch.gfm == 3 && ch.gfn == 2;
        if (!ok192 && !ok256)
            return set_error(SVTAD_ERR_INVALID,
                             "bwd_packed: SVTAD_BWD_FUSED shape is not 3x1, 3x3 or 4x3 (C = 192) or 3x2 (C = 256)");
    }
    // the split plan for ch.splits: whole 256-row units
    BwPlan p = p0;
    p.rows_per_split = cdiv(cdiv(n, (int64_t)ch.splits), 256) * 256;
    p.splits = (int)cdiv(n, p.rows_per_split);
    *gfm = ch.gfm;
    *gfn = ch.gfn;
    *p_out = p;
    return 1;
}

int bwd_fused_mfma(int dtype, const BwPlan& p0, const void* go, const void* x, const int32_t* nbr,
                   const void* w, const void* packed_bwd, uint32_t* flag, void* gi, void* gw, void* gb,
                   void* ws, size_t ws_bytes, int64_t n, int c_in, int c_out, int64_t tpb, hipStream_t s,
                   bool sym) {
    if (!aligned16(go) || !aligned16(x) || !aligned16(packed_bwd) || !aligned16(gi)) return 0;
    FusedChoice ch{0, 0, 0};
    BwPlan p;
    const int fp = bwd_fused_plan(dtype, p0, n, c_in, c_out, &ch.gfm, &ch.gfn, &p);
    if (fp != 1) return fp;
    const int st = check_split_plan("bwd_packed", p, n, fused_ws_bytes(p.splits, c_in, c_out), ws_bytes);
    if (st) return st;
    auto n_gg = [&](int fm, int fn) { return cdiv(n, 16 * fm) * (c_in / (64 * fn)); };
    float* part = (float*)ws;
    float* part_b = gb ? part + (int64_t)p.splits * (8 + kFusedCenterParts) * c_in * c_out : nullptr;
    const int64_t gg = n_gg(ch.gfm, ch.gfn), bw = (int64_t)fused_units(c_in) * p.splits;
    bool launched = false;
#define SVTAD_FUSED_CASE(C, FM, FN, BFM, BFN, BWM, BWN)                                                   \
    if (c_in == C && ch.gfm == FM && ch.gfn == FN) {                                                      \
        launched = true;                                                                                  \
        if (dtype == SVTAD_F16)                                                                           \
            launch_fused<f16, C, FM, FN, BFM, BFN, BWM, BWN>(go, nbr, packed_bwd, gi, flag, x, part,     \
                                                             part_b, n, tpb, p.rows_per_split, gg, bw, sym, s); \
        else                                                                                              \
            launch_fused<bf16, C, FM, FN, BFM, BFN, BWM, BWN>(go, nbr, packed_bwd, gi, flag, x, part,    \
                                                              part_b, n, tpb, p.rows_per_split, gg, bw, sym, s); \
    }
    SVTAD_FUSED_CASE(192, 3, 1, 6, 3, 2, 4)
    SVTAD_FUSED_CASE(192, 3, 3, 6, 3, 2, 4)
    SVTAD_FUSED_CASE(192, 4, 3, 6, 3, 2, 4)
    SVTAD_FUSED_CASE(256, 3, 2, 4, 4, 2, 4)
#undef SVTAD_FUSED_CASE
    // a plan without an instantiation leaves the partials unwritten: no
    // reduction of them, the caller runs the two launches instead
    if (!launched) return 0;
    const OrphanJob job{go, nbr, w, gi, n, c_in, c_out, tpb, flag};
    BigCfg bc;
    big_cfg(c_in, c_out, &bc);  // the configuration launch_fused used (6,3,2,4 / 4,4,2,4)
    bw_big_reduce(dtype, bc, p.splits, part, part_b, gw, gb, c_in, c_out, &job, kFusedCenterParts, s);
    return 1;
}

// Row-split plan of a linear layer's weight gradient (one offset): splits
// of whole 128-row pairs of stages, enough workgroups for every CU, at most
// kMaxSplitRows - 128 rows each.
BwPlan plan_wgrad(int64_t n, int c_in, int c_out) {
    BwPlan p;
    BigCfg c;
    p.path = big_cfg(c_in, c_out, &c) ? 1 : 0;
    const int64_t tiles = p.path ? (int64_t)(c_in / (16 * c.wgm * c.fm)) * (c_out / (16 * c.wgn * c.fn)) : 1;
    int64_t splits = std::max<int64_t>(cdiv(std::max<int64_t>(n, 1), kMaxSplitRows - 128),
                                       std::min<int64_t>(std::max<int64_t>(1, cu_count() / tiles),
                                                         cdiv(std::max<int64_t>(n, 1), 256)));
    int64_t rps = cdiv(cdiv(std::max<int64_t>(n, 1), splits), 128) * 128;
    splits = std::max<int64_t>(1, cdiv(n, rps));
    p.splits = (int)splits;
    p.rows_per_split = rps;
    p.ws_bytes = (size_t)splits * c_in * c_out * sizeof(float);
    return p;
}

template <typename T, int FM, int FN, int WGM, int WGN>
static int launch_wgrad(const BwPlan& p, const void* g, const int32_t* rows, const void* x, void* out,
                        float* part, size_t ws_bytes, int64_t n, int64_t n_src, int c_in, int c_out,
                        bool out_f32, hipStream_t s) {
    constexpr int BM = WGM * FM * 16, BN = WGN * FN * 16;
    if (c_in % BM != 0 || c_out % BN != 0)
        return set_error(SVTAD_ERR_INVALID, "linear_wgrad: widths are not whole tiles");
    const int nci = c_in / BM, nco = c_out / BN;
    const int64_t blocks = (int64_t)nci * nco * p.splits;
    const int st = check_split_plan("linear_wgrad", p, n, (size_t)blocks * BM * BN * 4, ws_bytes);
    if (st) return st;
    // the kernel's "x" (gathered, ci) is g and its "go" (linear, co) is x
    hipLaunchKernelGGL((k_bw_big<T, FM, FN, WGM, WGN>), dim3((unsigned)blocks),
                       dim3(bw_big_threads(FM, FN, WGM, WGN)), 0, s, (const T*)x, (const T*)g, rows,
                       part, (float*)nullptr, n, c_in, c_out, (int64_t)0, p.rows_per_split, nci, nco,
                       blocks, 1, n_src);
    const dim3 grid((unsigned)bw_quad_blocks((int64_t)c_in * c_out / 4, p.splits));
    const OrphanJob none{nullptr, nullptr, nullptr, nullptr, 0, 0, 0, 0, nullptr};
    if (out_f32)
        hipLaunchKernelGGL((k_bw_reduce<float, 2>), grid, dim3(256), 0, s, (const float*)part, (const float*)nullptr,
                           p.splits, 1, c_in, c_out, FM, FN, WGM, WGN, nci, nco, (float*)out, (float*)nullptr, none);
    else
        hipLaunchKernelGGL((k_bw_reduce<T, 2>), grid, dim3(256), 0, s, (const float*)part, (const float*)nullptr,
                           p.splits, 1, c_in, c_out, FM, FN, WGM, WGN, nci, nco, (T*)out, (T*)nullptr, none);
    return SVTAD_OK;
}

int wgrad_mfma(int dtype, const BwPlan& p, const void* g, const int32_t* rows, const void* x, void* out,
               void* ws, size_t ws_bytes, int64_t n, int64_t n_src, int c_in, int c_out, bool out_f32,
               hipStream_t s) {
    BigCfg bc;
    if (!p.path || !big_cfg(c_in, c_out, &bc))
        return set_error(SVTAD_ERR_UNSUPPORTED, "linear_wgrad: no tile configuration for these widths");
#define SVTAD_WG_CASE(M, N, WM, WN)                                                                           \
    if (bc.fm == M && bc.fn == N && bc.wgm == WM && bc.wgn == WN)                                             \
        return dtype == SVTAD_F16                                                                             \
                   ? launch_wgrad<f16, M, N, WM, WN>(p, g, rows, x, out, (float*)ws, ws_bytes, n, n_src, c_in, c_out, out_f32, s) \
                   : launch_wgrad<bf16, M, N, WM, WN>(p, g, rows, x, out, (float*)ws, ws_bytes, n, n_src, c_in, c_out, out_f32, s);
    SVTAD_WG_CASE(6, 3, 2, 4)
    SVTAD_WG_CASE(4, 4, 2, 4)
    SVTAD_WG_CASE(4, 2, 2, 4)
    SVTAD_WG_CASE(3, 3, 2, 2)
    SVTAD_WG_CASE(2, 2, 2, 2)
#undef SVTAD_WG_CASE
    return set_error(SVTAD_ERR_UNSUPPORTED, "linear_wgrad: no tile configuration for these widths");
}

}  // namespace svtad
