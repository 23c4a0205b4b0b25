// VALU (CUDA-core style) SparseConv2D kernels for every dtype. They carry the
// fp32/fp64 paths, the depthwise variant, the orphan pass of bwd_in and the
// row-split reduction of bwd_w; fp16/bf16 full convolutions normally take
// the MFMA kernels in conv_mfma.hip instead.
#include "sv_common.h"
#include "sv_conv.h"
#include "sv_internal.h"
#include "sv_mfma.h"

namespace svtad {

// ---------------------------------------------------------------------------
// Gathered GEMM: out[m, nn] = sum_k sum_c src[row(m,k), c] * B(k, c, nn)
//   MODE_FWD  : row = src(m,k),   B(k,c,nn) = w[k][c][nn]  (c over c_in)
//   MODE_BWDIN: row = src_t(m,k), B(k,c,nn) = w[k][nn][c]  (c over c_out)
// Tile 64 x 64, 256 threads, 4 x 4 outputs per thread, K step 16.
// ---------------------------------------------------------------------------
template <typename T, int MODE>
__global__ __launch_bounds__(256) void k_gg_valu(const T* __restrict__ src,
                                                 const int32_t* __restrict__ nbr,
                                                 const T* __restrict__ w,
                                                 const void* __restrict__ bias, int bias_mode,
                                                 T* __restrict__ out, int64_t n, int c_red,
                                                 int n_out, int64_t tpb) {
    typedef typename Acc<T>::type A;
    __shared__ int32_t sidx[9][64];
    __shared__ int any_k[9];
    __shared__ A As[16][64 + 4];
    __shared__ A Bs[16][64 + 4];
    const int tid = threadIdx.x;
    const int64_t row0 = (int64_t)blockIdx.x * 64;
    const int col0 = blockIdx.y * 64;
    if (tid < 9) any_k[tid] = 0;
    __syncthreads();
    for (int e = tid; e < 9 * 64; e += 256) {
        const int k = e >> 6, m = e & 63;
        const int64_t i = row0 + m;
        int64_t r = -1;
        if (i < n) r = MODE == MODE_FWD ? src_row(nbr, i, k, n, tpb) : src_row_t(nbr, i, k, n, tpb);
        sidx[k][m] = (int32_t)r;
        if (r >= 0) any_k[k] = 1;
    }
    __syncthreads();
    const int ty = tid >> 4, tx = tid & 15;
    A acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = 0;
    for (int k = 0; k < 9; ++k) {
        if (!any_k[k]) continue;  // uniform across the workgroup
        const T* wk = w + (int64_t)k * c_red * n_out;
        for (int c0 = 0; c0 < c_red; c0 += 16) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int e = tid + 256 * q;
                const int m = e >> 4, c = e & 15;
                const int32_t r = sidx[k][m];
                A v = 0;
                if (r >= 0 && c0 + c < c_red) v = to_acc<A>(src[(int64_t)r * c_red + c0 + c]);
                As[c][m] = v;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int e = tid + 256 * q;
                int c, nn;
                if (MODE == MODE_FWD) { c = e >> 6; nn = e & 63; }
                else { nn = e >> 4; c = e & 15; }
                A v = 0;
                if (c0 + c < c_red && col0 + nn < n_out) {
                    v = MODE == MODE_FWD
                            ? to_acc<A>(wk[(int64_t)(c0 + c) * n_out + col0 + nn])
                            : to_acc<A>(wk[(int64_t)(col0 + nn) * c_red + c0 + c]);
                }
                Bs[c][nn] = v;
            }
            __syncthreads();
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                A av[4], bv[4];
#pragma unroll
                for (int a = 0; a < 4; ++a) av[a] = As[c][ty * 4 + a];
#pragma unroll
                for (int b = 0; b < 4; ++b) bv[b] = Bs[c][tx * 4 + b];
#pragma unroll
                for (int a = 0; a < 4; ++a)
#pragma unroll
                    for (int b = 0; b < 4; ++b) acc[a][b] += av[a] * bv[b];
            }
            __syncthreads();
        }
    }
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        const int64_t i = row0 + ty * 4 + a;
        if (i >= n) continue;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int col = col0 + tx * 4 + b;
            if (col >= n_out) continue;
            A v = acc[a][b];
            T o;
            if (bias_mode == SVTAD_BIAS_FP32) {
                o = from_acc<T>(v + ((const A*)bias)[col]);
            } else if (bias_mode == SVTAD_BIAS_PRE) {
                o = from_acc<T>(v + to_acc<A>(((const T*)bias)[col]));
            } else if (bias_mode == SVTAD_BIAS_AFTER) {
                o = from_acc<T>(to_acc<A>(from_acc<T>(v)) + to_acc<A>(((const T*)bias)[col]));
            } else {
                o = from_acc<T>(v);
            }
            out[i * n_out + col] = o;
        }
    }
}

// ---------------------------------------------------------------------------
// Orphan pass of bwd_in: entries (i,k) -> j whose transpose (j, 8-k) -> i is
// not in the table are not covered by the transposed gather; the rows they
// reach are recomputed here (after the gather kernel has stored gi) by one
// workgroup, in fp32 with one rounding and a fixed order (orphan_exact).
// Tables built from a keep mask have none: with the flag the launch returns
// at once, without it the workgroup only scans the table.
// ---------------------------------------------------------------------------
template <typename T, bool DEPTHWISE>
__global__ __launch_bounds__(256) void k_orphans(const T* __restrict__ go,
                                                 const int32_t* __restrict__ nbr,
                                                 const T* __restrict__ w, T* __restrict__ gi,
                                                 int64_t n, int c_in, int c_out, int64_t tpb,
                                                 const uint32_t* __restrict__ flag) {
    if (flag && *flag == 0u) return;  // no entry without a symmetric partner
    orphan_exact<T, DEPTHWISE, 256>(go, nbr, w, gi, n, c_in, c_out, tpb);
}

// ---------------------------------------------------------------------------
// bwd_w partials: ws[s][k][ci][co] = sum over rows of split s of
// x[src(i,k), ci] * go[i, co]; ws_bias[s][co] = sum over the same rows of go.
// Grid (co tiles, 9 * ci tiles, splits); tile 64 x 64, K (rows) step 16.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void k_bw_valu(const T* __restrict__ go, const T* __restrict__ x,
                                                 const int32_t* __restrict__ nbr,
                                                 typename Acc<T>::type* __restrict__ ws,
                                                 typename Acc<T>::type* __restrict__ ws_bias,
                                                 int64_t n, int c_in, int c_out, int64_t tpb,
                                                 int64_t rows_per_split, int n_ci_tiles) {
    typedef typename Acc<T>::type A;
    __shared__ int32_t sidx[16];
    __shared__ A As[16][64 + 4];
    __shared__ A Bs[16][64 + 4];
    const int tid = threadIdx.x;
    const int co0 = blockIdx.x * 64;
    const int k = blockIdx.y / n_ci_tiles;
    const int ci0 = (blockIdx.y - k * n_ci_tiles) * 64;
    const int s = blockIdx.z;
    const int64_t r_begin = (int64_t)s * rows_per_split;
    const int64_t r_end = min(n, r_begin + rows_per_split);
    const bool do_bias = ws_bias != nullptr && k == 4 && ci0 == 0;
    const int ty = tid >> 4, tx = tid & 15;
    A acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = 0;
    A bsum = 0;
    for (int64_t r0 = r_begin; r0 < r_end; r0 += 16) {
        if (tid < 16) {
            const int64_t i = r0 + tid;
            sidx[tid] = i < r_end ? (int32_t)src_row(nbr, i, k, n, tpb) : -1;
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int e = tid + 256 * q;
            const int r = e >> 6, m = e & 63;
            const int32_t src = sidx[r];
            A v = 0;
            if (src >= 0 && ci0 + m < c_in) v = to_acc<A>(x[(int64_t)src * c_in + ci0 + m]);
            As[r][m] = v;
            const int64_t i = r0 + r;
            A g = 0;
            if (i < r_end && co0 + m < c_out) g = to_acc<A>(go[i * c_out + co0 + m]);
            Bs[r][m] = g;
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            A av[4], bv[4];
#pragma unroll
            for (int a = 0; a < 4; ++a) av[a] = As[r][ty * 4 + a];
#pragma unroll
            for (int b = 0; b < 4; ++b) bv[b] = Bs[r][tx * 4 + b];
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int b = 0; b < 4; ++b) acc[a][b] += av[a] * bv[b];
        }
        if (do_bias && tid < 64) {
#pragma unroll
            for (int r = 0; r < 16; ++r) bsum += Bs[r][tid];
        }
        __syncthreads();
    }
    A* dst = ws + ((int64_t)s * 9 + k) * c_in * c_out;
#pragma unroll
    for (int a = 0; a < 4; ++a) {
        const int ci = ci0 + ty * 4 + a;
        if (ci >= c_in) continue;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int co = co0 + tx * 4 + b;
            if (co < c_out) dst[(int64_t)ci * c_out + co] = acc[a][b];
        }
    }
    if (do_bias && tid < 64 && co0 + tid < c_out) ws_bias[(int64_t)s * c_out + co0 + tid] = bsum;
}

// Ordered sum of the split partials, rounded once: out[e] = T(sum_s ws[s][e]).
// out[e] = T(sum_s ws[s * stride + e]) for e < count0, out2[e - count0] for
// count0 <= e < count (two outputs from one partial row, e.g. weight and
// bias): a workgroup owns 64 outputs; its 16 groups of
// 64 threads each sum a contiguous sixteenth of the splits (eight loads in
// flight), and the 16 group sums are added in group order through LDS, so
// the order of the sum is fixed.
// Split reductions: a 1024-thread workgroup takes kRedLanes outputs; its
// kRedGroups thread groups each sum a contiguous range of the splits (up to
// 8 loads in flight), and the group sums are added in order through LDS. 32
// groups keep each group's range to one round of loads up to 256 splits (16
// groups of 64 outputs took two rounds at 150-254 splits).
constexpr int kRedGroups = 32, kRedLanes = 1024 / kRedGroups;

template <typename T, typename A>
__global__ __launch_bounds__(1024) void k_split_reduce(const A* __restrict__ ws, int64_t count,
                                                       int splits, T* __restrict__ out, int64_t stride,
                                                       int64_t count0, T* __restrict__ out2) {
    __shared__ A part[kRedGroups][kRedLanes];
    const int lane = threadIdx.x % kRedLanes, g = threadIdx.x / kRedLanes;
    const int64_t e = (int64_t)blockIdx.x * kRedLanes + lane;
    const int spt = (splits + kRedGroups - 1) / kRedGroups;
    const int q0 = min(splits, g * spt), q1 = min(splits, q0 + spt);
    A s = 0;
    if (e < count) {
        // eight loads in flight, the last batch's extra slots reading the
        // range's last split and adding zero (the sum and its order are those
        // of the plain loop; loads stay unconditional, so no branch waits)
        for (int q = q0; q < q1; q += 8) {
            A v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = ws[(int64_t)min(q + u, q1 - 1) * stride + e];
#pragma unroll
            for (int u = 0; u < 8; ++u) s += q + u < q1 ? v[u] : (A)0;
        }
    }
    part[g][lane] = s;
    __syncthreads();
    if (g != 0 || e >= count) return;
    A t = part[0][lane];
#pragma unroll
    for (int h = 1; h < kRedGroups; ++h) t += part[h][lane];
    if (e < count0) out[e] = from_acc<T>(t);
    else out2[e - count0] = from_acc<T>(t);
}

// ---------------------------------------------------------------------------
// Depthwise (groups = C): one thread per (row, channel).
// ---------------------------------------------------------------------------
template <typename T, int MODE>
__global__ __launch_bounds__(256) void k_dw_gather(const T* __restrict__ src,
                                                   const int32_t* __restrict__ nbr,
                                                   const T* __restrict__ w,
                                                   const T* __restrict__ bias,
                                                   T* __restrict__ out, int64_t n, int c,
                                                   int64_t tpb) {
    typedef typename Acc<T>::type A;
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= n * c) return;
    const int64_t i = e / c;
    const int ch = (int)(e - i * c);
    A s = bias ? to_acc<A>(bias[ch]) : (A)0;
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        const int64_t r = MODE == MODE_FWD ? src_row(nbr, i, k, n, tpb) : src_row_t(nbr, i, k, n, tpb);
        if (r >= 0) s += to_acc<A>(src[r * c + ch]) * to_acc<A>(w[k * c + ch]);
    }
    out[e] = from_acc<T>(s);
}

// ws[s][k][c] = sum over rows of split s of go[i,c] * x[src(i,k), c];
// ws_bias[s][c] = sum of go[i,c]. Grid (channel blocks of 64, splits);
// 4 waves split the rows, lanes the channels.
template <typename T>
__global__ __launch_bounds__(256) void k_dw_bw(const T* __restrict__ go, const T* __restrict__ x,
                                               const int32_t* __restrict__ nbr,
                                               typename Acc<T>::type* __restrict__ ws,
                                               typename Acc<T>::type* __restrict__ ws_bias,
                                               int64_t n, int c, int64_t tpb,
                                               int64_t rows_per_split) {
    typedef typename Acc<T>::type A;
    __shared__ A red[4][10][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int ch = blockIdx.x * 64 + lane;
    const int s = blockIdx.y;
    const int64_t r_begin = (int64_t)s * rows_per_split;
    const int64_t r_end = min(n, r_begin + rows_per_split);
    A acc[10];
#pragma unroll
    for (int k = 0; k < 10; ++k) acc[k] = 0;
    if (ch < c) {
        for (int64_t i = r_begin + wv; i < r_end; i += 4) {
            const A g = to_acc<A>(go[i * c + ch]);
            acc[9] += g;
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                const int64_t r = src_row(nbr, i, k, n, tpb);
                if (r >= 0) acc[k] += g * to_acc<A>(x[r * c + ch]);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < 10; ++k) red[wv][k][lane] = acc[k];
    __syncthreads();
    if (wv == 0 && ch < c) {
#pragma unroll
        for (int k = 0; k < 10; ++k) {
            const A v = red[0][k][lane] + red[1][k][lane] + red[2][k][lane] + red[3][k][lane];
            if (k < 9) ws[((int64_t)s * 9 + k) * c + ch] = v;
            else if (ws_bias) ws_bias[(int64_t)s * c + ch] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// Depthwise, vectorized (C a multiple of VEC = 16 / sizeof(T)): a thread owns
// VEC consecutive channels (16 bytes) of one row. The 9 gathered 16-byte
// loads are buffer loads whose offset is out of range for a missing neighbor
// (they return zeros: no branch around a load), all in flight before the
// first use; the row is written as one 16-byte store.
// ---------------------------------------------------------------------------
template <typename T> struct Vec16 {
    static constexpr int N = 16 / (int)sizeof(T);
    T e[N];
};

template <typename T, int MODE>
__global__ __launch_bounds__(256) void k_dw_vec(const T* __restrict__ src, const int32_t* __restrict__ nbr,
                                                const T* __restrict__ w, const T* __restrict__ bias,
                                                T* __restrict__ out, int64_t n, int c, int64_t tpb, bool sym) {
    constexpr int VEC = Vec16<T>::N;
    typedef typename Acc<T>::type A;
    const int cpr = c / VEC;
    // consecutive row blocks on one XCD: the rows a block gathers (within
    // about one image row of its own) are mostly in the same L2
    const int64_t e = xcd_tile(blockIdx.x, gridDim.x) * 256 + threadIdx.x;
    if (e >= n * cpr) return;
    const int64_t i = e / cpr;
    const int ch = (int)(e - i * cpr) * VEC;
    const rsrc_t rs = make_rsrc(src, (uint32_t)(n * c * (int64_t)sizeof(T)));
    // the row's table entries through a buffer resource: 32-bit offsets from
    // one scalar base (nine 64-bit address computations per thread made this
    // kernel 0.5-0.8 us slower)
    const rsrc_t rt = make_rsrc(nbr, (uint32_t)(n * 9 * 4));
    int tv[9];
#pragma unroll
    for (int k = 0; k < 9; ++k)
        tv[k] = (int)__builtin_amdgcn_raw_buffer_load_b32(rt, (uint32_t)(i * 9 + (MODE == MODE_FWD ? k : 8 - k)) * 4u, 0, 0);
    const int64_t shift = tpb > 0 ? (i / tpb) * tpb : 0;
    u32x4 v[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        int64_t r = tv[k] >= 0 ? (int64_t)tv[k] + shift : -1;
        if (r >= n) r = -1;
        // backward-input gathers row r through offset k only when r's entry
        // (r, k) points back to i (the transposed table, as src_row_t); sym:
        // the caller promises it does
        if (MODE != MODE_FWD && !sym && r >= 0 && src_row(nbr, r, k, n, tpb) != i) r = -1;
        v[k] = bload16(rs, r >= 0 ? (uint32_t)((r * c + ch) * (int64_t)sizeof(T)) : kOOB);
    }
    A acc[VEC];
    if (bias) {
        const Vec16<T> b = __builtin_bit_cast(Vec16<T>, *(const u32x4*)(bias + ch));
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[j] = to_acc<A>(b.e[j]);
    } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[j] = (A)0;
    }
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        const Vec16<T> xv = __builtin_bit_cast(Vec16<T>, v[k]);
        const Vec16<T> wv = __builtin_bit_cast(Vec16<T>, *(const u32x4*)(w + (int64_t)k * c + ch));
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[j] += to_acc<A>(xv.e[j]) * to_acc<A>(wv.e[j]);
    }
    Vec16<T> o;
#pragma unroll
    for (int j = 0; j < VEC; ++j) o.e[j] = from_acc<T>(acc[j]);
    // non-temporal: not read by this launch (saves the L2 write-back at its end)
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4, o), (u32x4*)(out + i * c + ch));
}

// The row lanes' sums of a depthwise backward-weight workgroup: thread (row
// lane rl, chunk q) holds acc[k][j] for channel q * VEC + j, k < 9 the
// offsets and k = 9 the bias. Each (k, channel) sum is added over the R row
// lanes in order 0 .. R-1 through LDS, five offsets at a time, eight LDS reads
// in flight, and stored at ws_split[k * c + channel]. LDS layout
// [kk][rl][j][q]: the 64 lanes of a store instruction write 64 consecutive
// words and a read instruction's lanes read consecutive (j, q) positions, so
// neither has bank conflicts (a [kk][rl][channel] layout, each lane storing
// its VEC consecutive channels, makes lanes 32 bytes apart collide 8 ways).
template <typename A, int VEC>
__device__ __forceinline__ void dw_row_lane_sums(const A (&acc)[10][VEC], A* __restrict__ red, bool active, int rl,
                                                 int q, int R, int c, int cpr, A* __restrict__ ws_split, int tid,
                                                 int nthreads) {
#pragma unroll
    for (int k0 = 0; k0 < 10; k0 += 5) {
        if (active) {
#pragma unroll
            for (int kk = 0; kk < 5; ++kk)
#pragma unroll
                for (int j = 0; j < VEC; ++j) red[((kk * R + rl) * VEC + j) * cpr + q] = acc[k0 + kk][j];
        }
        __syncthreads();
        for (int pi = tid; pi < 5 * c; pi += nthreads) {
            const int kk = pi / c, u = pi - kk * c;  // u = j * cpr + chunk
            const int j = u / cpr, qq = u - j * cpr;
            const A* col = red + (int64_t)kk * R * c + u;  // row lane stride VEC * cpr = c
            A v = (A)0;
            int h0 = 0;
            for (; h0 + 8 <= R; h0 += 8) {
                A t[8];
#pragma unroll
                for (int h = 0; h < 8; ++h) t[h] = col[(h0 + h) * c];
#pragma unroll
                for (int h = 0; h < 8; ++h) v += t[h];
            }
            for (; h0 < R; ++h0) v += col[h0 * c];
            ws_split[(int64_t)(k0 + kk) * c + qq * VEC + j] = v;
        }
        __syncthreads();
    }
}

// ws[s][k][c] = sum over the rows i of split s of go[i,c] x[src(i,k),c] for
// k < 9 and ws[s][9][c] = sum of go[i,c] (the bias; one partial row of 10 c
// per split, reduced in one launch): one workgroup of 512 threads per split,
// all channels. Thread (row lane rl, chunk q): R = 512 / cpr row lanes walk the
// split's rows two at a time (rows rl + 2uR and rl + (2u+1)R: the table
// reads and the 18 gathered loads of both are in flight together); each
// thread keeps 10 x VEC sums, added over the row lanes in order 0 .. R-1
// through LDS, five offsets at a time.
template <typename T>
__global__ __launch_bounds__(512) void k_dw_bw_vec(const T* __restrict__ go, const T* __restrict__ x,
                                                   const int32_t* __restrict__ nbr,
                                                   typename Acc<T>::type* __restrict__ ws, int64_t n, int c,
                                                   int64_t tpb, int64_t rows_per_split) {
    constexpr int VEC = Vec16<T>::N;
    typedef typename Acc<T>::type A;
    __shared__ __align__(16) A red[5 * 512 * VEC];
    const int cpr = c / VEC, R = 512 / cpr;
    const int tid = threadIdx.x, rl = tid / cpr, ch = (tid - rl * cpr) * VEC;
    const bool active = rl < R;
    const int s = (int)xcd_tile(blockIdx.x, gridDim.x);  // neighboring splits on one XCD (shared halo rows)
    const int64_t r_begin = (int64_t)s * rows_per_split;
    const int64_t r_end = min(n, r_begin + rows_per_split);
    const rsrc_t rs = make_rsrc(x, (uint32_t)(n * c * (int64_t)sizeof(T)));
    const rsrc_t rg = make_rsrc(go, (uint32_t)(n * c * (int64_t)sizeof(T)));
    A acc[10][VEC];
#pragma unroll
    for (int k = 0; k < 10; ++k)
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[k][j] = (A)0;
    auto offs = [&](int64_t i, uint32_t* off) {
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            const int64_t r = i < r_end ? src_row(nbr, i, k, n, tpb) : -1;
            off[k] = r >= 0 ? (uint32_t)((r * c + ch) * (int64_t)sizeof(T)) : kOOB;
        }
    };
    auto add = [&](const u32x4& gv, const u32x4* v) {
        const Vec16<T> g = __builtin_bit_cast(Vec16<T>, gv);
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[9][j] += to_acc<A>(g.e[j]);
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            const Vec16<T> xv = __builtin_bit_cast(Vec16<T>, v[k]);
#pragma unroll
            for (int j = 0; j < VEC; ++j) acc[k][j] += to_acc<A>(g.e[j]) * to_acc<A>(xv.e[j]);
        }
    };
    if (active) {
        for (int64_t i = r_begin + rl; i < r_end; i += 2 * R) {
            const int64_t i2 = i + R;  // may be past the split: zeros (go and x loads out of range)
            uint32_t o1[9], o2[9];
            offs(i, o1);
            offs(i2, o2);
            const u32x4 g1 = bload16(rg, (uint32_t)((i * c + ch) * (int64_t)sizeof(T)));
            const u32x4 g2 = bload16(rg, i2 < r_end ? (uint32_t)((i2 * c + ch) * (int64_t)sizeof(T)) : kOOB);
            u32x4 v1[9], v2[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) v1[k] = bload16(rs, o1[k]);
#pragma unroll
            for (int k = 0; k < 9; ++k) v2[k] = bload16(rs, o2[k]);
            add(g1, v1);
            add(g2, v2);
        }
    }
    // the 10 sums per channel over the row lanes, in order
    dw_row_lane_sums<A, VEC>(acc, red, active, rl, ch / VEC, R, c, cpr, ws + (int64_t)s * 10 * c, tid, 512);
}

// Depthwise backward in one pass over the rows: the backward-weight partials
// of k_dw_bw_vec and, for the same rows, the backward-input gather of
// k_dw_vec<MODE_BWDIN>. Row i's table entries give both the gathered x rows
// (weight gradient) and the candidates of its transposed entries: entry
// (i, 8-k) -> j is row i's transposed source for offset k when (j, k) -> i.
// Per chunk of rows, all threads first resolve both source rows of every
// (row, offset) into LDS (the table reads and the partner check are one
// parallel step, not a chain per row); then thread (row lane rl, chunk)
// takes rows rl, rl + R, ... of the chunk with every gathered load of a row
// in flight together. Chunks are a whole number of R rows, so a lane owns
// the rows k_dw_bw_vec gives it, in the same order, and the partial sums
// are bit-identical to k_dw_bw_vec's; each gi row is summed over k = 0 .. 8
// in k_dw_vec's order (fp16 results can still differ by an ulp in a few
// elements, where the compiler picks other multiply-add instructions). An
// entry without its partner (possible only in a table not built from a keep
// mask) is left to the orphan pass: the workgroup writes its flag word (0 or
// 1, every launch, so it needs no clearing) and the reduction kernel runs
// the pass when any word is set.
constexpr int kDwChunkRows = 512;
template <typename T>
__global__ __launch_bounds__(512) void k_dw_bwd_vec(const T* __restrict__ go, const T* __restrict__ x,
                                                    const int32_t* __restrict__ nbr, const T* __restrict__ w,
                                                    T* __restrict__ gi, typename Acc<T>::type* __restrict__ ws,
                                                    uint32_t* __restrict__ flags, int64_t n, int c, int64_t tpb,
                                                    int64_t rows_per_split, bool sym) {
    constexpr int VEC = Vec16<T>::N;
    typedef typename Acc<T>::type A;
    __shared__ __align__(16) A red[5 * 512 * VEC];
    __shared__ int sx[kDwChunkRows * 9], st[kDwChunkRows * 9];  // gathered x row / transposed go row, -1 none
    const int cpr = c / VEC, R = 512 / cpr;
    const int chunk = (kDwChunkRows / R) * R;
    const int tid = threadIdx.x, rl = tid / cpr, ch = (tid - rl * cpr) * VEC;
    const bool active = rl < R;
    const int s = (int)xcd_tile(blockIdx.x, gridDim.x);  // neighboring splits on one XCD (shared halo rows)
    const int64_t r_begin = (int64_t)s * rows_per_split;
    const int64_t r_end = min(n, r_begin + rows_per_split);
    const rsrc_t rs = make_rsrc(x, (uint32_t)(n * c * (int64_t)sizeof(T)));
    const rsrc_t rg = make_rsrc(go, (uint32_t)(n * c * (int64_t)sizeof(T)));
    A acc[10][VEC];
#pragma unroll
    for (int k = 0; k < 10; ++k)
#pragma unroll
        for (int j = 0; j < VEC; ++j) acc[k][j] = (A)0;
    Vec16<T> wk[9];
    if (active) {
#pragma unroll
        for (int k = 0; k < 9; ++k) wk[k] = __builtin_bit_cast(Vec16<T>, *(const u32x4*)(w + (int64_t)k * c + ch));
    }
    int orphan = 0;
    for (int64_t c0 = r_begin; c0 < r_end; c0 += chunk) {
        const int rows = (int)min<int64_t>(chunk, r_end - c0);
        __syncthreads();  // the previous chunk's rows are consumed
        for (int e = tid; e < rows * 9; e += 512) {
            const int r = e / 9, k = e - r * 9;
            const int64_t i = c0 + r;
            sx[e] = (int)src_row(nbr, i, k, n, tpb);
            const int64_t j = src_row(nbr, i, 8 - k, n, tpb);
            const bool ok = j >= 0 && (sym || src_row(nbr, j, k, n, tpb) == i);
            orphan |= (j >= 0 && !ok) ? 1 : 0;
            st[e] = ok ? (int)j : -1;
        }
        __syncthreads();
        if (!active) continue;
        for (int r = rl; r < rows; r += R) {
            const int64_t i = c0 + r;
            const u32x4 gv = bload16(rg, (uint32_t)((i * c + ch) * (int64_t)sizeof(T)));
            u32x4 v[9], t[9];
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                const int jx = sx[r * 9 + k], jt = st[r * 9 + k];
                v[k] = bload16(rs, jx >= 0 ? (uint32_t)(((int64_t)jx * c + ch) * (int64_t)sizeof(T)) : kOOB);
                t[k] = bload16(rg, jt >= 0 ? (uint32_t)(((int64_t)jt * c + ch) * (int64_t)sizeof(T)) : kOOB);
            }
            const Vec16<T> g = __builtin_bit_cast(Vec16<T>, gv);
#pragma unroll
            for (int j = 0; j < VEC; ++j) acc[9][j] += to_acc<A>(g.e[j]);
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                const Vec16<T> xv = __builtin_bit_cast(Vec16<T>, v[k]);
#pragma unroll
                for (int j = 0; j < VEC; ++j) acc[k][j] += to_acc<A>(g.e[j]) * to_acc<A>(xv.e[j]);
            }
            A gs[VEC];
#pragma unroll
            for (int j = 0; j < VEC; ++j) gs[j] = (A)0;
#pragma unroll
            for (int k = 0; k < 9; ++k) {
                const Vec16<T> tv = __builtin_bit_cast(Vec16<T>, t[k]);
#pragma unroll
                for (int j = 0; j < VEC; ++j) gs[j] += to_acc<A>(tv.e[j]) * to_acc<A>(wk[k].e[j]);
            }
            Vec16<T> o;
#pragma unroll
            for (int j = 0; j < VEC; ++j) o.e[j] = from_acc<T>(gs[j]);
            __builtin_nontemporal_store(__builtin_bit_cast(u32x4, o), (u32x4*)(gi + i * c + ch));  // as k_dw_vec
        }
    }
    // the weight / bias partials as in k_dw_bw_vec (red aliases nothing the
    // row loop uses)
    dw_row_lane_sums<A, VEC>(acc, red, active, rl, ch / VEC, R, c, cpr, ws + (int64_t)s * 10 * c, tid, 512);
    const int any = __syncthreads_or(orphan);
    if (tid == 0) flags[s] = any ? 1u : 0u;
}

// The split reduction of k_dw_bwd_vec's partials (as k_split_reduce, weight
// then bias from one partial row of 10 c), then, when any split's flag word
// is set, the depthwise pass for entries without a symmetric partner in the
// first workgroup (orphan_exact).
template <typename T, typename A>
__global__ __launch_bounds__(1024) void k_dw_bwd_reduce(const A* __restrict__ ws, int64_t count, int splits,
                                                        T* __restrict__ gw, int64_t stride, int64_t count0,
                                                        T* __restrict__ gb, const uint32_t* __restrict__ flags,
                                                        const T* __restrict__ go, const int32_t* __restrict__ nbr,
                                                        const T* __restrict__ w, T* __restrict__ gi, int64_t n,
                                                        int c, int64_t tpb) {
    __shared__ A part[kRedGroups][kRedLanes];
    const int lane = threadIdx.x % kRedLanes, g = threadIdx.x / kRedLanes;
    const int64_t e = (int64_t)blockIdx.x * kRedLanes + lane;
    const int spt = (splits + kRedGroups - 1) / kRedGroups;
    const int q0 = min(splits, g * spt), q1 = min(splits, q0 + spt);
    A sum = 0;
    if (e < count) {  // as k_split_reduce
        for (int q = q0; q < q1; q += 8) {
            A v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = ws[(int64_t)min(q + u, q1 - 1) * stride + e];
#pragma unroll
            for (int u = 0; u < 8; ++u) sum += q + u < q1 ? v[u] : (A)0;
        }
    }
    part[g][lane] = sum;
    __syncthreads();
    if (g == 0 && e < count) {
        A t = part[0][lane];
#pragma unroll
        for (int h = 1; h < kRedGroups; ++h) t += part[h][lane];
        if (e < count0) gw[e] = from_acc<T>(t);
        else gb[e - count0] = from_acc<T>(t);
    }
    int f = 0;
    for (int q = threadIdx.x; q < splits; q += 1024) f |= flags[q] != 0u ? 1 : 0;
    if (__syncthreads_or(f) == 0 || blockIdx.x != 0) return;
    orphan_exact<T, true, 1024>(go, nbr, w, gi, n, c, c, tpb);
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------

static bool al16v(const void* p) { return ((uintptr_t)p & 15) == 0; }

// the vectorized depthwise kernels apply: whole 16-byte chunks per row, at
// most 256 chunks per row, 32-bit buffer offsets, 16-byte aligned pointers
template <typename T>
static bool dw_vec_ok(int64_t n, int c, const void* a, const void* b, const void* d) {
    constexpr int VEC = Vec16<T>::N;
    return c % VEC == 0 && c / VEC <= 256 && n * c * (int64_t)sizeof(T) < (int64_t)INT32_MAX - 16 &&
           n * 36 < (int64_t)INT32_MAX - 16 && al16v(a) && al16v(b) && (!d || al16v(d));
}

template <typename T> constexpr int dtype_of();
template <> constexpr int dtype_of<float>() { return SVTAD_F32; }
template <> constexpr int dtype_of<f16>() { return SVTAD_F16; }
template <> constexpr int dtype_of<bf16>() { return SVTAD_BF16; }
template <> constexpr int dtype_of<double>() { return SVTAD_F64; }

template <typename T>
static void launch_split_reduce(const void* part, int64_t count, int splits, void* out,
                                hipStream_t s) {
    typedef typename Acc<T>::type A;
    hipLaunchKernelGGL((k_split_reduce<T, A>), dim3((unsigned)std::max<int64_t>(1, cdiv(count, kRedLanes))),
                       dim3(1024), 0, s, (const A*)part, count, splits, (T*)out, count, count, (T*)nullptr);
}

void split_reduce(int dtype, const void* part, int64_t count, int splits, void* out, hipStream_t s) {
    switch (dtype) {
        case SVTAD_F32: launch_split_reduce<float>(part, count, splits, out, s); break;
        case SVTAD_F16: launch_split_reduce<f16>(part, count, splits, out, s); break;
        case SVTAD_BF16: launch_split_reduce<bf16>(part, count, splits, out, s); break;
        case SVTAD_F64: launch_split_reduce<double>(part, count, splits, out, s); break;
    }
}

template <typename T>
static void launch_gg_valu(int mode, const void* src, const int32_t* nbr, const void* w,
                           const void* bias, int bias_mode, void* out, int64_t n, int c_red,
                           int n_out, int64_t tpb, hipStream_t s) {
    dim3 grid((unsigned)cdiv(n, 64), (unsigned)cdiv(n_out, 64));
    if (mode == MODE_FWD)
        hipLaunchKernelGGL((k_gg_valu<T, MODE_FWD>), grid, dim3(256), 0, s, (const T*)src, nbr,
                           (const T*)w, bias, bias_mode, (T*)out, n, c_red, n_out, tpb);
    else
        hipLaunchKernelGGL((k_gg_valu<T, MODE_BWDIN>), grid, dim3(256), 0, s, (const T*)src, nbr,
                           (const T*)w, (const void*)nullptr, 0, (T*)out, n, c_red, n_out, tpb);
}

void gg_valu(int dtype, int mode, const void* src, const int32_t* nbr, const void* w,
             const void* bias, int bias_mode, void* out, int64_t n, int c_red, int n_out,
             int64_t tpb, hipStream_t s) {
    switch (dtype) {
        case SVTAD_F32: launch_gg_valu<float>(mode, src, nbr, w, bias, bias_mode, out, n, c_red, n_out, tpb, s); break;
        case SVTAD_F16: launch_gg_valu<f16>(mode, src, nbr, w, bias, bias_mode, out, n, c_red, n_out, tpb, s); break;
        case SVTAD_BF16: launch_gg_valu<bf16>(mode, src, nbr, w, bias, bias_mode, out, n, c_red, n_out, tpb, s); break;
        case SVTAD_F64: launch_gg_valu<double>(mode, src, nbr, w, bias, bias_mode, out, n, c_red, n_out, tpb, s); break;
    }
}

template <typename T>
static void launch_orphans(bool dw, const void* go, const int32_t* nbr, const void* w, void* gi,
                           int64_t n, int c_in, int c_out, int64_t tpb, const uint32_t* flag,
                           hipStream_t s) {
    // one workgroup (the pass is exact and ordered, orphan_exact)
    dim3 grid(1);
    if (dw)
        hipLaunchKernelGGL((k_orphans<T, true>), grid, dim3(256), 0, s, (const T*)go, nbr,
                           (const T*)w, (T*)gi, n, c_in, c_out, tpb, flag);
    else
        hipLaunchKernelGGL((k_orphans<T, false>), grid, dim3(256), 0, s, (const T*)go, nbr,
                           (const T*)w, (T*)gi, n, c_in, c_out, tpb, flag);
}

void orphans(int dtype, bool dw, const void* go, const int32_t* nbr, const void* w, void* gi,
             int64_t n, int c_in, int c_out, int64_t tpb, const uint32_t* flag, hipStream_t s) {
    switch (dtype) {
        case SVTAD_F32: launch_orphans<float>(dw, go, nbr, w, gi, n, c_in, c_out, tpb, flag, s); break;
        case SVTAD_F16: launch_orphans<f16>(dw, go, nbr, w, gi, n, c_in, c_out, tpb, flag, s); break;
        case SVTAD_BF16: launch_orphans<bf16>(dw, go, nbr, w, gi, n, c_in, c_out, tpb, flag, s); break;
        case SVTAD_F64: launch_orphans<double>(dw, go, nbr, w, gi, n, c_in, c_out, tpb, flag, s); break;
    }
}

template <typename T>
static void launch_bw_valu(const BwPlan& p, const void* go, const void* x, const int32_t* nbr,
                           void* gw, void* gb, void* ws, int64_t n, int c_in, int c_out,
                           int64_t tpb, hipStream_t s) {
    typedef typename Acc<T>::type A;
    A* part = (A*)ws;
    A* part_b = gb ? part + (int64_t)p.splits * 9 * c_in * c_out : nullptr;
    const int n_ci_tiles = (int)cdiv(c_in, 64);
    dim3 grid((unsigned)cdiv(c_out, 64), (unsigned)(9 * n_ci_tiles), (unsigned)p.splits);
    hipLaunchKernelGGL((k_bw_valu<T>), grid, dim3(256), 0, s, (const T*)go, (const T*)x, nbr, part,
                       part_b, n, c_in, c_out, tpb, p.rows_per_split, n_ci_tiles);
    if (!gw) return;  // partials only
    split_reduce(dtype_of<T>(), part, 9LL * c_in * c_out, p.splits, gw, s);
    if (gb) split_reduce(dtype_of<T>(), part_b, (int64_t)c_out, p.splits, gb, s);
}

void bw_valu(int dtype, const BwPlan& p, const void* go, const void* x, const int32_t* nbr,
             void* gw, void* gb, void* ws, int64_t n, int c_in, int c_out, int64_t tpb,
             hipStream_t s) {
    switch (dtype) {
        case SVTAD_F32: launch_bw_valu<float>(p, go, x, nbr, gw, gb, ws, n, c_in, c_out, tpb, s); break;
        case SVTAD_F16: launch_bw_valu<f16>(p, go, x, nbr, gw, gb, ws, n, c_in, c_out, tpb, s); break;
        case SVTAD_BF16: launch_bw_valu<bf16>(p, go, x, nbr, gw, gb, ws, n, c_in, c_out, tpb, s); break;
        case SVTAD_F64: launch_bw_valu<double>(p, go, x, nbr, gw, gb, ws, n, c_in, c_out, tpb, s); break;
    }
}

template <typename T>
static void launch_dw(int mode, const void* src, const int32_t* nbr, const void* w,
                      const void* bias, void* out, int64_t n, int c, int64_t tpb, hipStream_t s, bool sym) {
    if (dw_vec_ok<T>(n, c, src, w, out) && (!bias || al16v(bias))) {
        const dim3 g((unsigned)cdiv(n * (c / Vec16<T>::N), 256));
        if (mode == MODE_FWD)
            hipLaunchKernelGGL((k_dw_vec<T, MODE_FWD>), g, dim3(256), 0, s, (const T*)src, nbr, (const T*)w,
                               (const T*)bias, (T*)out, n, c, tpb, false);
        else
            hipLaunchKernelGGL((k_dw_vec<T, MODE_BWDIN>), g, dim3(256), 0, s, (const T*)src, nbr, (const T*)w,
                               (const T*)nullptr, (T*)out, n, c, tpb, sym);
        return;
    }
    dim3 grid((unsigned)cdiv(n * c, 256));
    if (mode == MODE_FWD)
        hipLaunchKernelGGL((k_dw_gather<T, MODE_FWD>), grid, dim3(256), 0, s, (const T*)src, nbr,
                           (const T*)w, (const T*)bias, (T*)out, n, c, tpb);
    else
        hipLaunchKernelGGL((k_dw_gather<T, MODE_BWDIN>), grid, dim3(256), 0, s, (const T*)src, nbr,
                           (const T*)w, (const T*)nullptr, (T*)out, n, c, tpb);
}

void dw_gather(int dtype, int mode, const void* src, const int32_t* nbr, const void* w,
               const void* bias, void* out, int64_t n, int c, int64_t tpb, hipStream_t s, bool sym) {
    switch (dtype) {
        case SVTAD_F32: launch_dw<float>(mode, src, nbr, w, bias, out, n, c, tpb, s, sym); break;
        case SVTAD_F16: launch_dw<f16>(mode, src, nbr, w, bias, out, n, c, tpb, s, sym); break;
        case SVTAD_BF16: launch_dw<bf16>(mode, src, nbr, w, bias, out, n, c, tpb, s, sym); break;
        case SVTAD_F64: launch_dw<double>(mode, src, nbr, w, bias, out, n, c, tpb, s, sym); break;
    }
}

template <typename T>
static void launch_dw_bw(const BwPlan& p, const void* go, const void* x, const int32_t* nbr,
                         void* gw, void* gb, void* ws, int64_t n, int c, int64_t tpb,
                         hipStream_t s) {
    typedef typename Acc<T>::type A;
    A* part = (A*)ws;
    A* part_b = gb ? part + (int64_t)p.splits * 9 * c : nullptr;
    if (dw_vec_ok<T>(n, c, go, x, nullptr)) {
        hipLaunchKernelGGL((k_dw_bw_vec<T>), dim3((unsigned)p.splits), dim3(512), 0, s, (const T*)go,
                           (const T*)x, nbr, part, n, c, tpb, p.rows_per_split);
        const int64_t count = gb ? 10LL * c : 9LL * c;
        hipLaunchKernelGGL((k_split_reduce<T, A>), dim3((unsigned)std::max<int64_t>(1, cdiv(count, kRedLanes))),
                           dim3(1024), 0, s, (const A*)part, count, p.splits, (T*)gw, 10LL * c, 9LL * c,
                           (T*)gb);
        return;
    } else {
        dim3 grid((unsigned)cdiv(c, 64), (unsigned)p.splits);
        hipLaunchKernelGGL((k_dw_bw<T>), grid, dim3(256), 0, s, (const T*)go, (const T*)x, nbr, part,
                           part_b, n, c, tpb, p.rows_per_split);
    }
    split_reduce(dtype_of<T>(), part, 9LL * c, p.splits, gw, s);
    if (gb) split_reduce(dtype_of<T>(), part_b, (int64_t)c, p.splits, gb, s);
}

template <typename T>
static bool launch_dw_bwd(const BwPlan& p, const void* go, const void* x, const int32_t* nbr, const void* w,
                          void* gi, void* gw, void* gb, void* ws, uint32_t* flags, int64_t n, int c, int64_t tpb,
                          hipStream_t s, bool sym) {
    typedef typename Acc<T>::type A;
    if (!dw_vec_ok<T>(n, c, go, x, gi) || !al16v(w)) return false;
    hipLaunchKernelGGL((k_dw_bwd_vec<T>), dim3((unsigned)p.splits), dim3(512), 0, s, (const T*)go, (const T*)x,
                       nbr, (const T*)w, (T*)gi, (A*)ws, flags, n, c, tpb, p.rows_per_split, sym);
    const int64_t count = gb ? 10LL * c : 9LL * c;
    hipLaunchKernelGGL((k_dw_bwd_reduce<T, A>), dim3((unsigned)std::max<int64_t>(1, cdiv(count, kRedLanes))), dim3(1024),
                       0, s, (const A*)ws, count, p.splits, (T*)gw, 10LL * c, 9LL * c, (T*)gb, (const uint32_t*)flags,
                       (const T*)go, nbr, (const T*)w, (T*)gi, n, c, tpb);
    return true;
}

bool dw_bwd_fused(int dtype, const BwPlan& p, const void* go, const void* x, const int32_t* nbr, const void* w,
                  void* gi, void* gw, void* gb, void* ws, uint32_t* flags, int64_t n, int c, int64_t tpb,
                  hipStream_t s, bool sym) {
    switch (dtype) {
        case SVTAD_F32: return launch_dw_bwd<float>(p, go, x, nbr, w, gi, gw, gb, ws, flags, n, c, tpb, s, sym);
        case SVTAD_F16: return launch_dw_bwd<f16>(p, go, x, nbr, w, gi, gw, gb, ws, flags, n, c, tpb, s, sym);
        case SVTAD_BF16: return launch_dw_bwd<bf16>(p, go, x, nbr, w, gi, gw, gb, ws, flags, n, c, tpb, s, sym);
        case SVTAD_F64: return launch_dw_bwd<double>(p, go, x, nbr, w, gi, gw, gb, ws, flags, n, c, tpb, s, sym);
    }
    return false;
}

void dw_bw(int dtype, const BwPlan& p, const void* go, const void* x, const int32_t* nbr, void* gw,
           void* gb, void* ws, int64_t n, int c, int64_t tpb, hipStream_t s) {
    switch (dtype) {
        case SVTAD_F32: launch_dw_bw<float>(p, go, x, nbr, gw, gb, ws, n, c, tpb, s); break;
        case SVTAD_F16: launch_dw_bw<f16>(p, go, x, nbr, gw, gb, ws, n, c, tpb, s); break;
        case SVTAD_BF16: launch_dw_bw<bf16>(p, go, x, nbr, gw, gb, ws, n, c, tpb, s); break;
        case SVTAD_F64: launch_dw_bw<double>(p, go, x, nbr, gw, gb, ws, n, c, tpb, s); break;
    }
}

}  // namespace svtad
