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

// x as a stored fp32 value. The empty asm makes the value opaque, so the
// compiler cannot merge the operation that produced x with a later
// conversion to f16 (v_fma_mix*: one rounding of the exact result where the
// sequence of PyTorch ops rounds to fp32 first, then to f16).
__device__ __forceinline__ float f32_rounded(float x) {
    asm volatile("" : "+v"(x));
    return x;
}

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

__device__ __forceinline__ void atomic_add_out(float* p, float v) { atomicAdd(p, v); }
__device__ __forceinline__ void atomic_add_out(double* p, double v) { atomicAdd(p, v); }

template <typename H>
__device__ __forceinline__ void atomic_add_half(H* p, float v) {
    // CAS on the aligned 32-bit word that holds the 16-bit value.
    uintptr_t addr = (uintptr_t)p;
    unsigned int* word = (unsigned int*)(addr & ~(uintptr_t)3);
    const int shift = (addr & 2) ? 16 : 0;
    unsigned int old = *word, assumed;
    do {
        assumed = old;
        unsigned short bits = (unsigned short)((assumed >> shift) & 0xffffu);
        H h = __builtin_bit_cast(H, bits);
        H nh = (H)((float)h + v);
        unsigned int nb = (unsigned int)__builtin_bit_cast(unsigned short, nh);
        unsigned int nw = (assumed & ~(0xffffu << shift)) | (nb << shift);
        old = atomicCAS(word, assumed, nw);
    } while (old != assumed);
}
__device__ __forceinline__ void atomic_add_out(f16* p, float v) { atomic_add_half(p, v); }
__device__ __forceinline__ void atomic_add_out(bf16* p, float v) { atomic_add_half(p, v); }

// Backward-input contribution of table entry e = i*9 + k when (i, k) -> j has
// no symmetric partner (j, 8-k) -> i, which the transposed gathers cannot see:
// gi[j] += go[i] . W[k]^T (depthwise: go[i] * w[k]), added with atomics.
template <typename T, bool DEPTHWISE>
__device__ __forceinline__ void orphan_entry(int64_t e, const T* __restrict__ go,
                                             const int32_t* __restrict__ nbr,
                                             const T* __restrict__ w, T* __restrict__ gi, int64_t n,
                                             int c_in, int c_out, int64_t tpb) {
    typedef typename Acc<T>::type A;
    const int64_t i = e / 9;
    const int k = (int)(e - i * 9);
    const int64_t j = src_row(nbr, i, k, n, tpb);
    if (j < 0 || src_row(nbr, j, 8 - k, n, tpb) == i) return;
    if (DEPTHWISE) {
        for (int c = 0; c < c_in; ++c)
            atomic_add_out(gi + j * c_in + c,
                           to_acc<A>(go[i * c_in + c]) * to_acc<A>(w[(int64_t)k * c_in + c]));
    } else {
        const T* wk = w + (int64_t)k * c_in * c_out;
        for (int ci = 0; ci < c_in; ++ci) {
            A s = 0;
            for (int co = 0; co < c_out; ++co)
                s += to_acc<A>(go[i * c_out + co]) * to_acc<A>(wk[(int64_t)ci * c_out + co]);
            atomic_add_out(gi + j * c_in + ci, s);
        }
    }
}

// One-way entries handled exactly: the rows j that receive an entry (i, k) ->
// j whose partner (j, 8-k) -> i is absent are recomputed whole in fp32 and
// rounded once, as the reference accumulates gi in fp32 and casts it once
// (2d_sparse_v3.cu:825,834), and in a fixed order, so the result does not
// depend on scheduling. Run by every thread of ONE workgroup of NTH threads
// (the other rows keep what the transposed gather wrote):
//  1. the table is scanned in entry order and the one-way entries collected
//     in LDS as (target, entry) pairs, in that order;
//  2. the pairs are sorted by (target, entry) (bitonic network in LDS);
//  3. per target j, in increasing j: the one-way contributions in entry
//     order, then the symmetric ones (offsets 0..8, the partner-checked
//     transposed lookups that the gather also used), in fp32; gi[j] written
//     once. A thread owns output channels tid, tid + NTH, ... (c_in <= 4 NTH).
// More than kOrphanCap one-way entries, or a table of more than 2^31 entries:
// the atomic pass instead (each contribution added into gi with its own
// rounding, order unfixed).
constexpr int kOrphanCap = 2048;
// Inlined into each caller: as an out-of-line call it made the reduction
// kernels that hold it reserve registers for the call (58 -> 103 VGPRs).
template <typename T, bool DEPTHWISE, int NTH>
__device__ __forceinline__ void orphan_exact(const T* __restrict__ go, const int32_t* __restrict__ nbr,
                             const T* __restrict__ w, T* __restrict__ gi, int64_t n, int c_in, int c_out,
                             int64_t tpb) {
    typedef typename Acc<T>::type A;
    constexpr int NW = NTH / 64;
    constexpr int MAXS = 4;  // channel slots per thread
    __shared__ int sj[kOrphanCap], se[kOrphanCap];
    __shared__ int wcnt[NW];
    __shared__ int total;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int64_t ne = n * 9;
    if (ne > (int64_t)INT32_MAX) {  // entry numbers past 32 bits: the atomic pass
        for (int64_t e = tid; e < ne; e += NTH) orphan_entry<T, DEPTHWISE>(e, go, nbr, w, gi, n, c_in, c_out, tpb);
        return;
    }
    if (tid == 0) total = 0;
    __syncthreads();
    for (int64_t e0 = 0; e0 < ne; e0 += NTH) {
        const int64_t e = e0 + tid;
        int64_t j = -1;
        if (e < ne) {
            const int64_t i = e / 9;
            const int k = (int)(e - i * 9);
            j = src_row(nbr, i, k, n, tpb);
            if (j >= 0 && src_row(nbr, j, 8 - k, n, tpb) == i) j = -1;  // has its partner
        }
        const uint64_t m = __ballot(j >= 0);
        if (lane == 0) wcnt[wv] = __popcll(m);
        __syncthreads();
        int base = total;
        for (int q = 0; q < wv; ++q) base += wcnt[q];
        const int pos = base + __popcll(m & ((1ull << lane) - 1ull));
        if (j >= 0 && pos < kOrphanCap) {
            sj[pos] = (int)j;
            se[pos] = (int)e;
        }
        __syncthreads();
        if (tid == 0) {
            int t = total;
            for (int q = 0; q < NW; ++q) t += wcnt[q];
            total = t;
        }
        __syncthreads();
    }
    const int cnt = total;
    if (cnt == 0) return;
    if (cnt > kOrphanCap || c_in > MAXS * NTH) {
        for (int64_t e = tid; e < ne; e += NTH) orphan_entry<T, DEPTHWISE>(e, go, nbr, w, gi, n, c_in, c_out, tpb);
        return;
    }
    int P = 1;
    while (P < cnt) P <<= 1;
    for (int q = cnt + tid; q < P; q += NTH) {
        sj[q] = 0x7fffffff;
        se[q] = 0x7fffffff;
    }
    __syncthreads();
    for (int size = 2; size <= P; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int q = tid; q < P / 2; q += NTH) {
                const int lo = 2 * q - (q & (stride - 1)), hi = lo + stride;
                const bool up = (lo & size) == 0;
                const bool gt = sj[lo] > sj[hi] || (sj[lo] == sj[hi] && se[lo] > se[hi]);
                if (gt == up) {
                    const int tj = sj[lo], te = se[lo];
                    sj[lo] = sj[hi];
                    se[lo] = se[hi];
                    sj[hi] = tj;
                    se[hi] = te;
                }
            }
            __syncthreads();
        }
    }
    auto add = [&](A* acc, int64_t i, int k) {
#pragma unroll
        for (int s = 0; s < MAXS; ++s) {
            const int c = tid + s * NTH;
            if (c >= c_in) break;
            if (DEPTHWISE) {
                acc[s] += to_acc<A>(go[i * c_in + c]) * to_acc<A>(w[(int64_t)k * c_in + c]);
            } else {
                const T* wr = w + ((int64_t)k * c_in + c) * c_out;
                const T* gr = go + i * c_out;
                A t = 0;
                for (int co = 0; co < c_out; ++co) t += to_acc<A>(gr[co]) * to_acc<A>(wr[co]);
                acc[s] += t;
            }
        }
    };
    for (int a = 0; a < cnt;) {
        const int j = sj[a];
        int b = a + 1;
        while (b < cnt && sj[b] == j) ++b;
        A acc[MAXS];
#pragma unroll
        for (int s = 0; s < MAXS; ++s) acc[s] = 0;
        for (int q = a; q < b; ++q) {
            const int64_t e = se[q], i = e / 9;
            add(acc, i, (int)(e - i * 9));
        }
        for (int k = 0; k < 9; ++k) {
            const int64_t i = src_row(nbr, j, 8 - k, n, tpb);
            if (i >= 0 && src_row(nbr, i, k, n, tpb) == j) add(acc, i, k);
        }
#pragma unroll
        for (int s = 0; s < MAXS; ++s) {
            const int c = tid + s * NTH;
            if (c < c_in) gi[(int64_t)j * c_in + c] = from_acc<T>(acc[s]);
        }
        a = b;
    }
}

}  // namespace svtad
