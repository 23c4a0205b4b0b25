// Neighbor-index table kernels: build from a keep mask, remap after a prune,
// transpose, validate. Integer work; every output is bit-exact with the
// reference procedures (see the citations at each entry point).
#include "sv_common.h"
#include "sv_internal.h"

namespace svtad {

// ---------------------------------------------------------------------------
// build: per-frame counts -> exclusive scan -> per-frame fill
// ---------------------------------------------------------------------------

// One workgroup per frame: number of kept cells.
__global__ __launch_bounds__(256) void k_frame_count(const uint8_t* __restrict__ mask, int cells,
                                                     int32_t* __restrict__ counts) {
    const int64_t f = blockIdx.x;
    const uint8_t* m = mask + f * cells;
    int c = 0;
    for (int p = threadIdx.x; p < cells; p += 256) c += m[p] != 0;
    // wave64 reduction, then across the 4 waves
    for (int o = 32; o > 0; o >>= 1) c += __shfl_xor(c, o, 64);
    __shared__ int part[4];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = c;
    __syncthreads();
    if (threadIdx.x == 0) counts[f] = part[0] + part[1] + part[2] + part[3];
}

// Single workgroup: offsets[f] = sum_{g<f} counts[g], offsets[n] = total.
// counts and offsets may alias (in-place scan is done chunk by chunk with the
// reads of a chunk completed before its writes).
__global__ __launch_bounds__(1024) void k_exclusive_scan(const int32_t* counts, int64_t n,
                                                         int32_t* offsets) {
    __shared__ int32_t wsum[16];
    __shared__ int32_t carry_s;
    if (threadIdx.x == 0) carry_s = 0;
    __syncthreads();
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    for (int64_t base = 0; base < n; base += 1024) {
        const int64_t idx = base + threadIdx.x;
        int32_t v = idx < n ? counts[idx] : 0;
        // inclusive wave scan
        int32_t s = v;
        for (int o = 1; o < 64; o <<= 1) {
            int32_t t = __shfl_up(s, o, 64);
            if (lane >= o) s += t;
        }
        if (lane == 63) wsum[wid] = s;
        __syncthreads();
        int32_t wpre = 0;
        for (int w = 0; w < wid; ++w) wpre += wsum[w];
        const int32_t carry = carry_s;
        if (idx < n) offsets[idx] = carry + wpre + s - v;
        __syncthreads();
        if (threadIdx.x == 1023) carry_s = carry + wpre + s;
        __syncthreads();
    }
    if (threadIdx.x == 0) offsets[n] = carry_s;
}

// One workgroup per frame; dynamic LDS holds the local rank of every cell.
__global__ __launch_bounds__(256) void k_table_fill(const uint8_t* __restrict__ mask,
                                                    const int32_t* __restrict__ offsets, int h,
                                                    int w, int32_t* __restrict__ table) {
    extern __shared__ int16_t rank_s[];  // h*w entries (< 2^14); -1 for dropped cells
    __shared__ int32_t wsum[4];
    __shared__ int32_t carry_s;
    const int64_t f = blockIdx.x;
    const int cells = h * w;
    const uint8_t* m = mask + f * cells;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    if (threadIdx.x == 0) carry_s = 0;
    __syncthreads();
    for (int base = 0; base < cells; base += 256) {
        const int p = base + threadIdx.x;
        const bool kept = p < cells && m[p] != 0;
        const uint64_t bal = __ballot(kept);
        const int before = __popcll(bal & ((1ull << lane) - 1ull));
        if (lane == 0) wsum[wid] = __popcll(bal);
        __syncthreads();
        int pre = carry_s;
        for (int q = 0; q < wid; ++q) pre += wsum[q];
        if (p < cells) rank_s[p] = (int16_t)(kept ? pre + before : -1);
        __syncthreads();
        if (threadIdx.x == 0) carry_s += wsum[0] + wsum[1] + wsum[2] + wsum[3];
        __syncthreads();
    }
    const int32_t off = offsets[f];
    for (int p = threadIdx.x; p < cells; p += 256) {
        const int r = rank_s[p];
        if (r < 0) continue;
        const int y = p / w, x = p - (p / w) * w;
        int32_t* row = table + ((int64_t)off + r) * 9;
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            const int yy = y + k / 3 - 1, xx = x + k % 3 - 1;
            int32_t v = -1;
            if (yy >= 0 && yy < h && xx >= 0 && xx < w) {
                const int rq = rank_s[yy * w + xx];
                if (rq >= 0) v = off + rq;
            }
            row[k] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// remap (restates vit_sparse_adapter_poguise.py:913-977)
// ---------------------------------------------------------------------------

__global__ void k_fill_i32(int32_t* __restrict__ p, int64_t n, int32_t v) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

__global__ void k_remap_scatter(const int64_t* __restrict__ keep, int64_t batch, int64_t n_prev,
                                int64_t n_new, int32_t* __restrict__ mapping) {
    const int64_t total = batch * n_new;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t b = e / n_new;
        const int64_t kidx = keep[e];
        if (kidx >= 0 && kidx < n_prev) mapping[b * n_prev + kidx] = (int32_t)e;
    }
}

__global__ void k_remap_gather(const int32_t* __restrict__ table, const int64_t* __restrict__ keep,
                               int64_t batch, int64_t n_prev, int64_t n_new,
                               const int32_t* __restrict__ mapping, int32_t* __restrict__ out) {
    const int64_t total = batch * n_new * 9;
    const int64_t lim = batch * n_prev;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = e / 9;
        const int k = (int)(e - row * 9);
        const int64_t b = row / n_new;
        const int64_t kidx = keep[row];
        int32_t r = -1;
        if (kidx >= 0 && kidx < n_prev) {
            const int32_t v = table[(b * n_prev + kidx) * 9 + k];
            if (v != -1) {
                const int64_t q = v < 0 ? 0 : v;  // torch.clamp(min=0) of the reference
                r = q < lim ? mapping[q] : -1;
            }
        }
        out[e] = r;
    }
}

// ---------------------------------------------------------------------------
// fused prune step (restates vit_sparse_adapter_poguise.py:899-977)
// ---------------------------------------------------------------------------

// One pass over the output rows of x, one wave per row: the n_key key rows of
// each sample are copied, the kept token rows gathered
// (x[:, n_key + keep[b, j]]), in chunks of type V (16 bytes when the row
// allows it). For kept rows lane 0 also gathers last_idx (:908) and scatters
// the old -> new global mapping (:930-951) that k_remap_gather then reads.
// The row arithmetic is per wave (scalar), not per element. A keep index
// outside [0, n_prev) yields a zero row, idx_out -1 and no mapping entry.
// With x_out == NULL only the index work is done.
template <typename V>
__global__ __launch_bounds__(256) void k_prune_rows(const V* __restrict__ x, int64_t batch,
                                                    int64_t n_key, int64_t n_prev, int64_t row_chunks,
                                                    const int64_t* __restrict__ keep, int64_t n_new,
                                                    const int64_t* __restrict__ last_idx,
                                                    int32_t* __restrict__ mapping,
                                                    V* __restrict__ x_out, int64_t* __restrict__ idx_out) {
    const int64_t rows_out = n_key + n_new, rows_in = n_key + n_prev;
    const int64_t total = batch * rows_out;
    const int lane = threadIdx.x & 63;
    const int64_t w0 = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    for (int64_t r = w0; r < total; r += (int64_t)gridDim.x * 4) {
        const int64_t b = r / rows_out, q = r - b * rows_out;
        int64_t src = -1;
        if (q < n_key) {
            src = b * rows_in + q;
        } else {
            const int64_t j = q - n_key;
            const int64_t kidx = keep[b * n_new + j];
            const bool ok = kidx >= 0 && kidx < n_prev;
            if (ok) src = b * rows_in + n_key + kidx;
            if (lane == 0) {
                if (idx_out) idx_out[b * n_new + j] = ok ? last_idx[b * n_prev + kidx] : -1;
                if (mapping && ok) mapping[b * n_prev + kidx] = (int32_t)(b * n_new + j);
            }
        }
        if (x_out) {
            const V* sp = x + src * row_chunks;
            V* dp = x_out + r * row_chunks;
            for (int64_t c = lane; c < row_chunks; c += 64) dp[c] = src >= 0 ? sp[c] : V{};
        }
    }
}

// ---------------------------------------------------------------------------
// transpose + validate
// ---------------------------------------------------------------------------

__global__ void k_transpose_scatter(const int32_t* __restrict__ table, int64_t n, int64_t tpb,
                                    int32_t* __restrict__ table_t, int32_t* __restrict__ collisions) {
    const int64_t total = n * 9;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = e / 9;
        const int k = (int)(e - i * 9);
        const int64_t j = src_row(table, i, k, n, tpb);
        if (j < 0) continue;
        const int32_t old = atomicCAS(table_t + j * 9 + k, -1, (int32_t)i);
        if (old != -1) atomicAdd(collisions, 1);
    }
}

__global__ void k_validate_init(int32_t* stats) {
    stats[0] = 0;
    stats[1] = INT32_MAX;
    stats[2] = INT32_MIN;
}

__global__ __launch_bounds__(256) void k_validate(const int32_t* __restrict__ t, int64_t n,
                                                  int64_t bound, int32_t* stats) {
    int bad = 0, mn = INT32_MAX, mx = INT32_MIN;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int32_t v = t[e];
        if (v == -1) continue;
        bad += (v < 0 || v >= bound);
        mn = min(mn, v);
        mx = max(mx, v);
    }
    for (int o = 32; o > 0; o >>= 1) {
        bad += __shfl_xor(bad, o, 64);
        mn = min(mn, __shfl_xor(mn, o, 64));
        mx = max(mx, __shfl_xor(mx, o, 64));
    }
    if ((threadIdx.x & 63) == 0) {
        if (bad) atomicAdd(stats, bad);
        atomicMin(stats + 1, mn);
        atomicMax(stats + 2, mx);
    }
}

static inline unsigned grid_for(int64_t work, int threads) {
    int64_t g = cdiv(work, threads);
    if (g < 1) g = 1;
    if (g > 65536) g = 65536;
    return (unsigned)g;
}

}  // namespace svtad

using namespace svtad;

extern "C" int svtad_table_scan(const uint8_t* mask, int64_t n_frames, int h, int w,
                                int32_t* frame_offsets, void* stream) {
    if (n_frames < 0 || h <= 0 || w <= 0 || !frame_offsets || (n_frames > 0 && !mask))
        return set_error(SVTAD_ERR_INVALID, "table_scan: bad arguments");
    if ((int64_t)h * w > kMaxFrameCells)
        return set_error(SVTAD_ERR_UNSUPPORTED, "table_scan: h*w exceeds 16384 cells");
    if (n_frames * (int64_t)h * w >= (int64_t)INT32_MAX)
        return set_error(SVTAD_ERR_UNSUPPORTED, "table_scan: more than 2^31-1 cells");
    hipStream_t s = (hipStream_t)stream;
    if (n_frames > 0)
        hipLaunchKernelGGL(k_frame_count, dim3((unsigned)n_frames), dim3(256), 0, s, mask, h * w,
                           frame_offsets);
    hipLaunchKernelGGL(k_exclusive_scan, dim3(1), dim3(1024), 0, s, frame_offsets, n_frames,
                       frame_offsets);
    return launch_status();
}

extern "C" int svtad_table_fill(const uint8_t* mask, const int32_t* frame_offsets, int64_t n_frames,
                                int h, int w, int32_t* table, void* stream) {
    if (n_frames < 0 || h <= 0 || w <= 0 || (n_frames > 0 && (!mask || !frame_offsets || !table)))
        return set_error(SVTAD_ERR_INVALID, "table_fill: bad arguments");
    if ((int64_t)h * w > kMaxFrameCells)
        return set_error(SVTAD_ERR_UNSUPPORTED, "table_fill: h*w exceeds 16384 cells");
    if (n_frames == 0) return SVTAD_OK;
    const size_t lds = sizeof(int16_t) * (size_t)h * w;
    hipLaunchKernelGGL(k_table_fill, dim3((unsigned)n_frames), dim3(256), lds, (hipStream_t)stream,
                       mask, frame_offsets, h, w, table);
    return launch_status();
}

extern "C" int svtad_remap_table(const int32_t* table, int64_t batch, int64_t n_prev,
                                 const int64_t* keep_idx, int64_t n_new, int32_t* mapping_ws,
                                 int32_t* out, void* stream) {
    if (batch < 0 || n_prev < 0 || n_new < 0 || n_new > n_prev)
        return set_error(SVTAD_ERR_INVALID, "remap_table: bad sizes");
    if (batch * n_prev >= (int64_t)INT32_MAX)
        return set_error(SVTAD_ERR_UNSUPPORTED, "remap_table: more than 2^31-1 rows");
    if (batch * n_new == 0) return SVTAD_OK;
    if (!table || !keep_idx || !mapping_ws || !out)
        return set_error(SVTAD_ERR_INVALID, "remap_table: null pointer");
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(k_fill_i32, dim3(grid_for(batch * n_prev, 256)), dim3(256), 0, s, mapping_ws,
                       batch * n_prev, -1);
    hipLaunchKernelGGL(k_remap_scatter, dim3(grid_for(batch * n_new, 256)), dim3(256), 0, s,
                       keep_idx, batch, n_prev, n_new, mapping_ws);
    hipLaunchKernelGGL(k_remap_gather, dim3(grid_for(batch * n_new * 9, 256)), dim3(256), 0, s,
                       table, keep_idx, batch, n_prev, n_new, (const int32_t*)mapping_ws, out);
    return launch_status();
}

extern "C" int svtad_prune_step(const void* x, int64_t batch, int64_t n_key, int64_t n_prev,
                                int64_t row_bytes, const int64_t* keep_idx, int64_t n_new,
                                const int64_t* last_idx, const int32_t* table, int32_t* mapping_ws,
                                void* x_out, int64_t* idx_out, int32_t* table_out, void* stream) {
    if (batch < 0 || n_key < 0 || n_prev < 0 || n_new < 0 || n_new > n_prev || row_bytes < 0)
        return set_error(SVTAD_ERR_INVALID, "prune_step: bad sizes");
    if (batch * (n_key + n_prev) >= (int64_t)INT32_MAX)
        return set_error(SVTAD_ERR_UNSUPPORTED, "prune_step: more than 2^31-1 rows");
    const int64_t rows_out = batch * (n_key + n_new);
    if (batch * n_new == 0) {
        // nothing kept: no index or table output (their buffers may be empty)
        last_idx = nullptr, idx_out = nullptr, table = nullptr, table_out = nullptr;
    } else if ((last_idx == nullptr) != (idx_out == nullptr) ||
               (table == nullptr) != (table_out == nullptr) || (table && !mapping_ws)) {
        return set_error(SVTAD_ERR_INVALID,
                         "prune_step: last_idx/idx_out and table/table_out/mapping_ws go together");
    }
    if (rows_out == 0) return SVTAD_OK;
    if (!keep_idx || (row_bytes > 0 && (!x || !x_out)))
        return set_error(SVTAD_ERR_INVALID, "prune_step: null pointer");
    hipStream_t s = (hipStream_t)stream;
    if (table)
        hipLaunchKernelGGL(k_fill_i32, dim3(grid_for(batch * n_prev, 256)), dim3(256), 0, s, mapping_ws,
                           batch * n_prev, -1);
    // widest chunk that divides the row and both base addresses
    const uintptr_t al = (uintptr_t)x | (uintptr_t)x_out | (uintptr_t)row_bytes;
    const int64_t work_rows = row_bytes > 0 ? rows_out : 0;
    int32_t* map = table ? mapping_ws : nullptr;
    const unsigned g = grid_for(cdiv(rows_out, (int64_t)4), 1);
    if (work_rows == 0) {
        // no row bytes: only the index bookkeeping and the mapping
        hipLaunchKernelGGL((k_prune_rows<uint8_t>), dim3(g), dim3(256), 0, s, (const uint8_t*)nullptr,
                           batch, n_key, n_prev, (int64_t)0, keep_idx, n_new, last_idx, map,
                           (uint8_t*)nullptr, idx_out);
    } else if ((al & 15) == 0) {
        hipLaunchKernelGGL((k_prune_rows<uint4>), dim3(g), dim3(256), 0, s, (const uint4*)x, batch, n_key,
                           n_prev, row_bytes / 16, keep_idx, n_new, last_idx, map, (uint4*)x_out, idx_out);
    } else if ((al & 3) == 0) {
        hipLaunchKernelGGL((k_prune_rows<uint32_t>), dim3(g), dim3(256), 0, s, (const uint32_t*)x, batch,
                           n_key, n_prev, row_bytes / 4, keep_idx, n_new, last_idx, map,
                           (uint32_t*)x_out, idx_out);
    } else {
        hipLaunchKernelGGL((k_prune_rows<uint8_t>), dim3(g), dim3(256), 0, s, (const uint8_t*)x, batch,
                           n_key, n_prev, row_bytes, keep_idx, n_new, last_idx, map, (uint8_t*)x_out,
                           idx_out);
    }
    if (table)
        hipLaunchKernelGGL(k_remap_gather, dim3(grid_for(batch * n_new * 9, 256)), dim3(256), 0, s,
                           table, keep_idx, batch, n_prev, n_new, (const int32_t*)mapping_ws, table_out);
    return launch_status();
}

extern "C" int svtad_transpose_table(const int32_t* table, int64_t n, int64_t tokens_per_batch,
                                     int32_t* table_t, int32_t* collisions, void* stream) {
    if (n < 0 || tokens_per_batch < 0 || (n > 0 && (!table || !table_t || !collisions)))
        return set_error(SVTAD_ERR_INVALID, "transpose_table: bad arguments");
    if (n >= (int64_t)INT32_MAX)
        return set_error(SVTAD_ERR_UNSUPPORTED, "transpose_table: more than 2^31-1 rows");
    if (n == 0) return SVTAD_OK;
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(k_fill_i32, dim3(grid_for(n * 9, 256)), dim3(256), 0, s, table_t, n * 9, -1);
    hipLaunchKernelGGL(k_transpose_scatter, dim3(grid_for(n * 9, 256)), dim3(256), 0, s, table, n,
                       tokens_per_batch, table_t, collisions);
    return launch_status();
}

extern "C" int svtad_validate_table(const int32_t* table, int64_t n_entries, int64_t bound,
                                    int32_t* stats, void* stream) {
    if (n_entries < 0 || !stats || (n_entries > 0 && !table))
        return set_error(SVTAD_ERR_INVALID, "validate_table: bad arguments");
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(k_validate_init, dim3(1), dim3(1), 0, s, stats);
    if (n_entries > 0)
        hipLaunchKernelGGL(k_validate, dim3(grid_for(n_entries, 256 * 8)), dim3(256), 0, s, table,
                           n_entries, bound, stats);
    return launch_status();
}
