// Neighbor-index table kernels: build from a keep mask, remap after a prune,
// transpose, validate. Integer work; every output is bit-exact with the
// reference procedures (see the citations at each entry point).
#include <algorithm>

#include "sv_common.h"
#include "sv_internal.h"
#include "sv_mfma.h"

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

// ---------------------------------------------------------------------------
// one-launch builds: the table from a mask with a known row count (no host
// synchronisation), the full-grid table in closed form, and the
// local -> global conversion behind the tokens_per_batch heuristic
// ---------------------------------------------------------------------------

// Nonzero bytes of a 32-bit word: bit 7 of each byte is set iff the byte is
// nonzero ((b & 0x7f) + 0x7f carries into bit 7 unless b & 0x7f == 0; OR b
// adds b's own bit 7).
__device__ __forceinline__ int nonzero_bytes(uint32_t v) {
    return __popc((((v & 0x7f7f7f7fu) + 0x7f7f7f7fu) | v) & 0x80808080u);
}

// Workgroup g owns frames [g * fpw, (g + 1) * fpw). It counts the kept cells
// of every frame before its range itself (16-byte reads of the mask; mask is
// 16-byte aligned), which gives the rank of its first row without a scan
// launch; then per frame it ranks the cells in LDS (rank of each cell,
// cell of each rank) and writes the frame's rows entry by entry, so that
// consecutive threads store consecutive table entries. Rows at or past n_rows
// are not written; the workgroup that owns the last frame fills rows
// [total, n_rows) with -1 when the mask keeps fewer than n_rows cells.
template <typename I>
__global__ __launch_bounds__(256) void k_table_build(const uint8_t* __restrict__ mask, int64_t n_frames, int h,
                                                     int w, int fpw, int64_t n_rows, I* __restrict__ table) {
    extern __shared__ int16_t lds16[];
    int16_t* const rank_s = lds16;              // cells entries: rank of the cell in its frame, -1 if dropped
    int16_t* const cell_of = lds16 + h * w;     // cells entries: cell of each rank
    __shared__ int32_t wsum[4];
    __shared__ int32_t base_s;
    const int cells = h * w;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int64_t f0 = (int64_t)blockIdx.x * fpw;
    const int64_t f1 = min<int64_t>(n_frames, f0 + fpw);

    // kept cells before the range, eight 16-byte reads per thread in flight
    // at a time (buffer loads: a read past the prefix returns zeros, so the
    // batch has no branch; one read and its wait per iteration made the last
    // workgroup of a 160-frame mask wait for eight dependent rounds), plus
    // the prefix's last pre_bytes % 16 bytes
    const int pre_bytes = (int)(f0 * cells);  // < 4 MiB (host limit)
    const int nvec = pre_bytes / 16;
    const rsrc_t rm = make_rsrc(mask, (uint32_t)nvec * 16u);
    const int tail = nvec * 16 + tid;
    // the first 256 cells of the first frame, read with the prefix
    const rsrc_t rf = make_rsrc(mask, (uint32_t)(n_frames * cells));
    const bool first_kept = __builtin_amdgcn_raw_buffer_load_b8(
                                rf, f0 < f1 && tid < cells ? (uint32_t)(pre_bytes + tid) : kOOB, 0, 0) != 0;
    int cnt = 0;
    auto batch = [&](int c0, bool with_tail) {
        u32x4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = c0 + u * 256 + tid;
            v[u] = bload16(rm, c < nvec ? (uint32_t)c * 16u : kOOB);
        }
        if (with_tail)
            cnt += __builtin_amdgcn_raw_buffer_load_b8(make_rsrc(mask, (uint32_t)pre_bytes),
                                                       tail < pre_bytes ? (uint32_t)tail : kOOB, 0, 0) != 0;
#pragma unroll
        for (int u = 0; u < 8; ++u)
            cnt += nonzero_bytes(v[u][0]) + nonzero_bytes(v[u][1]) + nonzero_bytes(v[u][2]) + nonzero_bytes(v[u][3]);
    };
    batch(0, true);  // the whole prefix of masks up to 2048 x 16 bytes
    for (int c0 = 256 * 8; c0 < nvec; c0 += 256 * 8) batch(c0, false);
    for (int o = 32; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o, 64);
    if (tid == 0) base_s = 0;
    __syncthreads();
    if (lane == 0) atomicAdd(&base_s, cnt);
    __syncthreads();
    int64_t base = base_s;

    for (int64_t f = f0; f < f1; ++f) {
        const uint8_t* m = mask + f * cells;
        int kept_total = 0;
        for (int b0 = 0; b0 < cells; b0 += 256) {
            const int p = b0 + tid;
            const bool kept = f == f0 && b0 == 0 ? first_kept : p < cells && m[p] != 0;
            const uint64_t bal = __ballot(kept);
            const int before = __popcll(bal & ((1ull << lane) - 1ull));
            if (lane == 0) wsum[wid] = __popcll(bal);
            __syncthreads();
            int pre = kept_total;
            for (int q = 0; q < wid; ++q) pre += wsum[q];
            if (p < cells) {
                rank_s[p] = (int16_t)(kept ? pre + before : -1);
                if (kept) cell_of[pre + before] = (int16_t)p;
            }
            kept_total += wsum[0] + wsum[1] + wsum[2] + wsum[3];
            __syncthreads();
        }
        for (int e = tid; e < kept_total * 9; e += 256) {
            const int r = e / 9, k = e - r * 9;
            const int64_t row = base + r;
            if (row >= n_rows) break;  // rows grow with e
            const int p = cell_of[r];
            const int y = p / w, x = p - y * w;
            const int yy = y + k / 3 - 1, xx = x + k % 3 - 1;
            I v = -1;
            if (yy >= 0 && yy < h && xx >= 0 && xx < w) {
                const int rq = rank_s[yy * w + xx];
                if (rq >= 0) v = (I)(base + rq);
            }
            table[row * 9 + k] = v;
        }
        base += kept_total;
        __syncthreads();  // the next frame overwrites the rank arrays
    }
    if (f1 >= n_frames)
        for (int64_t e = base * 9 + tid; e < n_rows * 9; e += 256) table[e] = (I)-1;
}

// Full-grid table (every cell kept) in closed form: row i = f * h * w + y * w
// + x, entry k -> i + (dy * w + dx) when (y + dy, x + dx) is in the frame,
// else -1 (get_initial_neighbor_indices, vit_sparse_adapter_poguise.py:
// 1623-1670). One thread per entry, consecutive entries per thread block;
// the entry index and the divisions by 9, h * w and w in E (uint32_t when
// the table has fewer than 2^32 entries: a 64-bit division is a long
// software sequence on the GPU).
template <typename I, typename E>
__global__ __launch_bounds__(256) void k_table_grid(E n_entries, E h, E w, I* __restrict__ table) {
    const E cells = h * w;
    for (E e = blockIdx.x * (E)256 + threadIdx.x; e < n_entries; e += (E)gridDim.x * 256) {
        const E row = e / 9;
        const int k = (int)(e - row * 9);
        const E p = row % cells;
        const E y = p / w, x = p - y * w;
        const int dy = k / 3 - 1, dx = k % 3 - 1;
        const bool in = (dy >= 0 || y > 0) && (dy <= 0 || y + 1 < h) && (dx >= 0 || x > 0) && (dx <= 0 || x + 1 < w);
        table[e] = in ? (I)((int64_t)row + dy * (int64_t)w + dx) : (I)-1;
    }
}

// The reference wrapper's heuristic (sparse_conv_layer.py:170-177) without the
// host sync: with *vmax (the table's max, on the device) < tpb the entries are
// local to their batch and get the row's batch offset (i / tpb) * tpb, else
// they are global already. Negative entries and values past the int32 range
// become -1 (missing). Output int32.
template <typename I>
__global__ __launch_bounds__(256) void k_table_to_global(const I* __restrict__ in, int64_t n_entries,
                                                         int64_t tpb, const I* __restrict__ vmax,
                                                         int32_t* __restrict__ out) {
    const bool local = (int64_t)*vmax < tpb;
    for (int64_t e = blockIdx.x * (int64_t)256 + threadIdx.x; e < n_entries; e += (int64_t)gridDim.x * 256) {
        const int64_t v = (int64_t)in[e];
        int64_t o = v;
        if (v >= 0 && local) o += ((e / 9) / tpb) * tpb;
        out[e] = (v < 0 || o > (int64_t)INT32_MAX) ? -1 : (int32_t)o;
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

// the largest mask the one-launch build reads as prefix counts (each
// workgroup re-reads the mask before its frames); larger masks take the
// scan + fill launches
constexpr int64_t kBuildOneLaunchMaskBytes = (int64_t)4 << 20;

extern "C" int svtad_table_build(const uint8_t* mask, int64_t n_frames, int h, int w, int64_t n_rows, void* table,
                                 int index_bits, void* stream) {
    if (n_frames < 0 || h <= 0 || w <= 0 || n_rows < 0 || (index_bits != 32 && index_bits != 64))
        return set_error(SVTAD_ERR_INVALID, "table_build: bad arguments");
    if ((int64_t)h * w > kMaxFrameCells)
        return set_error(SVTAD_ERR_UNSUPPORTED, "table_build: h*w exceeds 16384 cells");
    if (n_frames * (int64_t)h * w >= (int64_t)INT32_MAX || n_rows >= (int64_t)INT32_MAX)
        return set_error(SVTAD_ERR_UNSUPPORTED, "table_build: more than 2^31-1 cells or rows");
    if (n_frames * (int64_t)h * w > kBuildOneLaunchMaskBytes)
        return set_error(SVTAD_ERR_UNSUPPORTED, "table_build: mask larger than 4 MiB (use svtad_table_scan / svtad_table_fill)");
    if (n_rows == 0) return SVTAD_OK;
    if (!table || (n_frames > 0 && !mask)) return set_error(SVTAD_ERR_INVALID, "table_build: null pointer");
    if (((uintptr_t)mask & 15) != 0) return set_error(SVTAD_ERR_INVALID, "table_build: mask must be 16-byte aligned");
    const int64_t groups_max = 256;
    const int fpw = (int)std::max<int64_t>(1, cdiv(n_frames, groups_max));
    const int64_t groups = std::max<int64_t>(1, cdiv(n_frames, fpw));
    const size_t lds = 2 * sizeof(int16_t) * (size_t)h * w;
    hipStream_t s = (hipStream_t)stream;
    if (index_bits == 32)
        hipLaunchKernelGGL(k_table_build<int32_t>, dim3((unsigned)groups), dim3(256), lds, s, mask, n_frames, h, w,
                           fpw, n_rows, (int32_t*)table);
    else
        hipLaunchKernelGGL(k_table_build<int64_t>, dim3((unsigned)groups), dim3(256), lds, s, mask, n_frames, h, w,
                           fpw, n_rows, (int64_t*)table);
    return launch_status();
}

extern "C" int svtad_table_grid(int64_t n_frames, int h, int w, void* table, int index_bits, void* stream) {
    if (n_frames < 0 || h <= 0 || w <= 0 || (index_bits != 32 && index_bits != 64))
        return set_error(SVTAD_ERR_INVALID, "table_grid: bad arguments");
    const int64_t rows = n_frames * (int64_t)h * w;
    if (rows >= (int64_t)INT32_MAX) return set_error(SVTAD_ERR_UNSUPPORTED, "table_grid: more than 2^31-1 rows");
    if (rows == 0) return SVTAD_OK;
    if (!table) return set_error(SVTAD_ERR_INVALID, "table_grid: null pointer");
    hipStream_t s = (hipStream_t)stream;
    const int64_t entries = rows * 9;
    const dim3 grid(grid_for(entries, 256));
    if (entries <= (int64_t)UINT32_MAX - (int64_t)grid.x * 256) {  // the loop's e + stride stays in 32 bits
        const uint32_t ne = (uint32_t)entries, hh = (uint32_t)h, ww = (uint32_t)w;
        if (index_bits == 32)
            hipLaunchKernelGGL((k_table_grid<int32_t, uint32_t>), grid, dim3(256), 0, s, ne, hh, ww, (int32_t*)table);
        else
            hipLaunchKernelGGL((k_table_grid<int64_t, uint32_t>), grid, dim3(256), 0, s, ne, hh, ww, (int64_t*)table);
    } else {
        if (index_bits == 32)
            hipLaunchKernelGGL((k_table_grid<int32_t, int64_t>), grid, dim3(256), 0, s, entries, (int64_t)h,
                               (int64_t)w, (int32_t*)table);
        else
            hipLaunchKernelGGL((k_table_grid<int64_t, int64_t>), grid, dim3(256), 0, s, entries, (int64_t)h,
                               (int64_t)w, (int64_t*)table);
    }
    return launch_status();
}

extern "C" int svtad_table_to_global(const void* table, int index_bits, int64_t n_rows, int64_t tokens_per_batch,
                                     const void* table_max, int32_t* out, void* stream) {
    if (n_rows < 0 || tokens_per_batch < 0 || (index_bits != 32 && index_bits != 64))
        return set_error(SVTAD_ERR_INVALID, "table_to_global: bad arguments");
    if (n_rows == 0) return SVTAD_OK;
    if (!table || !table_max || !out) return set_error(SVTAD_ERR_INVALID, "table_to_global: null pointer");
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid(grid_for(n_rows * 9, 256));
    if (index_bits == 32)
        hipLaunchKernelGGL(k_table_to_global<int32_t>, grid, dim3(256), 0, s, (const int32_t*)table, n_rows * 9,
                           tokens_per_batch, (const int32_t*)table_max, out);
    else
        hipLaunchKernelGGL(k_table_to_global<int64_t>, grid, dim3(256), 0, s, (const int64_t*)table, n_rows * 9,
                           tokens_per_batch, (const int64_t*)table_max, out);
    return launch_status();
}
