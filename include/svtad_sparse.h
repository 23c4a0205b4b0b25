/*
 * svtad_sparse.h — C ABI of the MI355X (gfx950) SparseConv2D library
 * (libsvtad_sparse.so).
 *
 * This is the drop-in boundary under the `opentad_sparse_ops` Python module.
 * Each entry point below names the reference interface it replaces
 * (paths relative to the pcr-upm/eccv26_tad repository root):
 *   2d_sparse_v3_bind.cpp = opentad/models/bricks/2d_sparse_v3_bind.cpp
 *   2d_sparse_v3.cu       = opentad/models/bricks/2d_sparse_v3.cu
 *   implicit_gemm_v2.cu   = opentad/models/bricks/implicit_gemm_v2.cu
 *   sparse_conv_layer.py  = opentad/models/bricks/sparse_conv_layer.py
 *   poguise.py            = opentad/models/backbones/vit_sparse_adapter_poguise.py
 *
 * Conventions
 *   - Every pointer argument is device memory, except where marked "host".
 *     Buffers are owned by the caller and 16-byte aligned; the library
 *     allocates nothing.
 *   - `stream` is a hipStream_t (NULL = the null stream). Every kernel of a
 *     call is enqueued on it; calls do not synchronise.
 *   - Tensors are dense row-major: x [n, c_in], out [n, c_out],
 *     nbr [n, 9] int32, weight [9, c_in, c_out] with k = ky*3 + kx
 *     (sparse_conv_layer.py:136,150-156), depthwise weight [9, c].
 *   - Neighbor entries: -1 = missing; otherwise the source row is
 *     nbr[i*9+k] + off(i), off(i) = (i / tokens_per_batch) * tokens_per_batch
 *     when tokens_per_batch > 0, else 0 (per-row rule, 2d_sparse_v3.cu:674-677).
 *     Any other negative entry, or a source row >= n, is treated as missing
 *     (the reference reads out of bounds there).
 *   - Return value: SVTAD_OK (0), a negative SVTAD_ERR_* for a rejected
 *     argument (message in svtad_last_error()), or a positive hipError_t from
 *     a kernel launch.
 *   - Accumulation is fp32 for f32/f16/bf16 and fp64 for f64; each output is
 *     rounded once to `dtype` (round-to-nearest-even).
 */
#ifndef SVTAD_SPARSE_H
#define SVTAD_SPARSE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum svtad_dtype { SVTAD_F32 = 0, SVTAD_F16 = 1, SVTAD_BF16 = 2, SVTAD_F64 = 3 };

enum svtad_status {
    SVTAD_OK = 0,
    SVTAD_ERR_INVALID = -1,      /* bad shape, dtype or pointer */
    SVTAD_ERR_WORKSPACE = -2,    /* workspace too small */
    SVTAD_ERR_UNSUPPORTED = -3   /* valid request this build does not handle */
};

/* bias_mode of svtad_fwd */
enum svtad_bias_mode {
    SVTAD_BIAS_NONE = 0,
    SVTAD_BIAS_FP32 = 1,   /* bias in the accumulator type (float32; float64 for
                              SVTAD_F64) added before rounding
                              (implicit_gemm_v2.cu:153-159, 291-294) */
    SVTAD_BIAS_AFTER = 2,  /* bias in `dtype`, added after rounding the conv to
                              dtype, then rounded again: `output += bias`
                              (sparse_conv_layer.py:86-87) */
    SVTAD_BIAS_PRE = 3     /* bias in `dtype`, widened exactly to the accumulator
                              type and added before rounding: the same result as
                              SVTAD_BIAS_FP32 given bias.to(float32)
                              (implicit_gemm_v2.cu:290-297) without the conversion */
};

/*
 * table_flags of the *_ex backward entry points (no counterpart in the
 * reference, which checks nothing: its backward-input scatters every entry).
 *   SVTAD_TABLE_SYMMETRIC: the caller promises that every entry
 *     (i, k) -> j has its partner (j, 8-k) -> i. Every table built from a
 *     keep mask has this property (svtad_table_build, svtad_table_grid,
 *     svtad_table_fill), and svtad_remap_table / svtad_prune_step /
 *     svtad_table_to_global keep it. The backward-input kernels then load no
 *     partners and no pass for entries without one runs. Results are
 *     identical to the unflagged call's for such tables; for a table without
 *     the property they are wrong (every access stays in bounds).
 */
enum svtad_table_flags { SVTAD_TABLE_SYMMETRIC = 1 };

/* Message of the last SVTAD_ERR_* returned on this host thread. */
const char* svtad_last_error(void);
const char* svtad_version(void);

/* Workspace bytes svtad_fwd / svtad_bwd_in need for this shape (0: none).
 * For f16/bf16 matrix-core shapes it holds the weight re-laid out in the
 * order the matrix-core operand fragments are read. */
size_t svtad_fwd_workspace_bytes(int c_in, int c_out, int dtype);
size_t svtad_bwd_in_workspace_bytes(int c_in, int c_out, int dtype);

/*
 * Forward SparseConv2D: out[i,co] = sum_k sum_ci x[src(i,k),ci] * w[k,ci,co]
 * (+ bias per bias_mode; bias may be NULL when mode = NONE).
 * Replaces `fwd` / launch_fwd (2d_sparse_v3_bind.cpp:9, 2d_sparse_v3.cu:751-822)
 * with SVTAD_BIAS_NONE, and `implicit_gemm_fwd_v2` / `implicit_gemm_fwd_v2_chunked`
 * (2d_sparse_v3_bind.cpp:12-13, implicit_gemm_v2.cu:197-300, 306-417) with
 * SVTAD_BIAS_FP32 / SVTAD_BIAS_PRE. Requires c_in % 4 == 0
 * (sparse_conv_layer.py:39-42). `workspace` must hold
 * svtad_fwd_workspace_bytes() bytes (may be NULL when that is 0).
 */
int svtad_fwd(const void* x, const int32_t* nbr, const void* weight, const void* bias,
              int bias_mode, void* out, void* workspace, size_t workspace_bytes, int64_t n,
              int c_in, int c_out, int64_t tokens_per_batch, int dtype, void* stream);

/*
 * Backward-input: gi[src(i,k),ci] += sum_co go[i,co] * w[k,ci,co], as a
 * scatter-free gather over the transposed table. The rows that receive an
 * entry whose transpose is not in the table ("one-way" entries; none in
 * tables built from a keep mask) are recomputed afterwards by one
 * workgroup, in fp32 with one rounding and a fixed order, so the result is
 * deterministic; with more than 2048 one-way entries they are added with
 * atomics instead (one rounding each, order unfixed).
 * Replaces `bwd_in` / launch_bwd_in (2d_sparse_v3_bind.cpp:10,
 * 2d_sparse_v3.cu:824-835). gi is fully written (no pre-zeroing needed).
 * `workspace` must hold svtad_bwd_in_workspace_bytes() bytes (may be NULL
 * when that is 0).
 */
int svtad_bwd_in(const void* grad_out, const int32_t* nbr, const void* weight, void* grad_in,
                 void* workspace, size_t workspace_bytes, int64_t n, int c_in, int c_out,
                 int64_t tokens_per_batch, int dtype, void* stream);

/*
 * Pre-packed weights (no counterpart in the reference; the autograd wrapper
 * packs once per forward and reuses the backward layout, where the entry
 * points above repack per call). svtad_pack_weight writes the weight
 * [9, c_in, c_out] in the order the matrix-core kernels read it: packed_fwd
 * holds svtad_fwd_workspace_bytes() bytes, packed_bwd
 * svtad_bwd_in_workspace_bytes(); either may be NULL. The packed entry points
 * compute exactly what svtad_fwd / svtad_bwd_in compute and return
 * SVTAD_ERR_UNSUPPORTED for shapes without a packed layout (both workspace
 * sizes 0). svtad_bwd_in_packed also takes the raw weight for table entries
 * whose transpose is absent.
 * The backward-input buffer (packed_bwd, and the svtad_bwd_in workspace) ends
 * with a 32-bit flag that the kernels maintain: svtad_pack_weight clears it,
 * the backward-input kernel sets it when the table holds an entry (i, k) -> j
 * without its partner (j, 8-k) -> i, and only then does the pass for such
 * entries do any work. packed_bwd is therefore written by
 * svtad_bwd_in_packed; calls that share one packed_bwd on one stream stay
 * correct (a set flag only costs the full pass), calls on different streams
 * must not share it.
 */
int svtad_pack_weight(const void* weight, void* packed_fwd, void* packed_bwd, int c_in, int c_out,
                      int dtype, void* stream);
int svtad_fwd_packed(const void* x, const int32_t* nbr, const void* packed_fwd, const void* bias,
                     int bias_mode, void* out, int64_t n, int c_in, int c_out,
                     int64_t tokens_per_batch, int dtype, void* stream);
int svtad_bwd_in_packed(const void* grad_out, const int32_t* nbr, const void* weight,
                        void* packed_bwd, void* grad_in, int64_t n, int c_in, int c_out,
                        int64_t tokens_per_batch, int dtype, void* stream);
/* svtad_bwd_in_packed with table_flags (svtad_table_flags; 0 = the same call). */
int svtad_bwd_in_packed_ex(const void* grad_out, const int32_t* nbr, const void* weight,
                           void* packed_bwd, void* grad_in, int64_t n, int c_in, int c_out,
                           int64_t tokens_per_batch, int dtype, unsigned table_flags, void* stream);

/*
 * Timing entry point (no counterpart in the reference): the gathered GEMM of
 * svtad_bwd_in_packed alone, without the launch of the pass for entries
 * whose symmetric partner is absent. grad_in equals svtad_bwd_in_packed's
 * for tables in which every entry has its partner (every table built from a
 * keep mask); the kernel still sets the flag in packed_bwd otherwise. For
 * measuring that kernel's duration by itself. One launch. table_flags as for
 * svtad_bwd_in_packed_ex.
 */
int svtad_bwd_in_gemm(const void* grad_out, const int32_t* nbr, void* packed_bwd, void* grad_in, int64_t n,
                      int c_in, int c_out, int64_t tokens_per_batch, int dtype, unsigned table_flags,
                      void* stream);

/*
 * Allocation-free forward. No counterpart in the reference: for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Computes exactly what svtad_fwd computes,
 * with its workspace (the packed weight) in a static device array of
 * svtad_fwd_noalloc_max_workspace_bytes() (8 MiB) that every GPU the library
 * runs on holds until the process ends; shapes whose svtad_fwd_workspace_bytes()
 * exceed it are rejected with SVTAD_ERR_UNSUPPORTED (square weights up to
 * C = 512 fit). Calls no hipMalloc/hipFree. All calls on one GPU share its
 * array: calls that overlap on one GPU (different streams, or host threads
 * without ordering) race. The first call on a device looks up the array's
 * device address (hipGetSymbolAddress); make that first call eagerly, before
 * a HIP graph capture of later calls on that device.
 */
size_t svtad_fwd_noalloc_max_workspace_bytes(void);
int svtad_fwd_noalloc(const void* x, const int32_t* nbr, const void* weight, const void* bias,
                      int bias_mode, void* out, int64_t n, int c_in, int c_out, int64_t tokens_per_batch,
                      int dtype, void* stream);

/*
 * The whole backward in one call: grad_in as svtad_bwd_in_packed computes it
 * and grad_w / grad_bias as svtad_bwd_w computes them (same kernels, same
 * results), with the pass for table entries without a symmetric partner run
 * inside the backward-weight reduction instead of a launch of its own.
 * Replaces the bwd_in + bwd_w pair the reference's autograd backward calls
 * (sparse_conv_layer.py:93-123, 2d_sparse_v3_bind.cpp:10-11). packed_bwd as for
 * svtad_bwd_in_packed; workspace holds svtad_bwd_w_workspace_bytes(); grad_w
 * must not be NULL (grad_bias may be). Returns SVTAD_ERR_UNSUPPORTED for shapes
 * without a packed backward-input layout.
 */
int svtad_bwd_packed(const void* grad_out, const void* x, const int32_t* nbr, const void* weight,
                     void* packed_bwd, void* grad_in, void* grad_w, void* grad_bias,
                     void* workspace, size_t workspace_bytes, int64_t n, int c_in, int c_out,
                     int64_t tokens_per_batch, int dtype, void* stream);
/* svtad_bwd_packed with table_flags (svtad_table_flags; 0 = the same call). */
int svtad_bwd_packed_ex(const void* grad_out, const void* x, const int32_t* nbr, const void* weight,
                        void* packed_bwd, void* grad_in, void* grad_w, void* grad_bias,
                        void* workspace, size_t workspace_bytes, int64_t n, int c_in, int c_out,
                        int64_t tokens_per_batch, int dtype, unsigned table_flags, void* stream);

/*
 * Where neither backward grid fills the GPU (C_in = C_out = 192 or 256, f16 /
 * bf16, low keep rates), svtad_bwd_packed runs backward-input and the
 * backward-weight partials in one launch. This host-only query (no GPU work)
 * returns 1 when it would (given 16-byte aligned grad_out, x, packed_bwd and
 * grad_in, which svtad_bwd_packed also needs for it), with the
 * backward-input tile shape (row fragments
 * of 16 rows, column fragments of 16 per wave) and the row-split count; 0
 * when the shape keeps two launches; SVTAD_ERR_INVALID for bad sizes or a bad
 * SVTAD_BWD_FUSED override ("off", "<rows>x<cols>[:<splits>]" with the shape
 * one of 3x1, 3x3, 4x3 at C = 192 or 3x2 at C = 256; read from the
 * environment on every call). It
 * describes how svtad_bwd_packed replaces the reference's two backward calls
 * (sparse_conv_layer.py:101-117); the reference has no such query.
 */
int svtad_bwd_fused_plan(int64_t n, int c_in, int c_out, int dtype, int* tile_row_frags, int* tile_col_frags,
                         int* splits);

/* Workspace bytes needed by svtad_bwd_w for this shape. */
size_t svtad_bwd_w_workspace_bytes(int64_t n, int c_in, int c_out, int dtype);

/*
 * Backward-weight: gw[k,ci,co] = sum_i go[i,co] * x[src(i,k),ci], as a
 * deterministic per-offset reduction (row-split fp32 partials in `workspace`,
 * then an ordered sum). If grad_bias is not NULL it also writes
 * grad_bias[co] = sum_i go[i,co] (sparse_conv_layer.py:120-121).
 * With grad_w == NULL only the row-split partial sums are written to the
 * workspace (for timing the partial-sum kernel alone; layout internal).
 * Replaces `bwd_w` / launch_bwd_w (2d_sparse_v3_bind.cpp:11, 2d_sparse_v3.cu:837-850).
 */
int svtad_bwd_w(const void* grad_out, const void* x, const int32_t* nbr, void* grad_w,
                void* grad_bias, void* workspace, size_t workspace_bytes, int64_t n, int c_in,
                int c_out, int64_t tokens_per_batch, int dtype, void* stream);

/*
 * Depthwise variant (groups = c), weight [9, c]. No counterpart in the
 * reference (SparseConv2d has no groups, sparse_conv_layer.py:126-141); same
 * index semantics as above. bias (dtype `dtype`) may be NULL; it is added to
 * the accumulator before rounding. Requires c % 4 == 0.
 */
int svtad_dw_fwd(const void* x, const int32_t* nbr, const void* weight, const void* bias,
                 void* out, int64_t n, int c, int64_t tokens_per_batch, int dtype, void* stream);
int svtad_dw_bwd_in(const void* grad_out, const int32_t* nbr, const void* weight, void* grad_in,
                    int64_t n, int c, int64_t tokens_per_batch, int dtype, void* stream);
/* svtad_dw_bwd_in with table_flags (svtad_table_flags; 0 = the same call). */
int svtad_dw_bwd_in_ex(const void* grad_out, const int32_t* nbr, const void* weight, void* grad_in,
                       int64_t n, int c, int64_t tokens_per_batch, int dtype, unsigned table_flags, void* stream);
size_t svtad_dw_bwd_w_workspace_bytes(int64_t n, int c, int dtype);
int svtad_dw_bwd_w(const void* grad_out, const void* x, const int32_t* nbr, void* grad_w,
                   void* grad_bias, void* workspace, size_t workspace_bytes, int64_t n, int c,
                   int64_t tokens_per_batch, int dtype, void* stream);
/*
 * Depthwise backward-input and backward-weight / bias in one call: one pass
 * over the rows computes grad_in and the row-split weight / bias partials
 * together (row i's table entries give both its gathered x rows and its
 * transposed go sources), and one reduction launch adds the partials in a
 * fixed order and runs the asymmetric-entry pass when the first pass met
 * such an entry. Results equal svtad_dw_bwd_in followed by svtad_dw_bwd_w.
 * grad_bias may be NULL. Workspace: svtad_dw_bwd_workspace_bytes(). Two
 * launches on `stream` (the two separate calls take four).
 */
size_t svtad_dw_bwd_workspace_bytes(int64_t n, int c, int dtype);
int svtad_dw_bwd(const void* grad_out, const void* x, const int32_t* nbr, const void* weight, void* grad_in,
                 void* grad_w, void* grad_bias, void* workspace, size_t workspace_bytes, int64_t n, int c,
                 int64_t tokens_per_batch, int dtype, void* stream);
/* svtad_dw_bwd with table_flags (svtad_table_flags; 0 = the same call). */
int svtad_dw_bwd_ex(const void* grad_out, const void* x, const int32_t* nbr, const void* weight, void* grad_in,
                    void* grad_w, void* grad_bias, void* workspace, size_t workspace_bytes, int64_t n, int c,
                    int64_t tokens_per_batch, int dtype, unsigned table_flags, void* stream);

/*
 * Neighbor table from a keep mask [n_frames, h, w] (uint8, nonzero = kept),
 * in two steps so the caller can size the table:
 *   1. svtad_table_scan writes frame_offsets[0..n_frames] (int32): the
 *      exclusive prefix count of kept cells per frame; frame_offsets[n_frames]
 *      is the total N.
 *   2. svtad_table_fill writes table [N, 9]: for the kept cell p with rank r,
 *      table[r,k] = rank(p + delta_k) if that cell is inside the frame and
 *      kept, else -1, with k = (dy+1)*3 + (dx+1).
 * For a full mask this is get_initial_neighbor_indices (poguise.py:1623-1670);
 * for a pruned mask with sorted keep lists it equals that table after the
 * Block remaps (poguise.py:913-977). Global indices (batch offsets included).
 * Requires h*w <= 16384 and n_frames*h*w < 2^31.
 */
int svtad_table_scan(const uint8_t* mask, int64_t n_frames, int h, int w, int32_t* frame_offsets,
                     void* stream);
int svtad_table_fill(const uint8_t* mask, const int32_t* frame_offsets, int64_t n_frames, int h,
                     int w, int32_t* table, void* stream);

/*
 * One-launch table builds, with no host synchronisation.
 *
 * svtad_table_build: the table svtad_table_scan + svtad_table_fill write,
 * for a caller that knows the row count N (the backbone's kept-token count,
 * e.g. B * ceil(r * T * h * w) after a top-k prune) and allocates
 * table [n_rows, 9] itself. Rows past the mask's kept count are -1; kept cells
 * past n_rows are not written. index_bits 32 (int32 entries,
 * vit_sparse_adapter_poguise.py) or 64 (int64, internvideo_next.py:1896-1945).
 * mask 16-byte aligned, at most 4 MiB (larger masks: scan + fill). One launch.
 *
 * svtad_table_grid: the full-grid table (every cell kept) in closed form,
 * table [n_frames * h * w, 9], as get_initial_neighbor_indices
 * (vit_sparse_adapter_poguise.py:1623-1670; int64 in internvideo_next.py).
 * One launch, no mask.
 *
 * svtad_table_to_global: the reference wrapper's tokens_per_batch heuristic
 * (sparse_conv_layer.py:170-177) on the device: with table_max (the table's
 * maximum entry, a device scalar of the table's type) < tokens_per_batch the
 * entries are per-sample (local) indices and each valid entry of row i gets
 * (i / tokens_per_batch) * tokens_per_batch added; otherwise they are copied.
 * Writes int32 out [n_rows, 9] (-1 for negative entries and values past the
 * int32 range), which every kernel then reads with tokens_per_batch = 0, the
 * same sources as the reference's tokens_per_batch = N. One launch.
 */
int svtad_table_build(const uint8_t* mask, int64_t n_frames, int h, int w, int64_t n_rows, void* table,
                      int index_bits, void* stream);
int svtad_table_grid(int64_t n_frames, int h, int w, void* table, int index_bits, void* stream);
int svtad_table_to_global(const void* table, int index_bits, int64_t n_rows, int64_t tokens_per_batch,
                          const void* table_max, int32_t* out, void* stream);

/*
 * Table remap after a prune (poguise.py:913-977; internvideo_next.py:1447-1492):
 * out[b*n_new+j, k] = mapping[table[b*n_prev + keep_idx[b,j], k]] for valid
 * entries, where mapping[b*n_prev + keep_idx[b,j]] = b*n_new + j and -1
 * elsewhere. keep_idx is int64 [B, n_new] (local indices into n_prev, as
 * returned by topk); mapping_ws holds B*n_prev int32.
 */
int svtad_remap_table(const int32_t* table, int64_t batch, int64_t n_prev, const int64_t* keep_idx,
                      int64_t n_new, int32_t* mapping_ws, int32_t* out, void* stream);

/*
 * Fused prune step of a Block (poguise.py:899-977; internvideo_next.py:1447-1492
 * for the table part), replacing the reference's gather / cat / gather /
 * fill / scatter / where sequence:
 *   x_out[b, :n_key]          = x[b, :n_key]                      (key tokens)
 *   x_out[b, n_key + j]       = x[b, n_key + keep_idx[b, j]]      (:901-910)
 *   idx_out[b, j]             = last_idx[b, keep_idx[b, j]]       (:908)
 *   table_out                 = svtad_remap_table(table, keep_idx) (:913-977)
 * x is [batch, n_key + n_prev] rows of row_bytes bytes (any element type),
 * x_out [batch, n_key + n_new] rows. last_idx / idx_out are int64 [batch,
 * n_prev] / [batch, n_new] and may both be NULL; table / table_out /
 * mapping_ws (batch*n_prev int32) may all be NULL (no table update, as when
 * the reference's neighbor_indices is None). With batch * n_new == 0 only the
 * key rows are written and the index / table pointers are ignored. A keep
 * index outside
 * [0, n_prev) gives a zero row, idx -1 and no mapping entry (the reference's
 * gather would raise). Two or three launches on `stream`.
 */
int svtad_prune_step(const void* x, int64_t batch, int64_t n_key, int64_t n_prev, int64_t row_bytes,
                     const int64_t* keep_idx, int64_t n_new, const int64_t* last_idx,
                     const int32_t* table, int32_t* mapping_ws, void* x_out, int64_t* idx_out,
                     int32_t* table_out, void* stream);

/*
 * Transposed table: table_t[j,k] = i for the entry with src(i,k) = j
 * (global indices), -1 where no entry maps there. When several entries map to
 * the same (j,k) one of them is kept and *collisions (device int32, caller
 * zeroes it) counts the others. For mask-built tables table_t[j,k] equals
 * table[j,8-k] and collisions stay 0.
 */
int svtad_transpose_table(const int32_t* table, int64_t n, int64_t tokens_per_batch,
                          int32_t* table_t, int32_t* collisions, void* stream);

/*
 * Table validation (the checks of _validate_neighbor_indices,
 * internvideo_next.py:41-70): stats[0] = number of entries that are neither
 * -1 nor in [0, bound), stats[1] = min and stats[2] = max over the entries
 * != -1 (INT32_MAX / INT32_MIN when there are none). stats is device int32[3];
 * the call initialises it.
 */
int svtad_validate_table(const int32_t* table, int64_t n_entries, int64_t bound, int32_t* stats,
                         void* stream);

/*
 * Adapter down projection with the GELU epilogue (the down_proj + act of the
 * sparse-conv adapter, vit_sparse_adapter_poguise.py:305-306, and the
 * special / patch split of :307-309):
 *   pre_act[m, :] = T(x[m, :] W^T + bias)                (nn.Linear, W [n, k])
 *   act[m, :]     = T(GELU(float(pre_act[m, :])))       (exact erf GELU)
 * x is [batch, n_tokens, k]; row r of sample b goes to act_special[b *
 * n_special + r] when r < n_special and to act_patch[b * (n_tokens -
 * n_special) + r - n_special] otherwise (the contiguous SparseConv2D input),
 * pre_act keeps the [batch, n_tokens, n] layout. bias may be NULL. f16 / bf16
 * only; k % 32 == 0, n % 64 == 0; x, weight and the outputs 16-byte aligned.
 * One launch on `stream`.
 */
int svtad_adapter_down(const void* x, const void* weight, const void* bias, void* pre_act,
                       void* act_special, void* act_patch, int64_t batch, int64_t n_tokens,
                       int64_t n_special, int k, int n, int dtype, void* stream);

/*
 * Adapter up projection with the scale-and-residual epilogue (the cat of
 * special tokens and SparseConv2D output, up_proj, gamma and residual of
 * vit_sparse_adapter_poguise.py:362,652-653):
 *   z[m, :]   = T(c[m, :] W^T + bias)       c = cat(a_special, a_patch) per sample
 *   out[m, :] = T(T(z * gamma[0]) + residual[m, :])
 * a_special [batch * n_special, k], a_patch [batch * (n_tokens - n_special), k]
 * are read in place of the concatenation; residual and out are [batch,
 * n_tokens, n]; gamma is one element of `dtype` on the device (no host read).
 * bias may be NULL. f16 / bf16 only; k % 32 == 0, n % 64 == 0; inputs,
 * weight, residual and out 16-byte aligned. One launch.
 */
int svtad_adapter_up(const void* a_special, const void* a_patch, const void* weight,
                     const void* bias, const void* gamma, const void* residual, void* out,
                     int64_t batch, int64_t n_tokens, int64_t n_special, int k, int n, int dtype,
                     void* stream);

/*
 * svtad_adapter_up with gamma, the residual and the output each in `dtype` or
 * in SVTAD_F32 (gamma_dtype, residual_dtype, out_dtype): the up projection of
 * the reference adapter under torch.autocast with float32 parameters
 * (opentad/cores/train_engine.py:672, vit_sparse_adapter_poguise.py:652-653),
 * where up_proj runs in the autocast dtype and `* self.gamma` promotes to
 * float32:
 *   z[m, :]   = T(c[m, :] W^T + bias)
 *   p         = float(z) * gamma[0]                 (gamma f32: fp32 product)
 *             = float(T(float(z) * gamma[0]))       (gamma of dtype)
 *   out[m, :] = p + float(residual[m, :])           (f32 out: stored as is;
 *                                                    out of dtype: rounded once)
 * An f32 residual or output needs an f32 gamma (with gamma, residual and out
 * all of `dtype` this is svtad_adapter_up). f32 residual and out rows are
 * n floats, 16-byte aligned. One launch.
 */
int svtad_adapter_up_mixed(const void* a_special, const void* a_patch, const void* weight,
                           const void* bias, const void* gamma, const void* residual, void* out,
                           int64_t batch, int64_t n_tokens, int64_t n_special, int k, int n, int dtype,
                           int gamma_dtype, int residual_dtype, int out_dtype, void* stream);

/*
 * A linear layer's weight gradient (the backward of the adapter's nn.Linear
 * layers, vit_sparse_adapter_poguise.py:305,652; PyTorch computes it as
 * grad_out^T @ input):
 *   out[i, j] = sum_{r < n} g[rows[r], i] * x[r, j]     (fp32 accumulation)
 * g has n_g_rows rows of c_g values (rows == NULL: row r of g, n_g_rows >= n),
 * x is [n, c_x], out [c_g, c_x] in `dtype`. The sum runs over row splits
 * whose fp32 partials (workspace, svtad_linear_wgrad_workspace_bytes) are
 * added in a fixed order, so the result is deterministic. f16 / bf16; c_g
 * and c_x need a tile configuration (multiples of 64 cover every case); g and
 * x 16-byte aligned. Two launches on `stream`.
 */
size_t svtad_linear_wgrad_workspace_bytes(int64_t n, int c_g, int c_x, int dtype);
int svtad_linear_wgrad(const void* g, const int32_t* rows, const void* x, void* out, void* workspace,
                       size_t workspace_bytes, int64_t n, int64_t n_g_rows, int c_g, int c_x, int dtype,
                       void* stream);
/* svtad_linear_wgrad with `out` in `dtype` or SVTAD_F32 (out_dtype): the
 * fp32 sums stored unrounded, for a caller that scales them before rounding
 * (the adapter's up projection, whose gradient the reference rounds once,
 * after the gamma scale). */
int svtad_linear_wgrad_mixed(const void* g, const int32_t* rows, const void* x, void* out, void* workspace,
                             size_t workspace_bytes, int64_t n, int64_t n_g_rows, int c_g, int c_x, int dtype,
                             int out_dtype, void* stream);

/*
 * Column sums out[c] = sum_r a[r, c] of a [rows, cols] matrix (the bias
 * gradient of a linear layer, vit_sparse_adapter_poguise.py:305,652), fp32
 * accumulation over 512-row splits added in a fixed order; out in `dtype`.
 * f16 / bf16, cols % 8 == 0, a 16-byte aligned. Two launches on `stream`.
 */
size_t svtad_column_sums_workspace_bytes(int64_t rows, int cols, int dtype);
int svtad_column_sums(const void* a, void* out, void* workspace, size_t workspace_bytes, int64_t rows, int cols,
                      int dtype, void* stream);

/*
 * GELU backward of the adapter's down projection, replacing the autograd of
 * nn.GELU plus the special / patch split (vit_sparse_adapter_poguise.py:305-309):
 *   grad_pre[m, c] = g(m, c) * (Phi(u) + u phi(u)),  u = pre_act[m, c],
 * with g read from grad_special [batch, n_special, n] for the first n_special
 * tokens of a sample and from grad_patch [batch * (n_tokens - n_special), n]
 * for the rest (NULL: zeros). pre_act and grad_pre are [batch, n_tokens, n].
 * fp32 evaluation, one rounding. f16 / bf16, n % 8 == 0, 16-byte aligned
 * buffers. One launch on `stream`.
 */
int svtad_gelu_backward_split(const void* grad_special, const void* grad_patch, const void* pre_act,
                              void* grad_pre, int64_t batch, int64_t n_tokens, int64_t n_special, int n,
                              int dtype, void* stream);

/*
 * Heatmap injection of the adapter, the forward of
 *   patch_tokens_proj + gather(heatmap_tokens, cell) * heatmap_gate
 * (vit_sparse_adapter_poguise.py:311-355), in place on the SparseConv2D input:
 *   patch[i, c] = T(patch[i, c] + T(special[src_rows[i], c] * gate[0]))
 * patch [rows, cols] (the patch tokens after down_proj + GELU), special
 * [n_special_rows, cols] (the special tokens of every sample, flattened),
 * src_rows int32 [rows]: the special row of the heatmap cell each patch token
 * samples (b * S + 1 + cell); rows whose entry is outside [0, n_special_rows)
 * are left unchanged. gate: one element (device). The products and sums are
 * rounded to `dtype` as in the unfused chain. f16 / bf16, cols % 8 == 0,
 * patch and special 16-byte aligned. One launch on `stream`.
 */
int svtad_heatmap_add(void* patch, const void* special, const int32_t* src_rows, const void* gate,
                      int64_t rows, int64_t n_special_rows, int cols, int dtype, void* stream);

/*
 * svtad_heatmap_add with the gate in `dtype` or SVTAD_F32 (gate_dtype). An
 * f32 gate is the reference chain under torch.autocast with float32
 * parameters (vit_sparse_adapter_poguise.py:355), where `sampled * gate` and
 * the add are float32 and SparseConv2d casts the sum to the autocast dtype
 * (sparse_conv_layer.py:191-202):
 *   patch[i, c] = T(float(patch[i, c]) + float(special[src_rows[i], c]) * gate[0])
 * One launch on `stream`.
 */
int svtad_heatmap_add_mixed(void* patch, const void* special, const int32_t* src_rows, const void* gate,
                            int64_t rows, int64_t n_special_rows, int cols, int dtype, int gate_dtype,
                            void* stream);

/*
 * Gradient of the adapter's gamma, replacing the autograd of `* self.gamma`
 * (vit_sparse_adapter_poguise.py:652-653): out[0] = sum_i w[i] g[i] +
 * sum_j b[j] gs[j], with w the up projection's weight, g = go^T c its
 * unscaled weight gradient, b its bias (NULL: none) and gs the column sums of
 * go. fp32 accumulation over 64 slices added in a fixed order, out (one
 * element) in `dtype`. With gamma (one element, device) the same pass writes
 * the scaled copies the up projection's backward uses in place of three
 * elementwise multiplies: w_scaled = w * gamma (for the input gradient),
 * g_scaled = g * gamma (the weight gradient), gs_scaled = gs * gamma (the
 * bias gradient); NULL skips one. f16 / bf16; counts multiples of 8; 16-byte
 * aligned; workspace of svtad_gamma_grad_workspace_bytes(). Two launches on
 * `stream`.
 */
size_t svtad_gamma_grad_workspace_bytes(void);
int svtad_gamma_grad(const void* w, const void* g, int64_t count, const void* b, const void* gs,
                     int64_t count_b, void* out, const void* gamma, void* w_scaled, void* g_scaled,
                     void* gs_scaled, void* workspace, size_t workspace_bytes, int dtype, void* stream);

/*
 * svtad_gamma_grad with g in `dtype` or SVTAD_F32 (g_dtype) and gamma in
 * `dtype` or SVTAD_F32 (gamma_dtype). An f32 g is the unrounded weight
 * gradient (svtad_linear_wgrad_mixed with an f32 output): the dot products
 * use it as is and g_scaled = T(g * gamma) is its single rounding, as the
 * reference rounds that gradient once. An f32 gamma is the float32 gamma of
 * the reference's autocast training (vit_sparse_adapter_poguise.py:652-653):
 * `out` (one element) is written in gamma_dtype. The other scaled copies
 * stay in `dtype`, each an fp32 product rounded once. Two launches.
 */
int svtad_gamma_grad_mixed(const void* w, const void* g, int64_t count, const void* b, const void* gs,
                           int64_t count_b, void* out, const void* gamma, void* w_scaled, void* g_scaled,
                           void* gs_scaled, void* workspace, size_t workspace_bytes, int dtype, int g_dtype,
                           int gamma_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SVTAD_SPARSE_H */
