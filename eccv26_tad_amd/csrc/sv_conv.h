// Internal interface between the C-ABI dispatch (conv.hip) and the kernel
// files (conv_valu.hip, conv_mfma.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

namespace svtad {

enum { MODE_FWD = 0, MODE_BWDIN = 1 };

// Row-split plan of a backward-weight reduction. Partials are stored as
// [splits][9][c_in][c_out] (+ [splits][c_out] for the bias) in the
// accumulator type.
struct BwPlan {
    int path;                 // 0 = VALU, 1 = MFMA
    int splits;
    int64_t rows_per_split;
    size_t ws_bytes;
};

// gathered GEMM on the VALU (any dtype)
void gg_valu(int dtype, int mode, const void* src, const int32_t* nbr, const void* w,
             const void* bias, int bias_mode, void* out, int64_t n, int c_red, int n_out,
             int64_t tpb, hipStream_t s);
// Backward-input contributions of table entries (i, k) -> j whose symmetric
// partner (j, 8-k) -> i is absent (the gathered kernels cannot see them),
// added with atomics. With a non-NULL flag the pass returns at once when the
// flag is 0 (the wide backward-input kernel sets it when it meets such an
// entry; the pack kernels clear it).
void orphans(int dtype, bool dw, const void* go, const int32_t* nbr, const void* w, void* gi,
             int64_t n, int c_in, int c_out, int64_t tpb, const uint32_t* flag, hipStream_t s);
void bw_valu(int dtype, const BwPlan& p, const void* go, const void* x, const int32_t* nbr,
             void* gw, void* gb, void* ws, int64_t n, int c_in, int c_out, int64_t tpb,
             hipStream_t s);
// sym (backward-input only): every entry has its partner, so the vectorized
// kernel loads no partners.
void dw_gather(int dtype, int mode, const void* src, const int32_t* nbr, const void* w,
               const void* bias, void* out, int64_t n, int c, int64_t tpb, hipStream_t s, bool sym = false);
void dw_bw(int dtype, const BwPlan& p, const void* go, const void* x, const int32_t* nbr, void* gw,
           void* gb, void* ws, int64_t n, int c, int64_t tpb, hipStream_t s);
// Depthwise backward-input and backward-weight / bias in one pass over the
// rows plus one reduction launch (which also runs the orphan pass when a
// split's flag word says so). ws holds the [splits][10][c] partials, flags
// one word per split. Returns false (nothing launched) when the vectorized
// kernels do not apply. sym: every entry has its partner (no partner loads;
// the flag words stay 0).
bool dw_bwd_fused(int dtype, const BwPlan& p, const void* go, const void* x, const int32_t* nbr, const void* w,
                  void* gi, void* gw, void* gb, void* ws, uint32_t* flags, int64_t n, int c, int64_t tpb,
                  hipStream_t s, bool sym = false);

// out[e] = T(sum_s part[s][e]) for e < count; partials in the accumulator type.
void split_reduce(int dtype, const void* part, int64_t count, int splits, void* out, hipStream_t s);

// MFMA path (f16 / bf16). Returns false when the shape is not handled, so the
// caller falls back to the VALU kernels.
bool gg_mfma_supported(int dtype, int c_red, int n_out);
// Workspace (the weight in MFMA fragment order) a gathered GEMM with
// reduction width c_red and n_out columns needs; 0 when the shape takes a
// kernel that reads w directly.
size_t gg_mfma_workspace(int dtype, int c_red, int n_out);
// The backward-input packed weight is followed by this many bytes holding the
// 32-bit orphan flag (see orphans).
constexpr size_t kOrphanFlagBytes = 256;
// w is the raw weight (ws holds room for its packed form, packed here) or,
// with prepacked, the fragment-ordered weight itself. For the backward-input
// mode, orphan_flag (may be NULL) is the flag word after the packed weight;
// the return value says whether the kernel that ran maintains it (if not,
// the orphan pass must run without the flag). sym is the caller's promise that
// every table entry (i, 8-k) -> p has its partner (p, k) -> i, as in every
// table built from a keep mask: the backward-input wide kernel then loads no
// partners (and never arms the flag).
bool gg_mfma(int dtype, int mode, const void* src, const int32_t* nbr, const void* w,
             const void* bias, int bias_mode, void* out, int64_t n, int c_red, int n_out,
             int64_t tpb, void* ws, bool prepacked, uint32_t* orphan_flag, hipStream_t s, bool sym = false);
// Whether the fragment-ordered (prepacked) entry points handle this shape.
bool gg_mfma_packed_ok(int dtype, int64_t n, int c_red, int n_out);
// Fragment-ordered weights for the forward (wf_fwd) and backward-input
// (wf_bwd) gathered GEMMs, one launch; either may be NULL. Clears the orphan
// flag after wf_bwd.
void pack_weight(const void* w, void* wf_fwd, void* wf_bwd, int c_in, int c_out, hipStream_t s);
bool bw_mfma_supported(int dtype, int64_t n, int c_in, int c_out);
// Rows per split of the MFMA backward-weight (its row list lives in LDS).
constexpr int kMaxSplitRows = 4096;
// compute units of the current device (256 on MI355X)
int cu_count();
int bw_mfma_tile(int c);
// (ci, co) tile edges of the MFMA backward-weight kernel chosen for a shape;
// true for the large-tile kernel, whose splits hold 10 work units (the 8
// off-center offsets over the split's rows, the center offset over each half)
// and whose rows_per_split is a multiple of 256.
bool bw_mfma_tiles(int c_in, int c_out, int* tm, int* tn);
// Orphan pass handed to the backward-weight reduction (one launch less when
// the backward-input and backward-weight run together): flag as for orphans
// (NULL: always run).
struct OrphanJob {
    const void* go;
    const int32_t* nbr;
    const void* w;
    void* gi;
    int64_t n;
    int c_in, c_out;
    int64_t tpb;
    const uint32_t* flag;
};
// Returns SVTAD_OK, or an SVTAD_ERR_* (message set, nothing launched) when
// the plan or the workspace (ws_bytes) does not fit what the kernels assume.
// *oj_taken says whether oj (may be NULL) was run by the reduction; false
// leaves it to the caller (gw NULL or a shape without the large-tile
// reduction).
int bw_mfma(int dtype, const BwPlan& p, const void* go, const void* x, const int32_t* nbr,
            void* gw, void* gb, void* ws, size_t ws_bytes, int64_t n, int c_in, int c_out, int64_t tpb,
            const OrphanJob* oj, bool* oj_taken, hipStream_t s);

// Backward-input and the backward-weight partials in one launch, then the
// ordered reduction (with the flag-gated orphan pass of flag, the word after
// packed_bwd), at C_in = C_out = 192 or 256 in f16 / bf16 when both grids
// together fit one workgroup per CU (low keep rates). p0 is plan_bw's plan (its
// split count, or fewer). Returns 1 when launched, 0 when the shape does not
// qualify (nothing launched), or an SVTAD_ERR_* (message set, nothing
// launched).
// The one-launch backward's plan for a shape (host only): 1 with the
// backward-input tile shape (gfm row fragments, gfn column fragments per
// wave) and the split plan, 0 when the shape keeps two launches, or an
// SVTAD_ERR_* for a bad SVTAD_BWD_FUSED override (message set).
int bwd_fused_plan(int dtype, const BwPlan& p0, int64_t n, int c_in, int c_out, int* gfm, int* gfn,
                   BwPlan* p_out);
int bwd_fused_mfma(int dtype, const BwPlan& p0, const void* go, const void* x, const int32_t* nbr,
                   const void* w, const void* packed_bwd, uint32_t* flag, void* gi, void* gw, void* gb,
                   void* ws, size_t ws_bytes, int64_t n, int c_in, int c_out, int64_t tpb, hipStream_t s,
                   bool sym = false);

// A linear layer's weight gradient out[ci][co] = sum_i g[rows[i]][ci] x[i][co]
// (rows NULL: row i of g), i < n, on the backward-weight partial kernel with
// one offset and its ordered reduction. path 0 in the plan: no large-tile
// configuration for (c_in, c_out); wgrad_mfma then returns
// SVTAD_ERR_UNSUPPORTED. Returns SVTAD_OK or an SVTAD_ERR_* (nothing
// launched) as bw_mfma.
BwPlan plan_wgrad(int64_t n, int c_in, int c_out);
int wgrad_mfma(int dtype, const BwPlan& p, const void* g, const int32_t* rows, const void* x, void* out,
               void* ws, size_t ws_bytes, int64_t n, int64_t n_src, int c_in, int c_out, bool out_f32,
               hipStream_t s);

}  // namespace svtad
