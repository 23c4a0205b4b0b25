// C-ABI entry points of the SparseConv2D convolution: argument checks, path
// selection (MFMA for f16/bf16 shapes it handles, VALU otherwise) and the
// backward-weight split plan.
#include <stdio.h>
#include <string.h>

#include "sv_common.h"
#include "sv_conv.h"
#include "sv_internal.h"

namespace svtad {

static bool dtype_ok(int d) { return d >= SVTAD_F32 && d <= SVTAD_F64; }
// The MFMA kernels read operands as 16-byte vectors.
static bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }
static size_t acc_bytes(int d) { return d == SVTAD_F64 ? 8 : 4; }

static int check_common(const char* who, int64_t n, int c_in, int c_out, int64_t tpb, int dtype) {
    static thread_local char buf[256];
    if (c_in % 4 != 0 && c_in == c_out && strncmp(who, "dw_", 3) == 0) {
        // depthwise: an even element count keeps the 16-bit atomics of the
        // orphan pass inside the buffer (they update aligned 32-bit words)
        snprintf(buf, sizeof(buf), "%s: C must be divisible by 4", who);
        return set_error(SVTAD_ERR_INVALID, buf);
    }
    if (!dtype_ok(dtype)) {
        snprintf(buf, sizeof(buf), "%s: unknown dtype %d", who, dtype);
        return set_error(SVTAD_ERR_INVALID, buf);
    }
    if (n < 0 || c_in <= 0 || c_out <= 0 || tpb < 0) {
        snprintf(buf, sizeof(buf), "%s: bad sizes n=%lld c_in=%d c_out=%d tokens_per_batch=%lld",
                 who, (long long)n, c_in, c_out, (long long)tpb);
        return set_error(SVTAD_ERR_INVALID, buf);
    }
    if (n >= (int64_t)INT32_MAX) {
        snprintf(buf, sizeof(buf), "%s: n=%lld exceeds the int32 table range", who, (long long)n);
        return set_error(SVTAD_ERR_UNSUPPORTED, buf);
    }
    return SVTAD_OK;
}

// Full conv plan. Rows are split so that the partial-tile workgroups fill the
// chip's compute units in whole rounds (a second round of workgroups on a few
// units would nearly double the kernel time), without splits shorter than 256
// rows where n allows, and so that no split is longer than kMaxSplitRows - 128
// rows.
static BwPlan plan_bw(int64_t n, int c_in, int c_out, int dtype) {
    BwPlan p;
    p.path = bw_mfma_supported(dtype, n, c_in, c_out) ? 1 : 0;
    int tm = 64, tn = 64;
    bool big = false;
    if (p.path) big = bw_mfma_tiles(c_in, c_out, &tm, &tn);
    // work units per split: the large-tile kernel splits the center offset's
    // rows in two halves (its off-center units only visit rows whose neighbor
    // exists, about half of them at moderate keep rates, so the center units
    // get half the rows to take about as long)
    const int units = big ? 10 : 9;
    const int gran = big ? 256 : 128;  // whole pairs of 64-row stages per unit
    const int64_t tiles = units * cdiv(c_in, tm) * cdiv(c_out, tn);
    int64_t splits;
    if (p.path) {
        // Fewest workgroup rounds times the longest unit, with a fixed cost
        // per workgroup worth about 256 rows, plus (large-tile kernel) the
        // partial tiles' write and read-back, worth about 3 rows per
        // workgroup over the whole grid. At c2 this picks 7 splits at 10 %
        // keep and 17 at 55 %; without the partial term it picked 13 and 23,
        // 3.4 and 4 µs slower per step. A weight of 5 rows picked 14 at
        // 55 %, 15 at 70 % and 18 at 100 %: the backward ran 0.2-1.5 µs
        // slower than with 17, 22 and 25. Splits are whole multiples of gran rows, at
        // most kMaxSplitRows (the LDS row list), at least 256 rows where n
        // allows. A partial second round costs a full round, so a count just
        // above the CU count loses to twice as many half-length splits.
        const int64_t cu = cu_count();
        const int64_t s_min = std::max<int64_t>(1, cdiv(n, kMaxSplitRows - gran));
        const int64_t s_cap = std::max<int64_t>(s_min, std::min<int64_t>(cdiv(n, 256), 4 * cu / tiles + 1));
        splits = s_min;
        int64_t best = INT64_MAX;
        for (int64_t sc = s_min; sc <= s_cap; ++sc) {
            const int64_t r = cdiv(cdiv(std::max<int64_t>(n, 1), sc), gran) * gran;
            const int64_t se = std::max<int64_t>(1, cdiv(n, r));
            const int64_t cost = cdiv(se * tiles, cu) * ((big ? r / 2 : r) + 256) + (big ? 3 * se * tiles : 0);
            if (cost < best) {
                best = cost;
                splits = se;
            }
        }
    } else {
        splits = std::min<int64_t>(cdiv(1024, tiles), std::max<int64_t>(1, n / 128));
    }
    splits = std::max<int64_t>(1, splits);
    int64_t rps = cdiv(std::max<int64_t>(n, 1), splits);
    // whole pairs of 64-row stages per unit: a split's row list (at most
    // kMaxSplitRows) is read two 64-row stages per iteration by the MFMA kernel
    rps = cdiv(rps, gran) * gran;
    splits = std::max<int64_t>(1, cdiv(n, rps));
    p.splits = (int)splits;
    p.rows_per_split = rps;
    p.ws_bytes = (size_t)splits * ((size_t)units * c_in * c_out + (size_t)2 * c_out) * acc_bytes(dtype);
    return p;
}

static BwPlan plan_dw_bw(int64_t n, int c, int dtype) {
    BwPlan p;
    p.path = 0;
    const int64_t cu = cu_count();
    const int vec = dtype == SVTAD_F64 ? 2 : dtype == SVTAD_F32 ? 4 : 8;  // elements per 16 bytes
    int64_t rps;
    if (c % vec == 0 && c / vec <= 256) {
        // The vectorized kernels: one 512-thread workgroup per split (it
        // holds a CU alone) walks its rows R = 512 / (c / vec) at a time, one
        // dependent gather round per pass. Every CU gets a split while each
        // has at least R rows: the fewest passes, and the last one partly
        // filled rather than fewer splits of full passes (at c = 192 fp16,
        // 3136 rows: 150 splits of one pass instead of 49 of four; 17248
        // rows: 254 splits of 68 rows, 0.6 us faster than 206 of 84).
        const int64_t r = 512 / (c / vec);
        const int64_t splits = std::min<int64_t>(cu, std::max<int64_t>(1, cdiv(n, r)));
        rps = cdiv(std::max<int64_t>(n, 1), splits);
    } else {
        // the scalar kernel (one workgroup per 64-channel block and split):
        // about 64 rows per split, at most one split per CU
        const int64_t splits = std::min<int64_t>(cu, std::max<int64_t>(1, cdiv(n, 64)));
        rps = cdiv(cdiv(std::max<int64_t>(n, 1), splits), 4) * 4;
    }
    const int64_t splits = std::max<int64_t>(1, cdiv(n, rps));
    p.splits = (int)splits;
    p.rows_per_split = rps;
    p.ws_bytes = (size_t)splits * ((size_t)9 * c + (size_t)c) * acc_bytes(dtype);
    return p;
}

}  // namespace svtad

using namespace svtad;

extern "C" size_t svtad_fwd_workspace_bytes(int c_in, int c_out, int dtype) {
    if (!dtype_ok(dtype) || c_in <= 0 || c_out <= 0) return 0;
    return gg_mfma_workspace(dtype, c_in, c_out);
}

// The packed backward-input weight is followed by the orphan flag word.
static size_t bwd_in_ws(int dtype, int c_in, int c_out) {
    const size_t w = gg_mfma_workspace(dtype, c_out, c_in);
    return w ? w + kOrphanFlagBytes : 0;
}

extern "C" size_t svtad_bwd_in_workspace_bytes(int c_in, int c_out, int dtype) {
    if (!dtype_ok(dtype) || c_in <= 0 || c_out <= 0) return 0;
    return bwd_in_ws(dtype, c_in, c_out);
}

extern "C" int svtad_fwd(const void* x, const int32_t* nbr, const void* weight, const void* bias,
                         int bias_mode, void* out, void* workspace, size_t workspace_bytes,
                         int64_t n, int c_in, int c_out, int64_t tokens_per_batch, int dtype,
                         void* stream) {
    int st = check_common("fwd", n, c_in, c_out, tokens_per_batch, dtype);
    if (st) return st;
    if (c_in % 4 != 0) return set_error(SVTAD_ERR_INVALID, "fwd: C_in must be divisible by 4");
    if (bias_mode < SVTAD_BIAS_NONE || bias_mode > SVTAD_BIAS_PRE)
        return set_error(SVTAD_ERR_INVALID, "fwd: bad bias_mode");
    if (bias_mode != SVTAD_BIAS_NONE && !bias)
        return set_error(SVTAD_ERR_INVALID, "fwd: bias_mode needs a bias pointer");
    const size_t need = gg_mfma_workspace(dtype, c_in, c_out);
    if (need && (!workspace || workspace_bytes < need))
        return set_error(SVTAD_ERR_WORKSPACE, "fwd: workspace smaller than svtad_fwd_workspace_bytes()");
    if (n == 0) return SVTAD_OK;
    if (!x || !nbr || !weight || !out) return set_error(SVTAD_ERR_INVALID, "fwd: null pointer");
    hipStream_t s = (hipStream_t)stream;
    if (gg_mfma_supported(dtype, c_in, c_out) && al16(x) && al16(weight) && al16(out) &&
        (!need || al16(workspace)))
        gg_mfma(dtype, MODE_FWD, x, nbr, weight, bias, bias_mode, out, n, c_in, c_out,
                tokens_per_batch, need ? workspace : nullptr, false, nullptr, s);
    else
        gg_valu(dtype, MODE_FWD, x, nbr, weight, bias, bias_mode, out, n, c_in, c_out,
                tokens_per_batch, s);
    return launch_status();
}

extern "C" int svtad_bwd_in(const void* grad_out, const int32_t* nbr, const void* weight,
                            void* grad_in, void* workspace, size_t workspace_bytes, int64_t n,
                            int c_in, int c_out, int64_t tokens_per_batch, int dtype, void* stream) {
    int st = check_common("bwd_in", n, c_in, c_out, tokens_per_batch, dtype);
    if (st) return st;
    const size_t need = bwd_in_ws(dtype, c_in, c_out);
    if (need && (!workspace || workspace_bytes < need))
        return set_error(SVTAD_ERR_WORKSPACE, "bwd_in: workspace smaller than svtad_bwd_in_workspace_bytes()");
    if (n == 0) return SVTAD_OK;
    if (!grad_out || !nbr || !weight || !grad_in)
        return set_error(SVTAD_ERR_INVALID, "bwd_in: null pointer");
    hipStream_t s = (hipStream_t)stream;
    // gi[j, ci] = sum_k sum_co go[src_t(j,k), co] * w[k][ci][co]
    uint32_t* flag = need ? (uint32_t*)((char*)workspace + need - kOrphanFlagBytes) : nullptr;
    bool flagged = false;
    if (gg_mfma_supported(dtype, c_out, c_in) && al16(grad_out) && al16(weight) && al16(grad_in) &&
        (!need || al16(workspace)))
        flagged = gg_mfma(dtype, MODE_BWDIN, grad_out, nbr, weight, nullptr, 0, grad_in, n, c_out, c_in,
                          tokens_per_batch, need ? workspace : nullptr, false, flag, s);
    else
        gg_valu(dtype, MODE_BWDIN, grad_out, nbr, weight, nullptr, 0, grad_in, n, c_out, c_in,
                tokens_per_batch, s);
    orphans(dtype, false, grad_out, nbr, weight, grad_in, n, c_in, c_out, tokens_per_batch,
            flagged ? flag : nullptr, s);
    return launch_status();
}

extern "C" int svtad_pack_weight(const void* weight, void* packed_fwd, void* packed_bwd, int c_in,
                                 int c_out, int dtype, void* stream) {
    if (!weight || (!packed_fwd && !packed_bwd) || c_in <= 0 || c_out <= 0)
        return set_error(SVTAD_ERR_INVALID, "pack_weight: bad arguments");
    if ((packed_fwd && !gg_mfma_workspace(dtype, c_in, c_out)) ||
        (packed_bwd && !gg_mfma_workspace(dtype, c_out, c_in)))
        return set_error(SVTAD_ERR_UNSUPPORTED, "pack_weight: shape/dtype has no packed layout");
    if (9LL * c_in * c_out * 2 >= (int64_t)INT32_MAX)  // the pack kernel reads w with 32-bit offsets
        return set_error(SVTAD_ERR_UNSUPPORTED, "pack_weight: weight of 2 GiB or more");
    if (!al16(packed_fwd) || !al16(packed_bwd))
        return set_error(SVTAD_ERR_INVALID, "pack_weight: packed buffers must be 16-byte aligned");
    pack_weight(weight, packed_fwd, packed_bwd, c_in, c_out, (hipStream_t)stream);
    return launch_status();
}

extern "C" int svtad_fwd_packed(const void* x, const int32_t* nbr, const void* packed_fwd,
                                const void* bias, int bias_mode, void* out, int64_t n, int c_in,
                                int c_out, int64_t tokens_per_batch, int dtype, void* stream) {
    int st = check_common("fwd_packed", n, c_in, c_out, tokens_per_batch, dtype);
    if (st) return st;
    if (bias_mode < SVTAD_BIAS_NONE || bias_mode > SVTAD_BIAS_PRE || (bias_mode != SVTAD_BIAS_NONE && !bias))
        return set_error(SVTAD_ERR_INVALID, "fwd_packed: bad bias_mode / bias");
    if (!gg_mfma_packed_ok(dtype, n, c_in, c_out))
        return set_error(SVTAD_ERR_UNSUPPORTED, "fwd_packed: shape/dtype has no packed layout");
    if (n == 0) return SVTAD_OK;
    if (!x || !nbr || !packed_fwd || !out) return set_error(SVTAD_ERR_INVALID, "fwd_packed: null pointer");
    if (!al16(x) || !al16(packed_fwd) || !al16(out))
        return set_error(SVTAD_ERR_INVALID, "fwd_packed: x, packed weight and out must be 16-byte aligned");
    gg_mfma(dtype, MODE_FWD, x, nbr, packed_fwd, bias, bias_mode, out, n, c_in, c_out,
            tokens_per_batch, nullptr, true, nullptr, (hipStream_t)stream);
    return launch_status();
}

// table_flags of the *_ex entry points: only SVTAD_TABLE_SYMMETRIC is defined
static int check_table_flags(const char* what, unsigned flags) {
    if (flags & ~(unsigned)SVTAD_TABLE_SYMMETRIC) {
        char msg[96];
        snprintf(msg, sizeof msg, "%s: unknown table_flags bits 0x%x", what, flags);
        return set_error(SVTAD_ERR_INVALID, msg);
    }
    return SVTAD_OK;
}

extern "C" int svtad_bwd_in_packed(const void* grad_out, const int32_t* nbr, const void* weight,
                                   void* packed_bwd, void* grad_in, int64_t n, int c_in,
                                   int c_out, int64_t tokens_per_batch, int dtype, void* stream) {
    return svtad_bwd_in_packed_ex(grad_out, nbr, weight, packed_bwd, grad_in, n, c_in, c_out, tokens_per_batch,
                                  dtype, 0u, stream);
}

extern "C" int svtad_bwd_in_packed_ex(const void* grad_out, const int32_t* nbr, const void* weight,
                                      void* packed_bwd, void* grad_in, int64_t n, int c_in, int c_out,
                                      int64_t tokens_per_batch, int dtype, unsigned table_flags, void* stream) {
    int st = check_common("bwd_in_packed", n, c_in, c_out, tokens_per_batch, dtype);
    if (!st) st = check_table_flags("bwd_in_packed", table_flags);
    if (st) return st;
    if (!gg_mfma_packed_ok(dtype, n, c_out, c_in))
        return set_error(SVTAD_ERR_UNSUPPORTED, "bwd_in_packed: shape/dtype has no packed layout");
    if (n == 0) return SVTAD_OK;
    if (!grad_out || !nbr || !weight || !packed_bwd || !grad_in)
        return set_error(SVTAD_ERR_INVALID, "bwd_in_packed: null pointer");
    if (!al16(grad_out) || !al16(packed_bwd) || !al16(grad_in))
        return set_error(SVTAD_ERR_INVALID, "bwd_in_packed: grad_out, packed weight and grad_in must be 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    // the orphan flag follows the packed layout (cleared by svtad_pack_weight)
    uint32_t* flag = (uint32_t*)((char*)packed_bwd + gg_mfma_workspace(dtype, c_out, c_in));
    const bool sym = table_flags & SVTAD_TABLE_SYMMETRIC;
    const bool flagged = gg_mfma(dtype, MODE_BWDIN, grad_out, nbr, packed_bwd, nullptr, 0, grad_in,
                                 n, c_out, c_in, tokens_per_batch, nullptr, true, flag, s, sym);
    // a symmetric table has no entries without a partner: no pass for them
    if (!sym)
        orphans(dtype, false, grad_out, nbr, weight, grad_in, n, c_in, c_out, tokens_per_batch,
                flagged ? flag : nullptr, s);
    return launch_status();
}

extern "C" int svtad_bwd_in_gemm(const void* grad_out, const int32_t* nbr, void* packed_bwd, void* grad_in,
                                 int64_t n, int c_in, int c_out, int64_t tokens_per_batch, int dtype,
                                 unsigned table_flags, void* stream) {
    int st = check_common("bwd_in_gemm", n, c_in, c_out, tokens_per_batch, dtype);
    if (!st) st = check_table_flags("bwd_in_gemm", table_flags);
    if (st) return st;
    if (!gg_mfma_packed_ok(dtype, n, c_out, c_in))
        return set_error(SVTAD_ERR_UNSUPPORTED, "bwd_in_gemm: shape/dtype has no packed layout");
    if (n == 0) return SVTAD_OK;
    if (!grad_out || !nbr || !packed_bwd || !grad_in) return set_error(SVTAD_ERR_INVALID, "bwd_in_gemm: null pointer");
    if (!al16(grad_out) || !al16(packed_bwd) || !al16(grad_in))
        return set_error(SVTAD_ERR_INVALID, "bwd_in_gemm: grad_out, packed weight and grad_in must be 16-byte aligned");
    uint32_t* flag = (uint32_t*)((char*)packed_bwd + gg_mfma_workspace(dtype, c_out, c_in));
    gg_mfma(dtype, MODE_BWDIN, grad_out, nbr, packed_bwd, nullptr, 0, grad_in, n, c_out, c_in, tokens_per_batch,
            nullptr, true, flag, (hipStream_t)stream, table_flags & SVTAD_TABLE_SYMMETRIC);
    return launch_status();
}

extern "C" size_t svtad_bwd_w_workspace_bytes(int64_t n, int c_in, int c_out, int dtype) {
    if (check_common("bwd_w_workspace_bytes", n, c_in, c_out, 0, dtype)) return 0;
    return plan_bw(n, c_in, c_out, dtype).ws_bytes;
}

extern "C" int svtad_bwd_fused_plan(int64_t n, int c_in, int c_out, int dtype, int* tile_row_frags,
                                    int* tile_col_frags, int* splits) {
    if (!tile_row_frags || !tile_col_frags || !splits)
        return set_error(SVTAD_ERR_INVALID, "bwd_fused_plan: null pointer");
    *tile_row_frags = *tile_col_frags = *splits = 0;
    const int st = check_common("bwd_fused_plan", n, c_in, c_out, 0, dtype);
    if (st) return st;
    BwPlan p;
    const int r = bwd_fused_plan(dtype, plan_bw(n, c_in, c_out, dtype), n, c_in, c_out, tile_row_frags,
                                 tile_col_frags, &p);
    if (r == 1) *splits = p.splits;
    return r;
}

extern "C" int svtad_bwd_w(const void* grad_out, const void* x, const int32_t* nbr, void* grad_w,
                           void* grad_bias, void* workspace, size_t workspace_bytes, int64_t n,
                           int c_in, int c_out, int64_t tokens_per_batch, int dtype, void* stream) {
    int st = check_common("bwd_w", n, c_in, c_out, tokens_per_batch, dtype);
    if (st) return st;
    BwPlan p = plan_bw(n, c_in, c_out, dtype);
    // grad_w NULL: only the row-split partial sums are written (to workspace)
    if (!workspace || (n > 0 && (!grad_out || !x || !nbr)))
        return set_error(SVTAD_ERR_INVALID, "bwd_w: null pointer");
    if (p.path == 1 && !(al16(grad_out) && al16(x))) p.path = 0;  // same workspace layout
    if (workspace_bytes < p.ws_bytes)
        return set_error(SVTAD_ERR_WORKSPACE, "bwd_w: workspace smaller than svtad_bwd_w_workspace_bytes()");
    hipStream_t s = (hipStream_t)stream;
    if (p.path == 1) {
        bool unused;
        st = bw_mfma(dtype, p, grad_out, x, nbr, grad_w, grad_bias, workspace, workspace_bytes, n, c_in, c_out,
                     tokens_per_batch, nullptr, &unused, s);
        if (st) return st;
    } else
        bw_valu(dtype, p, grad_out, x, nbr, grad_w, grad_bias, workspace, n, c_in, c_out,
                tokens_per_batch, s);
    return launch_status();
}

extern "C" int svtad_bwd_packed(const void* grad_out, const void* x, const int32_t* nbr,
                                const void* weight, void* packed_bwd, void* grad_in, void* grad_w,
                                void* grad_bias, void* workspace, size_t workspace_bytes, int64_t n,
                                int c_in, int c_out, int64_t tokens_per_batch, int dtype,
                                void* stream) {
    return svtad_bwd_packed_ex(grad_out, x, nbr, weight, packed_bwd, grad_in, grad_w, grad_bias, workspace,
                               workspace_bytes, n, c_in, c_out, tokens_per_batch, dtype, 0u, stream);
}

extern "C" int svtad_bwd_packed_ex(const void* grad_out, const void* x, const int32_t* nbr, const void* weight,
                                   void* packed_bwd, void* grad_in, void* grad_w, void* grad_bias, void* workspace,
                                   size_t workspace_bytes, int64_t n, int c_in, int c_out,
                                   int64_t tokens_per_batch, int dtype, unsigned table_flags, void* stream) {
    int st = check_common("bwd_packed", n, c_in, c_out, tokens_per_batch, dtype);
    if (!st) st = check_table_flags("bwd_packed", table_flags);
    if (st) return st;
    if (!gg_mfma_packed_ok(dtype, n, c_out, c_in))
        return set_error(SVTAD_ERR_UNSUPPORTED, "bwd_packed: shape/dtype has no packed layout");
    BwPlan p = plan_bw(n, c_in, c_out, dtype);
    if (!workspace || !grad_w || !weight || !packed_bwd ||
        (n > 0 && (!grad_out || !x || !nbr || !grad_in)))
        return set_error(SVTAD_ERR_INVALID, "bwd_packed: null pointer");
    if (n > 0 && !(al16(grad_out) && al16(packed_bwd) && al16(grad_in)))
        return set_error(SVTAD_ERR_INVALID, "bwd_packed: grad_out, packed weight and grad_in must be 16-byte aligned");
    if (p.path == 1 && !(al16(grad_out) && al16(x))) p.path = 0;
    if (workspace_bytes < p.ws_bytes)
        return set_error(SVTAD_ERR_WORKSPACE, "bwd_packed: workspace smaller than svtad_bwd_w_workspace_bytes()");
    hipStream_t s = (hipStream_t)stream;
    const bool sym = table_flags & SVTAD_TABLE_SYMMETRIC;
    // grad_in and the partials in one launch where neither fills the chip
    if (p.path == 1 && n > 0) {
        uint32_t* f = (uint32_t*)((char*)packed_bwd + gg_mfma_workspace(dtype, c_out, c_in));
        st = bwd_fused_mfma(dtype, p, grad_out, x, nbr, weight, packed_bwd, f, grad_in, grad_w, grad_bias,
                            workspace, workspace_bytes, n, c_in, c_out, tokens_per_batch, s, sym);
        if (st < 0) return st;
        if (st == 1) return launch_status();
    }
    // 1. grad_in (keeps the orphan flag after the packed layout)
    const uint32_t* flag = nullptr;
    if (n > 0) {
        uint32_t* f = (uint32_t*)((char*)packed_bwd + gg_mfma_workspace(dtype, c_out, c_in));
        if (gg_mfma(dtype, MODE_BWDIN, grad_out, nbr, packed_bwd, nullptr, 0, grad_in, n, c_out,
                    c_in, tokens_per_batch, nullptr, true, f, s, sym))
            flag = f;
    }
    // 2. grad_w / grad_bias; the reduction also runs the orphan pass of step 1
    // (none for a symmetric table)
    const OrphanJob job{grad_out, nbr, weight, grad_in, n, c_in, c_out, tokens_per_batch, flag};
    bool taken = false;
    if (p.path == 1) {
        st = bw_mfma(dtype, p, grad_out, x, nbr, grad_w, grad_bias, workspace, workspace_bytes, n, c_in, c_out,
                     tokens_per_batch, n > 0 && !sym ? &job : nullptr, &taken, s);
        if (st) return st;
    } else
        bw_valu(dtype, p, grad_out, x, nbr, grad_w, grad_bias, workspace, n, c_in, c_out,
                tokens_per_batch, s);
    if (n > 0 && !taken && !sym)
        orphans(dtype, false, grad_out, nbr, weight, grad_in, n, c_in, c_out, tokens_per_batch, flag, s);
    return launch_status();
}

extern "C" int svtad_dw_fwd(const void* x, const int32_t* nbr, const void* weight, const void* bias,
                            void* out, int64_t n, int c, int64_t tokens_per_batch, int dtype,
                            void* stream) {
    int st = check_common("dw_fwd", n, c, c, tokens_per_batch, dtype);
    if (st) return st;
    if (n == 0) return SVTAD_OK;
    if (!x || !nbr || !weight || !out) return set_error(SVTAD_ERR_INVALID, "dw_fwd: null pointer");
    dw_gather(dtype, MODE_FWD, x, nbr, weight, bias, out, n, c, tokens_per_batch, (hipStream_t)stream);
    return launch_status();
}

extern "C" int svtad_dw_bwd_in(const void* grad_out, const int32_t* nbr, const void* weight,
                               void* grad_in, int64_t n, int c, int64_t tokens_per_batch, int dtype,
                               void* stream) {
    return svtad_dw_bwd_in_ex(grad_out, nbr, weight, grad_in, n, c, tokens_per_batch, dtype, 0u, stream);
}

extern "C" int svtad_dw_bwd_in_ex(const void* grad_out, const int32_t* nbr, const void* weight, void* grad_in,
                                  int64_t n, int c, int64_t tokens_per_batch, int dtype, unsigned table_flags,
                                  void* stream) {
    int st = check_common("dw_bwd_in", n, c, c, tokens_per_batch, dtype);
    if (!st) st = check_table_flags("dw_bwd_in", table_flags);
    if (st) return st;
    if (n == 0) return SVTAD_OK;
    if (!grad_out || !nbr || !weight || !grad_in)
        return set_error(SVTAD_ERR_INVALID, "dw_bwd_in: null pointer");
    hipStream_t s = (hipStream_t)stream;
    const bool sym = table_flags & SVTAD_TABLE_SYMMETRIC;
    dw_gather(dtype, MODE_BWDIN, grad_out, nbr, weight, nullptr, grad_in, n, c, tokens_per_batch, s, sym);
    if (!sym) orphans(dtype, true, grad_out, nbr, weight, grad_in, n, c, c, tokens_per_batch, nullptr, s);
    return launch_status();
}

// partials of the depthwise backward ([splits][10][c] in the accumulator
// type), then one flag word per split, 16-byte aligned
static size_t dw_bwd_ws(const BwPlan& p) { return cdiv(p.ws_bytes, 16) * 16 + (size_t)p.splits * 4; }

extern "C" size_t svtad_dw_bwd_workspace_bytes(int64_t n, int c, int dtype) {
    if (check_common("dw_bwd_workspace_bytes", n, c, c, 0, dtype)) return 0;
    return dw_bwd_ws(plan_dw_bw(n, c, dtype));
}

extern "C" int svtad_dw_bwd(const void* grad_out, const void* x, const int32_t* nbr, const void* weight,
                            void* grad_in, void* grad_w, void* grad_bias, void* workspace, size_t workspace_bytes,
                            int64_t n, int c, int64_t tokens_per_batch, int dtype, void* stream) {
    return svtad_dw_bwd_ex(grad_out, x, nbr, weight, grad_in, grad_w, grad_bias, workspace, workspace_bytes, n, c,
                           tokens_per_batch, dtype, 0u, stream);
}

extern "C" int svtad_dw_bwd_ex(const void* grad_out, const void* x, const int32_t* nbr, const void* weight,
                               void* grad_in, void* grad_w, void* grad_bias, void* workspace, size_t workspace_bytes,
                               int64_t n, int c, int64_t tokens_per_batch, int dtype, unsigned table_flags,
                               void* stream) {
    int st = check_common("dw_bwd", n, c, c, tokens_per_batch, dtype);
    if (!st) st = check_table_flags("dw_bwd", table_flags);
    if (st) return st;
    const BwPlan p = plan_dw_bw(n, c, dtype);
    if (!grad_w || !workspace || !weight || (n > 0 && (!grad_out || !x || !nbr || !grad_in)))
        return set_error(SVTAD_ERR_INVALID, "dw_bwd: null pointer");
    if (workspace_bytes < dw_bwd_ws(p))
        return set_error(SVTAD_ERR_WORKSPACE, "dw_bwd: workspace smaller than svtad_dw_bwd_workspace_bytes()");
    hipStream_t s = (hipStream_t)stream;
    uint32_t* flags = (uint32_t*)((char*)workspace + cdiv(p.ws_bytes, 16) * 16);
    const bool sym = table_flags & SVTAD_TABLE_SYMMETRIC;
    if (n > 0 && dw_bwd_fused(dtype, p, grad_out, x, nbr, weight, grad_in, grad_w, grad_bias, workspace, flags, n,
                              c, tokens_per_batch, s, sym))
        return launch_status();
    // shapes / alignments the one-pass kernels do not take: the two passes
    if (n > 0) {
        dw_gather(dtype, MODE_BWDIN, grad_out, nbr, weight, nullptr, grad_in, n, c, tokens_per_batch, s, sym);
        if (!sym) orphans(dtype, true, grad_out, nbr, weight, grad_in, n, c, c, tokens_per_batch, nullptr, s);
    }
    dw_bw(dtype, p, grad_out, x, nbr, grad_w, grad_bias, workspace, n, c, tokens_per_batch, s);
    return launch_status();
}

extern "C" size_t svtad_dw_bwd_w_workspace_bytes(int64_t n, int c, int dtype) {
    if (check_common("dw_bwd_w_workspace_bytes", n, c, c, 0, dtype)) return 0;
    return plan_dw_bw(n, c, dtype).ws_bytes;
}

extern "C" int svtad_dw_bwd_w(const void* grad_out, const void* x, const int32_t* nbr, void* grad_w,
                              void* grad_bias, void* workspace, size_t workspace_bytes, int64_t n,
                              int c, int64_t tokens_per_batch, int dtype, void* stream) {
    int st = check_common("dw_bwd_w", n, c, c, tokens_per_batch, dtype);
    if (st) return st;
    const BwPlan p = plan_dw_bw(n, c, dtype);
    if (!grad_w || !workspace || (n > 0 && (!grad_out || !x || !nbr)))
        return set_error(SVTAD_ERR_INVALID, "dw_bwd_w: null pointer");
    if (workspace_bytes < p.ws_bytes)
        return set_error(SVTAD_ERR_WORKSPACE, "dw_bwd_w: workspace smaller than svtad_dw_bwd_w_workspace_bytes()");
    dw_bw(dtype, p, grad_out, x, nbr, grad_w, grad_bias, workspace, n, c, tokens_per_batch,
          (hipStream_t)stream);
    return launch_status();
}
