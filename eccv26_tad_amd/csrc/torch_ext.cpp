// `opentad_sparse_ops`: the PyTorch-ROCm extension module. Thin layer over the
// C ABI in include/svtad_sparse.h: argument checks, output allocation through
// the caching allocator, and the current HIP stream of the input's device.
//
// The five reference functions keep their names, argument order and meaning
// (opentad/models/bricks/2d_sparse_v3_bind.cpp:8-14); the rest are additions
// the autograd wrapper and the table utilities use.
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>

#include <tuple>

#include "../../include/svtad_sparse.h"

namespace {

int dtype_code(const at::Tensor& t) {
    switch (t.scalar_type()) {
        case at::kFloat: return SVTAD_F32;
        case at::kHalf: return SVTAD_F16;
        case at::kBFloat16: return SVTAD_BF16;
        case at::kDouble: return SVTAD_F64;
        default: TORCH_CHECK(false, "opentad_sparse_ops: unsupported dtype ", t.scalar_type());
    }
    return -1;
}

void* stream_of(const at::Tensor& t) {
    return (void*)c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

void check_status(int st, const char* who) {
    TORCH_CHECK(st == SVTAD_OK, "opentad_sparse_ops.", who, ": ", svtad_last_error(), " (status ",
                st, ")");
}

void check_gpu(const at::Tensor& t, const char* name) {
    TORCH_CHECK(t.is_cuda(), "opentad_sparse_ops: ", name, " must be a GPU tensor");
}

at::Tensor rows_view(const at::Tensor& t) {
    TORCH_CHECK(t.dim() >= 1, "expected at least 1 dimension");
    return t.contiguous();
}

int64_t n_rows(const at::Tensor& t) { return t.size(-1) == 0 ? 0 : t.numel() / t.size(-1); }

at::Tensor table_i32(const at::Tensor& nbr, int64_t n) {
    check_gpu(nbr, "neighbor_indices");
    TORCH_CHECK(nbr.scalar_type() == at::kInt, "neighbor_indices must be int32, got ",
                nbr.scalar_type());
    TORCH_CHECK(nbr.numel() == n * 9, "neighbor_indices has ", nbr.numel(), " entries, expected ",
                n, " x 9");
    return nbr.contiguous();
}

bool bias_present(const c10::optional<at::Tensor>& b) { return b.has_value() && b->defined() && b->numel() > 0; }

at::Tensor conv_fwd(const at::Tensor& x_in, const at::Tensor& nbr_in, const at::Tensor& w_in,
                    const c10::optional<at::Tensor>& bias_in, int64_t tpb, int bias_mode,
                    int64_t c_out_arg) {
    check_gpu(x_in, "x");
    check_gpu(w_in, "weight");
    at::Tensor x = rows_view(x_in);
    const int64_t c_in = x.size(-1);
    const int64_t n = n_rows(x);
    TORCH_CHECK(w_in.dim() == 3 && w_in.size(0) == 9 && w_in.size(1) == c_in,
                "weight must be (9, C_in, C_out) with C_in = ", c_in, ", got ", w_in.sizes());
    const int64_t c_out = w_in.size(2);
    TORCH_CHECK(c_out_arg < 0 || c_out_arg == c_out, "C_out argument ", c_out_arg,
                " does not match weight.size(2) = ", c_out);
    TORCH_CHECK(w_in.scalar_type() == x.scalar_type(), "x and weight dtypes differ: ",
                x.scalar_type(), " vs ", w_in.scalar_type());
    at::Tensor w = w_in.contiguous();
    at::Tensor nbr = table_i32(nbr_in, n);
    c10::DeviceGuard g(x.device());
    at::Tensor bias;
    if (bias_mode != SVTAD_BIAS_NONE && bias_present(bias_in)) {
        TORCH_CHECK(bias_in->numel() == c_out, "bias must have C_out = ", c_out, " elements");
        if (bias_mode == SVTAD_BIAS_FP32 && bias_in->scalar_type() == x.scalar_type()) {
            // widened exactly inside the kernel: no conversion launch
            bias_mode = SVTAD_BIAS_PRE;
            bias = bias_in->contiguous();
        } else {
            const at::ScalarType bt =
                bias_mode == SVTAD_BIAS_FP32
                    ? (x.scalar_type() == at::kDouble ? at::kDouble : at::kFloat)
                    : x.scalar_type();
            bias = bias_in->to(x.device(), bt).contiguous();
        }
        TORCH_CHECK(bias.device() == x.device(), "bias must be on x's device");
    } else {
        bias_mode = SVTAD_BIAS_NONE;
    }
    at::Tensor out = at::empty({n, c_out}, x.options());
    const int dt = dtype_code(x);
    const size_t ws_bytes = svtad_fwd_workspace_bytes((int)c_in, (int)c_out, dt);
    at::Tensor ws;
    if (ws_bytes && n > 0) ws = at::empty({(int64_t)ws_bytes}, x.options().dtype(at::kByte));
    const int st = svtad_fwd(x.data_ptr(), nbr.data_ptr<int32_t>(), w.data_ptr(),
                             bias.defined() ? bias.data_ptr() : nullptr, bias_mode, out.data_ptr(),
                             ws.defined() ? ws.data_ptr() : nullptr, ws_bytes, n, (int)c_in,
                             (int)c_out, tpb, dt, stream_of(x));
    check_status(st, "fwd");
    return out;
}

}  // namespace

// fwd(x, neighbor_indices, weight, C_out, tokens_per_batch) -> [N, C_out], no bias
// (2d_sparse_v3.cu:751-822)
at::Tensor op_fwd(const at::Tensor& x, const at::Tensor& nbr, const at::Tensor& w, int64_t c_out,
                  int64_t tpb) {
    return conv_fwd(x, nbr, w, c10::nullopt, tpb, SVTAD_BIAS_NONE, c_out);
}

// implicit_gemm_fwd_v2(x, neighbor_indices, weight, bias, tokens_per_batch); an empty
// bias means no bias, bias is added in fp32 (implicit_gemm_v2.cu:197-300)
at::Tensor op_implicit_gemm_fwd_v2(const at::Tensor& x, const at::Tensor& nbr, const at::Tensor& w,
                                   const c10::optional<at::Tensor>& bias, int64_t tpb) {
    return conv_fwd(x, nbr, w, bias, tpb, SVTAD_BIAS_FP32, -1);
}

// implicit_gemm_fwd_v2_chunked(..., chunk_size): same result; chunk_size was a
// memory knob of the reference's host chunk loop (implicit_gemm_v2.cu:306-417),
// which this implementation does not need.
at::Tensor op_implicit_gemm_fwd_v2_chunked(const at::Tensor& x, const at::Tensor& nbr,
                                           const at::Tensor& w,
                                           const c10::optional<at::Tensor>& bias, int64_t tpb,
                                           int64_t chunk_size) {
    TORCH_CHECK(chunk_size > 0, "chunk_size must be positive, got ", chunk_size);
    return conv_fwd(x, nbr, w, bias, tpb, SVTAD_BIAS_FP32, -1);
}

// fwd_bias(x, neighbor_indices, weight, bias, tokens_per_batch, bias_mode)
at::Tensor op_fwd_bias(const at::Tensor& x, const at::Tensor& nbr, const at::Tensor& w,
                       const c10::optional<at::Tensor>& bias, int64_t tpb, int64_t bias_mode) {
    TORCH_CHECK(bias_mode >= 0 && bias_mode <= 2, "bias_mode must be 0, 1 or 2");
    return conv_fwd(x, nbr, w, bias, tpb, (int)bias_mode, -1);
}

// pack_weight(weight, fwd, bwd) -> (packed_fwd, packed_bwd): the weight in the
// fragment order of the matrix-core kernels; an empty tensor for a layout not
// requested or not available for this shape / dtype.
std::tuple<at::Tensor, at::Tensor> op_pack_weight(const at::Tensor& w_in, bool fwd, bool bwd) {
    check_gpu(w_in, "weight");
    TORCH_CHECK(w_in.dim() == 3 && w_in.size(0) == 9, "weight must be (9, C_in, C_out)");
    at::Tensor w = w_in.contiguous();
    const int c_in = (int)w.size(1), c_out = (int)w.size(2);
    const int dt = dtype_code(w);
    const size_t bf = fwd ? svtad_fwd_workspace_bytes(c_in, c_out, dt) : 0;
    const size_t bb = bwd ? svtad_bwd_in_workspace_bytes(c_in, c_out, dt) : 0;
    c10::DeviceGuard g(w.device());
    at::Tensor pf = at::empty({(int64_t)bf}, w.options().dtype(at::kByte));
    at::Tensor pb = at::empty({(int64_t)bb}, w.options().dtype(at::kByte));
    if (bf || bb)
        check_status(svtad_pack_weight(w.data_ptr(), bf ? pf.data_ptr() : nullptr,
                                       bb ? pb.data_ptr() : nullptr, c_in, c_out, dt, stream_of(w)),
                     "pack_weight");
    return {pf, pb};
}

// fwd_packed(x, neighbor_indices, weight, packed_fwd, bias, tokens_per_batch,
// bias_mode): fwd_bias with a weight packed by pack_weight (falls back to
// fwd_bias when packed_fwd is empty or the shape has no packed path).
at::Tensor op_fwd_packed(const at::Tensor& x_in, const at::Tensor& nbr_in, const at::Tensor& w,
                         const at::Tensor& packed, const c10::optional<at::Tensor>& bias_in,
                         int64_t tpb, int64_t bias_mode) {
    TORCH_CHECK(bias_mode >= 0 && bias_mode <= 2, "bias_mode must be 0, 1 or 2");
    if (packed.numel() == 0) return conv_fwd(x_in, nbr_in, w, bias_in, tpb, (int)bias_mode, -1);
    check_gpu(x_in, "x");
    at::Tensor x = rows_view(x_in);
    const int64_t c_in = x.size(-1), n = n_rows(x);
    TORCH_CHECK(w.dim() == 3 && w.size(0) == 9 && w.size(1) == c_in, "weight must be (9, C_in, C_out)");
    TORCH_CHECK(w.scalar_type() == x.scalar_type(), "x and weight dtypes differ");
    const int64_t c_out = w.size(2);
    const int dt = dtype_code(x);
    TORCH_CHECK((size_t)packed.numel() == svtad_fwd_workspace_bytes((int)c_in, (int)c_out, dt),
                "packed_fwd does not match the weight");
    at::Tensor nbr = table_i32(nbr_in, n);
    c10::DeviceGuard g(x.device());
    int mode = (int)bias_mode;
    at::Tensor bias;
    if (mode != SVTAD_BIAS_NONE && bias_present(bias_in)) {
        TORCH_CHECK(bias_in->numel() == c_out, "bias must have C_out = ", c_out, " elements");
        if (mode == SVTAD_BIAS_FP32 && bias_in->scalar_type() == x.scalar_type()) {
            mode = SVTAD_BIAS_PRE;
            bias = bias_in->contiguous();
        } else {
            bias = bias_in->to(x.device(), mode == SVTAD_BIAS_FP32 ? at::kFloat : x.scalar_type()).contiguous();
        }
    } else {
        mode = SVTAD_BIAS_NONE;
    }
    at::Tensor out = at::empty({n, c_out}, x.options());
    const int st = svtad_fwd_packed(x.data_ptr(), nbr.data_ptr<int32_t>(), packed.data_ptr(),
                                    bias.defined() ? bias.data_ptr() : nullptr, mode, out.data_ptr(),
                                    n, (int)c_in, (int)c_out, tpb, dt, stream_of(x));
    if (st == SVTAD_ERR_UNSUPPORTED) return conv_fwd(x_in, nbr_in, w, bias_in, tpb, (int)bias_mode, -1);
    check_status(st, "fwd_packed");
    return out;
}

// bwd_in(grad_output, neighbor_indices, weight, n_kept, C_in, tokens_per_batch)
// -> [n_kept, C_in] in grad_output's dtype (2d_sparse_v3.cu:824-835)
at::Tensor op_bwd_in(const at::Tensor& go_in, const at::Tensor& nbr_in, const at::Tensor& w_in,
                     int64_t n_kept, int64_t c_in, int64_t tpb) {
    check_gpu(go_in, "grad_output");
    check_gpu(w_in, "weight");
    at::Tensor go = rows_view(go_in);
    const int64_t c_out = go.size(-1);
    TORCH_CHECK(n_rows(go) == n_kept, "grad_output has ", n_rows(go), " rows, n_kept = ", n_kept);
    TORCH_CHECK(w_in.dim() == 3 && w_in.size(0) == 9 && w_in.size(1) == c_in && w_in.size(2) == c_out,
                "weight must be (9, ", c_in, ", ", c_out, "), got ", w_in.sizes());
    TORCH_CHECK(w_in.scalar_type() == go.scalar_type(), "grad_output and weight dtypes differ");
    at::Tensor w = w_in.contiguous();
    at::Tensor nbr = table_i32(nbr_in, n_kept);
    c10::DeviceGuard g(go.device());
    at::Tensor gi = at::empty({n_kept, c_in}, go.options());
    const int dt = dtype_code(go);
    const size_t ws_bytes = svtad_bwd_in_workspace_bytes((int)c_in, (int)c_out, dt);
    at::Tensor ws;
    if (ws_bytes && n_kept > 0) ws = at::empty({(int64_t)ws_bytes}, go.options().dtype(at::kByte));
    const int st = svtad_bwd_in(go.data_ptr(), nbr.data_ptr<int32_t>(), w.data_ptr(), gi.data_ptr(),
                                ws.defined() ? ws.data_ptr() : nullptr, ws_bytes, n_kept, (int)c_in,
                                (int)c_out, tpb, dt, stream_of(go));
    check_status(st, "bwd_in");
    return gi;
}

// table_flags from the `symmetric` keyword of the backward ops: the caller's
// promise that every table entry has its partner (SVTAD_TABLE_SYMMETRIC)
static unsigned table_flags(bool symmetric) { return symmetric ? (unsigned)SVTAD_TABLE_SYMMETRIC : 0u; }

// bwd_in_packed(grad_output, neighbor_indices, weight, packed_bwd, n_kept, C_in,
// tokens_per_batch, symmetric=False): bwd_in with a weight packed by
// pack_weight (falls back to bwd_in when packed_bwd is empty or the shape has
// no packed path).
at::Tensor op_bwd_in_packed(const at::Tensor& go_in, const at::Tensor& nbr_in, const at::Tensor& w_in,
                            const at::Tensor& packed, int64_t n_kept, int64_t c_in, int64_t tpb,
                            bool symmetric) {
    if (packed.numel() == 0) return op_bwd_in(go_in, nbr_in, w_in, n_kept, c_in, tpb);
    check_gpu(go_in, "grad_output");
    at::Tensor go = rows_view(go_in);
    const int64_t c_out = go.size(-1);
    TORCH_CHECK(n_rows(go) == n_kept, "grad_output has ", n_rows(go), " rows, n_kept = ", n_kept);
    TORCH_CHECK(w_in.dim() == 3 && w_in.size(0) == 9 && w_in.size(1) == c_in && w_in.size(2) == c_out,
                "weight must be (9, ", c_in, ", ", c_out, ")");
    TORCH_CHECK(w_in.scalar_type() == go.scalar_type(), "grad_output and weight dtypes differ");
    const int dt = dtype_code(go);
    TORCH_CHECK((size_t)packed.numel() == svtad_bwd_in_workspace_bytes((int)c_in, (int)c_out, dt),
                "packed_bwd does not match the weight");
    at::Tensor w = w_in.contiguous();
    at::Tensor nbr = table_i32(nbr_in, n_kept);
    c10::DeviceGuard g(go.device());
    at::Tensor gi = at::empty({n_kept, c_in}, go.options());
    const int st = svtad_bwd_in_packed_ex(go.data_ptr(), nbr.data_ptr<int32_t>(), w.data_ptr(),
                                          packed.data_ptr(), gi.data_ptr(), n_kept, (int)c_in,
                                          (int)c_out, tpb, dt, table_flags(symmetric), stream_of(go));
    if (st == SVTAD_ERR_UNSUPPORTED) return op_bwd_in(go_in, nbr_in, w_in, n_kept, c_in, tpb);
    check_status(st, "bwd_in_packed");
    return gi;
}

// bwd_in_gemm(grad_output, neighbor_indices, packed_bwd, C_in, tokens_per_batch) -> [n, C_in]:
// backward-input's gathered GEMM alone (timing; equals bwd_in_packed for
// tables whose entries all have their symmetric partner)
at::Tensor op_bwd_in_gemm(const at::Tensor& go_in, const at::Tensor& nbr_in, const at::Tensor& packed,
                          int64_t c_in, int64_t tpb, bool symmetric) {
    check_gpu(go_in, "grad_output");
    at::Tensor go = rows_view(go_in);
    const int64_t n = n_rows(go), c_out = go.size(-1);
    const int dt = dtype_code(go);
    TORCH_CHECK(packed.numel() > 0 &&
                    (size_t)packed.numel() == svtad_bwd_in_workspace_bytes((int)c_in, (int)c_out, dt),
                "packed_bwd does not match C_in x C_out in grad_output's dtype");
    at::Tensor nbr = table_i32(nbr_in, n);
    c10::DeviceGuard g(go.device());
    at::Tensor gi = at::empty({n, c_in}, go.options());
    check_status(svtad_bwd_in_gemm(go.data_ptr(), nbr.data_ptr<int32_t>(), packed.data_ptr(), gi.data_ptr(), n,
                                   (int)c_in, (int)c_out, tpb, dt, table_flags(symmetric), stream_of(go)),
                 "bwd_in_gemm");
    return gi;
}

// bwd_w_bias(grad_output, x, neighbor_indices, C_in, tokens_per_batch, with_bias)
// -> (grad_weight [9, C_in, C_out] in x's dtype, grad_bias [C_out] or empty)
std::tuple<at::Tensor, at::Tensor> op_bwd_w_bias(const at::Tensor& go_in, const at::Tensor& x_in,
                                                 const at::Tensor& nbr_in, int64_t c_in,
                                                 int64_t tpb, bool with_bias) {
    check_gpu(go_in, "grad_output");
    check_gpu(x_in, "x");
    at::Tensor go = rows_view(go_in);
    at::Tensor x = rows_view(x_in);
    TORCH_CHECK(x.size(-1) == c_in, "x has ", x.size(-1), " channels, C_in = ", c_in);
    const int64_t n = n_rows(x);
    TORCH_CHECK(n_rows(go) == n, "grad_output has ", n_rows(go), " rows, x has ", n);
    TORCH_CHECK(go.scalar_type() == x.scalar_type(), "grad_output and x dtypes differ");
    const int64_t c_out = go.size(-1);
    at::Tensor nbr = table_i32(nbr_in, n);
    c10::DeviceGuard g(x.device());
    const int dt = dtype_code(x);
    const size_t ws_bytes = svtad_bwd_w_workspace_bytes(n, (int)c_in, (int)c_out, dt);
    TORCH_CHECK(ws_bytes > 0, "bwd_w: ", svtad_last_error());
    at::Tensor ws = at::empty({(int64_t)ws_bytes}, x.options().dtype(at::kByte));
    at::Tensor gw = at::empty({9, c_in, c_out}, x.options());
    at::Tensor gb = with_bias ? at::empty({c_out}, x.options()) : at::Tensor();
    const int st = svtad_bwd_w(go.data_ptr(), x.data_ptr(), nbr.data_ptr<int32_t>(), gw.data_ptr(),
                               with_bias ? gb.data_ptr() : nullptr, ws.data_ptr(), ws_bytes, n,
                               (int)c_in, (int)c_out, tpb, dt, stream_of(x));
    check_status(st, "bwd_w");
    return {gw, with_bias ? gb : at::empty({0}, x.options())};
}

// bwd_packed(grad_output, x, neighbor_indices, weight, packed_bwd, C_in,
// tokens_per_batch, with_bias) -> (grad_input [n, C_in], grad_weight, grad_bias
// or empty): the autograd backward in one call (what bwd_in_packed and
// bwd_w_bias give, with one launch less); falls back to those two when
// packed_bwd is empty or the shape has no packed path.
std::tuple<at::Tensor, at::Tensor, at::Tensor> op_bwd_packed(const at::Tensor& go_in, const at::Tensor& x_in,
                                                             const at::Tensor& nbr_in, const at::Tensor& w_in,
                                                             const at::Tensor& packed, int64_t c_in,
                                                             int64_t tpb, bool with_bias, bool symmetric) {
    check_gpu(go_in, "grad_output");
    check_gpu(x_in, "x");
    at::Tensor go = rows_view(go_in);
    at::Tensor x = rows_view(x_in);
    TORCH_CHECK(x.size(-1) == c_in, "x has ", x.size(-1), " channels, C_in = ", c_in);
    const int64_t n = n_rows(x), c_out = go.size(-1);
    auto separate = [&]() {
        at::Tensor gi = op_bwd_in_packed(go_in, nbr_in, w_in, packed, n, c_in, tpb, symmetric);
        auto gwb = op_bwd_w_bias(go_in, x_in, nbr_in, c_in, tpb, with_bias);
        return std::make_tuple(gi, std::get<0>(gwb), std::get<1>(gwb));
    };
    if (packed.numel() == 0) return separate();
    TORCH_CHECK(n_rows(go) == n, "grad_output has ", n_rows(go), " rows, x has ", n);
    TORCH_CHECK(go.scalar_type() == x.scalar_type() && w_in.scalar_type() == x.scalar_type(),
                "grad_output, x and weight dtypes differ");
    TORCH_CHECK(w_in.dim() == 3 && w_in.size(0) == 9 && w_in.size(1) == c_in && w_in.size(2) == c_out,
                "weight must be (9, ", c_in, ", ", c_out, ")");
    const int dt = dtype_code(x);
    TORCH_CHECK((size_t)packed.numel() == svtad_bwd_in_workspace_bytes((int)c_in, (int)c_out, dt),
                "packed_bwd does not match the weight");
    at::Tensor w = w_in.contiguous();
    at::Tensor nbr = table_i32(nbr_in, n);
    c10::DeviceGuard g(x.device());
    const size_t ws_bytes = svtad_bwd_w_workspace_bytes(n, (int)c_in, (int)c_out, dt);
    TORCH_CHECK(ws_bytes > 0, "bwd_packed: ", svtad_last_error());
    at::Tensor ws = at::empty({(int64_t)ws_bytes}, x.options().dtype(at::kByte));
    at::Tensor gi = at::empty({n, c_in}, x.options());
    at::Tensor gw = at::empty({9, c_in, c_out}, x.options());
    at::Tensor gb = with_bias ? at::empty({c_out}, x.options()) : at::Tensor();
    const int st = svtad_bwd_packed_ex(go.data_ptr(), x.data_ptr(), nbr.data_ptr<int32_t>(), w.data_ptr(),
                                       packed.data_ptr(), gi.data_ptr(), gw.data_ptr(),
                                       with_bias ? gb.data_ptr() : nullptr, ws.data_ptr(), ws_bytes, n,
                                       (int)c_in, (int)c_out, tpb, dt, table_flags(symmetric), stream_of(x));
    if (st == SVTAD_ERR_UNSUPPORTED) return separate();
    check_status(st, "bwd_packed");
    return {gi, gw, with_bias ? gb : at::empty({0}, x.options())};
}

// bwd_w_partials(grad_output, x, neighbor_indices, C_in, tokens_per_batch, with_bias)
// -> workspace bytes holding the row-split partial sums only (no reduction).
// For timing the partial-sum kernel of backward-weight on its own.
at::Tensor op_bwd_w_partials(const at::Tensor& go_in, const at::Tensor& x_in, const at::Tensor& nbr_in,
                             int64_t c_in, int64_t tpb, bool with_bias) {
    check_gpu(go_in, "grad_output");
    check_gpu(x_in, "x");
    at::Tensor go = rows_view(go_in);
    at::Tensor x = rows_view(x_in);
    TORCH_CHECK(x.size(-1) == c_in, "x has ", x.size(-1), " channels, C_in = ", c_in);
    const int64_t n = n_rows(x), c_out = go.size(-1);
    TORCH_CHECK(n_rows(go) == n && go.scalar_type() == x.scalar_type(), "grad_output must match x");
    at::Tensor nbr = table_i32(nbr_in, n);
    c10::DeviceGuard g(x.device());
    const int dt = dtype_code(x);
    const size_t ws_bytes = svtad_bwd_w_workspace_bytes(n, (int)c_in, (int)c_out, dt);
    TORCH_CHECK(ws_bytes > 0, "bwd_w_partials: ", svtad_last_error());
    at::Tensor ws = at::empty({(int64_t)ws_bytes}, x.options().dtype(at::kByte));
    at::Tensor gb = with_bias ? at::empty({c_out}, x.options()) : at::Tensor();
    check_status(svtad_bwd_w(go.data_ptr(), x.data_ptr(), nbr.data_ptr<int32_t>(), nullptr,
                             with_bias ? gb.data_ptr() : nullptr, ws.data_ptr(), ws_bytes, n,
                             (int)c_in, (int)c_out, tpb, dt, stream_of(x)),
                 "bwd_w_partials");
    return ws;
}

// bwd_w(grad_output, x, neighbor_indices, C_in, tokens_per_batch) -> [9, C_in, C_out]
// (2d_sparse_v3.cu:837-850)
at::Tensor op_bwd_w(const at::Tensor& go, const at::Tensor& x, const at::Tensor& nbr, int64_t c_in,
                    int64_t tpb) {
    return std::get<0>(op_bwd_w_bias(go, x, nbr, c_in, tpb, false));
}

// ---------------------------------------------------------------------------
// depthwise (groups = C), weight (9, C)
// ---------------------------------------------------------------------------

at::Tensor op_dw_fwd(const at::Tensor& x_in, const at::Tensor& nbr_in, const at::Tensor& w_in,
                     const c10::optional<at::Tensor>& bias_in, int64_t tpb) {
    check_gpu(x_in, "x");
    at::Tensor x = rows_view(x_in);
    const int64_t c = x.size(-1), n = n_rows(x);
    TORCH_CHECK(w_in.dim() == 2 && w_in.size(0) == 9 && w_in.size(1) == c,
                "depthwise weight must be (9, ", c, "), got ", w_in.sizes());
    TORCH_CHECK(w_in.scalar_type() == x.scalar_type(), "x and weight dtypes differ");
    at::Tensor w = w_in.contiguous();
    at::Tensor nbr = table_i32(nbr_in, n);
    c10::DeviceGuard g(x.device());
    at::Tensor bias;
    if (bias_present(bias_in)) bias = bias_in->to(x.device(), x.scalar_type()).contiguous();
    at::Tensor out = at::empty({n, c}, x.options());
    const int st = svtad_dw_fwd(x.data_ptr(), nbr.data_ptr<int32_t>(), w.data_ptr(),
                                bias.defined() ? bias.data_ptr() : nullptr, out.data_ptr(), n, (int)c,
                                tpb, dtype_code(x), stream_of(x));
    check_status(st, "dw_fwd");
    return out;
}

at::Tensor op_dw_bwd_in(const at::Tensor& go_in, const at::Tensor& nbr_in, const at::Tensor& w_in,
                        int64_t tpb, bool symmetric) {
    check_gpu(go_in, "grad_output");
    at::Tensor go = rows_view(go_in);
    const int64_t c = go.size(-1), n = n_rows(go);
    TORCH_CHECK(w_in.dim() == 2 && w_in.size(0) == 9 && w_in.size(1) == c,
                "depthwise weight must be (9, ", c, ")");
    TORCH_CHECK(w_in.scalar_type() == go.scalar_type(), "grad_output and weight dtypes differ");
    at::Tensor w = w_in.contiguous();
    at::Tensor nbr = table_i32(nbr_in, n);
    c10::DeviceGuard g(go.device());
    at::Tensor gi = at::empty({n, c}, go.options());
    const int st = svtad_dw_bwd_in_ex(go.data_ptr(), nbr.data_ptr<int32_t>(), w.data_ptr(), gi.data_ptr(), n,
                                      (int)c, tpb, dtype_code(go), table_flags(symmetric), stream_of(go));
    check_status(st, "dw_bwd_in");
    return gi;
}

std::tuple<at::Tensor, at::Tensor> op_dw_bwd_w(const at::Tensor& go_in, const at::Tensor& x_in,
                                               const at::Tensor& nbr_in, int64_t tpb,
                                               bool with_bias) {
    check_gpu(go_in, "grad_output");
    at::Tensor go = rows_view(go_in);
    at::Tensor x = rows_view(x_in);
    const int64_t c = x.size(-1), n = n_rows(x);
    TORCH_CHECK(go.size(-1) == c && n_rows(go) == n, "grad_output must match x's shape");
    TORCH_CHECK(go.scalar_type() == x.scalar_type(), "grad_output and x dtypes differ");
    at::Tensor nbr = table_i32(nbr_in, n);
    c10::DeviceGuard g(x.device());
    const int dt = dtype_code(x);
    const size_t ws_bytes = svtad_dw_bwd_w_workspace_bytes(n, (int)c, dt);
    TORCH_CHECK(ws_bytes > 0, "dw_bwd_w: ", svtad_last_error());
    at::Tensor ws = at::empty({(int64_t)ws_bytes}, x.options().dtype(at::kByte));
    at::Tensor gw = at::empty({9, c}, x.options());
    at::Tensor gb = with_bias ? at::empty({c}, x.options()) : at::empty({0}, x.options());
    const int st = svtad_dw_bwd_w(go.data_ptr(), x.data_ptr(), nbr.data_ptr<int32_t>(), gw.data_ptr(),
                                  with_bias ? gb.data_ptr() : nullptr, ws.data_ptr(), ws_bytes, n,
                                  (int)c, tpb, dt, stream_of(x));
    check_status(st, "dw_bwd_w");
    return {gw, gb};
}

// dw_bwd(grad_output, x, table, weight, tpb, with_bias) -> (grad_in, grad_w, grad_bias):
// dw_bwd_in and dw_bwd_w in one call (one pass over the rows + one reduction)
std::tuple<at::Tensor, at::Tensor, at::Tensor> op_dw_bwd(const at::Tensor& go_in, const at::Tensor& x_in,
                                                         const at::Tensor& nbr_in, const at::Tensor& w_in,
                                                         int64_t tpb, bool with_bias, bool symmetric) {
    check_gpu(go_in, "grad_output");
    at::Tensor go = rows_view(go_in);
    at::Tensor x = rows_view(x_in);
    const int64_t c = x.size(-1), n = n_rows(x);
    TORCH_CHECK(go.size(-1) == c && n_rows(go) == n, "grad_output must match x's shape");
    TORCH_CHECK(go.scalar_type() == x.scalar_type(), "grad_output and x dtypes differ");
    TORCH_CHECK(w_in.dim() == 2 && w_in.size(0) == 9 && w_in.size(1) == c,
                "depthwise weight must be (9, ", c, ")");
    TORCH_CHECK(w_in.scalar_type() == x.scalar_type(), "x and weight dtypes differ");
    at::Tensor w = w_in.contiguous();
    at::Tensor nbr = table_i32(nbr_in, n);
    c10::DeviceGuard g(x.device());
    const int dt = dtype_code(x);
    const size_t ws_bytes = svtad_dw_bwd_workspace_bytes(n, (int)c, dt);
    TORCH_CHECK(ws_bytes > 0, "dw_bwd: ", svtad_last_error());
    at::Tensor ws = at::empty({(int64_t)ws_bytes}, x.options().dtype(at::kByte));
    at::Tensor gi = at::empty({n, c}, x.options());
    at::Tensor gw = at::empty({9, c}, x.options());
    at::Tensor gb = with_bias ? at::empty({c}, x.options()) : at::empty({0}, x.options());
    const int st = svtad_dw_bwd_ex(go.data_ptr(), x.data_ptr(), nbr.data_ptr<int32_t>(), w.data_ptr(),
                                   gi.data_ptr(), gw.data_ptr(), with_bias ? gb.data_ptr() : nullptr, ws.data_ptr(),
                                   ws_bytes, n, (int)c, tpb, dt, table_flags(symmetric), stream_of(x));
    check_status(st, "dw_bwd");
    return {gi, gw, gb};
}

// ---------------------------------------------------------------------------
// neighbor tables
// ---------------------------------------------------------------------------

// build_neighbor_table(mask [..., H, W] bool/uint8) -> int32 [N, 9]
at::Tensor op_build_neighbor_table(const at::Tensor& mask_in) {
    check_gpu(mask_in, "mask");
    TORCH_CHECK(mask_in.dim() >= 2, "mask must be [..., H, W]");
    TORCH_CHECK(mask_in.scalar_type() == at::kBool || mask_in.scalar_type() == at::kByte,
                "mask must be bool or uint8");
    at::Tensor mask = mask_in.contiguous();
    if (mask.scalar_type() == at::kBool) mask = mask.view(at::kByte);
    const int64_t h = mask.size(-2), w = mask.size(-1);
    const int64_t frames = h * w == 0 ? 0 : mask.numel() / (h * w);
    c10::DeviceGuard g(mask.device());
    at::Tensor offs = at::empty({frames + 1}, mask.options().dtype(at::kInt));
    void* s = stream_of(mask);
    check_status(svtad_table_scan(mask.data_ptr<uint8_t>(), frames, (int)h, (int)w,
                                  offs.data_ptr<int32_t>(), s),
                 "build_neighbor_table");
    const int64_t n = offs[frames].item<int32_t>();  // host sync: sizes the output
    at::Tensor table = at::empty({n, 9}, mask.options().dtype(at::kInt));
    if (n == 0) return table;
    check_status(svtad_table_fill(mask.data_ptr<uint8_t>(), offs.data_ptr<int32_t>(), frames, (int)h,
                                  (int)w, table.data_ptr<int32_t>(), s),
                 "build_neighbor_table");
    return table;
}

// build_neighbor_table_n(mask [..., H, W], n_rows, int64_out) -> [n_rows, 9]: no host sync
// (the caller knows the kept count); masks past 4 MiB take scan + fill without a sync
at::Tensor op_build_neighbor_table_n(const at::Tensor& mask_in, int64_t n_rows, bool int64_out) {
    check_gpu(mask_in, "mask");
    TORCH_CHECK(mask_in.dim() >= 2, "mask must be [..., H, W]");
    TORCH_CHECK(mask_in.scalar_type() == at::kBool || mask_in.scalar_type() == at::kByte,
                "mask must be bool or uint8");
    TORCH_CHECK(n_rows >= 0, "n_rows must be >= 0");
    at::Tensor mask = mask_in.contiguous();
    if (mask.scalar_type() == at::kBool) mask = mask.view(at::kByte);
    if (((uintptr_t)mask.data_ptr() & 15) != 0) mask = mask.clone();
    const int64_t h = mask.size(-2), w = mask.size(-1);
    const int64_t frames = h * w == 0 ? 0 : mask.numel() / (h * w);
    c10::DeviceGuard g(mask.device());
    const auto idx_t = int64_out ? at::kLong : at::kInt;
    void* s = stream_of(mask);
    if (frames * h * w <= ((int64_t)4 << 20)) {
        at::Tensor table = at::empty({n_rows, 9}, mask.options().dtype(idx_t));
        check_status(svtad_table_build(mask.data_ptr<uint8_t>(), frames, (int)h, (int)w, n_rows, table.data_ptr(),
                                       int64_out ? 64 : 32, s),
                     "build_neighbor_table");
        return table;
    }
    // large masks: the scan + fill launches, into a buffer with a row for
    // every cell (the fill writes every kept cell, whatever n_rows says),
    // cut to n_rows
    at::Tensor offs = at::empty({frames + 1}, mask.options().dtype(at::kInt));
    check_status(svtad_table_scan(mask.data_ptr<uint8_t>(), frames, (int)h, (int)w, offs.data_ptr<int32_t>(), s),
                 "build_neighbor_table");
    at::Tensor t32 = at::full({std::max(n_rows, frames * h * w), 9}, -1, mask.options().dtype(at::kInt));
    check_status(svtad_table_fill(mask.data_ptr<uint8_t>(), offs.data_ptr<int32_t>(), frames, (int)h, (int)w,
                                  t32.data_ptr<int32_t>(), s),
                 "build_neighbor_table");
    t32 = t32.narrow(0, 0, n_rows).contiguous();
    return int64_out ? t32.to(at::kLong) : t32;
}

// grid_neighbor_table(frames, h, w, int64_out, like) -> [frames * h * w, 9] on like's device
at::Tensor op_grid_neighbor_table(int64_t frames, int64_t h, int64_t w, bool int64_out, const at::Tensor& like) {
    check_gpu(like, "like");
    TORCH_CHECK(frames >= 0 && h > 0 && w > 0, "bad grid");
    c10::DeviceGuard g(like.device());
    at::Tensor table = at::empty({frames * h * w, 9}, like.options().dtype(int64_out ? at::kLong : at::kInt));
    check_status(svtad_table_grid(frames, (int)h, (int)w, table.data_ptr(), int64_out ? 64 : 32, stream_of(like)),
                 "grid_neighbor_table");
    return table;
}

// table_to_global(table [..., 9] int32/int64, tokens_per_batch) -> int32 [rows, 9]: the
// max() < N heuristic on the device (no host sync)
at::Tensor op_table_to_global(const at::Tensor& table_in, int64_t tokens_per_batch) {
    check_gpu(table_in, "neighbor_indices");
    TORCH_CHECK(table_in.scalar_type() == at::kInt || table_in.scalar_type() == at::kLong,
                "neighbor_indices must be int32 or int64");
    TORCH_CHECK(table_in.numel() % 9 == 0, "neighbor_indices must have 9 entries per row");
    TORCH_CHECK(tokens_per_batch >= 0, "tokens_per_batch must be >= 0");
    at::Tensor table = table_in.contiguous();
    const int64_t rows = table.numel() / 9;
    c10::DeviceGuard g(table.device());
    at::Tensor out = at::empty({rows, 9}, table.options().dtype(at::kInt));
    if (rows == 0) return out;
    at::Tensor vmax = table.max();  // device scalar, no sync
    check_status(svtad_table_to_global(table.data_ptr(), table.scalar_type() == at::kLong ? 64 : 32, rows,
                                       tokens_per_batch, vmax.data_ptr(), out.data_ptr<int32_t>(), stream_of(table)),
                 "table_to_global");
    return out;
}

// remap_neighbor_table(table [B, N_prev, 9] int32, keep_idx [B, N_new] int64) -> [B, N_new, 9]
at::Tensor op_remap_neighbor_table(const at::Tensor& table_in, const at::Tensor& keep_in) {
    check_gpu(table_in, "table");
    check_gpu(keep_in, "keep_idx");
    TORCH_CHECK(table_in.dim() == 3 && table_in.size(2) == 9, "table must be [B, N_prev, 9]");
    TORCH_CHECK(table_in.scalar_type() == at::kInt, "table must be int32");
    TORCH_CHECK(keep_in.dim() == 2 && keep_in.size(0) == table_in.size(0), "keep_idx must be [B, N_new]");
    at::Tensor table = table_in.contiguous();
    at::Tensor keep = keep_in.to(at::kLong).contiguous();
    const int64_t B = table.size(0), n_prev = table.size(1), n_new = keep.size(1);
    c10::DeviceGuard g(table.device());
    at::Tensor mapping = at::empty({B * n_prev}, table.options());
    at::Tensor out = at::empty({B, n_new, 9}, table.options());
    check_status(svtad_remap_table(table.data_ptr<int32_t>(), B, n_prev, keep.data_ptr<int64_t>(),
                                   n_new, mapping.data_ptr<int32_t>(), out.data_ptr<int32_t>(),
                                   stream_of(table)),
                 "remap_neighbor_table");
    return out;
}

// prune_tokens(x [B, n_key + N_prev, ...], keep_idx [B, N_new] int64, last_idx [B, N_prev]
// int64 or empty, table [B, N_prev, 9] int32 or empty, n_key)
//   -> (x_out [B, n_key + N_new, ...], idx_out [B, N_new] or empty, table_out [B, N_new, 9] or empty)
std::tuple<at::Tensor, at::Tensor, at::Tensor> op_prune_tokens(const at::Tensor& x_in,
                                                               const at::Tensor& keep_in,
                                                               const at::Tensor& last_in,
                                                               const at::Tensor& table_in,
                                                               int64_t n_key) {
    check_gpu(x_in, "x");
    check_gpu(keep_in, "keep_idx");
    TORCH_CHECK(x_in.dim() >= 2, "x must be [B, n_key + N_prev, ...]");
    TORCH_CHECK(keep_in.dim() == 2 && keep_in.size(0) == x_in.size(0), "keep_idx must be [B, N_new]");
    const int64_t B = x_in.size(0);
    TORCH_CHECK(n_key >= 0 && n_key <= x_in.size(1), "num_key_tokens out of range");
    const int64_t n_prev = x_in.size(1) - n_key, n_new = keep_in.size(1);
    TORCH_CHECK(n_new <= n_prev, "keep_idx keeps more tokens than there are");
    at::Tensor x = x_in.contiguous();
    at::Tensor keep = keep_in.to(at::kLong).contiguous();
    const bool with_idx = last_in.defined() && last_in.numel() > 0;
    const bool with_table = table_in.defined() && table_in.numel() > 0;
    at::Tensor last, table;
    if (with_idx) {
        check_gpu(last_in, "last_idx");
        TORCH_CHECK(last_in.dim() == 2 && last_in.size(0) == B && last_in.size(1) == n_prev,
                    "last_idx must be [B, N_prev]");
        last = last_in.to(at::kLong).contiguous();
    }
    if (with_table) {
        check_gpu(table_in, "neighbor_indices");
        TORCH_CHECK(table_in.dim() == 3 && table_in.size(0) == B && table_in.size(1) == n_prev &&
                        table_in.size(2) == 9,
                    "neighbor_indices must be [B, N_prev, 9]");
        TORCH_CHECK(table_in.scalar_type() == at::kInt, "neighbor_indices must be int32");
        table = table_in.contiguous();
    }
    c10::DeviceGuard g(x.device());
    std::vector<int64_t> shape = x.sizes().vec();
    shape[1] = n_key + n_new;
    at::Tensor x_out = at::empty(shape, x.options());
    const int64_t rows_in = B * x.size(1);
    const int64_t row_bytes = rows_in > 0 ? x.numel() / rows_in * (int64_t)x.element_size() : 0;
    at::Tensor idx_out = with_idx ? at::empty({B, n_new}, last.options()) : at::empty({0}, keep.options());
    at::Tensor table_out = with_table ? at::empty({B, n_new, 9}, table.options())
                                      : at::empty({0}, keep.options().dtype(at::kInt));
    at::Tensor mapping = with_table ? at::empty({B * n_prev}, table.options()) : at::Tensor();
    check_status(svtad_prune_step(x.data_ptr(), B, n_key, n_prev, row_bytes, keep.data_ptr<int64_t>(),
                                  n_new, with_idx ? last.data_ptr<int64_t>() : nullptr,
                                  with_table ? table.data_ptr<int32_t>() : nullptr,
                                  with_table ? mapping.data_ptr<int32_t>() : nullptr, x_out.data_ptr(),
                                  with_idx ? idx_out.data_ptr<int64_t>() : nullptr,
                                  with_table ? table_out.data_ptr<int32_t>() : nullptr, stream_of(x)),
                 "prune_tokens");
    return {x_out, idx_out, table_out};
}

// transpose_neighbor_table(table [N, 9], tokens_per_batch) -> (table_t [N, 9], collisions [1])
std::tuple<at::Tensor, at::Tensor> op_transpose_neighbor_table(const at::Tensor& table_in,
                                                               int64_t tpb) {
    check_gpu(table_in, "table");
    TORCH_CHECK(table_in.scalar_type() == at::kInt, "table must be int32");
    TORCH_CHECK(table_in.numel() % 9 == 0, "table must have 9 entries per row");
    at::Tensor table = table_in.contiguous();
    const int64_t n = table.numel() / 9;
    c10::DeviceGuard g(table.device());
    at::Tensor tt = at::empty({n, 9}, table.options());
    at::Tensor coll = at::zeros({1}, table.options());
    check_status(svtad_transpose_table(table.data_ptr<int32_t>(), n, tpb, tt.data_ptr<int32_t>(),
                                       coll.data_ptr<int32_t>(), stream_of(table)),
                 "transpose_neighbor_table");
    return {tt, coll};
}

// validate_neighbor_table(table, bound) -> int32 [3] = (entries out of range, min, max)
at::Tensor op_validate_neighbor_table(const at::Tensor& table_in, int64_t bound) {
    check_gpu(table_in, "table");
    TORCH_CHECK(table_in.scalar_type() == at::kInt, "table must be int32");
    at::Tensor table = table_in.contiguous();
    c10::DeviceGuard g(table.device());
    at::Tensor stats = at::empty({3}, table.options());
    check_status(svtad_validate_table(table.data_ptr<int32_t>(), table.numel(), bound,
                                      stats.data_ptr<int32_t>(), stream_of(table)),
                 "validate_neighbor_table");
    return stats;
}

// Adapter GEMMs with fused epilogues (f16 / bf16).
void adapter_common(const at::Tensor& t, const at::Tensor& w, const char* name) {
    check_gpu(t, name);
    check_gpu(w, "weight");
    TORCH_CHECK(t.scalar_type() == w.scalar_type(), name, " and weight dtypes differ");
    TORCH_CHECK(t.scalar_type() == at::kHalf || t.scalar_type() == at::kBFloat16,
                "adapter GEMMs take float16 / bfloat16, got ", t.scalar_type());
    TORCH_CHECK(w.dim() == 2, "weight must be (out_features, in_features)");
}

const void* opt_ptr(const c10::optional<at::Tensor>& b, int64_t n, const at::Tensor& like) {
    if (!bias_present(b)) return nullptr;
    TORCH_CHECK(b->numel() == n && b->scalar_type() == like.scalar_type() && b->is_cuda(),
                "bias must have ", n, " elements of the input dtype");
    TORCH_CHECK(b->is_contiguous(), "bias must be contiguous");
    return b->data_ptr();
}

// adapter_down(x [B, N, k], weight [n, k], bias [n] or None, n_special)
//   -> (pre_act [B, N, n], act_special [B, S, n], act_patch [B * (N - S), n])
std::tuple<at::Tensor, at::Tensor, at::Tensor> op_adapter_down(const at::Tensor& x_in, const at::Tensor& w_in,
                                                               const c10::optional<at::Tensor>& bias,
                                                               int64_t n_special) {
    adapter_common(x_in, w_in, "x");
    TORCH_CHECK(x_in.dim() == 3, "x must be [B, N, C]");
    const int64_t B = x_in.size(0), N = x_in.size(1), k = x_in.size(2), n = w_in.size(0);
    TORCH_CHECK(w_in.size(1) == k, "weight must be (n, ", k, ")");
    TORCH_CHECK(n_special >= 0 && n_special <= N, "n_special out of range");
    at::Tensor x = x_in.contiguous(), w = w_in.contiguous();
    c10::DeviceGuard g(x.device());
    at::Tensor pre = at::empty({B, N, n}, x.options());
    at::Tensor sp = at::empty({B, n_special, n}, x.options());
    at::Tensor pa = at::empty({B * (N - n_special), n}, x.options());
    check_status(svtad_adapter_down(x.data_ptr(), w.data_ptr(), opt_ptr(bias, n, x), pre.data_ptr(),
                                    sp.numel() ? sp.data_ptr() : nullptr, pa.numel() ? pa.data_ptr() : nullptr,
                                    B, N, n_special, (int)k, (int)n, dtype_code(x), stream_of(x)),
                 "adapter_down");
    return {pre, sp, pa};
}

// adapter_up(a_special [B, S, k], a_patch [B * (N - S), k], weight [n, k], bias [n] or None,
//            gamma [1], residual [B, N, n], out_float32=False) -> out [B, N, n]
// a_special, a_patch, weight and bias share the compute dtype T (f16 / bf16).
// gamma and the residual are T, or float32 (the reference under autocast,
// where gamma is a float32 parameter): then z * gamma is an fp32 product and
// the add is fp32, and out is float32 with out_float32, else rounded once to
// T. With a T gamma, residual and out are T.
at::Tensor op_adapter_up(const at::Tensor& sp_in, const at::Tensor& pa_in, const at::Tensor& w_in,
                         const c10::optional<at::Tensor>& bias, const at::Tensor& gamma_in,
                         const at::Tensor& res_in, bool out_float32) {
    check_gpu(res_in, "residual");
    adapter_common(pa_in, w_in, "a_patch");
    TORCH_CHECK(res_in.dim() == 3, "residual must be [B, N, C]");
    const int64_t B = res_in.size(0), N = res_in.size(1), n = res_in.size(2), k = w_in.size(1);
    TORCH_CHECK(w_in.size(0) == n, "weight must be (", n, ", k)");
    TORCH_CHECK(sp_in.dim() == 3 && sp_in.size(0) == B && sp_in.size(2) == k, "a_special must be [B, S, k]");
    const int64_t S = sp_in.size(1);
    TORCH_CHECK(S <= N && pa_in.dim() == 2 && pa_in.size(0) == B * (N - S) && pa_in.size(1) == k,
                "a_patch must be [B * (N - S), k]");
    const at::ScalarType t = pa_in.scalar_type();
    TORCH_CHECK(sp_in.scalar_type() == t, "a_special and a_patch must share the dtype");
    auto t_or_f32 = [&](const at::Tensor& v) { return v.scalar_type() == t || v.scalar_type() == at::kFloat; };
    TORCH_CHECK(t_or_f32(gamma_in) && t_or_f32(res_in), "gamma and residual must be of the input dtype or float32");
    const bool g32 = gamma_in.scalar_type() == at::kFloat;
    TORCH_CHECK(g32 || (res_in.scalar_type() == t && !out_float32),
                "a float32 residual or output needs a float32 gamma");
    TORCH_CHECK(gamma_in.numel() == 1 && gamma_in.is_cuda(), "gamma must be one element on the GPU");
    at::Tensor sp = sp_in.contiguous(), pa = pa_in.contiguous(), w = w_in.contiguous(),
               res = res_in.contiguous(), gm = gamma_in.contiguous();
    c10::DeviceGuard g(res.device());
    at::Tensor out = at::empty({B, N, n}, res.options().dtype(out_float32 ? at::kFloat : t));
    const int dt = dtype_code(pa);
    check_status(svtad_adapter_up_mixed(sp.numel() ? sp.data_ptr() : nullptr, pa.numel() ? pa.data_ptr() : nullptr,
                                        w.data_ptr(), opt_ptr(bias, n, pa), gm.data_ptr(), res.data_ptr(),
                                        out.data_ptr(), B, N, S, (int)k, (int)n, dt, dtype_code(gm),
                                        dtype_code(res), dtype_code(out), stream_of(res)),
                 "adapter_up");
    return out;
}

// heatmap_add_(patch [R, C], special [*, C], src_rows int32 [R], gate [1]) -> patch,
// in place: patch[i] += special[src_rows[i]] * gate (rounded as the unfused chain)
at::Tensor op_heatmap_add_(at::Tensor patch, const at::Tensor& special_in, const at::Tensor& src_in,
                           const at::Tensor& gate_in) {
    adapter_common(patch, patch, "patch");
    TORCH_CHECK(patch.dim() == 2 && patch.is_contiguous(), "patch must be a contiguous [rows, cols] tensor");
    check_gpu(special_in, "special");
    check_gpu(src_in, "src_rows");
    check_gpu(gate_in, "gate");
    TORCH_CHECK(special_in.scalar_type() == patch.scalar_type() &&
                    (gate_in.scalar_type() == patch.scalar_type() || gate_in.scalar_type() == at::kFloat),
                "special and patch must share the dtype; gate is of that dtype or float32");
    const int64_t rows = patch.size(0), cols = patch.size(1);
    TORCH_CHECK(special_in.size(-1) == cols, "special must have ", cols, " columns");
    TORCH_CHECK(src_in.scalar_type() == at::kInt && src_in.numel() == rows, "src_rows must be int32 [rows]");
    TORCH_CHECK(gate_in.numel() == 1, "gate must be one element");
    at::Tensor sp = special_in.contiguous(), src = src_in.contiguous(), gate = gate_in.contiguous();
    c10::DeviceGuard g(patch.device());
    check_status(svtad_heatmap_add_mixed(patch.data_ptr(), sp.numel() ? sp.data_ptr() : nullptr,
                                         src.data_ptr<int32_t>(), gate.data_ptr(), rows, n_rows(sp), (int)cols,
                                         dtype_code(patch), dtype_code(gate), stream_of(patch)),
                 "heatmap_add_");
    return patch;
}

// linear_wgrad(g [*, c_g], rows int32 [n] or empty, x [n, c_x], out_float32=False) -> out [c_g, c_x]
// (in x's dtype, or the unrounded fp32 sums with out_float32)
// (out = g[rows]^T x, or g^T x with the first n rows of g when rows is empty)
at::Tensor op_linear_wgrad(const at::Tensor& g_in, const at::Tensor& rows_in, const at::Tensor& x_in,
                           bool out_float32) {
    adapter_common(g_in, g_in, "g");
    check_gpu(x_in, "x");
    TORCH_CHECK(x_in.scalar_type() == g_in.scalar_type(), "g and x dtypes differ");
    TORCH_CHECK(g_in.dim() == 2 && x_in.dim() == 2, "g and x must be 2-D");
    const int64_t n = x_in.size(0), c_g = g_in.size(1), c_x = x_in.size(1);
    const bool with_rows = rows_in.defined() && rows_in.numel() > 0;
    at::Tensor rows;
    if (with_rows) {
        check_gpu(rows_in, "rows");
        TORCH_CHECK(rows_in.scalar_type() == at::kInt && rows_in.numel() == n, "rows must be int32 [n]");
        rows = rows_in.contiguous();
    } else {
        TORCH_CHECK(g_in.size(0) >= n, "g has fewer rows than x");
    }
    at::Tensor g = g_in.contiguous(), x = x_in.contiguous();
    c10::DeviceGuard guard(x.device());
    at::Tensor out = at::empty({c_g, c_x}, x.options().dtype(out_float32 ? at::kFloat : x.scalar_type()));
    const size_t ws = svtad_linear_wgrad_workspace_bytes(n, (int)c_g, (int)c_x, dtype_code(x));
    at::Tensor work = at::empty({(int64_t)std::max<size_t>(ws, 1)}, x.options().dtype(at::kByte));
    check_status(svtad_linear_wgrad_mixed(g.data_ptr(), with_rows ? rows.data_ptr<int32_t>() : nullptr,
                                          x.data_ptr(), out.data_ptr(), work.data_ptr(), ws, n, g.size(0),
                                          (int)c_g, (int)c_x, dtype_code(x), dtype_code(out), stream_of(x)),
                 "linear_wgrad");
    return out;
}

// column_sums(a [rows, cols]) -> [cols]: sum over rows, fp32 accumulation, ordered
at::Tensor op_column_sums(const at::Tensor& a_in) {
    adapter_common(a_in, a_in, "a");
    at::Tensor a = a_in.contiguous();
    const int64_t rows = a.size(0), cols = a.size(1);
    c10::DeviceGuard guard(a.device());
    at::Tensor out = at::empty({cols}, a.options());
    const size_t ws = svtad_column_sums_workspace_bytes(rows, (int)cols, dtype_code(a));
    at::Tensor work = at::empty({(int64_t)std::max<size_t>(ws, 1)}, a.options().dtype(at::kByte));
    check_status(svtad_column_sums(a.data_ptr(), out.data_ptr(), work.data_ptr(), ws, rows, (int)cols,
                                   dtype_code(a), stream_of(a)),
                 "column_sums");
    return out;
}

// gelu_backward_split(grad_special [B, S, n] or None, grad_patch [B * (N - S), n] or None,
//                     pre_act [B, N, n], n_special) -> grad_pre [B, N, n]
at::Tensor op_gelu_backward_split(const c10::optional<at::Tensor>& g_sp, const c10::optional<at::Tensor>& g_pa,
                                  const at::Tensor& pre_in, int64_t n_special) {
    check_gpu(pre_in, "pre_act");
    TORCH_CHECK(pre_in.scalar_type() == at::kHalf || pre_in.scalar_type() == at::kBFloat16,
                "gelu_backward_split takes float16 / bfloat16, got ", pre_in.scalar_type());
    TORCH_CHECK(pre_in.dim() == 3, "pre_act must be [B, N, n]");
    const int64_t B = pre_in.size(0), N = pre_in.size(1), n = pre_in.size(2);
    TORCH_CHECK(n_special >= 0 && n_special <= N, "n_special out of range");
    at::Tensor pre = pre_in.contiguous(), sp, pa;
    if (g_sp.has_value() && g_sp->defined() && g_sp->numel() > 0) {
        check_gpu(*g_sp, "grad_special");
        TORCH_CHECK(g_sp->scalar_type() == pre.scalar_type() && g_sp->numel() == B * n_special * n,
                    "grad_special must be [B, S, n] of the pre_act dtype");
        sp = g_sp->contiguous();
    }
    if (g_pa.has_value() && g_pa->defined() && g_pa->numel() > 0) {
        check_gpu(*g_pa, "grad_patch");
        TORCH_CHECK(g_pa->scalar_type() == pre.scalar_type() && g_pa->numel() == B * (N - n_special) * n,
                    "grad_patch must be [B * (N - S), n] of the pre_act dtype");
        pa = g_pa->contiguous();
    }
    c10::DeviceGuard g(pre.device());
    at::Tensor out = at::empty_like(pre);
    check_status(svtad_gelu_backward_split(sp.defined() ? sp.data_ptr() : nullptr,
                                           pa.defined() ? pa.data_ptr() : nullptr, pre.data_ptr(),
                                           out.data_ptr(), B, N, n_special, (int)n, dtype_code(pre),
                                           stream_of(pre)),
                 "gelu_backward_split");
    return out;
}

// gamma_grad(w, g, b or None, gs or None) -> [1]: sum(w * g) + sum(b * gs), fp32, ordered
at::Tensor op_gamma_grad(const at::Tensor& w_in, const at::Tensor& g_in, const c10::optional<at::Tensor>& b_in,
                         const c10::optional<at::Tensor>& gs_in) {
    check_gpu(w_in, "w");
    check_gpu(g_in, "g");
    TORCH_CHECK(w_in.scalar_type() == g_in.scalar_type(), "w and g dtypes differ");
    TORCH_CHECK(w_in.scalar_type() == at::kHalf || w_in.scalar_type() == at::kBFloat16,
                "gamma_grad takes float16 / bfloat16, got ", w_in.scalar_type());
    TORCH_CHECK(w_in.numel() == g_in.numel(), "w and g must have the same size");
    at::Tensor w = w_in.contiguous(), g = g_in.contiguous(), b, gs;
    if (bias_present(b_in)) {
        TORCH_CHECK(gs_in.has_value() && gs_in->defined() && gs_in->numel() == b_in->numel(),
                    "gs must match b");
        check_gpu(*b_in, "b");
        check_gpu(*gs_in, "gs");
        TORCH_CHECK(b_in->scalar_type() == w.scalar_type() && gs_in->scalar_type() == w.scalar_type(),
                    "b and gs must have the dtype of w");
        b = b_in->contiguous();
        gs = gs_in->contiguous();
    }
    c10::DeviceGuard guard(w.device());
    at::Tensor out = at::empty({1}, w.options());
    const size_t wsb = svtad_gamma_grad_workspace_bytes();
    at::Tensor work = at::empty({(int64_t)wsb}, w.options().dtype(at::kByte));
    check_status(svtad_gamma_grad(w.data_ptr(), g.data_ptr(), w.numel(), b.defined() ? b.data_ptr() : nullptr,
                                  gs.defined() ? gs.data_ptr() : nullptr, b.defined() ? b.numel() : 0,
                                  out.data_ptr(), nullptr, nullptr, nullptr, nullptr, work.data_ptr(), wsb,
                                  dtype_code(w), stream_of(w)),
                 "gamma_grad");
    return out;
}

// up_proj_grads(w, g, b or None, gs or None, gamma [1]) ->
//   (grad_gamma [1], w * gamma, g * gamma, gs * gamma or empty): the gamma
//   gradient and the gamma-scaled tensors of the adapter's up-projection
//   backward in one pass. gamma is of w's dtype or float32 (the reference's
//   autocast training); grad_gamma has gamma's dtype, the scaled tensors w's.
//   g may be float32 (linear_wgrad's unrounded sums): g * gamma is then its
//   only rounding.
std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> op_up_proj_grads(
    const at::Tensor& w_in, const at::Tensor& g_in, const c10::optional<at::Tensor>& b_in,
    const c10::optional<at::Tensor>& gs_in, const at::Tensor& gamma_in) {
    check_gpu(w_in, "w");
    check_gpu(g_in, "g");
    check_gpu(gamma_in, "gamma");
    TORCH_CHECK((g_in.scalar_type() == w_in.scalar_type() || g_in.scalar_type() == at::kFloat) &&
                    (gamma_in.scalar_type() == w_in.scalar_type() || gamma_in.scalar_type() == at::kFloat),
                "g and gamma must be of w's dtype or float32");
    TORCH_CHECK(w_in.scalar_type() == at::kHalf || w_in.scalar_type() == at::kBFloat16,
                "up_proj_grads takes float16 / bfloat16, got ", w_in.scalar_type());
    TORCH_CHECK(w_in.numel() == g_in.numel() && gamma_in.numel() == 1, "w and g must match; gamma one element");
    at::Tensor w = w_in.contiguous(), g = g_in.contiguous(), gm = gamma_in.contiguous(), b, gs;
    if (bias_present(b_in)) {
        TORCH_CHECK(gs_in.has_value() && gs_in->defined() && gs_in->numel() == b_in->numel(), "gs must match b");
        check_gpu(*b_in, "b");
        check_gpu(*gs_in, "gs");
        TORCH_CHECK(b_in->scalar_type() == w.scalar_type() && gs_in->scalar_type() == w.scalar_type(),
                    "b and gs must have the dtype of w");
        b = b_in->contiguous();
        gs = gs_in->contiguous();
    }
    c10::DeviceGuard guard(w.device());
    at::Tensor out = at::empty({1}, gm.options());  // the gradient of gamma has gamma's dtype
    at::Tensor w_sc = at::empty_like(w), g_sc = at::empty_like(g, g.options().dtype(w.scalar_type()));
    at::Tensor gs_sc = b.defined() ? at::empty_like(gs) : at::empty({0}, w.options());
    const size_t wsb = svtad_gamma_grad_workspace_bytes();
    at::Tensor work = at::empty({(int64_t)wsb}, w.options().dtype(at::kByte));
    check_status(svtad_gamma_grad_mixed(w.data_ptr(), g.data_ptr(), w.numel(), b.defined() ? b.data_ptr() : nullptr,
                                        gs.defined() ? gs.data_ptr() : nullptr, b.defined() ? b.numel() : 0,
                                        out.data_ptr(), gm.data_ptr(), w_sc.data_ptr(), g_sc.data_ptr(),
                                        b.defined() ? gs_sc.data_ptr() : nullptr, work.data_ptr(), wsb,
                                        dtype_code(w), dtype_code(g), dtype_code(gm), stream_of(w)),
                 "up_proj_grads");
    return {out, w_sc, g_sc, gs_sc};
}

PYBIND11_MODULE(opentad_sparse_ops, m) {
    m.doc() = "MI355X (gfx950) SparseConv2D: drop-in for the reference opentad_sparse_ops";
    m.def("fwd", &op_fwd, "Forward", py::arg("x"), py::arg("neighbor_indices"), py::arg("weight"),
          py::arg("C_out"), py::arg("tokens_per_batch"));
    m.def("bwd_in", &op_bwd_in, "Backward Input", py::arg("grad_output"),
          py::arg("neighbor_indices"), py::arg("weight"), py::arg("n_kept"), py::arg("C_in"),
          py::arg("tokens_per_batch"));
    m.def("bwd_w", &op_bwd_w, "Backward Weight", py::arg("grad_output"), py::arg("x"),
          py::arg("neighbor_indices"), py::arg("C_in"), py::arg("tokens_per_batch"));
    m.def("implicit_gemm_fwd_v2", &op_implicit_gemm_fwd_v2, "Implicit GEMM forward (fused bias)",
          py::arg("x"), py::arg("neighbor_indices"), py::arg("weight"), py::arg("bias"),
          py::arg("tokens_per_batch"));
    m.def("implicit_gemm_fwd_v2_chunked", &op_implicit_gemm_fwd_v2_chunked,
          "Implicit GEMM forward (chunk_size accepted, not needed)", py::arg("x"),
          py::arg("neighbor_indices"), py::arg("weight"), py::arg("bias"),
          py::arg("tokens_per_batch"), py::arg("chunk_size"));
    m.def("fwd_bias", &op_fwd_bias, "Forward with bias_mode 0 none / 1 fp32 / 2 after rounding",
          py::arg("x"), py::arg("neighbor_indices"), py::arg("weight"), py::arg("bias"),
          py::arg("tokens_per_batch"), py::arg("bias_mode"));
    m.def("pack_weight", &op_pack_weight, "Weight in the matrix-core fragment order (fwd, bwd_in)",
          py::arg("weight"), py::arg("fwd") = true, py::arg("bwd") = true);
    m.def("fwd_packed", &op_fwd_packed, "fwd_bias with a packed weight", py::arg("x"),
          py::arg("neighbor_indices"), py::arg("weight"), py::arg("packed_fwd"), py::arg("bias"),
          py::arg("tokens_per_batch"), py::arg("bias_mode"));
    m.def("bwd_in_packed", &op_bwd_in_packed, "bwd_in with a packed weight", py::arg("grad_output"),
          py::arg("neighbor_indices"), py::arg("weight"), py::arg("packed_bwd"), py::arg("n_kept"),
          py::arg("C_in"), py::arg("tokens_per_batch"), py::arg("symmetric") = false);
    m.def("bwd_packed", &op_bwd_packed, "bwd_in_packed + bwd_w_bias in one call",
          py::arg("grad_output"), py::arg("x"), py::arg("neighbor_indices"), py::arg("weight"),
          py::arg("packed_bwd"), py::arg("C_in"), py::arg("tokens_per_batch"), py::arg("with_bias"),
          py::arg("symmetric") = false);
    m.def("bwd_in_gemm", &op_bwd_in_gemm, "Backward-input gathered GEMM only (timing)", py::arg("grad_output"),
          py::arg("neighbor_indices"), py::arg("packed_bwd"), py::arg("C_in"), py::arg("tokens_per_batch"),
          py::arg("symmetric") = false);
    m.def("bwd_w_partials", &op_bwd_w_partials, "Backward-weight partial sums only (timing)",
          py::arg("grad_output"), py::arg("x"), py::arg("neighbor_indices"), py::arg("C_in"),
          py::arg("tokens_per_batch"), py::arg("with_bias"));
    m.def("bwd_w_bias", &op_bwd_w_bias, "Backward weight and bias", py::arg("grad_output"),
          py::arg("x"), py::arg("neighbor_indices"), py::arg("C_in"), py::arg("tokens_per_batch"),
          py::arg("with_bias"));
    m.def("dw_fwd", &op_dw_fwd, "Depthwise forward", py::arg("x"), py::arg("neighbor_indices"),
          py::arg("weight"), py::arg("bias"), py::arg("tokens_per_batch"));
    m.def("dw_bwd_in", &op_dw_bwd_in, "Depthwise backward input", py::arg("grad_output"),
          py::arg("neighbor_indices"), py::arg("weight"), py::arg("tokens_per_batch"),
          py::arg("symmetric") = false);
    m.def("dw_bwd", &op_dw_bwd, "Depthwise backward input, weight and bias in one call",
          py::arg("grad_output"), py::arg("x"), py::arg("neighbor_indices"), py::arg("weight"),
          py::arg("tokens_per_batch"), py::arg("with_bias"), py::arg("symmetric") = false);
    m.def("dw_bwd_w", &op_dw_bwd_w, "Depthwise backward weight and bias", py::arg("grad_output"),
          py::arg("x"), py::arg("neighbor_indices"), py::arg("tokens_per_batch"),
          py::arg("with_bias"));
    m.def("build_neighbor_table", &op_build_neighbor_table, "Neighbor table from a keep mask",
          py::arg("mask"));
    m.def("build_neighbor_table_n", &op_build_neighbor_table_n,
          "Neighbor table from a keep mask with a known row count (one launch, no host sync)",
          py::arg("mask"), py::arg("n_rows"), py::arg("int64_out") = false);
    m.def("grid_neighbor_table", &op_grid_neighbor_table, "Full-grid neighbor table in closed form (one launch)",
          py::arg("frames"), py::arg("h"), py::arg("w"), py::arg("int64_out"), py::arg("like"));
    m.def("table_to_global", &op_table_to_global,
          "int32 global table from a local or global one by the max() < N rule, on the device",
          py::arg("neighbor_indices"), py::arg("tokens_per_batch"));
    m.def("remap_neighbor_table", &op_remap_neighbor_table, "Neighbor table remap after a prune",
          py::arg("table"), py::arg("keep_idx"));
    m.def("prune_tokens", &op_prune_tokens,
          "Fused prune step: kept-token gather, index gather and table remap",
          py::arg("x"), py::arg("keep_idx"), py::arg("last_idx"), py::arg("neighbor_indices"),
          py::arg("num_key_tokens"));
    m.def("transpose_neighbor_table", &op_transpose_neighbor_table, "Transposed neighbor table",
          py::arg("table"), py::arg("tokens_per_batch") = 0);
    m.def("validate_neighbor_table", &op_validate_neighbor_table,
          "(out-of-range count, min, max) of a neighbor table", py::arg("table"), py::arg("bound"));
    m.def("adapter_down", &op_adapter_down, "Adapter down_proj + GELU + special / patch split",
          py::arg("x"), py::arg("weight"), py::arg("bias"), py::arg("n_special"));
    m.def("adapter_up", &op_adapter_up, "Adapter up_proj on cat(special, patch) * gamma + residual",
          py::arg("a_special"), py::arg("a_patch"), py::arg("weight"), py::arg("bias"), py::arg("gamma"),
          py::arg("residual"), py::arg("out_float32") = false);
    m.def("heatmap_add_", &op_heatmap_add_, "In place: patch[i] += special[src_rows[i]] * gate (adapter heatmap injection)",
          py::arg("patch"), py::arg("special"), py::arg("src_rows"), py::arg("gate"));
    m.def("linear_wgrad", &op_linear_wgrad, "Linear-layer weight gradient g[rows]^T x (split rows, ordered sum)",
          py::arg("g"), py::arg("rows"), py::arg("x"), py::arg("out_float32") = false);
    m.def("column_sums", &op_column_sums, "Column sums of a [rows, cols] matrix (ordered, fp32 accumulation)",
          py::arg("a"));
    m.def("gelu_backward_split", &op_gelu_backward_split,
          "GELU backward of the adapter's down projection from split special / patch gradients",
          py::arg("grad_special"), py::arg("grad_patch"), py::arg("pre_act"), py::arg("n_special"));
    m.def("up_proj_grads", &op_up_proj_grads,
          "Adapter up projection: gamma gradient plus w, g, gs scaled by gamma, in one pass",
          py::arg("w"), py::arg("g"), py::arg("b"), py::arg("gs"), py::arg("gamma"));
    m.def("gamma_grad", &op_gamma_grad, "sum(w * g) + sum(b * gs) in fp32 (the adapter's gamma gradient)",
          py::arg("w"), py::arg("g"), py::arg("b"), py::arg("gs"));
    m.def("version", []() { return std::string(svtad_version()); });
}
