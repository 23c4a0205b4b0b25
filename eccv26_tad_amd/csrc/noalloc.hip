// Allocation-free SparseConv2D forward: svtad_fwd with its workspace (the
// weight in matrix-core fragment order) in a static device array instead of
// a caller buffer, for callers that cannot allocate (code under HIP graph
// capture, serving loops, harnesses that forbid hipMalloc).
#include <mutex>

#include "sv_common.h"
#include "sv_conv.h"
#include "sv_internal.h"

namespace svtad {

// Largest packed weight the array holds: 9 * c_in * c_out 16-bit values
// (C = 512: 4.5 MiB). Every GPU the library runs on holds its own copy until
// the process ends.
constexpr size_t kFwdScratchBytes = (size_t)8 << 20;

static __device__ __align__(256) unsigned char scratch[kFwdScratchBytes];

// Device address of `scratch` per device, looked up once per device with that
// device current (in host code the array's name is not a device address).
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64];

static int scratch_ptr(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return set_error(SVTAD_ERR_INVALID, "fwd_noalloc: no current device");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return set_error(SVTAD_ERR_INVALID, "fwd_noalloc: hipGetSymbolAddress failed");
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return SVTAD_OK;
}

}  // namespace svtad

using namespace svtad;

extern "C" size_t svtad_fwd_noalloc_max_workspace_bytes(void) { return kFwdScratchBytes; }

extern "C" int svtad_fwd_noalloc(const void* x, const int32_t* nbr, const void* weight, const void* bias,
                                 int bias_mode, void* out, int64_t n, int c_in, int c_out,
                                 int64_t tokens_per_batch, int dtype, void* stream) {
    const size_t need = svtad_fwd_workspace_bytes(c_in, c_out, dtype);
    if (need > kFwdScratchBytes)
        return set_error(SVTAD_ERR_UNSUPPORTED,
                         "fwd_noalloc: the packed weight (9 * c_in * c_out 16-bit values) exceeds the 8 MiB "
                         "static workspace; use svtad_fwd with a caller workspace");
    void* ws = nullptr;
    if (need) {
        const int st = scratch_ptr(&ws);
        if (st) return st;
    }
    return svtad_fwd(x, nbr, weight, bias, bias_mode, out, ws, need, n, c_in, c_out, tokens_per_batch, dtype,
                     stream);
}
