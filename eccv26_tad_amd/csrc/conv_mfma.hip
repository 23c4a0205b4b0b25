// MFMA (matrix core) SparseConv2D kernels for f16 / bf16.
#include "sv_common.h"
#include "sv_conv.h"

namespace svtad {

bool gg_mfma_supported(int, int, int) { return false; }
void gg_mfma(int, int, const void*, const int32_t*, const void*, const void*, int, void*, int64_t,
             int, int, int64_t, hipStream_t) {}
bool bw_mfma_supported(int, int, int) { return false; }
void bw_mfma(int, const BwPlan&, const void*, const void*, const int32_t*, void*, void*, void*,
             int64_t, int, int, int64_t, hipStream_t) {}

}  // namespace svtad
