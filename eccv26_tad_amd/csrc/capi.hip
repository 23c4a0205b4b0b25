// Error reporting and version of the C ABI.
#include <stdio.h>
#include <string.h>

#include "sv_common.h"
#include "sv_internal.h"

namespace svtad {

static thread_local char g_msg[512] = "";

int set_error(int code, const char* msg) {
    snprintf(g_msg, sizeof(g_msg), "%s", msg);
    return code;
}

int launch_status() {
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) return SVTAD_OK;
    snprintf(g_msg, sizeof(g_msg), "HIP launch failed: %s", hipGetErrorString(e));
    return (int)e;
}

}  // namespace svtad

extern "C" const char* svtad_last_error(void) { return svtad::g_msg; }

extern "C" const char* svtad_version(void) { return "svtad_sparse 0.1 gfx950"; }
