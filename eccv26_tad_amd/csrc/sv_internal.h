// Host-side helpers shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace svtad {

constexpr int64_t kMaxFrameCells = 16384;

// Records `msg` as this thread's last error and returns `code`.
int set_error(int code, const char* msg);

// hipGetLastError() after a launch sequence: SVTAD_OK or the HIP error code.
int launch_status();

}  // namespace svtad
