// Internal interface between the runtime core (runtime.cpp) and the compute
// entry points compiled into the same library (entry.hip).  Not part of the
// C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <functional>
#include <string>

namespace nkh_internal {

// Sets the calling thread's last-error text and returns `code`.
int set_error(int code, const std::string &msg);
// Formats a HIP error and returns NKH_ERR_HIP.
int hip_error(hipError_t e, const char *what);
// Runs fn(stream, device) under the runtime lock if the runtime is
// initialized; otherwise returns NKH_ERR_NOT_INIT.
int with_stream(const std::function<int(hipStream_t, int)> &fn);
// Per-device set-up of the entry points (entry.hip), run by nkh_init with
// the device current.
int device_setup(int device);

}  // namespace nkh_internal
