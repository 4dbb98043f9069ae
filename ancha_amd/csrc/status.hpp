// Failure reporting shared by every C entry point of include/ancha_hip.h: the calling thread's
// last-error text and the process-wide sticky HIP failure (defined in capi.hip).
//
// A HIP runtime error is sticky, like the reference's device::check (src/device.rs:11-41):
// once one is recorded every entry point returns it again without launching anything.
#pragma once
#include <hip/hip_runtime.h>

#include <string>

namespace ancha {

// Records `msg` as the calling thread's last error and returns `code`.
int fail(int code, const std::string& msg);

// Records the HIP failure `e` (the first one becomes the sticky state) and returns -(e).
int hip_fail(hipError_t e, const std::string& where);

// 0 for hipSuccess, else hip_fail(e, where).
inline int hip_status(hipError_t e, const char* where) {
  return e == hipSuccess ? 0 : hip_fail(e, where);
}

// The sticky failure code, or 0; a non-zero state also becomes the last-error text.
int sticky();

}  // namespace ancha
