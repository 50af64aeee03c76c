// C ABI housekeeping: version, error strings, per-thread error detail.
#include <stdarg.h>
#include <stdio.h>

#include "pgs_common.h"

namespace pgs {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(PGS_ERR_LAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  }
  return PGS_OK;
}

}  // namespace pgs

extern "C" {

int pgs_abi_version(void) { return 6; }

const char* pgs_error_string(int code) {
  switch (code) {
    case PGS_OK: return "ok";
    case PGS_ERR_INVALID_ARGUMENT: return "invalid argument";
    case PGS_ERR_MISALIGNED: return "misaligned pointer";
    case PGS_ERR_LAUNCH: return "kernel launch failed";
    case PGS_ERR_NO_DEVICE: return "no usable gfx950 device";
    default: return "unknown error";
  }
}

const char* pgs_last_error(void) { return pgs::g_last_error; }

}  // extern "C"
