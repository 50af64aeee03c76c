// C ABI housekeeping: version, error strings, per-thread error detail, the
// device check every launching entry point makes, the per-thread record of
// the last linear launch plan, and the stream capture query.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>

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

// Architecture of each device, checked once: 0 = not yet, 1 = gfx950, 2 = other.
static std::atomic<int> g_dev_arch[kMaxDevices];

int stream_device(hipStream_t st, int* dev) {
  hipError_t e = st ? hipStreamGetDevice(st, dev) : hipGetDevice(dev);
  if (e != hipSuccess || *dev < 0) {
    (void)hipGetLastError();
    return fail(PGS_ERR_NO_DEVICE, "no usable HIP device for the stream (%s)", hipGetErrorString(e));
  }
  return PGS_OK;
}

int require_device(const char* fn, hipStream_t st) {
  int dev = -1;
  if (stream_device(st, &dev)) return fail(PGS_ERR_NO_DEVICE, "%s: no HIP device is available", fn);
  if (dev >= kMaxDevices) return fail(PGS_ERR_NO_DEVICE, "%s: device index %d above %d", fn, dev, kMaxDevices - 1);
  int arch = g_dev_arch[dev].load(std::memory_order_relaxed);
  if (arch == 0) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
      (void)hipGetLastError();
      return fail(PGS_ERR_NO_DEVICE, "%s: cannot query device %d", fn, dev);
    }
    arch = strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 2;
    g_dev_arch[dev].store(arch, std::memory_order_relaxed);
    if (arch != 1)
      return fail(PGS_ERR_NO_DEVICE, "%s: device %d is %s; the kernels are built for gfx950 only", fn, dev,
                  prop.gcnArchName);
  }
  if (arch != 1) return fail(PGS_ERR_NO_DEVICE, "%s: device %d is not a gfx950", fn, dev);
  return PGS_OK;
}

// The last linear launch of the calling thread: the kernel (a static string
// naming its template instance), its grid and the K split.  Recorded by the
// launchers (two pointers and two ints per launch); formatted only on request.
struct LaunchNote {
  const char* kernel = nullptr;
  const char* second = nullptr;  // a follow-up kernel (split-K reduce), or null
  long long grid = 0;
  int splits = 0;
};
static thread_local LaunchNote g_note;
static thread_local char g_note_text[1024] = "";

void note_launch(const char* kernel, long long grid, int splits, const char* second) {
  g_note.kernel = kernel;
  g_note.second = second;
  g_note.grid = grid;
  g_note.splits = splits;
}

}  // namespace pgs

extern "C" {

int pgs_abi_version(void) { return 10; }

const char* pgs_error_string(int code) {
  switch (code) {
    case PGS_OK: return "ok";
    case PGS_ERR_INVALID_ARGUMENT: return "invalid argument";
    case PGS_ERR_MISALIGNED: return "misaligned pointer";
    case PGS_ERR_LAUNCH: return "kernel launch failed";
    case PGS_ERR_NO_DEVICE: return "no usable gfx950 device";
    case PGS_ERR_TIMEOUT: return "a bounded device-side wait gave up";
    default: return "unknown error";
  }
}

const char* pgs_last_error(void) { return pgs::g_last_error; }

const char* pgs_last_plan(void) {
  const pgs::LaunchNote& n = pgs::g_note;
  if (!n.kernel) return "";
  snprintf(pgs::g_note_text, sizeof(pgs::g_note_text), "%s | grid=%lld splits=%d%s%s", n.kernel, n.grid, n.splits,
           n.second ? " | then " : "", n.second ? n.second : "");
  return pgs::g_note_text;
}

int pgs_stream_capture_state(void* stream, int* capturing, unsigned long long* capture_id) {
  if (!capturing || !capture_id) return pgs::fail(PGS_ERR_INVALID_ARGUMENT, "pgs_stream_capture_state: null pointer");
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  unsigned long long id = 0;
  hipError_t e = hipStreamGetCaptureInfo(reinterpret_cast<hipStream_t>(stream), &status, &id);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return pgs::fail(PGS_ERR_NO_DEVICE, "pgs_stream_capture_state: %s", hipGetErrorString(e));
  }
  *capturing = status == hipStreamCaptureStatusActive ? 1 : status == hipStreamCaptureStatusInvalidated ? 2 : 0;
  *capture_id = *capturing ? id : 0;
  return PGS_OK;
}

}  // extern "C"
