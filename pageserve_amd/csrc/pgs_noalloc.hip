// pgs_w8a16_linear_noalloc: pgs_w8a16_linear for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  The K-split plans' scratch (pair slots
// and partial tiles) lives in a fixed file-scope device array instead of a
// caller workspace.  Each GPU holds its own copy of the array until the
// process ends; every call on a GPU shares it, so calls that overlap on one
// GPU (different streams, or graphs replayed concurrently) race.
#include <atomic>
#include <mutex>

#include "pgs_linear.h"

namespace pgs {
namespace {

// The largest workspace any launch plan of a 2048-hidden / 11008-intermediate
// model needs at up to 2048 tokens is 60.5 MiB (down_proj at 1793 to 1920
// tokens: 240 tiles of 128 x 128, K split 4, plus the pair slots); plans that
// need more are rejected.
constexpr size_t kScratchBytes = 64u << 20;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Per device: the array's device address (from hipGetSymbolAddress, taken
// once with that device current; the array's name is only a host-side
// stand-in).
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

int scratch_for(int dev, hipStream_t st, void** out) {
  void* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      int cur = -1;
      if (hipGetDevice(&cur) != hipSuccess || cur != dev) {
        (void)hipGetLastError();
        return fail(PGS_ERR_INVALID_ARGUMENT,
                    "pgs_w8a16_linear_noalloc: the stream's device %d must be the current device (%d)", dev, cur);
      }
      hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        return fail(PGS_ERR_LAUNCH, "pgs_w8a16_linear_noalloc: hipGetSymbolAddress failed on device %d: %s", dev,
                    hipGetErrorString(e));
      }
      // the pair slots must start empty (every call leaves them empty); the
      // loader zero-fills the array, this fill makes it explicit and runs
      // ahead of the first call's kernels on its stream
      if (int rc = fill_zero(p, static_cast<int64_t>(kPairBytes), st)) return rc;
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return PGS_OK;
}

}  // namespace
}  // namespace pgs

using namespace pgs;

extern "C" int pgs_w8a16_linear_noalloc(const void* x, const int8_t* qp, const float* scale, const void* bias,
                                        void* y, int y_dtype, int64_t m, int64_t n, int64_t k, void* stream) {
  const char* fn = "pgs_w8a16_linear_noalloc";
  if (m < 0 || n < 0 || k < 0)
    return fail(PGS_ERR_INVALID_ARGUMENT, "%s: negative size m=%lld n=%lld k=%lld", fn, (long long)m, (long long)n,
                (long long)k);
  size_t need = 0;
  if (m > 0 && n > 0 && k > 0) {
    need = pgs_w8a16_workspace_bytes(m, &n, 1, k, 0);
    if (need > kScratchBytes)
      return fail(PGS_ERR_INVALID_ARGUMENT, "%s: m=%lld n=%lld k=%lld needs %zu bytes of scratch, above the %zu-byte maximum",
                  fn, (long long)m, (long long)n, (long long)k, need, kScratchBytes);
  }
  // the scratch goes to every non-empty call, so its plan is the one
  // pgs_w8a16_linear makes with a workspace (some plans need none but are
  // only taken where a split would be possible)
  void* ws = nullptr;
  if (m > 0 && n > 0 && k > 0) {
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (int rc = require_device(fn, st)) return rc;
    int dev = -1;
    if (int rc = stream_device(st, &dev)) return rc;
    if (int rc = scratch_for(dev, st, &ws)) return rc;
  }
  pgs_linear_out o{qp, scale, bias, y, n};
  return linear_call(fn, x, &o, 1, y_dtype, m, k, ws, ws ? kScratchBytes : 0, stream);
}
