// RMSNorm of the activations feeding the q|k|v and gate|up projections
// (engine/model.py:29-34, called at engine/model.py:166 and :187), as one
// kernel instead of the reference's chain of elementwise and reduction ops:
//
//   var  = mean_j x[i, j]^2           (fp32)
//   r    = 1 / sqrt(var + eps)         (torch.rsqrt; IEEE sqrt and divide here)
//   h    = bf16( w[j] * bf16( x[i, j] * r ) )
//
// The two bf16 roundings are the reference's: x * r is cast back to the model
// dtype before the multiply by the bf16 norm weight.  One workgroup per row;
// the sum of squares is reduced in a fixed order (per-thread strided sums,
// then a fixed butterfly inside each wave, then the waves in order), so
// results do not depend on timing.  Memory bound: 2 B read twice (L2 the
// second time) and 2 B written per element.
#include "pgs_linear.h"

namespace pgs {
namespace {

constexpr int kNormThreads = 256;

__device__ __forceinline__ float bf16_round(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

template <bool VEC>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ w, float eps,
                                                               uint16_t* __restrict__ h, int K) {
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * K;
  uint16_t* hr = h + row * K;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  float ss = 0.f;
  if constexpr (VEC) {
    for (int j = tid * 8; j < K; j += kNormThreads * 8) {
      const u32x4 v = ld16(xr + j);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = bf16_bits_to_f32(static_cast<uint16_t>(v[e])), hi = bf16_bits_to_f32(static_cast<uint16_t>(v[e] >> 16));
        ss += lo * lo;
        ss += hi * hi;
      }
    }
  } else {
    for (int j = tid; j < K; j += kNormThreads) {
      const float f = bf16_bits_to_f32(xr[j]);
      ss += f * f;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  __shared__ float part[kNormThreads / 64];
  if (lane == 0) part[wave] = ss;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / 64; ++i) total += part[i];
  const float r = 1.0f / sqrtf(total / static_cast<float>(K) + eps);

  if constexpr (VEC) {
    for (int j = tid * 8; j < K; j += kNormThreads * 8) {
      const u32x4 v = ld16(xr + j);
      const u32x4 g = ld16(w + j);
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = bf16_bits_to_f32(static_cast<uint16_t>(v[e])), x1 = bf16_bits_to_f32(static_cast<uint16_t>(v[e] >> 16));
        const float g0 = bf16_bits_to_f32(static_cast<uint16_t>(g[e])), g1 = bf16_bits_to_f32(static_cast<uint16_t>(g[e] >> 16));
        o[e] = pack_bf16x2(g0 * bf16_round(x0 * r), g1 * bf16_round(x1 * r));
      }
      *reinterpret_cast<u32x4*>(hr + j) = o;
    }
  } else {
    for (int j = tid; j < K; j += kNormThreads)
      hr[j] = f32_to_bf16_bits(bf16_bits_to_f32(w[j]) * bf16_round(bf16_bits_to_f32(xr[j]) * r));
  }
}

}  // namespace
}  // namespace pgs

using namespace pgs;

extern "C" int pgs_rmsnorm(const void* x, const void* weight, float eps, void* h, int64_t m, int64_t k, void* stream) {
  if (m < 0 || k < 0 || m > 0x7fffffff || k > 0x7fffffff)
    return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_rmsnorm: bad size m=%lld k=%lld", (long long)m, (long long)k);
  if (m == 0) return PGS_OK;
  if (k == 0) return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_rmsnorm: hidden size k=0");
  if (!x || !weight || !h) return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_rmsnorm: null pointer");
  if (!aligned(x, 2) || !aligned(weight, 2) || !aligned(h, 2)) return fail(PGS_ERR_MISALIGNED, "pgs_rmsnorm: misaligned");
  if (!(eps >= 0.f)) return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_rmsnorm: eps must be >= 0");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (int rc = require_device("pgs_rmsnorm", st)) return rc;
  const bool vec = k % 8 == 0 && aligned(x, 16) && aligned(weight, 16) && aligned(h, 16);
  const auto* xp = reinterpret_cast<const uint16_t*>(x);
  const auto* wp = reinterpret_cast<const uint16_t*>(weight);
  auto* hp = reinterpret_cast<uint16_t*>(h);
  if (vec)
    hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3(static_cast<unsigned>(m)), dim3(kNormThreads), 0, st, xp, wp, eps, hp,
                       static_cast<int>(k));
  else
    hipLaunchKernelGGL(rmsnorm_kernel<false>, dim3(static_cast<unsigned>(m)), dim3(kNormThreads), 0, st, xp, wp, eps,
                       hp, static_cast<int>(k));
  return check_launch("rmsnorm kernel");
}
