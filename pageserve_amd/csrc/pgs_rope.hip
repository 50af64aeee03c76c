// Rotary position embedding of the q and k projections (engine/model.py:37-56,
// apply_rope / rotate_half, applied at engine/model.py:172-173) as one kernel
// for both tensors, in place or out of place.  With h = head_dim / 2 and the
// reference's bf16 op chain x * cos + rotate_half(x) * sin, each op computed
// in fp32 and rounded once to bf16:
//
//   out[i]     = bf16( bf16(x[i]     * cos[i])     + bf16(-x[i + h] * sin[i]) )      i < h
//   out[i + h] = bf16( bf16(x[i + h] * cos[i + h]) + bf16( x[i]     * sin[i + h]) )
//
// (rotate_half negates exactly, and round-to-nearest-even is symmetric, so
// bf16(-a * s) = -bf16(a * s)).  cos / sin: bf16 [m, head_dim], the rows of
// the reference's cos_cache / sin_cache for the m tokens' positions.  One
// thread owns eight consecutive dimensions of the first half of one
// (token, head) and their eight partners, so in-place updates are safe.
// Memory bound: 2 B read and 2 B written per element, plus the tables (L2).
#include "pgs_linear.h"

namespace pgs {
namespace {

constexpr int kRopeThreads = 256;

__device__ __forceinline__ float bf16r(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

__device__ __forceinline__ void rope_pair(float x1, float x2, float c1, float s1, float c2, float s2, float& o1,
                                          float& o2) {
  o1 = bf16r(x1 * c1) + bf16r(-x2 * s1);
  o2 = bf16r(x2 * c2) + bf16r(x1 * s2);
}

// x / out: [m, heads, 2h] bf16; the first `units_q` work units belong to q,
// the rest to k (vector path: a unit is 8 dimensions of one (token, head)).
template <bool VEC>
__global__ __launch_bounds__(kRopeThreads) void rope_kernel(const uint16_t* __restrict__ q, uint16_t* qo, int q_heads,
                                                            const uint16_t* __restrict__ k, uint16_t* ko, int k_heads,
                                                            const uint16_t* __restrict__ cs,
                                                            const uint16_t* __restrict__ sn, int64_t m, int h) {
  constexpr int W = VEC ? 8 : 1;  // dimensions per unit
  const int per_row = h / W;      // units per (token, head)
  const int64_t units_q = m * q_heads * per_row;
  const int64_t units = units_q + m * k_heads * per_row;
  const int64_t u = static_cast<int64_t>(blockIdx.x) * kRopeThreads + threadIdx.x;
  if (u >= units) return;
  const bool is_q = u < units_q;
  const int64_t v = is_q ? u : u - units_q;
  const int heads = is_q ? q_heads : k_heads;
  const int64_t row = v / per_row;  // (token, head) row
  const int i0 = static_cast<int>(v - row * per_row) * W;
  const int64_t token = row / heads;
  const uint16_t* xr = (is_q ? q : k) + row * (2 * h);
  uint16_t* orow = (is_q ? qo : ko) + row * (2 * h);
  const uint16_t* cr = cs + token * (2 * h);
  const uint16_t* sr = sn + token * (2 * h);
  if constexpr (VEC) {
    const u32x4 xa = ld16(xr + i0), xb = ld16(xr + i0 + h);
    const u32x4 ca = ld16(cr + i0), cb = ld16(cr + i0 + h);
    const u32x4 sa = ld16(sr + i0), sb = ld16(sr + i0 + h);
    u32x4 oa, ob;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float o1[2], o2[2];
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        const int sh = 16 * w;
        rope_pair(bf16_bits_to_f32(static_cast<uint16_t>(xa[e] >> sh)), bf16_bits_to_f32(static_cast<uint16_t>(xb[e] >> sh)),
                  bf16_bits_to_f32(static_cast<uint16_t>(ca[e] >> sh)), bf16_bits_to_f32(static_cast<uint16_t>(sa[e] >> sh)),
                  bf16_bits_to_f32(static_cast<uint16_t>(cb[e] >> sh)), bf16_bits_to_f32(static_cast<uint16_t>(sb[e] >> sh)),
                  o1[w], o2[w]);
      }
      oa[e] = pack_bf16x2(o1[0], o1[1]);
      ob[e] = pack_bf16x2(o2[0], o2[1]);
    }
    *reinterpret_cast<u32x4*>(orow + i0) = oa;
    *reinterpret_cast<u32x4*>(orow + i0 + h) = ob;
  } else {
    float o1, o2;
    rope_pair(bf16_bits_to_f32(xr[i0]), bf16_bits_to_f32(xr[i0 + h]), bf16_bits_to_f32(cr[i0]),
              bf16_bits_to_f32(sr[i0]), bf16_bits_to_f32(cr[i0 + h]), bf16_bits_to_f32(sr[i0 + h]), o1, o2);
    orow[i0] = f32_to_bf16_bits(o1);
    orow[i0 + h] = f32_to_bf16_bits(o2);
  }
}

}  // namespace
}  // namespace pgs

using namespace pgs;

extern "C" int pgs_rope(const void* q, void* q_out, int64_t q_heads, const void* k, void* k_out, int64_t k_heads,
                        const void* cos, const void* sin, int64_t m, int64_t head_dim, void* stream) {
  if (m < 0 || q_heads < 0 || k_heads < 0 || head_dim < 0)
    return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_rope: negative size");
  if (head_dim % 2 != 0 || head_dim > 0x10000)
    return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_rope: head_dim=%lld must be even and at most 65536", (long long)head_dim);
  if (q_heads > 0x10000 || k_heads > 0x10000) return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_rope: too many heads");
  if (m == 0 || head_dim == 0 || (q_heads == 0 && k_heads == 0)) return PGS_OK;
  if ((q_heads > 0 && (!q || !q_out)) || (k_heads > 0 && (!k || !k_out)) || !cos || !sin)
    return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_rope: null pointer");
  if (!aligned(q, 2) || !aligned(q_out, 2) || !aligned(k, 2) || !aligned(k_out, 2) || !aligned(cos, 2) ||
      !aligned(sin, 2))
    return fail(PGS_ERR_MISALIGNED, "pgs_rope: misaligned");
  const int h = static_cast<int>(head_dim / 2);
  const bool vec = h % 8 == 0 && aligned(q, 16) && aligned(q_out, 16) && aligned(k, 16) && aligned(k_out, 16) &&
                   aligned(cos, 16) && aligned(sin, 16);
  const int64_t units = m * (q_heads + k_heads) * (vec ? h / 8 : h);
  const int64_t blocks = (units + kRopeThreads - 1) / kRopeThreads;
  if (blocks > 0x7fffffff) return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_rope: too large");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (int rc = require_device("pgs_rope", st)) return rc;
  const auto* qp = reinterpret_cast<const uint16_t*>(q);
  const auto* kp = reinterpret_cast<const uint16_t*>(k);
  auto* qo = reinterpret_cast<uint16_t*>(q_out);
  auto* ko = reinterpret_cast<uint16_t*>(k_out);
  const auto* cp = reinterpret_cast<const uint16_t*>(cos);
  const auto* sp = reinterpret_cast<const uint16_t*>(sin);
  if (vec)
    hipLaunchKernelGGL(rope_kernel<true>, dim3(static_cast<unsigned>(blocks)), dim3(kRopeThreads), 0, st, qp, qo,
                       static_cast<int>(q_heads), kp, ko, static_cast<int>(k_heads), cp, sp, m, h);
  else
    hipLaunchKernelGGL(rope_kernel<false>, dim3(static_cast<unsigned>(blocks)), dim3(kRopeThreads), 0, st, qp, qo,
                       static_cast<int>(q_heads), kp, ko, static_cast<int>(k_heads), cp, sp, m, h);
  return check_launch("rope kernel");
}
