// Packed weight layout: pack / unpack between the reference's row-major
// [n, k] int8 (QuantizedWeight.q, engine/quantization.py:22,38) and the
// MFMA tile order the linear kernels stream (layout in pgs_common.h), and
// dequantize straight from the packed form (engine/quantization.py:27).
// One thread per 16-byte lane segment of a 1 KiB block: the packed side is
// always a 16-byte access; the row-major side is 16 bytes when k % 16 == 0.
#include "pgs_common.h"

namespace pgs {
namespace {

__global__ __launch_bounds__(256) void fill_zero_kernel(u32x4* __restrict__ p, int64_t n16) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n16) p[i] = u32x4{0u, 0u, 0u, 0u};
}

// segment index -> (row, first column) of the [n, k] matrix
__device__ __forceinline__ void segment_origin(int64_t seg, int64_t kb, int64_t& r, int64_t& j) {
  const int64_t block = seg >> 6;
  const int lane = static_cast<int>(seg & 63);
  r = (block / kb) * 16 + (lane & 15);
  j = (block % kb) * 64 + (lane >> 4) * 16;
}

template <bool K16>
__global__ __launch_bounds__(256) void pack_kernel(const int8_t* __restrict__ q, int64_t n, int64_t k, int64_t kb,
                                                   int64_t nseg, int8_t* __restrict__ packed) {
  const int64_t seg = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (seg >= nseg) return;
  int64_t r, j;
  segment_origin(seg, kb, r, j);
  u32x4 v = {0u, 0u, 0u, 0u};
  if (r < n && j < k) {
    const int8_t* src = q + r * k + j;
    if (K16) {
      v = *reinterpret_cast<const u32x4*>(src);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (j + i < k) v[i >> 2] |= static_cast<uint32_t>(static_cast<uint8_t>(src[i])) << (8 * (i & 3));
    }
  }
  *reinterpret_cast<u32x4*>(packed + seg * 16) = v;
}

template <bool K16>
__global__ __launch_bounds__(256) void unpack_kernel(const int8_t* __restrict__ packed, int64_t n, int64_t k,
                                                     int64_t kb, int64_t nseg, int8_t* __restrict__ q) {
  const int64_t seg = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (seg >= nseg) return;
  int64_t r, j;
  segment_origin(seg, kb, r, j);
  if (r >= n || j >= k) return;
  const u32x4 v = *reinterpret_cast<const u32x4*>(packed + seg * 16);
  int8_t* dst = q + r * k + j;
  if (K16) {
    *reinterpret_cast<u32x4*>(dst) = v;
  } else {
    for (int i = 0; i < 16 && j + i < k; ++i) dst[i] = static_cast<int8_t>(v[i >> 2] >> (8 * (i & 3)));
  }
}

template <int OUT>
__device__ __forceinline__ void store_one(void* out, int64_t e, float v) {
  if constexpr (OUT == PGS_DTYPE_F32)
    reinterpret_cast<float*>(out)[e] = v;
  else if constexpr (OUT == PGS_DTYPE_BF16)
    reinterpret_cast<uint16_t*>(out)[e] = f32_to_bf16_bits(v);
  else
    reinterpret_cast<_Float16*>(out)[e] = static_cast<_Float16>(v);
}

// out[r, j] = dtype(float(q[r, j]) * scale[r]), row-major output
template <int OUT>
__global__ __launch_bounds__(256) void dequantize_packed_kernel(const int8_t* __restrict__ packed,
                                                                const float* __restrict__ scale, int64_t n,
                                                                int64_t k, int64_t kb, int64_t nseg,
                                                                void* __restrict__ out) {
  const int64_t seg = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (seg >= nseg) return;
  int64_t r, j;
  segment_origin(seg, kb, r, j);
  if (r >= n || j >= k) return;
  const u32x4 v = *reinterpret_cast<const u32x4*>(packed + seg * 16);
  const float s = scale[r];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (j + i < k) {
      const float f = static_cast<float>(static_cast<int8_t>(v[i >> 2] >> (8 * (i & 3)))) * s;
      store_one<OUT>(out, r * k + j + i, f);
    }
  }
}

int check_nk(const char* fn, int64_t n, int64_t k) {
  if (n < 0 || k < 0)
    return fail(PGS_ERR_INVALID_ARGUMENT, "%s: negative size n=%lld k=%lld", fn, (long long)n, (long long)k);
  if (packed_bytes(n, k) / 16 > 0x7fffffffLL * 256LL) return fail(PGS_ERR_INVALID_ARGUMENT, "%s: too large", fn);
  return PGS_OK;
}

unsigned blocks_for(int64_t nseg) { return static_cast<unsigned>((nseg + 255) / 256); }

}  // namespace

int fill_zero(void* p, int64_t bytes, hipStream_t st) {
  if (bytes <= 0) return PGS_OK;
  if (!aligned(p, 16) || bytes % 16) return fail(PGS_ERR_MISALIGNED, "fill_zero: buffer not 16-byte granular");
  const int64_t n16 = bytes / 16;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks_for(n16)), dim3(256), 0, st, reinterpret_cast<u32x4*>(p), n16);
  return check_launch("fill_zero");
}

}  // namespace pgs

using namespace pgs;

extern "C" int64_t pgs_packed_bytes(int64_t n, int64_t k) {
  if (n < 0 || k < 0) return -1;
  return packed_bytes(n, k);
}

extern "C" int pgs_pack_weight(const int8_t* q, int64_t n, int64_t k, int8_t* packed, void* stream) {
  int rc = check_nk("pgs_pack_weight", n, k);
  if (rc) return rc;
  if (n == 0 || k == 0) return PGS_OK;
  if (!q || !packed) return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_pack_weight: null pointer");
  if (!aligned(packed, 16)) return fail(PGS_ERR_MISALIGNED, "pgs_pack_weight: packed buffer not 16-byte aligned");
  const int64_t kb = packed_kblocks(k), nseg = packed_bytes(n, k) / 16;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if ((rc = require_device("pgs_pack_weight", st))) return rc;
  if (k % 16 == 0 && aligned(q, 16))
    hipLaunchKernelGGL(pack_kernel<true>, dim3(blocks_for(nseg)), dim3(256), 0, st, q, n, k, kb, nseg, packed);
  else
    hipLaunchKernelGGL(pack_kernel<false>, dim3(blocks_for(nseg)), dim3(256), 0, st, q, n, k, kb, nseg, packed);
  return check_launch("pgs_pack_weight");
}

extern "C" int pgs_unpack_weight(const int8_t* packed, int64_t n, int64_t k, int8_t* q, void* stream) {
  int rc = check_nk("pgs_unpack_weight", n, k);
  if (rc) return rc;
  if (n == 0 || k == 0) return PGS_OK;
  if (!q || !packed) return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_unpack_weight: null pointer");
  if (!aligned(packed, 16)) return fail(PGS_ERR_MISALIGNED, "pgs_unpack_weight: packed buffer not 16-byte aligned");
  const int64_t kb = packed_kblocks(k), nseg = packed_bytes(n, k) / 16;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if ((rc = require_device("pgs_unpack_weight", st))) return rc;
  if (k % 16 == 0 && aligned(q, 16))
    hipLaunchKernelGGL(unpack_kernel<true>, dim3(blocks_for(nseg)), dim3(256), 0, st, packed, n, k, kb, nseg, q);
  else
    hipLaunchKernelGGL(unpack_kernel<false>, dim3(blocks_for(nseg)), dim3(256), 0, st, packed, n, k, kb, nseg, q);
  return check_launch("pgs_unpack_weight");
}

extern "C" int pgs_dequantize_packed(const int8_t* packed, const float* scale, int64_t n, int64_t k, void* out,
                                     int out_dtype, void* stream) {
  int rc = check_nk("pgs_dequantize_packed", n, k);
  if (rc) return rc;
  if (n == 0 || k == 0) return PGS_OK;
  if (!packed || !scale || !out) return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_dequantize_packed: null pointer");
  if (!aligned(packed, 16) || !aligned(scale, 4))
    return fail(PGS_ERR_MISALIGNED, "pgs_dequantize_packed: packed/scale misaligned");
  const int64_t kb = packed_kblocks(k), nseg = packed_bytes(n, k) / 16;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (out_dtype != PGS_DTYPE_F32 && out_dtype != PGS_DTYPE_BF16 && out_dtype != PGS_DTYPE_F16)
    return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_dequantize_packed: output dtype code %d not supported", out_dtype);
  if ((rc = require_device("pgs_dequantize_packed", st))) return rc;
  switch (out_dtype) {
    case PGS_DTYPE_F32:
      if (!aligned(out, 4)) return fail(PGS_ERR_MISALIGNED, "pgs_dequantize_packed: output misaligned");
      hipLaunchKernelGGL(dequantize_packed_kernel<PGS_DTYPE_F32>, dim3(blocks_for(nseg)), dim3(256), 0, st, packed,
                         scale, n, k, kb, nseg, out);
      break;
    case PGS_DTYPE_BF16:
    case PGS_DTYPE_F16:
      if (!aligned(out, 2)) return fail(PGS_ERR_MISALIGNED, "pgs_dequantize_packed: output misaligned");
      if (out_dtype == PGS_DTYPE_BF16)
        hipLaunchKernelGGL(dequantize_packed_kernel<PGS_DTYPE_BF16>, dim3(blocks_for(nseg)), dim3(256), 0, st, packed,
                           scale, n, k, kb, nseg, out);
      else
        hipLaunchKernelGGL(dequantize_packed_kernel<PGS_DTYPE_F16>, dim3(blocks_for(nseg)), dim3(256), 0, st, packed,
                           scale, n, k, kb, nseg, out);
      break;
    default:
      return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_dequantize_packed: output dtype code %d not supported", out_dtype);
  }
  return check_launch("pgs_dequantize_packed");
}
