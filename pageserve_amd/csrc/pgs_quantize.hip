// Per-output-row symmetric INT8 quantizer and dequantizer (gfx950).
//
// quantize_per_channel: engine/quantization.py:16-23.  One workgroup per
// weight row: pass 1 reduces max|w| (exact: a max is order independent), the
// scale is absmax / 127 with a correctly rounded IEEE divide, pass 2 re-reads
// the row (now L2-resident) and writes rint(w / scale) clamped to +-127.
// The division is a true IEEE divide (never a reciprocal multiply) and rint
// is round-half-to-even, which is what the reference's CPU arithmetic does;
// the results are bit-identical.
//
// dequantize: engine/quantization.py:26-27.  fp32 product q * scale, then one
// round-to-nearest-even conversion to the output type.
#include "pgs_common.h"

namespace pgs {
namespace {

constexpr int kQuantThreads = 256;

template <bool BF16, int VEC>
__device__ __forceinline__ void load_row_vec(const void* __restrict__ base, int64_t elem, float (&f)[VEC]) {
  if constexpr (BF16) {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(base) + elem;
    if constexpr (VEC == 8) {
      u32x4 v = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f[2 * i] = __uint_as_float(v[i] << 16);
        f[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) f[i] = bf16_bits_to_f32(p[i]);
    }
  } else {
    const float* p = reinterpret_cast<const float*>(base) + elem;
    if constexpr (VEC == 4) {
      f32x4 v = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
      for (int i = 0; i < 4; ++i) f[i] = v[i];
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) f[i] = p[i];
    }
  }
}

// max that propagates NaN, as torch's amax does (fmaxf would drop it): a row
// holding a NaN gets a NaN scale, as in the reference
__device__ __forceinline__ float nan_max(float a, float b) {
  return a != a ? a : (b != b ? b : fmaxf(a, b));
}

__device__ __forceinline__ uint32_t quantize_one(float w, float s) {
  float r = rintf(w / s);  // IEEE divide, ties-to-even
  // NaN (a NaN or infinite weight, or a row with a NaN scale): 0, which is
  // what the reference's int8 conversion of NaN gives on the CPU
  if (!(r == r)) return 0u;
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(static_cast<int>(r))));
}

// PACKED: write q in the packed tile layout (kb = packed_kblocks(k)) instead
// of row-major; a VEC-element group never straddles a 16-byte lane segment.
template <bool BF16, int VEC, bool PACKED>
__global__ __launch_bounds__(kQuantThreads) void quantize_rows_kernel(
    const void* __restrict__ w, int64_t k, int64_t kb, int8_t* __restrict__ q, float* __restrict__ scale) {
  const int64_t row = blockIdx.x;
  const int64_t nvec = k / VEC;
  const int64_t base = row * k;
  __shared__ float red[kQuantThreads / kWave];

  float amax = 0.0f;
  for (int64_t v = threadIdx.x; v < nvec; v += kQuantThreads) {
    float f[VEC];
    load_row_vec<BF16, VEC>(w, base + v * VEC, f);
#pragma unroll
    for (int i = 0; i < VEC; ++i) amax = nan_max(amax, fabsf(f[i]));
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) amax = nan_max(amax, __shfl_xor(amax, off));
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int i = 1; i < kQuantThreads / kWave; ++i) amax = nan_max(amax, red[i]);

  // :20 clamp(min=1e-8) (a NaN stays NaN, as torch's clamp keeps it), :21 / 127.0
  const float s = (amax != amax ? amax : fmaxf(amax, 1e-8f)) / 127.0f;
  if (threadIdx.x == 0) scale[row] = s;

  for (int64_t v = threadIdx.x; v < nvec; v += kQuantThreads) {
    float f[VEC];
    load_row_vec<BF16, VEC>(w, base + v * VEC, f);
    const int64_t dst = PACKED ? packed_offset(row, v * VEC, kb) : base + v * VEC;
    if constexpr (VEC == 8) {
      u32x2 out;
      out[0] = quantize_one(f[0], s) | (quantize_one(f[1], s) << 8) | (quantize_one(f[2], s) << 16) |
               (quantize_one(f[3], s) << 24);
      out[1] = quantize_one(f[4], s) | (quantize_one(f[5], s) << 8) | (quantize_one(f[6], s) << 16) |
               (quantize_one(f[7], s) << 24);
      *reinterpret_cast<u32x2*>(q + dst) = out;
    } else if constexpr (VEC == 4) {
      uint32_t out = quantize_one(f[0], s) | (quantize_one(f[1], s) << 8) | (quantize_one(f[2], s) << 16) |
                     (quantize_one(f[3], s) << 24);
      *reinterpret_cast<uint32_t*>(q + dst) = out;
    } else {
#pragma unroll
      for (int i = 0; i < VEC; ++i) {
        const int64_t d = PACKED ? packed_offset(row, v * VEC + i, kb) : base + v * VEC + i;
        q[d] = static_cast<int8_t>(quantize_one(f[i], s));
      }
    }
  }
}

template <int OUT>  // PGS_DTYPE_*
__device__ __forceinline__ void store_dequant(void* out, int64_t e, float v) {
  if constexpr (OUT == PGS_DTYPE_F32) {
    reinterpret_cast<float*>(out)[e] = v;
  } else if constexpr (OUT == PGS_DTYPE_BF16) {
    reinterpret_cast<uint16_t*>(out)[e] = f32_to_bf16_bits(v);
  } else {
    reinterpret_cast<_Float16*>(out)[e] = static_cast<_Float16>(v);
  }
}

// 16 weights per thread; requires k % 16 == 0 and 16-byte aligned q/out.
template <int OUT>
__global__ __launch_bounds__(256) void dequantize16_kernel(const int8_t* __restrict__ q,
                                                           const float* __restrict__ scale, int64_t k,
                                                           int64_t nchunks, void* __restrict__ out) {
  const int64_t c = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (c >= nchunks) return;
  const int64_t e = c * 16;
  const float s = scale[e / k];
  const u32x4 w = *reinterpret_cast<const u32x4*>(q + e);
  float f[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int b = 0; b < 4; ++b) f[4 * i + b] = static_cast<float>(static_cast<int8_t>(w[i] >> (8 * b))) * s;
  }
  if constexpr (OUT == PGS_DTYPE_F32) {
    f32x4* o = reinterpret_cast<f32x4*>(reinterpret_cast<float*>(out) + e);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f32x4{f[4 * i], f[4 * i + 1], f[4 * i + 2], f[4 * i + 3]};
  } else if constexpr (OUT == PGS_DTYPE_BF16) {
    u32x4* o = reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(out) + e);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      o[i] = u32x4{pack_bf16x2(f[8 * i], f[8 * i + 1]), pack_bf16x2(f[8 * i + 2], f[8 * i + 3]),
                   pack_bf16x2(f[8 * i + 4], f[8 * i + 5]), pack_bf16x2(f[8 * i + 6], f[8 * i + 7])};
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) store_dequant<OUT>(out, e + i, f[i]);
  }
}

template <int OUT>
__global__ __launch_bounds__(256) void dequantize1_kernel(const int8_t* __restrict__ q,
                                                          const float* __restrict__ scale, int64_t k,
                                                          int64_t total, void* __restrict__ out) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= total) return;
  store_dequant<OUT>(out, e, static_cast<float>(q[e]) * scale[e / k]);
}

template <int OUT>
int launch_dequant(const int8_t* q, const float* scale, int64_t n, int64_t k, void* out, hipStream_t st) {
  const int64_t total = n * k;
  const size_t out_align = (OUT == PGS_DTYPE_F32) ? 16 : 16;
  if (k % 16 == 0 && aligned(q, 16) && aligned(out, out_align)) {
    const int64_t nchunks = total / 16;
    const int64_t blocks = (nchunks + 255) / 256;
    hipLaunchKernelGGL(dequantize16_kernel<OUT>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, q,
                       scale, k, nchunks, out);
  } else {
    const int64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(dequantize1_kernel<OUT>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, q, scale,
                       k, total, out);
  }
  return check_launch("pgs_dequantize");
}

template <bool PACKED>
int launch_quantize(const char* fn, const void* w, int w_dtype, int64_t n, int64_t k, int8_t* q, float* scale,
                    void* stream) {
  if (n < 0 || k < 0)
    return fail(PGS_ERR_INVALID_ARGUMENT, "%s: negative size n=%lld k=%lld", fn, (long long)n, (long long)k);
  if (w_dtype != PGS_DTYPE_F32 && w_dtype != PGS_DTYPE_BF16)
    return fail(PGS_ERR_INVALID_ARGUMENT, "%s: weight dtype code %d not fp32/bf16", fn, w_dtype);
  if (n == 0) return PGS_OK;
  if (n > 0x7fffffff) return fail(PGS_ERR_INVALID_ARGUMENT, "%s: n=%lld too large", fn, (long long)n);
  if (!scale || (k > 0 && (!w || !q))) return fail(PGS_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  const size_t esz = (w_dtype == PGS_DTYPE_F32) ? 4 : 2;
  if (!aligned(w, esz) || !aligned(scale, 4))
    return fail(PGS_ERR_MISALIGNED, "%s: weight/scale not aligned to element size", fn);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (int rc = require_device(fn, st)) return rc;
  const int64_t kb = packed_kblocks(k);
  if (PACKED && k > 0 && (n % 16 != 0 || k % 64 != 0)) {
    // padding rows/columns of the packed buffer must read as zero
    int rc = fill_zero(q, packed_bytes(n, k), st);
    if (rc) return rc;
  }
  dim3 grid(static_cast<unsigned>(n)), block(kQuantThreads);
  if (w_dtype == PGS_DTYPE_F32) {
    if (k % 4 == 0 && aligned(w, 16) && aligned(q, 4))
      hipLaunchKernelGGL((quantize_rows_kernel<false, 4, PACKED>), grid, block, 0, st, w, k, kb, q, scale);
    else
      hipLaunchKernelGGL((quantize_rows_kernel<false, 1, PACKED>), grid, block, 0, st, w, k, kb, q, scale);
  } else {
    if (k % 8 == 0 && aligned(w, 16) && aligned(q, 8))
      hipLaunchKernelGGL((quantize_rows_kernel<true, 8, PACKED>), grid, block, 0, st, w, k, kb, q, scale);
    else
      hipLaunchKernelGGL((quantize_rows_kernel<true, 1, PACKED>), grid, block, 0, st, w, k, kb, q, scale);
  }
  return check_launch(fn);
}

}  // namespace
}  // namespace pgs

using namespace pgs;

extern "C" int pgs_quantize_per_channel(const void* w, int w_dtype, int64_t n, int64_t k, int8_t* q,
                                        float* scale, void* stream) {
  return launch_quantize<false>("pgs_quantize_per_channel", w, w_dtype, n, k, q, scale, stream);
}

extern "C" int pgs_quantize_per_channel_packed(const void* w, int w_dtype, int64_t n, int64_t k, int8_t* packed,
                                               float* scale, void* stream) {
  return launch_quantize<true>("pgs_quantize_per_channel_packed", w, w_dtype, n, k, packed, scale, stream);
}

extern "C" int pgs_dequantize(const int8_t* q, const float* scale, int64_t n, int64_t k, void* out, int out_dtype,
                              void* stream) {
  if (n < 0 || k < 0)
    return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_dequantize: negative size n=%lld k=%lld", (long long)n, (long long)k);
  if (n == 0 || k == 0) return PGS_OK;
  if (!q || !scale || !out) return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_dequantize: null pointer");
  if (!aligned(scale, 4)) return fail(PGS_ERR_MISALIGNED, "pgs_dequantize: scale not 4-byte aligned");
  if (n * k / 16 > 0x7fffffffLL * 256LL)
    return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_dequantize: tensor too large");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (out_dtype != PGS_DTYPE_F32 && out_dtype != PGS_DTYPE_BF16 && out_dtype != PGS_DTYPE_F16)
    return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_dequantize: output dtype code %d not supported", out_dtype);
  if (int rc = require_device("pgs_dequantize", st)) return rc;
  switch (out_dtype) {
    case PGS_DTYPE_F32:
      if (!aligned(out, 4)) return fail(PGS_ERR_MISALIGNED, "pgs_dequantize: fp32 output not 4-byte aligned");
      return launch_dequant<PGS_DTYPE_F32>(q, scale, n, k, out, st);
    case PGS_DTYPE_BF16:
      if (!aligned(out, 2)) return fail(PGS_ERR_MISALIGNED, "pgs_dequantize: bf16 output not 2-byte aligned");
      return launch_dequant<PGS_DTYPE_BF16>(q, scale, n, k, out, st);
    case PGS_DTYPE_F16:
      if (!aligned(out, 2)) return fail(PGS_ERR_MISALIGNED, "pgs_dequantize: fp16 output not 2-byte aligned");
      return launch_dequant<PGS_DTYPE_F16>(q, scale, n, k, out, st);
    default:
      return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_dequantize: output dtype code %d not supported", out_dtype);
  }
}
