// Shared device types, conversions and host-side error plumbing for the
// gfx950 INT8 weight-only linear kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "pageserve_amd.h"

namespace pgs {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// conversions
// ---------------------------------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Signed byte B of v as fp32, one VALU instruction: v_cvt_f32_i32 with an
// SDWA source selecting and sign-extending the byte.  (Left to itself the
// compiler extracts bytes 1 and 3 with an extra 16-bit shift each.)
template <int B>
__device__ __forceinline__ float sbyte_to_f32(uint32_t v) {
  float r;
  if constexpr (B == 0)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(v));
  else if constexpr (B == 1)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(v));
  else if constexpr (B == 2)
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(v));
  else
    asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(v));
  return r;
}

// 8 signed bytes (two dwords) -> 8 bf16, exact (|q| <= 127 fits bf16's 8-bit
// significand): 8 SDWA conversions + 4 v_cvt_pk_bf16_f32 (1.5 VALU/element).
__device__ __forceinline__ bf16x8 i8x8_to_bf16x8(uint32_t lo, uint32_t hi) {
  f32x8 f = {sbyte_to_f32<0>(lo), sbyte_to_f32<1>(lo), sbyte_to_f32<2>(lo), sbyte_to_f32<3>(lo),
             sbyte_to_f32<0>(hi), sbyte_to_f32<1>(hi), sbyte_to_f32<2>(hi), sbyte_to_f32<3>(hi)};
  return __builtin_convertvector(f, bf16x8);
}

// fp32 -> bf16 bits, round to nearest even (hardware v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  __bf16 b = (__bf16)f;
  return __builtin_bit_cast(uint16_t, b);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// x * sigmoid(x) in fp32 (F.silu): x / (1 + e^-x) with the hardware
// base-2 exponential (v_exp_f32, e^-x = 2^(-x log2 e)) and the hardware
// reciprocal (v_rcp_f32), each within about one fp32 ulp, in about 5
// instructions instead of the library exponential and IEEE division (~30).
// The rounding of the exponent y = -x log2 e (half an ulp of |y|) scales
// e^-x by up to 2^(|y| u / 2), so the relative error is about
// (4 + |x| log2 e) ulps: a few ulps for the |x| of a layer's gate values,
// more where e^-x is huge (x far below zero, silu(x) then tiny).
// x -> +inf: x; x -> -inf: -0 (NaN at -inf itself, as x * sigmoid(x) gives).
__device__ __forceinline__ float silu_f32(float x) {
  const float e = __builtin_amdgcn_exp2f(x * -1.4426950408889634f);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// packed weight layout
// ---------------------------------------------------------------------------
//
// The linear kernels read int8 weights in "MFMA tile" order: the [n, k]
// matrix is cut into 16-row x 64-k blocks, stored block-row by block-row
// ([ceil(n/16)][ceil(k/64)] blocks of 1 KiB), and inside a block the 16 bytes
// of lane l (0..63) are row l%16, columns 16*(l/16) .. +15.  One 128-bit load
// per lane then fetches a whole contiguous KiB that is exactly the A operand
// of two v_mfma_f32_16x16x32_bf16.  Padding rows/columns are zero.

__host__ __device__ inline int64_t packed_kblocks(int64_t k) { return (k + 63) / 64; }
__host__ __device__ inline int64_t packed_bytes(int64_t n, int64_t k) {
  return ((n + 15) / 16) * packed_kblocks(k) * 1024;
}
// byte offset of element (r, j) of an [n, k] matrix with kb = packed_kblocks(k)
__host__ __device__ inline int64_t packed_offset(int64_t r, int64_t j, int64_t kb) {
  return ((r >> 4) * kb + (j >> 6)) * 1024 + (((r & 15) + 16 * ((j & 63) >> 4)) << 4) + (j & 15);
}

// ---------------------------------------------------------------------------
// host-side error handling (defined in pgs_api.hip)
// ---------------------------------------------------------------------------

int fail(int code, const char* fmt, ...);
int check_launch(const char* what);
int fill_zero(void* p, int64_t bytes, hipStream_t st);  // kernel fill (no memset node in captured graphs)

// Devices the library tracks per device state for (architecture, scratch).
constexpr int kMaxDevices = 64;
// The device a stream launches on (the current device for the null stream).
int stream_device(hipStream_t st, int* dev);
// PGS_OK when the stream's device is a gfx950 (checked once per device),
// else PGS_ERR_NO_DEVICE with a message.  Every launching entry point calls
// it after its argument checks and before its first launch.
int require_device(const char* fn, hipStream_t st);

// Records the calling thread's last linear launch (pgs_last_plan): `kernel`
// is a static string naming the kernel instance, `second` an optional
// follow-up kernel (the split-K reduce).
void note_launch(const char* kernel, long long grid, int splits, const char* second = nullptr);

inline bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

}  // namespace pgs
