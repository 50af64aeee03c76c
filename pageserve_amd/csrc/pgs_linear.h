// Shared definitions of the W8A16 linear kernels (skinny and tile GEMM).
//
// Operand convention of every kernel: v_mfma_f32_16x16x32_bf16 with the
// weight as A (16 weight rows) and the activations as B (16 tokens).  Lane l
// supplies A row l%16 and B column l%16, both over the same 8 consecutive k
// values 8*(l/16)..+7 of a 32-k step, so a 16-byte load of 16 int8 weights
// feeds two MFMAs.  The accumulator lane l holds D[4*(l/16)+r][l%16], r=0..3.
#pragma once

#include "pgs_common.h"

namespace pgs {

// Members of one launch that share the activations x (q/k/v), or the SwiGLU
// pair (member 0 = gate, member 1 = up, output in member 0's y).
struct GroupArgs {
  const int8_t* q[PGS_MAX_GROUP];
  const float* scale[PGS_MAX_GROUP];
  const uint16_t* bias[PGS_MAX_GROUP];
  void* y[PGS_MAX_GROUP];
  const uint16_t* res[PGS_MAX_GROUP];  // bf16 [m, n] residual added to the output, or null
  int32_t n[PGS_MAX_GROUP];
  int32_t unit_begin[PGS_MAX_GROUP + 1];  // first work unit (tile) of each member
  int32_t n_outs;
};

struct Problem {
  const uint16_t* x;
  GroupArgs args;
  int m, k;
  int nmat;  // 1 = linear / group, 2 = SwiGLU pair
  bool out_f32;
  float* partials;  // split-K partial tiles (null: no split)
  size_t partial_bytes;
  unsigned long long* pairs;  // zeroed pair slots (skinny two-way split), or null
  const uint16_t* norm_w;     // rms_norm weight fused in front of the linear (bf16 [k]), or null
  float eps;
  // Row-argmax mode (fp32 single matrix, skinny kernel, no K split): instead
  // of the outputs, workgroup b writes the key of its best output of token t
  // to keys[b * m + t] (argmax_key); null otherwise
  unsigned long long* keys;
};

// Largest in_features of the linear kernels: their buffer offsets
// (row * K * 2 bytes for up to 128 activation rows) are 32-bit.
constexpr int kMaxK = 1 << 22;

// Workspace layout: kPairBytes of pair slots (zero before first use, left
// zero by every call), then the split-K partial tiles.  One 8-byte slot per
// output of a 16-row tile: 256 tiles x 16 rows x 16 tokens (128 tiles at up
// to 32 tokens).
constexpr size_t kPairBytes = 256u * 256u * 8u;

// Launch plan of the skinny kernel (m <= 32).
struct SkinnyPlan {
  int tiles;   // 16-row tiles over all members
  int splits;  // workgroups per tile (split K across workgroups)
  bool pair;   // two K halves combined through pair slots (no reduce launch)
  int shape;   // launch shape: waves per workgroup and K slots per wave
  bool fold;   // two workgroups of 8 rows per tile, two chunks per MFMA (m <= 8)
  int tm;      // 16-token column blocks per tile (1: m <= 16, 2: m <= 32)
};

// Launch plan of the tile GEMM (m > 16).
struct GemmPlan {
  int bm, bn;     // output tile (tokens x weight rows)
  int kg;         // K groups of four waves per workgroup (K % 64 == 0 kernel)
  int tiles_m, tiles_n, tiles;
  int splits;     // workgroups per output tile along K
  bool once;      // the one-shot tile (16 or 32 tokens, K <= 2048)
};

SkinnyPlan plan_skinny(int m, int k, int nmat, int tiles, bool can_split);
// workgroups of a skinny launch
int64_t skinny_grid(const SkinnyPlan& p);
size_t skinny_partial_bytes(const SkinnyPlan& p, int nmat);
// whether the skinny kernel can apply rms_norm to its staged activations
// (bf16 output, m <= 4, K % 64 == 0, no K split, an issue-once shape)
bool skinny_norm_fusable(const SkinnyPlan& p, int m, int k, bool out_f32, int nmat);
int launch_skinny(Problem& p, const SkinnyPlan& plan, hipStream_t st);

// pgs_w8a16_linear_group with the entry point's name `fn` in its messages
// (for entry points that supply their own workspace).
int linear_call(const char* fn, const void* x, const pgs_linear_out* outs, int n_outs, int y_dtype, int64_t m,
                int64_t k, void* workspace, size_t workspace_bytes, void* stream);

GemmPlan plan_gemm(int m, int k, int nmat, const int32_t* n, int members, bool can_split);
size_t gemm_partial_bytes(const GemmPlan& p, int nmat);
int launch_gemm(Problem& p, const GemmPlan& plan, hipStream_t st);

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------

// Selects member [g] with constant indices only (a dynamic index into a
// kernel-argument array would spill the struct to scratch).
template <typename T, int L>
__device__ __forceinline__ T pick(const T (&arr)[L], int g) {
  T v = arr[0];
#pragma unroll
  for (int i = 1; i < L; ++i) v = (g == i) ? arr[i] : v;
  return v;
}

// The same choice with every element read into a scalar register first, so
// the choice is a register select.  The compiler otherwise folds the selects
// into one load from a computed kernel-argument offset, which puts a second,
// dependent scalar memory round trip in front of the kernel's first vector
// load: worth avoiding in short (decode) kernels, whose run time is mostly
// such latencies.  Pointers pass the barrier as global-memory pointers, so
// accesses through the result stay global (not flat) loads and stores.
template <typename T, int L>
__device__ __forceinline__ T pick_early(const T (&arr)[L], int g) {
  T v[L];
#pragma unroll
  for (int i = 0; i < L; ++i) {
    v[i] = arr[i];
    asm volatile("" : "+s"(v[i]));
  }
  T r = v[0];
#pragma unroll
  for (int i = 1; i < L; ++i) r = (g == i) ? v[i] : r;
  return r;
}
template <typename T, int L>
__device__ __forceinline__ T* pick_early(T* const (&arr)[L], int g) {
  using GT = __attribute__((address_space(1))) T;
  GT* v[L];
#pragma unroll
  for (int i = 0; i < L; ++i) {
    v[i] = (GT*)arr[i];
    asm volatile("" : "+s"(v[i]));
  }
  GT* r = v[0];
#pragma unroll
  for (int i = 1; i < L; ++i) r = (g == i) ? v[i] : r;
  return (T*)r;
}

// Row-argmax key of output `row` with value f: ordered as (f, then smaller
// row) under unsigned comparison, so that the maximum key is torch.argmax's
// choice -- the first index of the maximum, every NaN counting as the
// maximum -- and max is exact, commutative and associative (any reduction
// order gives the same key).  -0.0 counts as +0.0.  The high word maps the
// float's bits monotonically onto unsigned order; the low word is the
// row's complement.  Key 0 is below every output's key.
__device__ __forceinline__ unsigned long long argmax_key(float f, uint32_t row) {
  const uint32_t b = __float_as_uint(f == 0.f ? 0.f : f);
  const uint32_t hi = f != f ? 0xffffffffu : ((b & 0x80000000u) ? ~b : (b | 0x80000000u));
  return (static_cast<unsigned long long>(hi) << 32) | (0xffffffffu - row);
}
__device__ __forceinline__ float argmax_key_value(unsigned long long key) {
  const uint32_t hi = static_cast<uint32_t>(key >> 32);
  if (hi == 0xffffffffu) return __uint_as_float(0x7fc00000u);
  return __uint_as_float((hi & 0x80000000u) ? (hi & 0x7fffffffu) : ~hi);
}
__device__ __forceinline__ uint32_t argmax_key_row(unsigned long long key) {
  return 0xffffffffu - static_cast<uint32_t>(key);
}

// Workgroup b of a grid of `total` runs on XCD b % 8 (round robin over the
// eight XCDs); the remap numbers the workgroups of each XCD consecutively, so
// that units with neighbouring numbers share an L2.  A bijection of
// [0, total) for any total.
__device__ __forceinline__ int xcd_remap(int b, int total) {
  const int xcd = b & 7, slot = b >> 3;
  const int per = total >> 3, rem = total & 7;
  return (xcd < rem) ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
}

__device__ __forceinline__ int member_of(const GroupArgs& a, int unit) {
  int g = 0;
#pragma unroll
  for (int i = 1; i < PGS_MAX_GROUP; ++i) g = (i < a.n_outs && unit >= a.unit_begin[i]) ? i : g;
  return g;
}

// Buffer loads: a resource (base, byte size) in scalar registers, a
// per-lane offset and a wave-uniform offset; the hardware range check
// returns zeros for bytes past the size, without a memory access.
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer, 32-bit data format
constexpr int kLoadNT = 2;              // cache policy: non-temporal (streamed once)

// A buffer resource must live in scalar registers; values the compiler cannot
// prove wave-uniform (pointers picked from the argument arrays) are moved
// there explicitly.  The inputs are uniform by construction.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ const void* uniform(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const void*>((static_cast<uint64_t>(hi) << 32) | lo);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int n = bytes > 0x7fffffff ? 0x7fffffff : static_cast<int>(bytes);  // integer clamp (no fp round trip)
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(uniform(base)), 0, uniform(n), kRsrcWord3);
}

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// Streaming load: the weights are read once per call, so keep them from
// displacing reusable lines (activations, partials) in the caches.
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// y = residual + linear with the reference's roundings (engine/model.py:184,
// 190): the linear output is rounded to the output type first, then added.
template <bool OUT_F32>
__device__ __forceinline__ float add_residual(float lin, const uint16_t* res, int64_t idx) {
  if (!res) return lin;
  const float l = OUT_F32 ? lin : bf16_bits_to_f32(f32_to_bf16_bits(lin));
  return l + bf16_bits_to_f32(res[idx]);
}

template <bool OUT_F32>
__device__ __forceinline__ void store_out(void* y, int64_t idx, float v) {
  if constexpr (OUT_F32)
    reinterpret_cast<float*>(y)[idx] = v;
  else
    reinterpret_cast<uint16_t*>(y)[idx] = f32_to_bf16_bits(v);
}

}  // namespace pgs
