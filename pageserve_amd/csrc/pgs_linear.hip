// W8A16 linear kernels for gfx950: y = x . (q * scale)^T (+ bias).
//
// Replaces the reference's per-call "dequantize to a dense weight, then GEMM"
// (engine/quantization.py:26-27 via engine/model.py:25-26 feeding F.linear at
// engine/model.py:168-170, 184, 188-190, 193).  The int8 weight is read once
// from HBM and widened to bf16 in registers (exact: |q| <= 127); products are
// accumulated in fp32 on the matrix cores; the per-row scale (and bias) is
// applied once per output in the epilogue.
//
// Two kernel families share one MFMA shape, v_mfma_f32_16x16x32_bf16, with the
// weight as the A operand (16 weight rows) and the activations as B (16
// tokens).  Per lane l the A and B operands carry the same 8 consecutive k
// values, so a 16-byte load of 16 int8 weights feeds two MFMAs.  The
// accumulator lane l holds D[4*(l/16)+r][l%16], r = 0..3.
//
//  * skinny (m <= 16, decode): no LDS staging of operands.  Each wave streams
//    16-row weight tiles with 128-bit loads (16 rows x 64 contiguous bytes per
//    instruction), the workgroup's waves split K, and the partial 16x16 tiles
//    are summed through LDS in a fixed order before the epilogue.
//  * tile GEMM (m > 16, prefill): 128x128 output tiles, BK = 64.  Activation
//    tiles are copied to LDS; int8 weight tiles are widened to bf16 on the way
//    into LDS (each weight converted once per workgroup); LDS is double
//    buffered with register prefetch of the next K step; 16-byte chunks are
//    XOR-swizzled by row so MFMA operand reads are bank-conflict free.
//    Workgroup ids are remapped so tiles that share a weight panel run on the
//    same XCD (dispatch is round-robin over the 8 XCDs, each with its own L2).
//
// Both fuse the SwiGLU pair (engine/model.py:188-190): the gate and up tiles
// of the same rows are accumulated side by side and the epilogue writes
// silu(g * s_g) * (u * s_u).
#include <algorithm>
#include <atomic>

#include "pgs_common.h"

namespace pgs {
namespace {

struct GroupArgs {
  const int8_t* q[PGS_MAX_GROUP];
  const float* scale[PGS_MAX_GROUP];
  const uint16_t* bias[PGS_MAX_GROUP];
  void* y[PGS_MAX_GROUP];
  int32_t n[PGS_MAX_GROUP];
  int32_t unit_begin[PGS_MAX_GROUP + 1];
  int32_t n_outs;
};

// Selects member [g] with constant indices only (a dynamic index into a
// kernel-argument array would spill the struct to scratch).
template <typename T, int L>
__device__ __forceinline__ T pick(const T (&arr)[L], int g) {
  T v = arr[0];
#pragma unroll
  for (int i = 1; i < PGS_MAX_GROUP; ++i) v = (g == i) ? arr[i] : v;
  return v;
}

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

template <bool OUT_F32>
__device__ __forceinline__ void store_out(void* y, int64_t idx, float v) {
  if constexpr (OUT_F32)
    reinterpret_cast<float*>(y)[idx] = v;
  else
    reinterpret_cast<uint16_t*>(y)[idx] = f32_to_bf16_bits(v);
}

// ===========================================================================
// skinny kernel, m <= 16
// ===========================================================================
//
// Grid: one workgroup per "unit" of RT 16-row tiles of one output (group
// member g).  NW waves split the K chunks (64 k each) round-robin; each wave
// keeps U chunks of loads in flight.  NMAT = 2 is the SwiGLU pair: member 0
// is the gate, member 1 the up projection, one output (member 0's y).
template <int RT, int NW, int U, int NMAT, bool OUT_F32>
__global__ __launch_bounds__(64 * NW) void skinny_kernel(const uint16_t* __restrict__ x, GroupArgs a, int M,
                                                         int K) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int unit = blockIdx.x;

  int g = 0;
#pragma unroll
  for (int i = 1; i < PGS_MAX_GROUP; ++i) g = (i < a.n_outs && unit >= a.unit_begin[i] && NMAT == 1) ? i : g;

  const int N = pick(a.n, g);
  const int row0 = (unit - pick(a.unit_begin, g)) * RT * 16;
  const int lrow = lane & 15;
  const int kgrp = lane >> 4;

  const int8_t* wrow[NMAT][RT];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) {
    const int8_t* qg = (NMAT == 2) ? a.q[mat] : pick(a.q, g);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int r = min(row0 + rt * 16 + lrow, N - 1);
      wrow[mat][rt] = qg + static_cast<int64_t>(r) * K + kgrp * 16;
    }
  }
  const uint16_t* xrow = x + static_cast<int64_t>(min(lrow, M - 1)) * K + kgrp * 16;

  f32x4 acc[NMAT][RT];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[mat][rt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nchunks = K >> 6;
  for (int c0 = wave * U; c0 < nchunks; c0 += NW * U) {
    u32x4 wv[U][NMAT][RT];
    u32x4 xv[U][2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = c0 + u;
      if (c < nchunks) {
        const int koff = c * 64;
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) wv[u][mat][rt] = ld16(wrow[mat][rt] + koff);
        xv[u][0] = ld16(xrow + koff);
        xv[u][1] = ld16(xrow + koff + 8);
      } else {
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
          for (int rt = 0; rt < RT; ++rt) wv[u][mat][rt] = u32x4{0u, 0u, 0u, 0u};
        xv[u][0] = u32x4{0u, 0u, 0u, 0u};
        xv[u][1] = u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bf16x8 b0 = __builtin_bit_cast(bf16x8, xv[u][0]);
      const bf16x8 b1 = __builtin_bit_cast(bf16x8, xv[u][1]);
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) {
          const u32x4 w = wv[u][mat][rt];
          acc[mat][rt] = mfma16x16x32(i8x8_to_bf16x8(w[0], w[1]), b0, acc[mat][rt]);
          acc[mat][rt] = mfma16x16x32(i8x8_to_bf16x8(w[2], w[3]), b1, acc[mat][rt]);
        }
    }
  }
  // K tail: 16 <= K % 64 < 64 (K is a multiple of 16); handled by the last wave.
  const int ktail = K & 63;
  if (ktail != 0 && wave == NW - 1) {
    const int koff = nchunks * 64;
    const bool on = kgrp * 16 < ktail;
    u32x4 x0 = on ? ld16(xrow + koff) : u32x4{0u, 0u, 0u, 0u};
    u32x4 x1 = on ? ld16(xrow + koff + 8) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const u32x4 w = on ? ld16(wrow[mat][rt] + koff) : u32x4{0u, 0u, 0u, 0u};
        acc[mat][rt] = mfma16x16x32(i8x8_to_bf16x8(w[0], w[1]), __builtin_bit_cast(bf16x8, x0), acc[mat][rt]);
        acc[mat][rt] = mfma16x16x32(i8x8_to_bf16x8(w[2], w[3]), __builtin_bit_cast(bf16x8, x1), acc[mat][rt]);
      }
  }

  __shared__ f32x4 red[NW][NMAT][RT][64];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) red[wave][mat][rt][lane] = acc[mat][rt];
  __syncthreads();

  const float* sc0 = (NMAT == 2) ? a.scale[0] : pick(a.scale, g);
  const float* sc1 = a.scale[1];
  const uint16_t* bias = (NMAT == 2) ? nullptr : pick(a.bias, g);
  void* y = (NMAT == 2) ? a.y[0] : pick(a.y, g);
  const int total = M * RT * 16;
  for (int idx = threadIdx.x; idx < total; idx += 64 * NW) {
    const int mm = idx / (RT * 16);
    const int nl = idx - mm * (RT * 16);
    const int n = row0 + nl;
    if (n >= N) continue;
    const int rt = nl >> 4;
    const int i = nl & 15;
    const int ln = (i >> 2) * 16 + mm;
    const int r = i & 3;
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      s0 += red[w][0][rt][ln][r];
      if constexpr (NMAT == 2) s1 += red[w][NMAT - 1][rt][ln][r];
    }
    float v;
    if constexpr (NMAT == 2) {
      v = silu_f32(s0 * sc0[n]) * (s1 * sc1[n]);
    } else {
      v = s0 * sc0[n];
      if (bias) v += bf16_bits_to_f32(bias[n]);
    }
    store_out<OUT_F32>(y, static_cast<int64_t>(mm) * N + n, v);
  }
}

// ===========================================================================
// tile GEMM, m > 16
// ===========================================================================

constexpr int kBK = 64;          // k per LDS stage: 128 bytes of bf16 per row
constexpr int kGemmThreads = 256;  // 4 waves, 2 (m) x 2 (n)

// Maps the dispatch-order workgroup id to a logical tile so that each XCD
// (which receives ids xcd, xcd + 8, ...) gets one contiguous run of tiles.
__device__ __forceinline__ int xcd_remap(int b, int total) {
  const int xcd = b & 7, slot = b >> 3;
  const int per = total >> 3, rem = total & 7;
  return (xcd < rem) ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
}

// LDS element offset (bf16 units) of logical 16-byte chunk `ch` of row `row`
// in a [rows][64] tile; chunks are XOR-swizzled with the row's low 3 bits.
__device__ __forceinline__ int swz(int row, int ch) { return row * kBK + ((ch ^ (row & 7)) << 3); }

template <int BM, int BN, int NMAT, bool OUT_F32>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(const uint16_t* __restrict__ x, GroupArgs a, int M,
                                                            int K, int tiles_m, int tiles_total) {
  constexpr int XS = BM * kBK;  // bf16 elements of one X stage
  constexpr int WS = BN * kBK;  // bf16 elements of one W stage (per matrix)
  constexpr int STAGE = XS + NMAT * WS;
  constexpr int XL = BM / 32;   // 16-byte X chunk loads per thread
  constexpr int WL = BN / 64;   // 16-byte int8 W loads per thread per matrix
  constexpr int TM = BM / 32;   // 16-token MFMA tiles per wave
  constexpr int TN = BN / 32;   // 16-row MFMA tiles per wave
  static_assert(BM % 32 == 0 && BN % 64 == 0, "tile shape");

  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;

  const int t = xcd_remap(blockIdx.x, tiles_total);
  // locate the group member owning this tile (units are counted in tiles)
  int g = 0;
#pragma unroll
  for (int i = 1; i < PGS_MAX_GROUP; ++i) g = (i < a.n_outs && t >= a.unit_begin[i] * tiles_m && NMAT == 1) ? i : g;
  const int tl = t - pick(a.unit_begin, g) * tiles_m;
  const int N = pick(a.n, g);
  const int n0 = (tl / tiles_m) * BN;
  const int m0 = (tl % tiles_m) * BM;

  // global source pointers of this thread's chunks
  const uint16_t* xsrc[XL];
  int xoff[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int ci = tid + kGemmThreads * i;
    const int row = ci >> 3, ch = ci & 7;
    xsrc[i] = x + static_cast<int64_t>(min(m0 + row, M - 1)) * K + ch * 8;
    xoff[i] = swz(row, ch);
  }
  const int8_t* wsrc[NMAT][WL];
  int woff[WL];
#pragma unroll
  for (int i = 0; i < WL; ++i) {
    const int ci = tid + kGemmThreads * i;
    const int row = ci >> 2, c4 = ci & 3;
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) {
      const int8_t* qg = (NMAT == 2) ? a.q[mat] : pick(a.q, g);
      wsrc[mat][i] = qg + static_cast<int64_t>(min(n0 + row, N - 1)) * K + c4 * 16;
    }
    woff[i] = row * kBK;  // chunk index 2*c4 (+1) swizzled below
  }
  u32x4 xr[XL];
  u32x4 wr[NMAT][WL];
  const int ktiles = (K + kBK - 1) / kBK;

  auto gload = [&](int kt) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const int ci = tid + kGemmThreads * i;
      const bool on = k0 + (ci & 7) * 8 < K;
      xr[i] = on ? ld16(xsrc[i] + k0) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < WL; ++i) {
      const int ci = tid + kGemmThreads * i;
      const bool on = k0 + (ci & 3) * 16 < K;
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat) wr[mat][i] = on ? ld16(wsrc[mat][i] + k0) : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto lstore = [&](int stage) {
    uint16_t* s = smem + stage * STAGE;
#pragma unroll
    for (int i = 0; i < XL; ++i) *reinterpret_cast<u32x4*>(s + xoff[i]) = xr[i];
#pragma unroll
    for (int i = 0; i < WL; ++i) {
      const int ci = tid + kGemmThreads * i;
      const int row = ci >> 2, c4 = ci & 3;
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat) {
        uint16_t* ws = s + XS + mat * WS;
        const u32x4 w = wr[mat][i];
        *reinterpret_cast<bf16x8*>(ws + swz(row, 2 * c4)) = i8x8_to_bf16x8(w[0], w[1]);
        *reinterpret_cast<bf16x8*>(ws + swz(row, 2 * c4 + 1)) = i8x8_to_bf16x8(w[2], w[3]);
      }
    }
  };

  f32x4 acc[NMAT][TN][TM];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
    for (int nt = 0; nt < TN; ++nt)
#pragma unroll
      for (int mt = 0; mt < TM; ++mt) acc[mat][nt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  gload(0);
  lstore(0);
  __syncthreads();

  const int lr = lane & 15, lg = lane >> 4;
  for (int kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < ktiles) gload(kt + 1);
    const uint16_t* s = smem + cur * STAGE;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int ch = 4 * h + lg;
      bf16x8 bx[TM];
#pragma unroll
      for (int mt = 0; mt < TM; ++mt) {
        const int row = wm * (BM / 2) + mt * 16 + lr;
        bx[mt] = *reinterpret_cast<const bf16x8*>(s + swz(row, ch));
      }
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat) {
        const uint16_t* ws = s + XS + mat * WS;
#pragma unroll
        for (int nt = 0; nt < TN; ++nt) {
          const int row = wn * (BN / 2) + nt * 16 + lr;
          const bf16x8 aw = *reinterpret_cast<const bf16x8*>(ws + swz(row, ch));
#pragma unroll
          for (int mt = 0; mt < TM; ++mt) acc[mat][nt][mt] = mfma16x16x32(aw, bx[mt], acc[mat][nt][mt]);
        }
      }
    }
    if (kt + 1 < ktiles) lstore(cur ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds rows n = base + 4*lg + r, token m = base + lr
  const float* sc0 = (NMAT == 2) ? a.scale[0] : pick(a.scale, g);
  const float* sc1 = a.scale[1];
  const uint16_t* bias = (NMAT == 2) ? nullptr : pick(a.bias, g);
  void* y = (NMAT == 2) ? a.y[0] : pick(a.y, g);
  // 4 consecutive outputs per lane: vector store when every row start is aligned
  const bool yvec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & (OUT_F32 ? 15 : 7)) == 0;
#pragma unroll
  for (int nt = 0; nt < TN; ++nt) {
    const int nb = n0 + wn * (BN / 2) + nt * 16 + 4 * lg;
    float s0[4], s1[4], bv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int n = min(nb + r, N - 1);
      s0[r] = sc0[n];
      s1[r] = (NMAT == 2) ? sc1[n] : 0.f;
      bv[r] = (NMAT == 1 && bias) ? bf16_bits_to_f32(bias[n]) : 0.f;
    }
#pragma unroll
    for (int mt = 0; mt < TM; ++mt) {
      const int m = m0 + wm * (BM / 2) + mt * 16 + lr;
      if (m >= M) continue;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if constexpr (NMAT == 2)
          v[r] = silu_f32(acc[0][nt][mt][r] * s0[r]) * (acc[1][nt][mt][r] * s1[r]);
        else
          v[r] = acc[0][nt][mt][r] * s0[r] + bv[r];
      }
      const int64_t base = static_cast<int64_t>(m) * N + nb;
      if (yvec && nb + 3 < N) {
        if constexpr (OUT_F32) {
          *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(y) + base) = f32x4{v[0], v[1], v[2], v[3]};
        } else {
          *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(y) + base) =
              u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        }
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (nb + r < N) store_out<OUT_F32>(y, base + r, v[r]);
      }
    }
  }
}

// ===========================================================================
// host side
// ===========================================================================

struct Problem {
  const uint16_t* x;
  GroupArgs args;
  int m, k;
  int nmat;  // 1 = plain / grouped, 2 = SwiGLU pair
  bool out_f32;
};

template <int RT, int NW, int U, int NMAT, bool OUT_F32>
int launch_skinny(Problem& p, hipStream_t st) {
  int units = 0;
  const int members = (NMAT == 2) ? 1 : p.args.n_outs;
  for (int i = 0; i < members; ++i) {
    p.args.unit_begin[i] = units;
    const int tiles = (p.args.n[i] + 15) / 16;
    units += (tiles + RT - 1) / RT;
  }
  for (int i = members; i <= PGS_MAX_GROUP; ++i) p.args.unit_begin[i] = units;
  hipLaunchKernelGGL((skinny_kernel<RT, NW, U, NMAT, OUT_F32>), dim3(units), dim3(64 * NW), 0, st, p.x, p.args,
                     p.m, p.k);
  return check_launch("w8a16 skinny kernel");
}

template <int NMAT, bool OUT_F32>
int dispatch_skinny(Problem& p, hipStream_t st) {
  // total 16-row tiles across members decides how many waves split K
  int64_t tiles = 0;
  const int members = (NMAT == 2) ? 1 : p.args.n_outs;
  for (int i = 0; i < members; ++i) tiles += (p.args.n[i] + 15) / 16;
  const int chunks = p.k / 64;
  // aim for >= ~2048 waves on the 256 CUs while giving each wave >= 4 chunks
  if (tiles >= 512 || chunks < 16) return launch_skinny<1, 4, 4, NMAT, OUT_F32>(p, st);
  if (tiles >= 256 || chunks < 32) return launch_skinny<1, 8, 4, NMAT, OUT_F32>(p, st);
  return launch_skinny<1, 16, 4, NMAT, OUT_F32>(p, st);
}

template <int BM, int BN, int NMAT, bool OUT_F32>
int launch_gemm(Problem& p, hipStream_t st) {
  const int tiles_m = (p.m + BM - 1) / BM;
  int units = 0;  // n-tiles
  const int members = (NMAT == 2) ? 1 : p.args.n_outs;
  for (int i = 0; i < members; ++i) {
    p.args.unit_begin[i] = units;
    units += (p.args.n[i] + BN - 1) / BN;
  }
  for (int i = members; i <= PGS_MAX_GROUP; ++i) p.args.unit_begin[i] = units;
  const int64_t total = static_cast<int64_t>(units) * tiles_m;
  if (total > 0x7fffffff) return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16 gemm: too many tiles");
  constexpr size_t lds = sizeof(uint16_t) * 2 * (BM * kBK + NMAT * BN * kBK);
  // the dynamic-LDS limit is a per-function, per-device attribute: set it once per device
  static std::atomic<uint64_t> attr_done{0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(PGS_ERR_NO_DEVICE, "w8a16 gemm: hipGetDevice failed");
  const uint64_t bit = 1ull << (dev & 63);
  if (!(attr_done.load(std::memory_order_acquire) & bit)) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kernel<BM, BN, NMAT, OUT_F32>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess) return fail(PGS_ERR_LAUNCH, "w8a16 gemm: cannot reserve %zu bytes of LDS: %s", lds,
                                     hipGetErrorString(e));
    attr_done.fetch_or(bit, std::memory_order_acq_rel);
  }
  hipLaunchKernelGGL((gemm_kernel<BM, BN, NMAT, OUT_F32>), dim3(static_cast<unsigned>(total)), dim3(kGemmThreads),
                     lds, st, p.x, p.args, p.m, p.k, tiles_m, static_cast<int>(total));
  return check_launch("w8a16 gemm kernel");
}

template <int NMAT, bool OUT_F32>
int dispatch(Problem& p, hipStream_t st) {
  if (p.m <= 16) return dispatch_skinny<NMAT, OUT_F32>(p, st);
  return launch_gemm<128, 128, NMAT, OUT_F32>(p, st);
}

int run(Problem& p, hipStream_t st) {
  if (p.nmat == 2) return dispatch<2, false>(p, st);
  return p.out_f32 ? dispatch<1, true>(p, st) : dispatch<1, false>(p, st);
}

int check_common(const char* fn, const void* x, int64_t m, int64_t k) {
  if (m < 0 || k < 0) return fail(PGS_ERR_INVALID_ARGUMENT, "%s: negative size m=%lld k=%lld", fn, (long long)m,
                                  (long long)k);
  if (m > 0x7fffffff || k > 0x7fffffff) return fail(PGS_ERR_INVALID_ARGUMENT, "%s: size too large", fn);
  if (k % 16 != 0)
    return fail(PGS_ERR_INVALID_ARGUMENT, "%s: in_features k=%lld must be a multiple of 16", fn, (long long)k);
  if (m > 0 && k > 0 && !x) return fail(PGS_ERR_INVALID_ARGUMENT, "%s: null activation pointer", fn);
  if (!aligned(x, 16)) return fail(PGS_ERR_MISALIGNED, "%s: activations must be 16-byte aligned", fn);
  return PGS_OK;
}

int check_member(const char* fn, const int8_t* q, const float* scale, const void* bias, const void* y, int64_t n,
                 int64_t m, int64_t k) {
  if (n < 0 || n > 0x7fffffff) return fail(PGS_ERR_INVALID_ARGUMENT, "%s: bad out_features n=%lld", fn, (long long)n);
  if (n == 0 || m == 0) return PGS_OK;
  if (!y || !scale || (k > 0 && !q)) return fail(PGS_ERR_INVALID_ARGUMENT, "%s: null pointer", fn);
  if (!aligned(q, 16)) return fail(PGS_ERR_MISALIGNED, "%s: int8 weights must be 16-byte aligned", fn);
  if (!aligned(scale, 4) || !aligned(bias, 2) || !aligned(y, 4))
    return fail(PGS_ERR_MISALIGNED, "%s: scale/bias/output misaligned", fn);
  if (static_cast<double>(m) * static_cast<double>(n) > 9.0e18)
    return fail(PGS_ERR_INVALID_ARGUMENT, "%s: output too large", fn);
  return PGS_OK;
}

}  // namespace
}  // namespace pgs

using namespace pgs;

extern "C" int pgs_w8a16_linear_group(const void* x, const pgs_linear_out* outs, int n_outs, int y_dtype,
                                      int64_t m, int64_t k, void* stream) {
  const char* fn = "pgs_w8a16_linear_group";
  int rc = check_common(fn, x, m, k);
  if (rc) return rc;
  if (!outs || n_outs < 1 || n_outs > PGS_MAX_GROUP)
    return fail(PGS_ERR_INVALID_ARGUMENT, "%s: n_outs=%d must be in [1, %d]", fn, n_outs, PGS_MAX_GROUP);
  if (y_dtype != PGS_DTYPE_BF16 && y_dtype != PGS_DTYPE_F32)
    return fail(PGS_ERR_INVALID_ARGUMENT, "%s: output dtype code %d not bf16/fp32", fn, y_dtype);
  Problem p{};
  p.x = reinterpret_cast<const uint16_t*>(x);
  p.m = static_cast<int>(m);
  p.k = static_cast<int>(k);
  p.nmat = 1;
  p.out_f32 = (y_dtype == PGS_DTYPE_F32);
  int used = 0;
  for (int i = 0; i < n_outs; ++i) {
    rc = check_member(fn, outs[i].q, outs[i].scale, outs[i].bias, outs[i].y, outs[i].n, m, k);
    if (rc) return rc;
    if (outs[i].n == 0) continue;
    p.args.q[used] = outs[i].q;
    p.args.scale[used] = outs[i].scale;
    p.args.bias[used] = reinterpret_cast<const uint16_t*>(outs[i].bias);
    p.args.y[used] = outs[i].y;
    p.args.n[used] = static_cast<int32_t>(outs[i].n);
    ++used;
  }
  if (m == 0 || used == 0) return PGS_OK;
  if (k == 0) {
    return fail(PGS_ERR_INVALID_ARGUMENT, "%s: in_features k=0 is not supported", fn);
  }
  p.args.n_outs = used;
  for (int i = used; i < PGS_MAX_GROUP; ++i) {
    p.args.q[i] = p.args.q[0];
    p.args.scale[i] = p.args.scale[0];
    p.args.bias[i] = nullptr;
    p.args.y[i] = p.args.y[0];
    p.args.n[i] = 0;
  }
  return run(p, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int pgs_w8a16_linear(const void* x, const int8_t* q, const float* scale, const void* bias, void* y,
                                int y_dtype, int64_t m, int64_t n, int64_t k, void* stream) {
  pgs_linear_out o{q, scale, bias, y, n};
  return pgs_w8a16_linear_group(x, &o, 1, y_dtype, m, k, stream);
}

extern "C" int pgs_w8a16_swiglu(const void* x, const int8_t* q_gate, const float* s_gate, const int8_t* q_up,
                                const float* s_up, void* act, int64_t m, int64_t n, int64_t k, void* stream) {
  const char* fn = "pgs_w8a16_swiglu";
  int rc = check_common(fn, x, m, k);
  if (rc) return rc;
  rc = check_member(fn, q_gate, s_gate, nullptr, act, n, m, k);
  if (rc) return rc;
  rc = check_member(fn, q_up, s_up, nullptr, act, n, m, k);
  if (rc) return rc;
  if (m == 0 || n == 0) return PGS_OK;
  if (k == 0) return fail(PGS_ERR_INVALID_ARGUMENT, "%s: in_features k=0 is not supported", fn);
  Problem p{};
  p.x = reinterpret_cast<const uint16_t*>(x);
  p.m = static_cast<int>(m);
  p.k = static_cast<int>(k);
  p.nmat = 2;
  p.out_f32 = false;
  p.args.n_outs = 1;
  p.args.q[0] = q_gate;
  p.args.q[1] = q_up;
  p.args.scale[0] = s_gate;
  p.args.scale[1] = s_up;
  p.args.y[0] = act;
  p.args.y[1] = act;
  p.args.n[0] = static_cast<int32_t>(n);
  p.args.n[1] = static_cast<int32_t>(n);
  for (int i = 2; i < PGS_MAX_GROUP; ++i) {
    p.args.q[i] = q_gate;
    p.args.scale[i] = s_gate;
    p.args.y[i] = act;
    p.args.n[i] = 0;
  }
  return run(p, reinterpret_cast<hipStream_t>(stream));
}
