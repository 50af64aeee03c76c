// LDS-tiled W8A16 MFMA GEMM for prefill-sized inputs (m > 16 tokens).
//
// 128x128 output tiles (tokens x weight rows), BK = 64, 4 waves (2 x 2), each
// wave 64x64 via v_mfma_f32_16x16x32_bf16.  Activation tiles are copied to
// LDS; int8 weight tiles are widened to bf16 on their way into LDS (each
// weight converted once per workgroup).  LDS is double buffered with register
// prefetch of the next K step, and 16-byte chunks are XOR-swizzled by row so
// the MFMA operand reads do not conflict on banks.  Workgroup ids are
// remapped so that the tiles sharing a weight panel run on the same XCD
// (dispatch is round robin over the 8 XCDs, each with its own L2).  NMAT = 2
// is the fused SwiGLU pair: gate and up tiles accumulate side by side and the
// epilogue writes silu(g * s_g) * (u * s_u).
#include <atomic>

#include "pgs_linear.h"

namespace pgs {
namespace {

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
  // packed weights: thread ci reads lane (ci % 64) of 16-row block (ci / 64),
  // i.e. row 16*(ci/64) + ci%16, k bytes 16*((ci%64)/16) .. +15 of the step
  const int kb = (K + kBK - 1) / kBK;
  const int last_block = (N + 15) / 16 - 1;
  const int8_t* wsrc[NMAT][WL];
#pragma unroll
  for (int i = 0; i < WL; ++i) {
    const int ci = tid + kGemmThreads * i;
    const int blk = min((n0 >> 4) + (ci >> 6), last_block);
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) {
      const int8_t* qg = (NMAT == 2) ? a.q[mat] : pick(a.q, g);
      wsrc[mat][i] = qg + static_cast<int64_t>(blk) * kb * 1024 + (ci & 63) * 16;
    }
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
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat) wr[mat][i] = ld16(wsrc[mat][i] + kt * 1024);
    }
  };
  auto lstore = [&](int stage) {
    uint16_t* s = smem + stage * STAGE;
#pragma unroll
    for (int i = 0; i < XL; ++i) *reinterpret_cast<u32x4*>(s + xoff[i]) = xr[i];
#pragma unroll
    for (int i = 0; i < WL; ++i) {
      const int ci = tid + kGemmThreads * i;
      const int row = ((ci >> 6) << 4) + (ci & 15), c4 = (ci & 63) >> 4;
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


template <int BM, int BN, int NMAT, bool OUT_F32>
int launch_cfg(Problem& p, const GemmPlan& plan, hipStream_t st) {
  constexpr size_t lds = sizeof(uint16_t) * 2 * (BM * kBK + NMAT * BN * kBK);
  // the dynamic-LDS limit is a per-function, per-device attribute: set it once per device
  static std::atomic<uint64_t> attr_done{0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(PGS_ERR_NO_DEVICE, "w8a16 gemm: hipGetDevice failed");
  const uint64_t bit = 1ull << (dev & 63);
  if (!(attr_done.load(std::memory_order_acquire) & bit)) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kernel<BM, BN, NMAT, OUT_F32>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    if (e != hipSuccess)
      return fail(PGS_ERR_LAUNCH, "w8a16 gemm: cannot reserve %zu bytes of LDS: %s", lds, hipGetErrorString(e));
    attr_done.fetch_or(bit, std::memory_order_acq_rel);
  }
  hipLaunchKernelGGL((gemm_kernel<BM, BN, NMAT, OUT_F32>), dim3(static_cast<unsigned>(plan.tiles)),
                     dim3(kGemmThreads), lds, st, p.x, p.args, p.m, p.k, plan.tiles_m, plan.tiles);
  return check_launch("w8a16 gemm kernel");
}

}  // namespace

GemmPlan plan_gemm(int m, int k, int nmat, const int32_t* n, int members, bool can_split) {
  (void)k;
  (void)nmat;
  (void)can_split;
  GemmPlan p{};
  p.bm = 128;
  p.bn = 128;
  p.tiles_m = (m + p.bm - 1) / p.bm;
  p.tiles_n = 0;
  for (int i = 0; i < members; ++i) p.tiles_n += (n[i] + p.bn - 1) / p.bn;
  p.tiles = p.tiles_m * p.tiles_n;
  p.splits = 1;
  return p;
}

size_t gemm_partial_bytes(const GemmPlan& p, int nmat) {
  (void)p;
  (void)nmat;
  return 0;
}

int launch_gemm(Problem& p, const GemmPlan& plan, hipStream_t st) {
  // member boundaries in units of n-tiles
  int units = 0;
  const int members = (p.nmat == 2) ? 1 : p.args.n_outs;
  for (int i = 0; i < members; ++i) {
    p.args.unit_begin[i] = units;
    units += (p.args.n[i] + plan.bn - 1) / plan.bn;
  }
  for (int i = members; i <= PGS_MAX_GROUP; ++i) p.args.unit_begin[i] = units;
  if (p.nmat == 2) return launch_cfg<128, 128, 2, false>(p, plan, st);
  return p.out_f32 ? launch_cfg<128, 128, 1, true>(p, plan, st) : launch_cfg<128, 128, 1, false>(p, plan, st);
}

}  // namespace pgs
