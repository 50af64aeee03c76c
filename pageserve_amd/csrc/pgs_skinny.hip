// Skinny W8A16 kernel for decode-sized inputs (m <= 16 tokens).
//
// Memory bound: every int8 weight byte is read from HBM exactly once, from
// the packed tile layout (pgs_common.h) with 128-bit non-temporal loads, so
// each wave instruction streams one contiguous KiB that is already the A
// operand of two MFMAs; the weights are widened to bf16 in registers and fed to
// v_mfma_f32_16x16x32_bf16 (tokens padded to 16 columns; for m = 1 the idle
// columns cost nothing, the kernel is far from MFMA bound).
//
// Work decomposition: one workgroup per (16-row tile, K split).  The NW waves
// of a workgroup take 64-k chunks of its K range round robin, U chunks per
// batch with every load of a batch in flight together, and their partial
// 16x16 tiles are summed through LDS in a fixed order.  Short-N shapes
// (o_proj, down_proj: 128 tiles) would leave half of the 256 CUs idle, so
// their K range is split over several workgroups: each writes its partial
// tile to the workspace and a second small kernel sums the partials in split
// order and runs the epilogue.  (Combining them inside one kernel would need
// an agent-scope release per workgroup, which writes back the whole L2 and
// costs far more than the extra launch.)  Results never depend on timing:
// every sum has a fixed order.
#include "pgs_linear.h"

namespace pgs {
namespace {

// output (token mm, row i of a 16-row tile) lives in accumulator lane
// (i/4)*16 + mm, register i%4
__device__ __forceinline__ int acc_lane(int i, int mm) { return (i >> 2) * 16 + mm; }

template <int NMAT, bool OUT_F32>
__device__ __forceinline__ void epilogue(const GroupArgs& a, int g, int n, int mm, int N, const float (&v)[NMAT]) {
  const float* sc0 = (NMAT == 2) ? a.scale[0] : pick(a.scale, g);
  void* y = (NMAT == 2) ? a.y[0] : pick(a.y, g);
  float out;
  if constexpr (NMAT == 2) {
    out = silu_f32(v[0] * sc0[n]) * (v[1] * a.scale[1][n]);
  } else {
    out = v[0] * sc0[n];
    const uint16_t* bias = pick(a.bias, g);
    if (bias) out += bf16_bits_to_f32(bias[n]);
    out = add_residual<OUT_F32>(out, pick(a.res, g), static_cast<int64_t>(mm) * N + n);
  }
  store_out<OUT_F32>(y, static_cast<int64_t>(mm) * N + n, out);
}

template <int NW, int U, int NMAT, bool OUT_F32, bool K64>
__global__ __launch_bounds__(64 * NW) void skinny_kernel(const uint16_t* __restrict__ x, GroupArgs a, int M,
                                                         int K, int splits, float* __restrict__ partials,
                                                         unsigned long long* __restrict__ pairs) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int tile = blockIdx.x / splits;
  const int s = blockIdx.x - tile * splits;

  const int g = (NMAT == 2) ? 0 : member_of(a, tile);
  const int N = pick(a.n, g);
  const int row0 = (tile - pick(a.unit_begin, g)) * 16;
  const int lrow = lane & 15;
  const int kgrp = lane >> 4;

  // packed weights: block (tile, chunk) is 1 KiB, this lane's 16 bytes at lane*16
  const int nchunks = (K + 63) >> 6;
  const int8_t* wrow[NMAT];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) {
    const int8_t* qg = (NMAT == 2) ? a.q[mat] : pick(a.q, g);
    wrow[mat] = qg + static_cast<int64_t>(row0 >> 4) * nchunks * 1024 + lane * 16;
  }
  const uint16_t* xrow = x + static_cast<int64_t>(min(lrow, M - 1)) * K + kgrp * 16;

  const int cb = static_cast<int>(static_cast<int64_t>(s) * nchunks / splits);
  const int ce = static_cast<int>(static_cast<int64_t>(s + 1) * nchunks / splits);

  f32x4 acc[NMAT];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) acc[mat] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto mac = [&](const u32x4 (&wv)[NMAT], u32x4 x0, u32x4 x1) {
    const bf16x8 b0 = __builtin_bit_cast(bf16x8, x0);
    const bf16x8 b1 = __builtin_bit_cast(bf16x8, x1);
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) {
      acc[mat] = mfma16x16x32(i8x8_to_bf16x8(wv[mat][0], wv[mat][1]), b0, acc[mat]);
      acc[mat] = mfma16x16x32(i8x8_to_bf16x8(wv[mat][2], wv[mat][3]), b1, acc[mat]);
    }
  };

  // Full batches of U chunks, software pipelined: the loads of the next batch
  // are issued before the MFMAs of the current one, so every wave keeps a
  // batch in flight while it computes.
  struct Batch {
    u32x4 w[U][NMAT];
    u32x4 x[U][2];
  };
  auto load_batch = [&](Batch& b, int c) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int koff = (c + u) * 64;
      // activations are not padded: a chunk past K reloads the first 16
      // columns of the row (in bounds, K >= 16) and mac_batch zeroes it
      // (branch free; masking here would wait at issue)
      const int xo = (K64 || koff + kgrp * 16 < K) ? koff : -kgrp * 16;
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat) b.w[u][mat] = ld16_stream(wrow[mat] + (c + u) * 1024);
      b.x[u][0] = ld16(xrow + xo);
      b.x[u][1] = ld16(xrow + xo + 8);
    }
  };
  auto mac_batch = [&](const Batch& b, int c) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t mask = (K64 || (c + u) * 64 + kgrp * 16 < K) ? 0xffffffffu : 0u;
      mac(b.w[u], b.x[u][0] & mask, b.x[u][1] & mask);
    }
  };
  constexpr int kStep = NW * U;
  int c0 = cb + wave * U;
  if (c0 + U <= ce) {
    Batch cur;
    load_batch(cur, c0);
    while (c0 + kStep + U <= ce) {
      Batch nxt;
      load_batch(nxt, c0 + kStep);
      mac_batch(cur, c0);
      cur = nxt;
      c0 += kStep;
    }
    mac_batch(cur, c0);
    c0 += kStep;
  }
  // the last partial batch of this wave, one chunk at a time
  for (int c = c0; c < min(c0 + U, ce); ++c) {
    const int koff = c * 64;
    const bool on = K64 || koff + kgrp * 16 < K;
    u32x4 wv[NMAT];
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) wv[mat] = ld16_stream(wrow[mat] + c * 1024);
    const uint32_t mask = on ? 0xffffffffu : 0u;
    const int xo = on ? koff : -kgrp * 16;
    const u32x4 x0 = ld16(xrow + xo) & mask;
    const u32x4 x1 = ld16(xrow + xo + 8) & mask;
    mac(wv, x0, x1);
  }

  __shared__ f32x4 red[NW][NMAT][64];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) red[wave][mat][lane] = acc[mat];
  __syncthreads();

  const int outs = M * 16;
  float* mine = partials + (static_cast<int64_t>(tile) * splits + s) * (NMAT * 256);
  for (int idx = threadIdx.x; idx < outs; idx += 64 * NW) {
    const int mm = idx >> 4, i = idx & 15;
    const int ln = acc_lane(i, mm), r = i & 3;
    float v[NMAT];
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) t += red[w][mat][ln][r];
      v[mat] = t;
    }
    if (NMAT == 1 && pairs) {
      // The two K halves of this tile meet in one 64-bit slot per output.
      // The first to arrive leaves (1, its partial); the second takes it,
      // empties the slot for the next call and finishes the output.  The data
      // travels inside the atomic, so no fence or wait is needed, and the sum
      // does not depend on the arrival order (fp32 addition is commutative).
      // System scope: the two workgroups run on different XCDs, and the
      // exchange is then performed beyond their L2s.
      unsigned long long* slot = pairs + static_cast<int64_t>(tile) * 256 + idx;
      const unsigned long long prev = __hip_atomic_exchange(slot, (1ull << 32) | __float_as_uint(v[0]), __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_SYSTEM);
      if (prev >> 32) {
        __hip_atomic_exchange(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        v[0] += __uint_as_float(static_cast<uint32_t>(prev));
        if (row0 + i < N) epilogue<NMAT, OUT_F32>(a, g, row0 + i, mm, N, v);
      }
    } else if (splits > 1) {
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat) mine[mat * 256 + idx] = v[mat];
    } else if (row0 + i < N) {
      epilogue<NMAT, OUT_F32>(a, g, row0 + i, mm, N, v);
    }
  }
}

// Sums the split partial tiles of each 16-row tile in split order, then runs
// the epilogue.  One 256-thread workgroup per tile (<= 16 x 16 outputs).
template <int NMAT, bool OUT_F32>
__global__ __launch_bounds__(256) void skinny_reduce_kernel(GroupArgs a, int M, int splits,
                                                            const float* __restrict__ partials) {
  const int tile = blockIdx.x;
  const int g = (NMAT == 2) ? 0 : member_of(a, tile);
  const int N = pick(a.n, g);
  const int row0 = (tile - pick(a.unit_begin, g)) * 16;
  const int idx = threadIdx.x;
  if (idx >= M * 16) return;
  const int mm = idx >> 4, i = idx & 15;
  if (row0 + i >= N) return;
  const float* base = partials + static_cast<int64_t>(tile) * splits * (NMAT * 256);
  float v[NMAT];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) {
    float t = 0.f;
    for (int sp = 0; sp < splits; ++sp) t += base[sp * (NMAT * 256) + mat * 256 + idx];
    v[mat] = t;
  }
  epilogue<NMAT, OUT_F32>(a, g, row0 + i, mm, N, v);
}

template <int NW, int U, int NMAT, bool OUT_F32>
int launch_cfg(Problem& p, const SkinnyPlan& plan, hipStream_t st) {
  const int64_t grid = static_cast<int64_t>(plan.tiles) * plan.splits;
  unsigned long long* pairs = plan.pair ? p.pairs : nullptr;
  if (p.k % 64 == 0)
    hipLaunchKernelGGL((skinny_kernel<NW, U, NMAT, OUT_F32, true>), dim3(static_cast<unsigned>(grid)), dim3(64 * NW),
                       0, st, p.x, p.args, p.m, p.k, plan.splits, p.partials, pairs);
  else
    hipLaunchKernelGGL((skinny_kernel<NW, U, NMAT, OUT_F32, false>), dim3(static_cast<unsigned>(grid)),
                       dim3(64 * NW), 0, st, p.x, p.args, p.m, p.k, plan.splits, p.partials, pairs);
  int rc = check_launch("w8a16 skinny kernel");
  if (rc || plan.splits == 1 || plan.pair) return rc;
  hipLaunchKernelGGL((skinny_reduce_kernel<NMAT, OUT_F32>), dim3(static_cast<unsigned>(plan.tiles)), dim3(256), 0, st,
                     p.args, p.m, plan.splits, p.partials);
  return check_launch("w8a16 skinny reduce kernel");
}

template <int NMAT, bool OUT_F32>
int launch_nw(Problem& p, const SkinnyPlan& plan, hipStream_t st) {
  switch (plan.nw) {
    case 4: return launch_cfg<4, 2, NMAT, OUT_F32>(p, plan, st);
    case 8: return launch_cfg<8, 2, NMAT, OUT_F32>(p, plan, st);
    default: return launch_cfg<16, 2, NMAT, OUT_F32>(p, plan, st);
  }
}

}  // namespace

SkinnyPlan plan_skinny(int m, int k, int nmat, int tiles, bool can_split) {
  (void)m;
  (void)nmat;
  // Measured on MI355X inside HIP graphs (decode shapes of a 2048-hidden
  // model): 8 waves per workgroup with 2-chunk pipelined batches is best for
  // K = 2048; a long K (down_proj, K = 11008) over few tiles wants 16 waves
  // and a 2-way K split so that twice as many CUs stream it.
  SkinnyPlan p{tiles, 8, 1, false};
  const int chunks = (k + 63) / 64;
  if (can_split && tiles < 256) {
    if (nmat == 1 && chunks >= 16) {
      p.splits = 2;  // K halves combined through pair slots
      p.pair = true;
    } else if (chunks >= 128) {
      p.splits = 2;  // SwiGLU pair: partial tiles and a reduce kernel
    }
  }
  const int per_wg = (chunks + p.splits - 1) / p.splits;
  p.nw = per_wg >= 64 ? 16 : per_wg >= 16 ? 8 : 4;
  return p;
}

size_t skinny_partial_bytes(const SkinnyPlan& p, int nmat) {
  return (p.splits > 1 && !p.pair) ? static_cast<size_t>(p.tiles) * p.splits * nmat * 256 * sizeof(float) : 0;
}

int launch_skinny(Problem& p, const SkinnyPlan& plan, hipStream_t st) {
  if (plan.pair && (!p.pairs || plan.tiles * 256 * sizeof(unsigned long long) > kPairBytes || p.nmat != 1))
    return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16 skinny: paired split without pair slots");
  if (plan.splits > 1 && !plan.pair && (!p.partials || p.partial_bytes < skinny_partial_bytes(plan, p.nmat)))
    return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16 skinny: split-K plan without a large enough workspace");
  if (p.nmat == 2) return launch_nw<2, false>(p, plan, st);
  return p.out_f32 ? launch_nw<1, true>(p, plan, st) : launch_nw<1, false>(p, plan, st);
}

}  // namespace pgs
