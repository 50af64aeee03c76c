// W8A16 MFMA GEMM for prefill-sized inputs (m > 32 tokens).
//
// Output tile BM tokens x BN weight rows per workgroup of 4 waves, K stepped
// 64 at a time (one packed weight block column).  The waves split the tile
// along N: wave w owns weight rows [w*BN/4, (w+1)*BN/4) for all BM tokens.
//
//  * Weights never touch LDS.  In the packed layout (pgs_common.h) a 16-row x
//    64-k block is one contiguous KiB whose lane-l 16 bytes are exactly lane
//    l's A operand for two v_mfma_f32_16x16x32_bf16, so each wave loads its
//    own blocks with 128-bit loads straight into registers and widens them to
//    bf16 there; every weight is read and converted once per workgroup.
//  * Activations go through LDS, double buffered: [BM][64] bf16 per stage,
//    16-byte chunks XOR-swizzled with (row/2)%8 so that the 16 lanes of a
//    ds_read_b128 cover all 64 banks once.  All 4 waves read them as B.
//  * Global loads run ahead of the MFMAs: one K step (LEAD = 1, predicated)
//    or two (LEAD = 2, rotating register sets).  Weights stay in registers,
//    activations go registers -> LDS one step before their use, or, in
//    gemm_dma_kernel (the SwiGLU pair above 128 tokens, lm_head, and single
//    matrices with many tiles), straight from memory into S LDS stages by
//    the buffer unit's LDS DMA, S - 1 steps ahead and without registers.
//  * Weight loads are ordinary cached loads: the tiles_m workgroups of one
//    weight panel run together on one XCD and share it through its L2.
//  * NMAT = 2 is the SwiGLU pair: gate and up blocks of the same rows are
//    accumulated side by side; the epilogue writes silu(g*s_g) * (u*s_u).
//  * Split K: with few output tiles (o_proj / down_proj at prefill sizes) the
//    K range is split over `splits` workgroups per tile; each writes its fp32
//    partial tile to the workspace and a second kernel sums the partials in
//    split order and runs the epilogue (a fixed order: reproducible).
//  * Workgroup ids are remapped so the units sharing a weight panel (same
//    weight rows and K split) run on the same XCD (dispatch is round robin
//    over the 8 XCDs, each with its own L2).
#include <type_traits>
#include <utility>

#include "pgs_linear.h"

namespace pgs {
namespace {

constexpr int kBK = 64;
constexpr int kBN = 128;  // weight rows per tile and matrix: 4 waves x 32
constexpr int kThreads = 256;

// Element offset (bf16 units) of 16-byte chunk `ch` of row `row` in a
// [rows][64] stage.  The chunk is XOR-swizzled with bits 0..2 of the row and
// bit 3 folded into bit 0, so that the 16 lanes a 128-bit LDS access serves
// per cycle (16 consecutive rows, one chunk column: the B-operand reads; or
// two rows' eight chunks: the stores) hit 16 distinct 16-byte bank groups of
// gfx950's 64 banks (measured: zero bank-conflict cycles).
__device__ __forceinline__ int swz(int row, int ch) { return row * kBK + ((ch ^ (row & 7) ^ ((row >> 3) & 1)) << 3); }

struct GemmArgs {
  GroupArgs g;
  int M, K;
  int tiles_m;     // token tiles
  int tiles;       // output tiles (tiles_m x weight-row tiles over all members)
  int splits;
  float* partials;
};

// Split-K partial tile in lane order: [tile][split][mat][nt][mt][lane] x f32x4
// (the reduce kernel reads the same order).  Written and read once each,
// with the non-temporal policy (down_proj at 128 / 512 tokens 18.4 / 37.5
// against 19.2 / 37.9 us with the default one).
template <int TN, int TM, int NMAT, typename Args>
__device__ __forceinline__ void store_partials(const f32x4 (&acc)[NMAT][TN][TM], const Args& ga, int t, int s, int wave,
                                               int lane) {
  constexpr int SLOTS = 4 * TN * TM * 64;
  f32x4* part = reinterpret_cast<f32x4*>(ga.partials) + (static_cast<int64_t>(t) * ga.splits + s) * NMAT * SLOTS;
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
    for (int nt = 0; nt < TN; ++nt)
#pragma unroll
      for (int mt = 0; mt < TM; ++mt)
        __builtin_nontemporal_store(acc[mat][nt][mt], part + mat * SLOTS + ((wave * TN + nt) * TM + mt) * 64 + lane);
}

// Epilogue operands of four consecutive output rows nb .. nb+3 (clamped to
// N - 1 past the end): scales, bias (single matrices) or the pair's second
// scale.
template <int NMAT>
struct Rows4 {
  float s0[4], s1[4], bv[4];
};
template <int NMAT>
__device__ __forceinline__ Rows4<NMAT> rows4(const GroupArgs& a, int g, int N, int nb) {
  const float* sc0 = (NMAT == 2) ? a.scale[0] : pick(a.scale, g);
  const float* sc1 = a.scale[NMAT - 1];
  const uint16_t* bias = (NMAT == 2) ? nullptr : pick(a.bias, g);
  // the bias is loaded unconditionally (an absent one reads the scales as a
  // dummy address) and selected afterwards: a load under a branch makes the
  // compiler wait for every earlier load, the kernels' activation DMAs
  // included, before continuing
  const uint16_t* bsrc = bias ? bias : reinterpret_cast<const uint16_t*>(sc0);
  Rows4<NMAT> e;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int n = min(nb + r, N - 1);
    e.s0[r] = sc0[n];
    e.s1[r] = (NMAT == 2) ? sc1[n] : 0.f;
    if constexpr (NMAT == 1) {
      const float bvr = bf16_bits_to_f32(bsrc[n]);
      e.bv[r] = bias ? bvr : 0.f;
    } else {
      e.bv[r] = 0.f;
    }
  }
  return e;
}

// Rows nb .. nb+3 of token m from their fp32 sums: scale and bias, or SwiGLU,
// then the residual (single matrices) and one vector store when the four
// outputs are in range and aligned (`yvec`), else element stores.
template <int NMAT, bool OUT_F32>
__device__ __forceinline__ void store_rows4(const GroupArgs& a, int g, int N, int m, int nb, const Rows4<NMAT>& e,
                                            const f32x4& v0, const f32x4& v1, void* y, bool yvec) {
  float v[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if constexpr (NMAT == 2)
      v[r] = silu_f32(v0[r] * e.s0[r]) * (v1[r] * e.s1[r]);
    else
      v[r] = v0[r] * e.s0[r] + e.bv[r];
  }
  const int64_t base = static_cast<int64_t>(m) * N + nb;
  const uint16_t* res = (NMAT == 2) ? nullptr : pick(a.res, g);
  if (NMAT == 1 && res) {
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = add_residual<OUT_F32>(v[r], res, base + min(r, N - 1 - nb));
  }
  if (yvec && nb + 3 < N) {
    if constexpr (OUT_F32)
      *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(y) + base) = f32x4{v[0], v[1], v[2], v[3]};
    else
      *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(y) + base) =
          u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (nb + r < N) store_out<OUT_F32>(y, base + r, v[r]);
  }
}

template <bool OUT_F32>
__device__ __forceinline__ bool vec_out(const void* y, int N) {
  return (N & 3) == 0 && (reinterpret_cast<uintptr_t>(y) & (OUT_F32 ? 15 : 7)) == 0;
}

// Epilogue of one workgroup tile: lane (lr, lg) of wave `wave` holds, for
// weight tile nt and token tile mt, rows nb + r (r = 0..3) of token
// m0 + mt*16 + lr, nb = n0 + wave*BN/4 + nt*16 + 4*lg.  Applies scale, bias
// or SwiGLU and stores bf16 / fp32.
template <int BN, int TN, int TM, int NMAT, bool OUT_F32>
__device__ __forceinline__ void store_tile(const f32x4 (&acc)[NMAT][TN][TM], const GroupArgs& a, int g, int M,
                                           int N, int m0, int n0, int wave, int lr, int lg) {
  void* y = (NMAT == 2) ? a.y[0] : pick(a.y, g);
  const bool yvec = vec_out<OUT_F32>(y, N);
#pragma unroll
  for (int nt = 0; nt < TN; ++nt) {
    const int nb = n0 + wave * (BN / 4) + nt * 16 + 4 * lg;
    const Rows4<NMAT> e = rows4<NMAT>(a, g, N, nb);
#pragma unroll
    for (int mt = 0; mt < TM; ++mt) {
      const int m = m0 + mt * 16 + lr;
      if (m >= M) continue;
      store_rows4<NMAT, OUT_F32>(a, g, N, m, nb, e, acc[0][nt][mt], acc[NMAT - 1][nt][mt], y, yvec);
    }
  }
}

template <int BM, int BN, int NMAT, bool OUT_F32, int OCC, int LEAD>
__global__ __launch_bounds__(kThreads, OCC) void gemm_kernel(const uint16_t* __restrict__ x, GemmArgs ga) {
  constexpr int TM = BM / 16;        // token tiles per wave
  constexpr int TN = BN / 64;        // 16-row weight tiles per wave (per matrix)
  constexpr int XS = BM * kBK;       // bf16 elements of one activation stage
  constexpr int XL = BM * 8 / kThreads;  // 16-byte activation chunks per thread per stage
  static_assert(BM % 32 == 0 && BN % 64 == 0 && XL >= 1, "tile shape");
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][XS];

  const GroupArgs& a = ga.g;
  const int M = ga.M, K = ga.K;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // work unit u = (weight-row tile, split, token tile), token tile fastest:
  // the tiles_m units that read the same weight blocks are consecutive, and
  // the remap puts consecutive units on one XCD (one L2)
  const int u = xcd_remap(blockIdx.x, ga.tiles * ga.splits);
  const int tm = u % ga.tiles_m, r = u / ga.tiles_m;
  const int s = r % ga.splits;
  const int t = (r / ga.splits) * ga.tiles_m + tm;

  // tile -> (member, n0, m0); members are counted in n-tiles of BN rows
  int g = 0;
#pragma unroll
  for (int i = 1; i < PGS_MAX_GROUP; ++i)
    g = (NMAT == 1 && i < a.n_outs && t >= a.unit_begin[i] * ga.tiles_m) ? i : g;
  const int tl = t - pick(a.unit_begin, g) * ga.tiles_m;
  const int N = pick(a.n, g);
  const int n0 = (tl / ga.tiles_m) * BN;
  const int m0 = (tl % ga.tiles_m) * BM;

  const int kb = (K + kBK - 1) / kBK;  // packed block columns = K steps
  const int kt0 = static_cast<int>(static_cast<int64_t>(s) * kb / ga.splits);
  const int kt1 = static_cast<int>(static_cast<int64_t>(s + 1) * kb / ga.splits);

  // this wave's weight blocks: rows n0 + wave*BN/4 + nt*16 .. +15 (clamped to the
  // last real block; rows past N are padding zeros or discarded)
  const int last_blk = (N + 15) / 16 - 1;
  const int8_t* wptr[NMAT][TN];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) {
    const int8_t* qg = (NMAT == 2) ? a.q[mat] : pick(a.q, g);
#pragma unroll
    for (int nt = 0; nt < TN; ++nt) {
      const int blk = min((n0 >> 4) + wave * TN + nt, last_blk);
      wptr[mat][nt] = qg + static_cast<int64_t>(blk) * kb * 1024 + lane * 16;
    }
  }
  // this thread's activation chunks: row ci/8, chunk ci%8 of the stage
  const uint16_t* xptr[XL];
  int xoff[XL], xcol[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int ci = tid + kThreads * i;
    const int row = ci >> 3, ch = ci & 7;
    xptr[i] = x + static_cast<int64_t>(min(m0 + row, M - 1)) * K + ch * 8;
    xoff[i] = swz(row, ch);
    xcol[i] = ch * 8;
  }

  using WRegs = u32x4[NMAT][TN];
  using XRegs = u32x4[XL];
  auto wload = [&](int kt, WRegs& w) {
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
      for (int nt = 0; nt < TN; ++nt) w[mat][nt] = ld16(wptr[mat][nt] + kt * 1024);
  };
  // K tail: an activation chunk past K is zeroed when it is stored to LDS
  // (masking the loaded value would wait for the load right away)
  auto xstore = [&](uint16_t* stage, const XRegs& xv, int kt) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      const uint32_t mask = (k0 + xcol[i] < K) ? 0xffffffffu : 0u;
      *reinterpret_cast<u32x4*>(stage + xoff[i]) = xv[i] & mask;
    }
  };

  f32x4 acc[NMAT][TN][TM];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
    for (int nt = 0; nt < TN; ++nt)
#pragma unroll
      for (int mt = 0; mt < TM; ++mt) acc[mat][nt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int lr = lane & 15, lg = lane >> 4;
  auto compute = [&](const WRegs& wc, const uint16_t* stage) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      bf16x8 aw[NMAT][TN];
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
        for (int nt = 0; nt < TN; ++nt)
          aw[mat][nt] = i8x8_to_bf16x8(wc[mat][nt][2 * h], wc[mat][nt][2 * h + 1]);
      // the packed A operand of lane group lg holds k = 16*lg + 8*h .. +7:
      // the matching activation chunk (8 bf16) is 2*lg + h
      const int ch = 2 * lg + h;
#pragma unroll
      for (int mt = 0; mt < TM; ++mt) {
        const bf16x8 bx = *reinterpret_cast<const bf16x8*>(stage + swz(mt * 16 + lr, ch));
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
          for (int nt = 0; nt < TN; ++nt) acc[mat][nt][mt] = mfma16x16x32(aw[mat][nt], bx, acc[mat][nt][mt]);
      }
    }
  };

  if constexpr (LEAD == 1) {
    // One-step prefetch, predicated: step kt + 1's loads are issued before
    // step kt's MFMAs and land in LDS (activations) / registers (weights)
    // after them.
    WRegs wa, wc;
    XRegs xa;
    auto xload = [&](int kt) {
      const int k0 = kt * kBK;
#pragma unroll
      for (int i = 0; i < XL; ++i) xa[i] = (k0 + xcol[i] < K) ? ld16(xptr[i] + k0) : u32x4{0u, 0u, 0u, 0u};
    };
    if (kt0 < kt1) {
      wload(kt0, wa);
      xload(kt0);
      xstore(xs[0], xa, kt0);
    }
    __syncthreads();
    for (int kt = kt0; kt < kt1; ++kt) {
      const int cur = (kt - kt0) & 1;
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
        for (int nt = 0; nt < TN; ++nt) wc[mat][nt] = wa[mat][nt];
      if (kt + 1 < kt1) {
        wload(kt + 1, wa);
        xload(kt + 1);
      }
      compute(wc, xs[cur]);
      if (kt + 1 < kt1) xstore(xs[cur ^ 1], xa, kt + 1);
      __syncthreads();
    }
  } else {
    // Two-step lead in rotating register sets (no copies): weights in three
    // sets, activations in two (they reach LDS one step before their use).
    // The loop is unrolled by six so every set index is static.  Loads past
    // the end of the range are clamped to the last step (redundant, in
    // bounds): a branch around them would make the compiler wait for every
    // outstanding load where the paths join.  For the same reason an
    // activation chunk past K reloads the row's first 8 columns (in bounds)
    // and xstore zeroes it.  Activation loads are issued
    // before weight loads, so the wait before their LDS store leaves the
    // younger weight loads in flight.
    WRegs wset[3];
    XRegs xset[2];
    const int last = kt1 - 1;
    auto xload = [&](int kt, XRegs& xv) {
      const int k0 = kt * kBK;
#pragma unroll
      for (int i = 0; i < XL; ++i) xv[i] = ld16(xptr[i] + (k0 + xcol[i] < K ? k0 : -xcol[i]));
    };
    auto step = [&](auto I, int kt) {
      constexpr int i = decltype(I)::value;
      xload(min(kt + 2, last), xset[i % 2]);
      wload(min(kt + 2, last), wset[(i + 2) % 3]);
      __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the MFMAs
      compute(wset[i % 3], xs[(kt - kt0) & 1]);
      // step kt + 1's activations were loaded one step ago
      if (kt + 1 < kt1) xstore(xs[(kt - kt0 + 1) & 1], xset[(i + 1) % 2], kt + 1);
      __syncthreads();
    };
    if (kt0 < kt1) {
      xload(kt0, xset[0]);
      wload(kt0, wset[0]);
      xload(min(kt0 + 1, last), xset[1]);
      wload(min(kt0 + 1, last), wset[1]);
      xstore(xs[0], xset[0], kt0);
      __syncthreads();
      for (int kt = kt0;;) {
        step(std::integral_constant<int, 0>{}, kt);
        if (++kt >= kt1) break;
        step(std::integral_constant<int, 1>{}, kt);
        if (++kt >= kt1) break;
        step(std::integral_constant<int, 2>{}, kt);
        if (++kt >= kt1) break;
        step(std::integral_constant<int, 3>{}, kt);
        if (++kt >= kt1) break;
        step(std::integral_constant<int, 4>{}, kt);
        if (++kt >= kt1) break;
        step(std::integral_constant<int, 5>{}, kt);
        if (++kt >= kt1) break;
      }
    }
  }

  // ---- epilogue: lane holds rows nb + r (r = 0..3) for token m0 + mt*16 + lr
  if (ga.splits > 1) {
    store_partials<TN, TM, NMAT>(acc, ga, t, s, wave, lane);
    return;
  }
  store_tile<BN, TN, TM, NMAT, OUT_F32>(acc, a, g, M, N, m0, n0, wave, lr, lg);
}

// The kernel for K % 64 == 0 (every shape of the Qwen2 family): BM tokens x
// 128 weight rows (per matrix) per workgroup, optional K split.
//  * A 16x16x32 MFMA leaves the vector ALU only a few cycles of its issue
//    time, so the int8 -> bf16 widening (1.5 VALU per weight element) bounds
//    the loop unless each widened operand feeds enough MFMAs: it feeds one
//    per 16-token tile, BM/16 of them (BM = 128: 1.5 VALU per MFMA).
//  * Both operands use buffer loads: K is stepped through the scalar offset
//    (no per-step address arithmetic) and the hardware range check returns
//    zeros for weight blocks past the matrix and activation rows past M (no
//    clamping or masking); the loop carries no VALU beyond the widening.
//  * Weights run two K steps ahead in three rotating register sets,
//    activations XLEAD steps ahead through double-buffered LDS; the loop is
//    unrolled by six so every set and stage index is static.

// Runs step(integral_constant<i>, kt) for kt = kt0 .. kt1-1 with the loop
// body unrolled over i = 0 .. sizeof...(Is)-1; the fold stops after the step
// that ends the range.
template <typename Step, int... Is>
__device__ __forceinline__ void run_steps(Step& step, int kt0, int kt1, std::integer_sequence<int, Is...>) {
  for (int kt = kt0;;)
    if (!((step(std::integral_constant<int, Is>{}, kt), ++kt < kt1) && ...)) break;
}

// f(integral_constant<J>) for J in Js, in order.
template <typename F, int... Js>
__device__ __forceinline__ void static_for(F&& f, std::integer_sequence<int, Js...>) {
  (f(std::integral_constant<int, Js>{}), ...);
}

// The same steps as whole unrolled blocks in a loop with a single exit, then
// the remainder (fewer than sizeof...(Is) steps, positions 0, 1, ...) after
// it.  For loops that read LDS filled by buffer-to-LDS DMA: at the head of a
// loop with an exit after every step the compiler's wait insertion loses
// track of which LDS object each DMA in flight targets and waits for all of
// them; with one exit it keeps them apart.
template <typename Step, int... Is>
__device__ __forceinline__ void run_blocks(Step& step, int iters, std::integer_sequence<int, Is...>) {
  constexpr int U = sizeof...(Is);
  int j = 0;
  for (; j + U <= iters; j += U) (step(std::integral_constant<int, Is>{}, j + Is), ...);
  const int r = iters - j;
  ((Is < r ? step(std::integral_constant<int, Is>{}, j + Is) : void()), ...);
}

constexpr int gcd2(int a, int b) { return b ? gcd2(b, a % b) : a; }
constexpr int lcm3(int a, int b, int c) { return a / gcd2(a, b) * b / gcd2(a / gcd2(a, b) * b, c) * c; }

// Linear tile index -> (weight tile, token tile) in blocks of kGroup x kGroup
// (partial blocks at the edges), weight-tile blocks outermost, token tiles
// fastest inside a block: the units of one weight tile stay contiguous, so
// the contiguous range each XCD receives splits at most one weight panel.
constexpr int kGroup = 8;
__device__ __forceinline__ void block_order(int t, int tiles_n, int tiles_m, int& tn, int& tm) {
  const int per_ngroup = kGroup * tiles_m;
  const int gn = t / per_ngroup;
  const int gn_size = min(kGroup, tiles_n - gn * kGroup);
  const int r = t - gn * per_ngroup;
  const int mb = r / (gn_size * kGroup);
  const int gm_size = min(kGroup, tiles_m - mb * kGroup);
  const int rem = r - mb * gn_size * kGroup;
  tn = gn * kGroup + rem / gm_size;
  tm = mb * kGroup + rem % gm_size;
}

//  * KG = 2 or 4 runs that many groups of four waves per workgroup on
//    interleaved K steps (each group with its own LDS stages), so a workgroup
//    of a small tile still gives every SIMD KG waves and keeps KG times the
//    weight bytes in flight; the other groups hand their accumulators to
//    group 0 through LDS at the end, one at a time in a fixed order.  All
//    groups run the same number of iterations (a group past its last step
//    loads its last step again and skips the MFMAs), so every barrier is
//    reached by all waves.
template <int BM, int BN, int NMAT, bool OUT_F32, int WLEAD, int XLEAD, int OCC, int KG>
__global__ __launch_bounds__(kThreads * KG, OCC) void gemm_k64_kernel(const uint16_t* __restrict__ x, GemmArgs ga) {
  constexpr int TM = BM / 16, TN = BN / 64;
  static_assert(BN % 64 == 0, "weight rows per tile: 4 waves x 16-row multiples");
  constexpr int WSETS = WLEAD + 1;               // rotating weight register sets
  constexpr int UNROLL = lcm3(WSETS, XLEAD, 2);  // static set and stage indices
  static_assert(BM % 32 == 0 && WLEAD >= 1 && XLEAD >= 1 && (KG == 1 || KG == 2 || KG == 4), "tile shape / pipeline");
  constexpr int XS = BM * kBK;           // bf16 elements of one activation stage
  constexpr int XL = BM * 8 / kThreads;  // 16-byte activation chunks per thread per stage
  constexpr int kStageBytes = KG * 2 * XS * 2;
  constexpr int kRedBytes = KG > 1 ? 4 * NMAT * TN * TM * 64 * 16 : 0;
  __shared__ __attribute__((aligned(16))) char smem[kStageBytes > kRedBytes ? kStageBytes : kRedBytes];

  const GroupArgs& a = ga.g;
  const int M = ga.M, K = ga.K;
  // (kg is wave-uniform; readfirstlane makes that visible to the compiler, so
  // the K offsets derived from it stay in scalar registers: a buffer load
  // whose scalar offset sits in a vector register is wrapped in a loop over
  // its distinct values)
  const int tid = threadIdx.x, lane = tid & 63, wave = (tid >> 6) & 3, kg = __builtin_amdgcn_readfirstlane(tid >> 8);
  const int tid_g = tid & (kThreads - 1);
  uint16_t* const xs = reinterpret_cast<uint16_t*>(smem) + kg * 2 * XS;
  // Work units: (weight tile, K split, token tile).  (split, weight tile)
  // pairs form "virtual" weight tiles, split-major, ordered in blocks of
  // kGroup virtual weight tiles x kGroup token tiles, so the ~64 workgroups
  // an XCD runs at once share 8 weight panels and 8 activation tiles through
  // its L2; the remap keeps consecutive units on one XCD.
  const int tiles_n = ga.tiles / ga.tiles_m;
  int vn, mt_all;
  block_order(xcd_remap(blockIdx.x, ga.tiles * ga.splits), tiles_n * ga.splits, ga.tiles_m, vn, mt_all);
  const int s = vn / tiles_n, nt_all = vn - s * tiles_n;
  const int t = nt_all * ga.tiles_m + mt_all;  // tile index of the split partials
  int g = 0;
#pragma unroll
  for (int i = 1; i < PGS_MAX_GROUP; ++i) g = (NMAT == 1 && i < a.n_outs && nt_all >= a.unit_begin[i]) ? i : g;
  const int N = pick(a.n, g);
  const int n0 = (nt_all - pick(a.unit_begin, g)) * BN;
  const int m0 = mt_all * BM;
  const int kb = K / kBK;
  const int kt0 = static_cast<int>(static_cast<int64_t>(s) * kb / ga.splits);
  const int kt1 = static_cast<int>(static_cast<int64_t>(s + 1) * kb / ga.splits);
  // this group's K steps: kt0 + kg, kt0 + kg + KG, ... < kt1
  // (a group with no step at all, range <= kg, only loads step kt0 and computes nothing)
  const int range = kt1 - kt0;
  const int iters = (range + KG - 1) / KG;
  const int first = kt0 + kg;
  const int last = range > kg ? kt0 + kg + ((range - 1 - kg) / KG) * KG : kt0;

  // weights: one resource per matrix starting at this tile's first row block
  const int blk0 = n0 >> 4, blocks = (N + 15) >> 4;
  __amdgpu_buffer_rsrc_t wres[NMAT];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) {
    const int8_t* qg = (NMAT == 2) ? a.q[mat] : pick(a.q, g);
    wres[mat] = make_rsrc(qg + static_cast<int64_t>(blk0) * kb * 1024, static_cast<int64_t>(blocks - blk0) * kb * 1024);
  }
  int woff[TN];
#pragma unroll
  for (int nt = 0; nt < TN; ++nt) woff[nt] = (wave * TN + nt) * kb * 1024 + lane * 16;
  // activations: rows m0.. of x; rows past M read as zero
  const __amdgpu_buffer_rsrc_t xres = make_rsrc(x + static_cast<int64_t>(m0) * K, static_cast<int64_t>(M - m0) * K * 2);
  int xoff_g[XL], xoff_s[XL];
#pragma unroll
  for (int i = 0; i < XL; ++i) {
    const int ci = tid_g + kThreads * i;
    const int row = ci >> 3, ch = ci & 7;
    xoff_g[i] = row * K * 2 + ch * 16;
    xoff_s[i] = swz(row, ch);
  }
  const int lr = lane & 15, lg = lane >> 4;
  // B operand of token tile mt, K half h: swz(mt*16 + lr, 2*lg + h) = mt*1024 + swz(lr, 2*lg + h)
  const int bofs0 = swz(lr, 2 * lg), bofs1 = swz(lr, 2 * lg + 1);

  using WRegs = u32x4[NMAT][TN];
  using XRegs = u32x4[XL];
  WRegs wset[WSETS];
  XRegs xset[XLEAD];
  auto wload = [&](int kt, WRegs& w) {
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
      for (int nt = 0; nt < TN; ++nt) w[mat][nt] = __builtin_amdgcn_raw_buffer_load_b128(wres[mat], woff[nt], kt * 1024, 0);
  };
  auto xload = [&](int kt, XRegs& xr) {
#pragma unroll
    for (int i = 0; i < XL; ++i) xr[i] = __builtin_amdgcn_raw_buffer_load_b128(xres, xoff_g[i], kt * (kBK * 2), 0);
  };
  auto xstore = [&](int stage, const XRegs& xr) {
#pragma unroll
    for (int i = 0; i < XL; ++i) *reinterpret_cast<u32x4*>(xs + stage * XS + xoff_s[i]) = xr[i];
  };

  f32x4 acc[NMAT][TN][TM];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
    for (int nt = 0; nt < TN; ++nt)
#pragma unroll
      for (int mt = 0; mt < TM; ++mt) acc[mat][nt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Per K half: every B fragment of the half is read before its MFMAs (all
  // TM reads in flight at once; the compiler otherwise reuses one register
  // and waits out the LDS latency before every MFMA pair), then the weights
  // are widened and the MFMAs issued.
  auto compute = [&](const WRegs& wc, int stage) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint16_t* bsrc = xs + stage * XS + (h ? bofs1 : bofs0);
      bf16x8 bx[TM];
#pragma unroll
      for (int mt = 0; mt < TM; ++mt) bx[mt] = *reinterpret_cast<const bf16x8*>(bsrc + mt * 1024);
      __builtin_amdgcn_sched_barrier(0);
      bf16x8 aw[NMAT][TN];
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
        for (int nt = 0; nt < TN; ++nt) aw[mat][nt] = i8x8_to_bf16x8(wc[mat][nt][2 * h], wc[mat][nt][2 * h + 1]);
#pragma unroll
      for (int mt = 0; mt < TM; ++mt)
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
          for (int nt = 0; nt < TN; ++nt) acc[mat][nt][mt] = mfma16x16x32(aw[mat][nt], bx[mt], acc[mat][nt][mt]);
    }
  };

  // Iteration j (position i of the unrolled loop) handles this group's K
  // step kt = first + j*KG: load the weights of iteration j + WLEAD into set
  // (i + WLEAD) % WSETS and the activations of iteration j + XLEAD into set
  // i % XLEAD, run the MFMAs of step kt (weights in set i % WSETS,
  // activations in LDS stage i % 2), then store iteration j + 1's activations
  // (loaded XLEAD - 1 iterations ago, set (i + 1) % XLEAD) to the other
  // stage.  Loads past the group's last step are clamped to it (redundant).
  auto step = [&](auto I, int j) {
    constexpr int i = decltype(I)::value;
    const int kt = first + j * KG;
    xload(min(kt + XLEAD * KG, last), xset[i % XLEAD]);
    wload(min(kt + WLEAD * KG, last), wset[(i + WLEAD) % WSETS]);
    __builtin_amdgcn_sched_barrier(0);  // keep the loads ahead of the MFMAs
    // the MFMA phase at raised wave priority, so that when two workgroups
    // share a SIMD the one in its MFMA phase issues first (the SwiGLU pair at
    // 512 and 2048 tokens: 52.3 -> 50.5 us, 182 -> 175.5 us; single
    // matrices unchanged)
    __builtin_amdgcn_s_setprio(1);
    if (KG == 1 || kt < kt1) compute(wset[i % WSETS], i % 2);
    __builtin_amdgcn_s_setprio(0);
    if (j + 1 < iters) xstore((i + 1) % 2, xset[(i + 1) % XLEAD]);
    __syncthreads();
  };
#pragma unroll
  for (int j = 0; j < XLEAD; ++j) xload(min(first + j * KG, last), xset[j]);
#pragma unroll
  for (int j = 0; j < WLEAD; ++j) wload(min(first + j * KG, last), wset[j]);
  xstore(0, xset[0]);
  __syncthreads();
  run_steps(step, 0, iters, std::make_integer_sequence<int, UNROLL>{});

  if constexpr (KG > 1) {
    // groups KG-1 .. 1 hand their accumulators to group 0 through LDS, one
    // group at a time (fixed order; the stages are free after the last barrier)
    f32x4* red = reinterpret_cast<f32x4*>(smem);
#pragma unroll
    for (int src = KG - 1; src >= 1; --src) {
      if (kg == src) {
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
          for (int nt = 0; nt < TN; ++nt)
#pragma unroll
            for (int mt = 0; mt < TM; ++mt) red[(((wave * NMAT + mat) * TN + nt) * TM + mt) * 64 + lane] = acc[mat][nt][mt];
      }
      __syncthreads();
      if (kg == 0) {
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
          for (int nt = 0; nt < TN; ++nt)
#pragma unroll
            for (int mt = 0; mt < TM; ++mt) acc[mat][nt][mt] += red[(((wave * NMAT + mat) * TN + nt) * TM + mt) * 64 + lane];
      }
      __syncthreads();
    }
    if (kg != 0) return;
  }
  if (ga.splits > 1) {
    store_partials<TN, TM, NMAT>(acc, ga, t, s, wave, lane);
    return;
  }
  store_tile<BN, TN, TM, NMAT, OUT_F32>(acc, a, g, M, N, m0, n0, wave, lr, lg);
}
// The same tile with the activations moved from HBM/L2 into LDS by the
// buffer unit itself (buffer_load_dwordx4 ... lds, gfx950's 16-byte LDS DMA)
// instead of through registers: S stages of [BM][64] bf16, each the target of
// DMAs issued S - 1 K steps before its use, so an activation tile has S - 1
// steps to arrive and costs no registers while in flight (the register path
// could afford one step of lead, and its waves stalled at the end of every
// step on the LDS store of the next step's activations).  Each stage is its
// own LDS object, so the compiler's LDS-DMA tracking waits for exactly the
// DMAs of the stage a read touches; the waits that make a stage visible to
// the other waves are explicit: every wave waits for its own DMAs of the
// next stage (a vmcnt count: the loop issues the same loads every step),
// then one barrier per step.  Weights go to registers as in gemm_k64_kernel.
// Each lane's DMA writes 16 bytes at a fixed position of its wave's 1 KiB
// slice; the lane fetches the activation piece whose swizzled home (swz) is
// that position.
// 16 bytes per lane from a buffer into LDS: lane l's bytes land at lds + 16 l
// (the LDS address is wave-uniform; it goes to M0).  A __device__ function of
// its own: used directly in a kernel template, the builtin makes the host
// pass drop that kernel's launch stub.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint16_t* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

template <int BM, int BN, int NMAT, bool OUT_F32, int WLEAD, int S, int OCC>
__global__ __launch_bounds__(kThreads, OCC) void gemm_dma_kernel(const uint16_t* __restrict__ x, GemmArgs ga) {
  constexpr int TM = BM / 16, TN = BN / 64;
  constexpr int WSETS = WLEAD + 1;
  constexpr int UNROLL = lcm3(WSETS, S, 1);
  constexpr int XS = BM * kBK;           // bf16 elements of one stage
  constexpr int XL = BM * 8 / kThreads;  // DMA instructions per lane per stage
  constexpr int WL = NMAT * TN;          // weight loads per lane per step
  // (WLEAD >= S - 3: the per-step wait below counts the loads issued after
  // a stage's DMA; the first steps' stages come from the prologue, after
  // which only WLEAD weight steps were issued)
  static_assert(BM % 32 == 0 && BN % 64 == 0 && XL >= 1 && S >= 2 && S <= 8 && WLEAD >= 1 && WLEAD >= S - 3,
                "tile / pipeline");
  __shared__ __attribute__((aligned(16))) uint16_t st0[XS];
  __shared__ __attribute__((aligned(16))) uint16_t st1[XS];
  __shared__ __attribute__((aligned(16))) uint16_t st2[S > 2 ? XS : 1];
  __shared__ __attribute__((aligned(16))) uint16_t st3[S > 3 ? XS : 1];
  __shared__ __attribute__((aligned(16))) uint16_t st4[S > 4 ? XS : 1];
  __shared__ __attribute__((aligned(16))) uint16_t st5[S > 5 ? XS : 1];
  __shared__ __attribute__((aligned(16))) uint16_t st6[S > 6 ? XS : 1];
  __shared__ __attribute__((aligned(16))) uint16_t st7[S > 7 ? XS : 1];
  auto stage = [&](auto I) -> uint16_t* {
    constexpr int i = decltype(I)::value;
    if constexpr (i == 0) return st0;
    else if constexpr (i == 1) return st1;
    else if constexpr (i == 2) return st2;
    else if constexpr (i == 3) return st3;
    else if constexpr (i == 4) return st4;
    else if constexpr (i == 5) return st5;
    else if constexpr (i == 6) return st6;
    else return st7;
  };

  const GroupArgs& a = ga.g;
  const int M = ga.M, K = ga.K;
  // (the wave index is wave-uniform; readfirstlane makes that visible, so the
  // DMA's LDS address -- it goes to M0 -- stays a scalar)
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tiles_n = ga.tiles / ga.tiles_m;
  int vn, mt_all;
  block_order(xcd_remap(blockIdx.x, ga.tiles * ga.splits), tiles_n * ga.splits, ga.tiles_m, vn, mt_all);
  const int s = vn / tiles_n, nt_all = vn - s * tiles_n;
  const int t = nt_all * ga.tiles_m + mt_all;
  int g = 0;
#pragma unroll
  for (int i = 1; i < PGS_MAX_GROUP; ++i) g = (NMAT == 1 && i < a.n_outs && nt_all >= a.unit_begin[i]) ? i : g;
  const int N = pick(a.n, g);
  const int n0 = (nt_all - pick(a.unit_begin, g)) * BN;
  const int m0 = mt_all * BM;
  const int kb = K / kBK;
  const int kt0 = static_cast<int>(static_cast<int64_t>(s) * kb / ga.splits);
  const int kt1 = static_cast<int>(static_cast<int64_t>(s + 1) * kb / ga.splits);
  const int iters = kt1 - kt0, last = kt1 - 1;

  const int blk0 = n0 >> 4, blocks = (N + 15) >> 4;
  __amdgpu_buffer_rsrc_t wres[NMAT];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) {
    const int8_t* qg = (NMAT == 2) ? a.q[mat] : pick(a.q, g);
    wres[mat] = make_rsrc(qg + static_cast<int64_t>(blk0) * kb * 1024, static_cast<int64_t>(blocks - blk0) * kb * 1024);
  }
  int woff[TN];
#pragma unroll
  for (int nt = 0; nt < TN; ++nt) woff[nt] = (wave * TN + nt) * kb * 1024 + lane * 16;
  // activations: rows m0.. of x; rows past M read as zero
  const __amdgpu_buffer_rsrc_t xres = make_rsrc(x + static_cast<int64_t>(m0) * K, static_cast<int64_t>(M - m0) * K * 2);
  // DMA j of this wave fills 16-byte positions p = (wave*XL + j)*64 + lane of
  // a stage: row p / 8, physical chunk p % 8, i.e. logical chunk
  // (p % 8) ^ f(row), the inverse of swz
  int xoff_g[XL];
#pragma unroll
  for (int j = 0; j < XL; ++j) {
    const int p = (wave * XL + j) * 64 + lane;
    const int row = p >> 3;
    const int ch = (p & 7) ^ (row & 7) ^ ((row >> 3) & 1);
    xoff_g[j] = row * K * 2 + ch * 16;
  }
  const int lr = lane & 15, lg = lane >> 4;
  const int bofs0 = swz(lr, 2 * lg), bofs1 = swz(lr, 2 * lg + 1);

  using WRegs = u32x4[NMAT][TN];
  WRegs wset[WSETS];
  auto wload = [&](int kt, WRegs& w) {
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
      for (int nt = 0; nt < TN; ++nt) w[mat][nt] = __builtin_amdgcn_raw_buffer_load_b128(wres[mat], woff[nt], kt * 1024, 0);
  };
  auto dma = [&](uint16_t* dst, int kt) {
#pragma unroll
    for (int j = 0; j < XL; ++j)
      dma16(xres, dst + (wave * XL + j) * 512, xoff_g[j], kt * (kBK * 2));
  };

  f32x4 acc[NMAT][TN][TM];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
    for (int nt = 0; nt < TN; ++nt)
#pragma unroll
      for (int mt = 0; mt < TM; ++mt) acc[mat][nt][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const WRegs& wc, const uint16_t* stg) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint16_t* bsrc = stg + (h ? bofs1 : bofs0);
      bf16x8 bx[TM];
#pragma unroll
      for (int mt = 0; mt < TM; ++mt) bx[mt] = *reinterpret_cast<const bf16x8*>(bsrc + mt * 1024);
      __builtin_amdgcn_sched_barrier(0);
      bf16x8 aw[NMAT][TN];
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
        for (int nt = 0; nt < TN; ++nt) aw[mat][nt] = i8x8_to_bf16x8(wc[mat][nt][2 * h], wc[mat][nt][2 * h + 1]);
#pragma unroll
      for (int mt = 0; mt < TM; ++mt)
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
          for (int nt = 0; nt < TN; ++nt) acc[mat][nt][mt] = mfma16x16x32(aw[mat][nt], bx[mt], acc[mat][nt][mt]);
    }
  };
  // Every wave waits for its own DMAs into the stage the next step reads
  // (issued S - 2 steps before this one; each later step issued WL weight
  // loads, then XL DMAs), then one barrier makes the stage visible to all
  // and frees the stage just read for the DMA of the next step.
  constexpr int kAfter = (S - 2) * (WL + XL);
  constexpr int kWait = 0xF70 | (kAfter & 15) | ((kAfter >> 4) << 14);
  static_assert(kAfter < 64, "vmcnt range");
  auto step_barrier = [&] {
    __builtin_amdgcn_s_waitcnt(kWait);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // Iteration j (position i of the unrolled loop): weights of j + WLEAD into
  // set (i + WLEAD) % WSETS, DMA of j + S - 1 into stage (i + S - 1) % S
  // (loads past the last step repeat it: in bounds, counts unchanged), the
  // MFMAs of j on set i % WSETS and stage i % S, then the barrier.
  auto step = [&](auto I, int j) {
    constexpr int i = decltype(I)::value;
    const int kt = kt0 + j;
    wload(min(kt + WLEAD, last), wset[(i + WLEAD) % WSETS]);
    dma(stage(std::integral_constant<int, (i + S - 1) % S>{}), min(kt + S - 1, last));
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(1);
    compute(wset[i % WSETS], stage(std::integral_constant<int, i % S>{}));
    __builtin_amdgcn_s_setprio(0);
    step_barrier();
  };
  // (the planner gives every split at least one K step; a guard on iters here
  // costs the accumulators their registers: the compiler then spills them)
  {
    // prologue: stages 0 .. S-2, then weights 0 .. WLEAD-1; wait for stage 0
    static_for([&](auto J) { dma(stage(J), min(kt0 + decltype(J)::value, last)); },
               std::make_integer_sequence<int, S - 1>{});
#pragma unroll
    for (int j = 0; j < WLEAD; ++j) wload(min(kt0 + j, last), wset[j]);
    constexpr int kPro = (S - 2) * XL + WLEAD * WL;
    constexpr int kProWait = 0xF70 | (kPro & 15) | ((kPro >> 4) << 14);
    static_assert(kPro < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(kProWait);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    run_blocks(step, iters, std::make_integer_sequence<int, UNROLL>{});
    // the last steps' repeated loads (DMAs into LDS among them) land before
    // the workgroup ends and its LDS is handed to the next one
    __builtin_amdgcn_s_waitcnt(0xF70);
  }
  if (ga.splits > 1) {
    store_partials<TN, TM, NMAT>(acc, ga, t, s, wave, lane);
    return;
  }
  store_tile<BN, TN, TM, NMAT, OUT_F32>(acc, a, g, M, N, m0, n0, wave, lr, lg);
}

// Sums the split partial tiles in split order and runs the epilogue.  One
// thread per accumulator slot (4 consecutive output rows of one token) over
// all tiles; partial reads are coalesced 16-byte loads.  With the split
// count known (SPL = 2, 4, 8; 0: read at run time) every partial load is in
// flight before the first add (a runtime loop waits for each in turn), and
// the epilogue operands are requested before them; the sum is the same
// ((0 + p0) + p1) + ... either way.
template <int BM, int BN, int NMAT, bool OUT_F32, int SPL>
__global__ __launch_bounds__(kThreads) void gemm_reduce_kernel(GemmArgs ga) {
  constexpr int TM = BM / 16, TN = BN / 64;
  constexpr int SLOTS = 4 * TN * TM * 64;  // per tile and matrix
  const GroupArgs& a = ga.g;
  const int M = ga.M;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (gid >= static_cast<int64_t>(ga.tiles) * SLOTS) return;
  const int t = static_cast<int>(gid / SLOTS);
  const int slot = static_cast<int>(gid - static_cast<int64_t>(t) * SLOTS);
  const int lane = slot & 63;
  const int mt = (slot >> 6) % TM;
  const int nt = (slot >> 6) / TM % TN;
  const int wave = (slot >> 6) / (TM * TN);
  int g = 0;
#pragma unroll
  for (int i = 1; i < PGS_MAX_GROUP; ++i)
    g = (NMAT == 1 && i < a.n_outs && t >= a.unit_begin[i] * ga.tiles_m) ? i : g;
  const int tl = t - pick(a.unit_begin, g) * ga.tiles_m;
  const int N = pick(a.n, g);
  const int n0 = (tl / ga.tiles_m) * BN;
  const int m0 = (tl % ga.tiles_m) * BM;
  const int m = m0 + mt * 16 + (lane & 15);
  const int nb = n0 + wave * (BN / 4) + nt * 16 + 4 * (lane >> 4);
  if (m >= M) return;
  const Rows4<NMAT> e = rows4<NMAT>(a, g, N, nb);
  const f32x4* part = reinterpret_cast<const f32x4*>(ga.partials) + static_cast<int64_t>(t) * ga.splits * NMAT * SLOTS;
  f32x4 v[NMAT];
  if constexpr (SPL > 0) {
    f32x4 pv[NMAT][SPL];
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
      for (int sp = 0; sp < SPL; ++sp) pv[mat][sp] = __builtin_nontemporal_load(part + (sp * NMAT + mat) * SLOTS + slot);
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) {
      v[mat] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int sp = 0; sp < SPL; ++sp) v[mat] += pv[mat][sp];
    }
  } else {
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) {
      v[mat] = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int sp = 0; sp < ga.splits; ++sp) v[mat] += part[(static_cast<int64_t>(sp) * NMAT + mat) * SLOTS + slot];
    }
  }
  void* y = (NMAT == 2) ? a.y[0] : pick(a.y, g);
  store_rows4<NMAT, OUT_F32>(a, g, N, m, nb, e, v[0], v[NMAT - 1], y, vec_out<OUT_F32>(y, N));
}

template <int BM, int BN, int NMAT, bool OUT_F32>
int launch_reduce(const GemmArgs& ga, hipStream_t st) {
  const int64_t slots = static_cast<int64_t>(ga.tiles) * BM * BN / 4;
  const dim3 grid(static_cast<unsigned>((slots + kThreads - 1) / kThreads));
  if (ga.splits == 2)
    hipLaunchKernelGGL((gemm_reduce_kernel<BM, BN, NMAT, OUT_F32, 2>), grid, dim3(kThreads), 0, st, ga);
  else if (ga.splits == 4)
    hipLaunchKernelGGL((gemm_reduce_kernel<BM, BN, NMAT, OUT_F32, 4>), grid, dim3(kThreads), 0, st, ga);
  else if (ga.splits == 8)
    hipLaunchKernelGGL((gemm_reduce_kernel<BM, BN, NMAT, OUT_F32, 8>), grid, dim3(kThreads), 0, st, ga);
  else
    hipLaunchKernelGGL((gemm_reduce_kernel<BM, BN, NMAT, OUT_F32, 0>), grid, dim3(kThreads), 0, st, ga);
  return check_launch("w8a16 gemm reduce kernel");
}

template <int BM, int BN, int NMAT, bool OUT_F32, int OCC, int LEAD>
int launch_cfg(const uint16_t* x, const GemmArgs& ga, hipStream_t st) {
  const int64_t grid = static_cast<int64_t>(ga.tiles) * ga.splits;
  note_launch(__PRETTY_FUNCTION__, grid, ga.splits, ga.splits > 1 ? "gemm_reduce_kernel" : nullptr);
  hipLaunchKernelGGL((gemm_kernel<BM, BN, NMAT, OUT_F32, OCC, LEAD>), dim3(static_cast<unsigned>(grid)),
                     dim3(kThreads), 0, st, x, ga);
  int rc = check_launch("w8a16 gemm kernel");
  if (rc || ga.splits == 1) return rc;
  return launch_reduce<BM, BN, NMAT, OUT_F32>(ga, st);
}

template <int BM, int BN, int NMAT, bool OUT_F32, int WLEAD, int XLEAD, int OCC, int KG = 1>
int launch_k64(const uint16_t* x, const GemmArgs& ga, hipStream_t st) {
  const int64_t grid = static_cast<int64_t>(ga.tiles) * ga.splits;
  note_launch(__PRETTY_FUNCTION__, grid, ga.splits, ga.splits > 1 ? "gemm_reduce_kernel" : nullptr);
  hipLaunchKernelGGL((gemm_k64_kernel<BM, BN, NMAT, OUT_F32, WLEAD, XLEAD, OCC, KG>), dim3(static_cast<unsigned>(grid)),
                     dim3(kThreads * KG), 0, st, x, ga);
  int rc = check_launch("w8a16 gemm kernel");
  if (rc || ga.splits == 1) return rc;
  return launch_reduce<BM, BN, NMAT, OUT_F32>(ga, st);
}

template <int BM, int BN, int NMAT, bool OUT_F32, int WLEAD, int S, int OCC>
int launch_dma(const uint16_t* x, const GemmArgs& ga, hipStream_t st) {
  const int64_t grid = static_cast<int64_t>(ga.tiles) * ga.splits;
  note_launch(__PRETTY_FUNCTION__, grid, ga.splits, ga.splits > 1 ? "gemm_reduce_kernel" : nullptr);
  hipLaunchKernelGGL((gemm_dma_kernel<BM, BN, NMAT, OUT_F32, WLEAD, S, OCC>), dim3(static_cast<unsigned>(grid)),
                     dim3(kThreads), 0, st, x, ga);
  int rc = check_launch("w8a16 gemm kernel");
  if (rc || ga.splits == 1) return rc;
  return launch_reduce<BM, BN, NMAT, OUT_F32>(ga, st);
}

// A short K over few tokens in one round trip (single matrices at 33..128
// tokens with K <= 64 NG CPG, e.g. q|k|v and o_proj of a 2048-hidden model).
// The stepped kernels spend ~1 us per 64-k step there waiting on their own
// pipeline (every step's loads, LDS stores and barrier on the critical path
// of few waves) while the work per step is tiny.  Here a workgroup of 16
// waves owns 16 TM tokens x 16 NT weight rows: every wave issues all of its
// loads at once -- a sixteenth of the 16 TM x K activation tile by LDS DMA
// (each lane's 16 bytes placed at their swizzled home, rows past M read as
// zero) and its weight blocks (one 16-row tile, every NG-th 64-k chunk, CPG
// blocks) into registers -- then one wait and one barrier, its MFMAs, and
// the NG K groups summed through LDS in a fixed order.  NT = 4, 2 or 1
// 16-row tiles per workgroup (NG = 16 / NT K groups); TM = 1 or 2 16-token
// tiles.  Once the data is in, the int8 -> bf16 widening (12 VALU per 8
// weights) is what takes the time: with TM = 2 each widened operand feeds
// two MFMAs (o_proj at 128 tokens: 2.5 us of the 16-token tile's 6.6 us
// launch span are its MFMA phase, with every byte already landed).
template <int CPG, int NT, bool OUT_F32, int TM = 1>
__global__ __launch_bounds__(1024) void gemm_once_kernel(const uint16_t* __restrict__ x, GemmArgs ga) {
  constexpr int BM = 16 * TM, BN = 16 * NT, NG = 16 / NT;
  constexpr int CH = NG * CPG;       // chunks (64 k) the activation tile holds
  constexpr int CHUNK = BM * kBK;    // bf16 elements of one chunk block (2 TM KiB)
  constexpr int SLICES = CH * CHUNK * 2 / 1024;  // 1 KiB DMA slices of the tile
  constexpr int SPW = SLICES / 16;               // per wave
  static_assert(SPW * 16 == SLICES && NT * NG == 16 && (TM == 1 || TM == 2), "whole slices per wave; 16 waves");
  static_assert(CH * CHUNK * 2 <= 128 * 1024, "the activation tile fits the LDS");
  __shared__ __attribute__((aligned(16))) uint16_t xs[CH * CHUNK];
  const GroupArgs& a = ga.g;
  const int M = ga.M, K = ga.K;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nt = wave % NT, grp = wave / NT;  // 16-row tile, K group
  const int tiles_n = ga.tiles / ga.tiles_m;
  int vn, mt_all;
  block_order(xcd_remap(blockIdx.x, ga.tiles), tiles_n, ga.tiles_m, vn, mt_all);
  int g = 0;
#pragma unroll
  for (int i = 1; i < PGS_MAX_GROUP; ++i) g = (i < a.n_outs && vn >= a.unit_begin[i]) ? i : g;
  const int N = pick(a.n, g);
  const int n0 = (vn - pick(a.unit_begin, g)) * BN;
  const int m0 = mt_all * BM;
  const int kb = K / kBK;  // <= CH (the planner's bound)

  // activations: 16-byte position p of the tile is chunk p / 128, row
  // (p % 128) / 8, physical piece p % 8, i.e. logical piece (p % 8) ^ f(row)
  const __amdgpu_buffer_rsrc_t xres = make_rsrc(x + static_cast<int64_t>(m0) * K, static_cast<int64_t>(M - m0) * K * 2);
  const int nslices = kb * CHUNK * 2 / 1024;
#pragma unroll
  for (int j = 0; j < SPW; ++j) {
    const int sl = wave * SPW + j;
    if (sl < nslices) {
      const int p = sl * 64 + lane;
      const int c = p / (BM * 8), row = (p >> 3) % BM, pc = p & 7;
      const int lc = pc ^ (row & 7) ^ ((row >> 3) & 1);
      dma16(xres, xs + sl * 512, row * K * 2 + c * 128 + lc * 16, 0);
    }
  }
  // the vmcnt wait below counts on the DMAs being issued before everything
  // else: keep the scheduler from moving later loads above them
  __builtin_amdgcn_sched_barrier(0);
  // epilogue operands
  const int lr = lane & 15, lg = lane >> 4;
  const int nb = n0 + nt * 16 + 4 * lg;
  const Rows4<1> e = rows4<1>(a, g, N, nb);
  // weights, last: this wave's tile, chunks grp, grp + NG, ... (CPG of
  // them; a chunk past K is never used)
  const int blk0 = n0 >> 4, blocks = (N + 15) >> 4;
  const __amdgpu_buffer_rsrc_t wres =
      make_rsrc(pick(a.q, g) + static_cast<int64_t>(blk0) * kb * 1024, static_cast<int64_t>(blocks - blk0) * kb * 1024);
  const int woff = nt * kb * 1024 + lane * 16;
  u32x4 w[CPG];
#pragma unroll
  for (int j = 0; j < CPG; ++j) w[j] = __builtin_amdgcn_raw_buffer_load_b128(wres, woff, (j * NG + grp) * 1024, 0);

  // this wave's DMAs (and everything else but the weight loads, issued
  // last) have landed when at most CPG loads are outstanding; the barrier
  // then makes the whole tile visible, and each weight block is waited for
  // only where its MFMAs use it
  constexpr int kWait = 0xF70 | (CPG & 15) | ((CPG >> 4) << 14);
  __builtin_amdgcn_s_waitcnt(kWait);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  // token tile t's rows sit 16 t rows on, with the same swizzle
  const int bofs0 = swz(lr, 2 * lg), bofs1 = swz(lr, 2 * lg + 1);
  f32x4 acc[TM];
#pragma unroll
  for (int t = 0; t < TM; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int j = 0; j < CPG; ++j) {
    const int c = j * NG + grp;
    if (c < kb) {
      const uint16_t* blk = xs + c * CHUNK;
      const bf16x8 a0 = i8x8_to_bf16x8(w[j][0], w[j][1]), a1 = i8x8_to_bf16x8(w[j][2], w[j][3]);
#pragma unroll
      for (int t = 0; t < TM; ++t) {
        const bf16x8 b0 = *reinterpret_cast<const bf16x8*>(blk + t * 16 * kBK + bofs0);
        const bf16x8 b1 = *reinterpret_cast<const bf16x8*>(blk + t * 16 * kBK + bofs1);
        acc[t] = mfma16x16x32(a0, b0, acc[t]);
        acc[t] = mfma16x16x32(a1, b1, acc[t]);
      }
    }
  }
  __builtin_amdgcn_s_setprio(0);
  // the K groups meet in LDS (the tile's space, free after this barrier)
  __syncthreads();
  f32x4* red = reinterpret_cast<f32x4*>(xs);
#pragma unroll
  for (int t = 0; t < TM; ++t) red[((grp * NT + nt) * TM + t) * 64 + lane] = acc[t];
  __syncthreads();
  if (grp != 0) return;
  void* y = pick(a.y, g);
#pragma unroll
  for (int t = 0; t < TM; ++t) {
    f32x4 v = red[(nt * TM + t) * 64 + lane];
#pragma unroll
    for (int q = 1; q < NG; ++q) v += red[((q * NT + nt) * TM + t) * 64 + lane];
    const int m = m0 + 16 * t + lr;
    if (m < M) store_rows4<1, OUT_F32>(a, g, N, m, nb, e, v, v, y, vec_out<OUT_F32>(y, N));
  }
}

template <int CPG, int NT, bool OUT_F32, int TM = 1>
int launch_once(const uint16_t* x, const GemmArgs& ga, hipStream_t st) {
  if (ga.splits != 1 || ga.K % kBK != 0 || ga.K > 16 / NT * CPG * kBK)
    return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16 gemm: one-shot tile for K=%d", ga.K);
  note_launch(__PRETTY_FUNCTION__, ga.tiles, 1);
  hipLaunchKernelGGL((gemm_once_kernel<CPG, NT, OUT_F32, TM>), dim3(static_cast<unsigned>(ga.tiles)), dim3(1024), 0, st,
                     x, ga);
  return check_launch("w8a16 gemm kernel");
}

// Measured on MI355X (Qwen2.5-3B projections, 512, 1024 and 2048 tokens).
// K % 64 == 0: at least two work units per CU without a K split (q|k|v, o
// and down_proj at 2048 tokens): the LDS-DMA kernel, 4 waves per SIMD
// (o 23.4 vs 24.6 us, q|k|v 29.5 vs 30.5 us at 2048 tokens); at most two
// work units per CU (o / q|k|v / down_proj at 512 and 1024 tokens): the
// buffer-load kernel in two K groups per workgroup, or, for a long K over
// at most one work unit per CU (measured on down_proj at 1024 tokens, which
// now takes the 128 x 128 split plan, as fast there), four.  Other K:
// the pointer kernel (SwiGLU: one-step pipeline at the compiler's register
// budget; single matrices: two-step pipeline at 4 waves per SIMD).
template <int BM, int NMAT, bool OUT_F32>
int launch_bm(const uint16_t* x, const GemmArgs& ga, hipStream_t st) {
  if (ga.K % kBK == 0) {
    if constexpr (NMAT == 2) return launch_k64<BM, kBN, 2, OUT_F32, 2, 2, 2>(x, ga, st);
    const int64_t units = static_cast<int64_t>(ga.tiles) * ga.splits;
    // a long K over at most one workgroup per CU: four K groups
    if (units <= 256 && ga.K / kBK > 64) return launch_k64<BM, kBN, 1, OUT_F32, 2, 2, 1, 4>(x, ga, st);
    if (units >= 512 && ga.splits == 1) return launch_dma<BM, kBN, 1, OUT_F32, 2, 3, 4>(x, ga, st);
    return launch_k64<BM, kBN, 1, OUT_F32, 2, 2, 2, 2>(x, ga, st);
  }
  if constexpr (NMAT == 2)
    return launch_cfg<BM, kBN, 2, OUT_F32, 1, 1>(x, ga, st);
  else
    return launch_cfg<BM, kBN, 1, OUT_F32, 4, 2>(x, ga, st);
}

template <int NMAT, bool OUT_F32>
int launch_plan(const uint16_t* x, const GemmArgs& ga, const GemmPlan& plan, hipStream_t st) {
  if constexpr (NMAT == 1) {
    // one-shot 16- or 32-token tiles (K <= 2048): 64, 32 or 16 rows in 4, 8
    // or 16 K groups
    if (plan.once) {
      if (plan.bm == 32) {
        if (plan.bn == 64) return launch_once<8, 4, OUT_F32, 2>(x, ga, st);
        if (plan.bn == 32) return launch_once<4, 2, OUT_F32, 2>(x, ga, st);
        return launch_once<2, 1, OUT_F32, 2>(x, ga, st);
      }
      if (plan.bn == 64) return launch_once<8, 4, OUT_F32>(x, ga, st);
      if (plan.bn == 32) return launch_once<4, 2, OUT_F32>(x, ga, st);
      return launch_once<2, 1, OUT_F32>(x, ga, st);
    }
  }
  if (ga.K % kBK == 0 && plan.bn == 64) {
    if constexpr (NMAT == 2) {
      // the SwiGLU pair in 128-token tiles (the planner's choice above 96
      // tokens): 128 tokens x 64 rows per matrix (each widened weight operand
      // feeds 8 MFMAs; B operands are reused across the pair's two A tiles
      // per wave)
      // (LDS-DMA activations, three stages, 3 waves per SIMD: 46.3 vs 47.8 us
      // at 512 tokens, 159 vs 169 us at 2048 over the register-staged kernel)
      if (plan.bm == 128) return launch_dma<128, 64, 2, OUT_F32, 2, 3, 3>(x, ga, st);
      // 64-token tiles above 64 tokens: LDS-DMA activations, four stages (80
      // / 96 tokens: 20.5 / 21.0 vs 22.9 / 23.9 us for the two-K-group kernel);
      // at 64 tokens and below the two-K-group kernel is as fast
      if (ga.M > 64) return launch_dma<64, 64, 2, OUT_F32, 3, 4, 3>(x, ga, st);
      return launch_k64<64, 64, 2, OUT_F32, 2, 2, 1, 2>(x, ga, st);
    } else {
      // single matrices above 128 tokens (short K, few tiles): 32 x 64 tiles
      // in two K groups
      if (ga.M > 128) return launch_k64<32, 64, 1, OUT_F32, 2, 2, 2, 2>(x, ga, st);
      // single matrices at 33..128 tokens: 64-row tiles in four K groups
      return plan.bm == 32 ? launch_k64<32, 64, 1, OUT_F32, 2, 2, 1, 4>(x, ga, st)
                           : launch_k64<64, 64, 1, OUT_F32, 2, 2, 1, 4>(x, ga, st);
    }
  }
  if constexpr (NMAT == 1) {
    // (lm_head at 256 tokens: 155-161 vs 174-184 us with register-staged activations)
    if (plan.bm == 128 && plan.bn == kBN && ga.K % kBK == 0) return launch_dma<128, kBN, 1, OUT_F32, 2, 3, 2>(x, ga, st);
  }
  if (plan.bm == 128) return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16 gemm: no 128-token tile kernel for this shape");
  return plan.bm == 32 ? launch_bm<32, NMAT, OUT_F32>(x, ga, st) : launch_bm<64, NMAT, OUT_F32>(x, ga, st);
}

}  // namespace

GemmPlan plan_gemm(int m, int k, int nmat, const int32_t* n, int members, bool can_split) {
  GemmPlan p{};
  const int kb = (k + kBK - 1) / kBK;
  // 33..128 tokens (K % 64 == 0): weight streaming dominates, so 64-row
  // tiles and K groups keep more workgroups and more weight bytes in flight
  const bool mid = k % kBK == 0 && m <= 128;
  p.bn = (mid || (nmat == 2 && k % kBK == 0)) ? 64 : kBN;
  p.kg = 1;
  int tiles_n = 0;
  for (int i = 0; i < members; ++i) tiles_n += (n[i] + p.bn - 1) / p.bn;
  auto tiles_for = [&](int bm) { return static_cast<int64_t>((m + bm - 1) / bm) * tiles_n; };
  // a single matrix with a short K above 128 tokens whose 32 x 128 tiles
  // would number at most 384 (o at 129..768 tokens, q|k|v at 129..608):
  // 32 x 64 tiles in two K groups, twice the workgroups and an even spread
  // over the CUs (o at 160 / 256 / 512 / 768 tokens 9.2 / 9.3 / 11.8 / 15.2
  // vs 13.8 / 11.9 / 12.5 / 17.1 us, q|k|v at 160 / 256 / 512 9.7 / 11.9 /
  // 15.1 vs 15.2 / 12.6 / 17.3; no faster for q|k|v at 768, 480 tiles, and
  // slower at 1024 tokens, 512+ tiles: o 19.0 vs 17.2)
  const bool narrow = !mid && nmat == 1 && k % kBK == 0 && kb <= 64 && tiles_for(32) <= 384;
  if (narrow) {
    p.bn = 64;
    tiles_n = 0;
    for (int i = 0; i < members; ++i) tiles_n += (n[i] + p.bn - 1) / p.bn;
  }
  if (mid) {
    // a single matrix with K <= 2048: one-shot tiles of 16 or 32 tokens and
    // 16, 32 or 64 rows, the fewest rows whose count fills the 256 CUs at
    // most once (o_proj at 64 tokens 6.1 vs 9.3 us, q|k|v at 96 tokens 7.8 vs
    // 9.2 us); more tiles than that run past one round and lose to the
    // stepped kernel (q|k|v at 128 tokens 11.0 vs 9.2 us).  Of the two token
    // heights the one with more tiles, and at equal counts 32 tokens (each
    // widened weight feeds two MFMAs: o_proj at 96 / 128 tokens 7.0 / 7.1 vs
    // 7.4 / 7.7 us); 16 tokens up to 64 (6.0 vs 6.9 us for o_proj at 64,
    // where 32 would halve the tiles)
    if (nmat == 1 && kb <= 32) {
      int best_bm = 0, best_nt = 0, best_tn = 0;
      int64_t best_tiles = 0;
      for (int bm = 16; bm <= 32; bm *= 2) {
        if (bm == 32 && m <= 64) continue;
        for (int nt = 1; nt <= 4; nt *= 2) {
          int tn = 0;
          for (int i = 0; i < members; ++i) tn += (n[i] + 16 * nt - 1) / (16 * nt);
          const int64_t tiles = static_cast<int64_t>((m + bm - 1) / bm) * tn;
          if (tiles <= 256) {
            if (tiles > best_tiles || (tiles == best_tiles && bm == 32)) {
              best_bm = bm;
              best_nt = nt;
              best_tn = tn;
              best_tiles = tiles;
            }
            break;
          }
        }
      }
      if (best_tiles > 0) {
        p.once = true;
        p.bm = best_bm;
        p.bn = 16 * best_nt;
        p.kg = 16 / best_nt;
        p.tiles_m = (m + best_bm - 1) / best_bm;
        p.tiles_n = best_tn;
        p.tiles = static_cast<int>(best_tiles);
        p.splits = 1;
        return p;
      }
    }
    p.bm = (nmat == 1 && kb <= 64) ? 32 : 64;
    // the SwiGLU pair above 96 tokens: one 128-token tile row, each weight
    // panel read once (128 tokens 21.9 vs 23.5 us; at 96 tokens within noise)
    if (nmat == 2 && m > 96) p.bm = 128;
    p.kg = nmat == 2 ? 2 : 4;
    p.tiles_m = (m + p.bm - 1) / p.bm;
    p.tiles_n = tiles_n;
    p.tiles = p.tiles_m * p.tiles_n;
    p.splits = 1;
    // long K (down_proj): split K up to 8 ways until one workgroup per CU,
    // keeping >= 4 K steps per K group (down_proj at 40 / 64 tokens, 32
    // tiles: 16.1 / 17.3 us with 8 splits against 17.3 / 18.75 with 4)
    if (can_split && nmat == 1 && kb > 64) {
      while (p.splits < 8 && static_cast<int64_t>(p.tiles) * p.splits < 256 && kb / (p.splits * 2) >= 4 * p.kg)
        p.splits *= 2;
    }
    return p;
  }
  p.bm = narrow ? 32 : p.bn == 64 ? 128 : m <= 32 ? 32 : 64;
  // the SwiGLU pair keeps 64-token tiles when its last 128-token tile would be
  // at most half full (160 tokens 27.6 vs 31.6 us, 192: 28.7 vs 30.9, 320:
  // 37.2 vs 41.7, 448: 46.8 vs 47.5; at 384 the 128-token tiles win, 42.7 vs 44.2)
  if (nmat == 2 && p.bn == 64 && m % 128 != 0 && m % 128 <= 64) p.bm = 64;
  // a single matrix with very many 128-token tiles (lm_head at 256 tokens):
  // 128 x 128 tiles read each weight panel half as often (lm_head [151936,
  // 2048] at 256 tokens 165-176 vs 173-184 us; at 320..1376 tiles they are
  // no faster or slower: q|k|v at 2048 tokens 32.5 vs 29.3 us)
  if (nmat == 1 && k % kBK == 0 && p.bn == kBN && m >= 256 && tiles_for(128) >= 2048) p.bm = 128;
  // a long K (down_proj) above 256 tokens: 128 x 128 tiles, split K (up to
  // 8 ways) until 512 workgroups (down_proj [2048, 11008] at 384 tokens
  // 33.6-34.1 vs 35.6-36.9 us with eight splits, at 768 52.4-54.1 vs
  // 57.3-58.8, at 1280 69.8 vs 79.3 and at 1536 78.7 vs 87-90 with four, at
  // 2048 94.5 vs 99-104 with two; at 512 and 1024 tokens within noise of the
  // plans below, at 256 no faster)
  // (without a workspace only where the split would stop at one anyway, 512
  // tiles and more, so that a call plans alike with or without one)
  const bool long128 = nmat == 1 && k % kBK == 0 && p.bn == kBN && kb > 64 && m > 256 &&
                       (can_split || tiles_for(128) >= 512);
  if (long128) p.bm = 128;
  // a single matrix with a short K and few 64-token tiles: 32-token tiles
  // give the CUs work without splitting K
  if (nmat == 1 && p.bm == 64 && kb <= 64 && tiles_for(64) < 256) p.bm = 32;
  p.tiles_m = (m + p.bm - 1) / p.bm;
  p.tiles_n = tiles_n;
  p.tiles = p.tiles_m * p.tiles_n;
  p.splits = 1;
  if (long128) {
    while (p.splits < 8 && static_cast<int64_t>(p.tiles) * p.splits < 512) p.splits *= 2;
    return p;
  }
  // fewer than 256 output tiles: split K until about four workgroups per CU,
  // keeping >= 32 K steps per split (>= 8 when there are very few tiles).
  // From 256 tiles on, K groups inside the workgroup beat a split and its
  // reduce launch (down_proj at 1024 tokens 54 vs 58.5-64 us, at 2048: 99
  // vs 105-110; above 256 tokens down_proj now takes the 128 x 128 plan).
  if (can_split && p.tiles < 256) {
    const int min_steps = p.tiles < 128 ? 8 : 32;
    while (p.splits < 8 && static_cast<int64_t>(p.tiles) * p.splits < 1024 && kb / (p.splits * 2) >= min_steps)
      p.splits *= 2;
  }
  return p;
}

size_t gemm_partial_bytes(const GemmPlan& p, int nmat) {
  if (p.splits <= 1) return 0;
  return static_cast<size_t>(p.tiles) * p.splits * nmat * p.bm * p.bn * sizeof(float);
}

int launch_gemm(Problem& p, const GemmPlan& plan, hipStream_t st) {
  if (plan.splits > 1 && (!p.partials || p.partial_bytes < gemm_partial_bytes(plan, p.nmat)))
    return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16 gemm: split-K plan without a large enough workspace");
  // member boundaries in units of n-tiles
  GemmArgs ga{};
  ga.g = p.args;
  int units = 0;
  const int members = (p.nmat == 2) ? 1 : p.args.n_outs;
  for (int i = 0; i < members; ++i) {
    ga.g.unit_begin[i] = units;
    units += (p.args.n[i] + plan.bn - 1) / plan.bn;
  }
  for (int i = members; i <= PGS_MAX_GROUP; ++i) ga.g.unit_begin[i] = units;
  ga.M = p.m;
  ga.K = p.k;
  ga.tiles_m = plan.tiles_m;
  ga.tiles = plan.tiles;
  ga.splits = plan.splits;
  ga.partials = p.partials;
  if (p.nmat == 2) return launch_plan<2, false>(p.x, ga, plan, st);
  return p.out_f32 ? launch_plan<1, true>(p.x, ga, plan, st) : launch_plan<1, false>(p.x, ga, plan, st);
}

}  // namespace pgs
