// Skinny W8A16 kernel for decode-sized inputs (m <= 32 tokens).
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
// batch; for the K ranges of the usual shapes a wave issues all of its
// batches at once, so a short launch costs one memory round trip rather than
// one per batch.  The waves' partial 16x16 tiles are summed through LDS in a
// fixed order.  Short-N shapes (o_proj, down_proj: 128 tiles) would leave
// half of the 256 CUs idle, so their K range may be split over two
// workgroups that meet in a pair slot (below); the SwiGLU pair splits
// through workspace partials and a second small kernel instead.  At up to 8
// tokens a short-N matrix is "folded" instead: two workgroups per tile, each
// owning 8 of its rows over the whole K range, with two 64-k chunks per MFMA
// (A rows 0-7: its rows in chunk c, A rows 8-15: the same rows in chunk c+1;
// B columns 0..m-1: the tokens in chunk c, m..2m-1: the tokens in chunk c+1),
// so that output (token t, row r) is C[r][t] + C[r+8][t+m].  Each lane's
// 16 bytes are still one contiguous piece of the packed block, the
// instruction stream equals that of a K split, and nothing crosses
// workgroups.  17..32 tokens use two 16-token column blocks (TM = 2): each
// widened weight fragment feeds one MFMA per block, and every wave still
// issues its loads at once with no barrier inside its K range (a tiled GEMM
// with activations shared through LDS synchronises its waves at every K
// step).  Results never depend on timing: every sum has a fixed order.
#include "pgs_linear.h"

namespace pgs {
namespace {

// output (token mm, row i of a 16-row tile) lives in accumulator lane
// (i/4)*16 + mm, register i%4
__device__ __forceinline__ int acc_lane(int i, int mm) { return (i >> 2) * 16 + mm; }

// Operands of one output's epilogue (scales, bias, residual), loaded before
// the weight stream so that their memory round trip overlaps it instead of
// following it.  The loads are unconditional (an absent bias or residual
// reads a valid dummy address instead and is ignored), so no branch makes
// the kernel wait for them before the weight loads are issued; the bf16
// values stay raw until the epilogue.
template <int NMAT>
struct EpiIn {
  float s[NMAT];
  uint16_t bias, res;
};

template <int NMAT>
__device__ __forceinline__ EpiIn<NMAT> epilogue_load(const GroupArgs& a, int g, int n, int mm, int N,
                                                     const uint16_t* dummy) {
  EpiIn<NMAT> e;
  if constexpr (NMAT == 2) {
    e.s[0] = a.scale[0][n];
    e.s[1] = a.scale[1][n];
    e.bias = e.res = 0;
  } else {
    const float* sc = pick_early(a.scale, g);
    const uint16_t* bias = pick_early(a.bias, g);
    const uint16_t* res = pick_early(a.res, g);
    e.s[0] = sc[n];
    e.bias = *(bias ? bias + n : dummy);
    e.res = *(res ? res + static_cast<int64_t>(mm) * N + n : dummy);
  }
  return e;
}

template <int NMAT, bool OUT_F32>
__device__ __forceinline__ void epilogue(const GroupArgs& a, int g, int n, int mm, int N, const float (&v)[NMAT],
                                         const EpiIn<NMAT>& e) {
  void* y = (NMAT == 2) ? a.y[0] : pick_early(a.y, g);
  float out;
  if constexpr (NMAT == 2) {
    out = silu_f32(v[0] * e.s[0]) * (v[1] * e.s[1]);
  } else {
    out = v[0] * e.s[0];
    if (pick_early(a.bias, g)) out += bf16_bits_to_f32(e.bias);
    if (pick_early(a.res, g)) {
      // the reference's roundings (engine/model.py:184, 190): the linear
      // output is rounded to the output type first, then added
      const float l = OUT_F32 ? out : bf16_bits_to_f32(f32_to_bf16_bits(out));
      out = l + bf16_bits_to_f32(e.res);
    }
  }
  store_out<OUT_F32>(y, static_cast<int64_t>(mm) * N + n, out);
}

// Waves per SIMD the compiler must leave room for: the SwiGLU pair at
// 8 waves x 2 batches holds 64 registers of loads per lane, and three of its
// workgroups per CU (all 688 of a 2048 x 11008 pair resident at once) need
// <= 80 registers.
constexpr int skinny_occ(int nw, int nb, int nmat, int tm) {
  return (tm == 1 && nmat == 2 && nw == 8 && nb == 2) ? 6 : 1;
}

// LDS of a kernel with xm staged tokens (slots of s chunks; 8 or 16 tokens
// are staged one batch at a time; the fused norm adds its per-wave partial sums);
// at most 160 KiB per workgroup on gfx950.
constexpr int kLdsLimit = 160 * 1024;
constexpr int skinny_lds_bytes(int nw, int u, int nb, int nmat, int s, int xm, bool norm) {
  return (xm > 0 ? nw * (xm >= 8 ? 1 : nb) * u * s * xm * 9 * 16 : 0) + nw * nmat * 64 * 16 + (norm ? nw * xm * 4 : 0);
}

// Template parameters:
//   NW, U, NB  waves per workgroup, 64-k slots per batch, batches per wave
//              issued at once (NB = 0: a loop over pairs of batches)
//   NMAT       1 single matrix (q|k|v group members, o, down, lm_head);
//              2 the SwiGLU pair (gate and up rows of the same index)
//   OUT_F32    fp32 output (lm_head logits) instead of bf16
//   K64        K % 64 == 0 (no masked K tail)
//   FOLD       two workgroups per tile (splits == 1, M <= 8), workgroup 2t + h
//              owns rows 8h .. 8h+7 of tile t
//   XM         > 0: up to XM tokens (M <= XM, NB > 0, K % 64 == 0), their
//              activations staged through LDS (below)
//   NORM       the activations are the rows of x after rms_norm with weight nw
//              and eps (engine/model.py:29-34), computed on the staged pieces
//              (splits == 1: the workgroup holds whole rows)
//   TM         16-token column blocks (M <= 16 TM; 2: unfolded, direct loads)
// The launcher picks one combination per call (launch_kernel); the static
// asserts below list the combinations that exist.
template <int NW, int U, int NB, int NMAT, bool OUT_F32, bool K64, bool FOLD, int XM, bool NORM, int TM = 1>
__global__ __launch_bounds__(64 * NW, skinny_occ(NW, NB, NMAT, TM)) void skinny_kernel(const uint16_t* __restrict__ x, GroupArgs a, int M,
                                                         int K, int splits, float* __restrict__ partials,
                                                         unsigned long long* __restrict__ pairs,
                                                         const uint16_t* __restrict__ nw, float eps,
                                                         unsigned long long* __restrict__ keys) {
  static_assert(!FOLD || NMAT == 1, "folding serves single matrices");
  static_assert(XM == 0 || (NB > 0 && K64 && (8 % XM == 0 || (XM == 16 && !NORM && !FOLD))),
                "activation staging covers issue-once shapes");
  static_assert(!NORM || (XM > 0 && !OUT_F32), "the fused norm works on staged activations");
  static_assert(TM == 1 || (TM == 2 && !FOLD && XM == 0), "two token blocks: unfolded, direct activation loads");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar loop control
  // (folded: the two halves of a tile run back to back on one XCD)
  const int unit = FOLD ? xcd_remap(blockIdx.x, gridDim.x) : blockIdx.x / splits;
  const int tile = FOLD ? unit >> 1 : unit;
  const int half = FOLD ? unit & 1 : 0;
  const int s = FOLD ? 0 : blockIdx.x - unit * splits;  // K split

  const int g = (NMAT == 2) ? 0 : member_of(a, tile);
  const int N = pick_early(a.n, g);
  const int row0 = (tile - pick_early(a.unit_begin, g)) * 16;
  const int lrow = lane & 15;
  const int kgrp = lane >> 4;

  // one output per thread (M * 16 <= 256 TM <= 64 * NW): token mm, tile row oi
  static_assert(NW >= 4 && 64 * NW >= 256 * TM, "the epilogue gives each thread at most one output");
  const int idx = threadIdx.x;
  const int mm = FOLD ? idx >> 3 : idx >> 4;
  const int oi = FOLD ? 8 * half + (idx & 7) : idx & 15;
  const int nout = M * (FOLD ? 8 : 16);
  const bool has_out = idx < nout && row0 + oi < N;

  // (splits <= 2 and nchunks <= 2^16: 32-bit arithmetic)
  const int nchunks = (K + 63) >> 6;
  const int cb = s * nchunks / splits;
  const int ce = (s + 1) * nchunks / splits;
  // The range is walked in slots of S chunks (S = 2 folded: chunks
  // cb + S*j .. cb + S*j + S-1 for slot j).
  constexpr int S = FOLD ? 2 : 1;
  const int nslots = (ce - cb + S - 1) / S;
  // Packed weights: block (tile, chunk) is 1 KiB, the 16 bytes of tile row
  // i, k group g at (i + 16 g) * 16.  One buffer resource per matrix spans
  // exactly this workgroup's chunks [cb, ce) of its 16-row block row, so a
  // chunk past the range reads zeros without touching memory.
  __amdgpu_buffer_rsrc_t wres[NMAT];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) {
    const int8_t* qg = (NMAT == 2) ? a.q[mat] : pick_early(a.q, g);
    wres[mat] = make_rsrc(qg + (static_cast<int64_t>(row0 >> 4) * nchunks + cb) * 1024,
                          static_cast<int64_t>(ce - cb) * 1024);
  }
  // A operand row lrow: tile row lrow, or (folded) row 8 half + lrow % 8 of
  // the slot's chunk lrow / 8
  const int woff = FOLD ? (lrow >> 3) * 1024 + (8 * half + (lrow & 7) + 16 * kgrp) * 16 : lane * 16;
  // B operand column lrow: token min(lrow, M - 1), or (folded) token lrow % M
  // of the slot's chunk lrow / M (columns >= 2M repeat column 0, unused); this
  // lane's 16 k of the chunk
  const int xsub = (FOLD && lrow >= M && lrow < 2 * M) ? 1 : 0;
  const int xrow = FOLD ? (lrow < M ? lrow : (xsub ? lrow - M : 0)) : min(lrow, M - 1);
  const __amdgpu_buffer_rsrc_t xres = make_rsrc(x, static_cast<int64_t>(M) * K * 2);
  const int xoff = xrow * K * 2 + xsub * 128 + kgrp * 32;
  // (TM = 2) B operand column lrow of the second block: token min(16 + lrow, M - 1)
  const int xoff2 = min(16 + lrow, M - 1) * K * 2 + kgrp * 32;

  f32x4 acc[NMAT], acc2[NMAT];  // acc2: second token block (TM = 2)
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) acc[mat] = acc2[mat] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto mac = [&](const u32x4 (&wv)[NMAT], u32x4 x0, u32x4 x1) {
    const bf16x8 b0 = __builtin_bit_cast(bf16x8, x0);
    const bf16x8 b1 = __builtin_bit_cast(bf16x8, x1);
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) {
      acc[mat] = mfma16x16x32(i8x8_to_bf16x8(wv[mat][0], wv[mat][1]), b0, acc[mat]);
      acc[mat] = mfma16x16x32(i8x8_to_bf16x8(wv[mat][2], wv[mat][3]), b1, acc[mat]);
    }
  };
  // both token blocks: each weight fragment widened once, used twice
  auto mac2 = [&](const u32x4 (&wv)[NMAT], u32x4 x0, u32x4 x1, u32x4 y0, u32x4 y1) {
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) {
      const bf16x8 w0 = i8x8_to_bf16x8(wv[mat][0], wv[mat][1]);
      const bf16x8 w1 = i8x8_to_bf16x8(wv[mat][2], wv[mat][3]);
      acc[mat] = mfma16x16x32(w0, __builtin_bit_cast(bf16x8, x0), acc[mat]);
      acc[mat] = mfma16x16x32(w1, __builtin_bit_cast(bf16x8, x1), acc[mat]);
      acc2[mat] = mfma16x16x32(w0, __builtin_bit_cast(bf16x8, y0), acc2[mat]);
      acc2[mat] = mfma16x16x32(w1, __builtin_bit_cast(bf16x8, y1), acc2[mat]);
    }
  };

  // Batches of U slots: batch j of this wave covers slots c(j) .. c(j)+U-1,
  // c(j) = (j * NW + wave) * U.  Every load is issued and every MFMA
  // run unconditionally, in a fixed order (a chunk at or past ce reads zero
  // weights, and its activations are masked to zero as well, so that
  // non-finite inputs of other K ranges cannot leak in); with no branch the
  // compiler can neither sink a load towards its use nor lose count: its
  // wait before each batch's MFMAs counts exactly the loads issued after it,
  // and nothing waits for more than its own data.  The loads carry no address
  // arithmetic: K advances in the scalar offset.  NB > 0: the wave's NB
  // batches are all issued up front (one memory round trip for the whole
  // workgroup); NB = 0 (long K): groups of two batches in a loop.
  struct Batch {
    u32x4 w[U][NMAT];
    u32x4 x[U][2 * TM];
  };
  auto load_w = [&](Batch& b, int c) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat)
        b.w[u][mat] = __builtin_amdgcn_raw_buffer_load_b128(wres[mat], woff, (c + u) * S * 1024, kLoadNT);
  };
  auto load_batch = [&](Batch& b, int c) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c0 = (c + u) * S;  // first chunk of the slot, from cb
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat)
        b.w[u][mat] = __builtin_amdgcn_raw_buffer_load_b128(wres[mat], woff, c0 * 1024, kLoadNT);
      // (chunks past the range, and K % 64 != 0 columns past K, read the
      // next row or zeros; mac_batch masks them)
      b.x[u][0] = __builtin_amdgcn_raw_buffer_load_b128(xres, xoff, (cb + c0) * 128, 0);
      b.x[u][1] = __builtin_amdgcn_raw_buffer_load_b128(xres, xoff + 16, (cb + c0) * 128, 0);
      if constexpr (TM == 2) {
        b.x[u][2] = __builtin_amdgcn_raw_buffer_load_b128(xres, xoff2, (cb + c0) * 128, 0);
        b.x[u][3] = __builtin_amdgcn_raw_buffer_load_b128(xres, xoff2 + 16, (cb + c0) * 128, 0);
      }
    }
  };

  // XM > 0: the tokens' activations for this wave's NB * U slots (S chunk
  // rows of 128 bytes per token) are fetched once, as XP 16-byte pieces
  // (piece p by lane p % 64 in pass p / 64), parked in the wave's own slice
  // of LDS and read back as B operands.  That replaces two vector loads per
  // chunk, each returning 1 KiB to the registers although the M real columns
  // use M * 64 bytes of it (M = 1: all 16 lanes of a k group read one
  // address, an LDS broadcast), by XPASS loads per wave.  Only this wave
  // touches its slice.  Slice layout: row (slot chunk, token) of 8 pieces,
  // rows 9 pieces apart, so that the B reads of up to eight rows (XM tokens
  // x 2 chunks) fall on distinct banks (and those of 16 tokens: row r starts
  // at 144 r bytes, distinct 16-byte bank groups mod 256).  XM = 8 and 16
  // park one batch at a time into a slice of one batch (PHASED): all of a
  // wave's batches would need 4.5 / 9 KiB per wave, LDS that the resident
  // workgroups the weight stream needs do not have (lm_head [151936, 2048]
  // at 5 / 8 tokens 51.9-54.2 / 56.9-57.9 us phased, 54.9-55.6 / 58.5-59.5
  // with every batch parked at once).
  constexpr bool PHASED = XM >= 8;
  constexpr int XP = XM > 0 ? NB * U * S * XM * 8 : 1;
  constexpr int XPASS = (XP + 63) / 64;
  constexpr int XROWS = XM > 0 ? (PHASED ? U * S * XM : NB * U * S * XM) : 1;
  constexpr int PPB = PHASED ? U * S * XM * 8 / 64 : 1;  // passes per batch
  static_assert(!PHASED || PPB * 64 == U * S * XM * 8, "whole passes per batch");
  __shared__ u32x4 xst[XM > 0 ? NW * XROWS * 9 : 1];
  u32x4* const xw = xst + (XM > 0 ? wave * XROWS * 9 : 0);

  auto mac_batch = [&](const Batch& b, int c, int j) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int ch = cb + (c + u) * S + xsub;  // this lane's activation chunk
      const bool on = ch < ce && (K64 || ch * 64 + kgrp * 16 < K);
      const uint32_t mask = on ? 0xffffffffu : 0u;
      if constexpr (XM > 0) {
        const u32x4* src = xw + ((((PHASED ? 0 : j) * U + u) * S + xsub) * XM + xrow) * 9 + kgrp * 2;
        mac(b.w[u], src[0] & mask, src[1] & mask);
      } else if constexpr (TM == 2) {
        mac2(b.w[u], b.x[u][0] & mask, b.x[u][1] & mask, b.x[u][2] & mask, b.x[u][3] & mask);
      } else {
        mac(b.w[u], b.x[u][0] & mask, b.x[u][1] & mask);
      }
    }
  };
  constexpr int kStep = NW * U;
  const int first = wave * U;
  // epilogue operands (clamped to a valid output, so the loads need no branch)
  auto load_epi = [&] { return epilogue_load<NMAT>(a, g, min(row0 + oi, N - 1), min(mm, M - 1), N, x); };
  EpiIn<NMAT> epi;
  if constexpr (NB > 0) {
    Batch bt[NB];
    u32x4 xpiece[XM > 0 ? XPASS : 1];
    u32x4 wpiece[NORM ? XPASS : 1];  // NORM: the norm weights of the same columns
    if constexpr (XM > 0) {
      // the pieces first, so that parking them waits for them alone
      const __amdgpu_buffer_rsrc_t nres = make_rsrc(NORM ? nw : x, NORM ? static_cast<int64_t>(K) * 2 : 0);
#pragma unroll
      for (int i = 0; i < XPASS; ++i) {
        const int p = lane + 64 * i;
        // piece p: 16-byte piece p % 8 of token (p / 8) % XM in chunk row
        // p / (8 XM) (slot of the wave, then chunk of the slot)
        const int t = (p >> 3) % XM, cr = p / (8 * XM);
        const int sw = cr / S;
        const int ch = cb + (first + (sw / U) * kStep + sw % U) * S + cr % S;
        // (pieces past XP, chunks past the range and tokens past M read
        // zeros: an offset past the buffer; a chunk past K of token t would
        // otherwise be the start of token t + 1, which the sum of squares
        // must not see)
        const bool in = p < XP && ch < ce;
        const int off = in ? t * K * 2 + ch * 128 + (p & 7) * 16 : 0x7ffffff0;
        xpiece[i] = __builtin_amdgcn_raw_buffer_load_b128(xres, off, 0, 0);
        if constexpr (NORM)
          wpiece[i] = __builtin_amdgcn_raw_buffer_load_b128(nres, in ? ch * 128 + (p & 7) * 16 : 0x7ffffff0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < NB; ++j) load_w(bt[j], first + j * kStep);
    } else {
#pragma unroll
      for (int j = 0; j < NB; ++j) load_batch(bt[j], first + j * kStep);
    }
    epi = load_epi();  // behind the weight loads
    __builtin_amdgcn_sched_barrier(0);  // every load issued before the first wait
    if constexpr (NORM) {
      // rms_norm on the staged pieces.  All pieces of a lane belong to token
      // (lane / 8) % XM (XM divides 8).  Sum of squares in a fixed order:
      // each lane over its pieces, the lanes of a token by a butterfly, the
      // waves in order through LDS; then r = 1 / sqrt(mean + eps) and
      // h = bf16(w * bf16(x * r)), the reference's roundings.
      const int tl = (lane >> 3) % XM;
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < XPASS; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = bf16_bits_to_f32(static_cast<uint16_t>(xpiece[i][e]));
          const float hi = bf16_bits_to_f32(static_cast<uint16_t>(xpiece[i][e] >> 16));
          ss += lo * lo;
          ss += hi * hi;
        }
#pragma unroll
      for (int off = 1; off < 64; off <<= 1)
        if ((off >> 3) % XM == 0 || off < 8) ss += __shfl_xor(ss, off);  // lanes of the same token
      __shared__ float npart[NW][XM];
      if ((lane & ~(8 * XM - 1) & ~7) == 0 && (lane & 7) == 0) npart[wave][tl] = ss;
      __syncthreads();
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) tot += npart[w][tl];
      const float r = 1.0f / sqrtf(tot / static_cast<float>(K) + eps);
#pragma unroll
      for (int i = 0; i < XPASS; ++i) {
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x0 = bf16_bits_to_f32(static_cast<uint16_t>(xpiece[i][e]));
          const float x1 = bf16_bits_to_f32(static_cast<uint16_t>(xpiece[i][e] >> 16));
          const float g0 = bf16_bits_to_f32(static_cast<uint16_t>(wpiece[i][e]));
          const float g1 = bf16_bits_to_f32(static_cast<uint16_t>(wpiece[i][e] >> 16));
          o[e] = pack_bf16x2(g0 * bf16_bits_to_f32(f32_to_bf16_bits(x0 * r)),
                             g1 * bf16_bits_to_f32(f32_to_bf16_bits(x1 * r)));
        }
        xpiece[i] = tl < M ? o : u32x4{0u, 0u, 0u, 0u};  // (tokens past M: never read)
      }
    }
    if constexpr (XM > 0 && !PHASED) {
#pragma unroll
      for (int i = 0; i < XPASS; ++i) {
        const int p = lane + 64 * i;
        if (p < XP) xw[(p >> 3) * 9 + (p & 7)] = xpiece[i];
      }
      // the same wave reads the slice back: its LDS operations complete in
      // order; keep the compiler from moving the reads above the stores
      __builtin_amdgcn_wave_barrier();
      asm volatile("" ::: "memory");
    }
    // (raised wave priority: a wave whose data has arrived issues its MFMAs
    // ahead of the other workgroups' waves; down_proj at one token 6.31 ->
    // 6.28 us, q|k|v 3.36 -> 3.34)
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      if constexpr (PHASED) {
        // batch j's passes into the slice (the previous batch's reads of it
        // were issued before these stores: one wave's LDS operations run in
        // order), then its MFMAs
#pragma unroll
        for (int i = j * PPB; i < (j + 1) * PPB; ++i) {
          const int p = lane + 64 * i - j * PPB * 64;
          xw[(p >> 3) * 9 + (p & 7)] = xpiece[i];
        }
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
      }
      mac_batch(bt[j], first + j * kStep, j);
      if constexpr (PHASED) asm volatile("" ::: "memory");
    }
    __builtin_amdgcn_s_setprio(0);
  } else {
    epi = load_epi();
    for (int c = first; c < nslots; c += 2 * kStep) {
      Batch b0, b1;
      load_batch(b0, c);
      load_batch(b1, c + kStep);
      mac_batch(b0, c, 0);
      mac_batch(b1, c + kStep, 0);
    }
  }

  __shared__ f32x4 red[NW][NMAT * TM][64];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) {
    red[wave][mat * TM][lane] = acc[mat];
    if constexpr (TM == 2) red[wave][mat * TM + 1][lane] = acc2[mat];
  }
  __syncthreads();

  const bool live = idx < nout;
  // token mm is column mm % 16 of block mm / 16
  const int ln = acc_lane(FOLD ? oi & 7 : oi, mm & 15), r = oi & 3, tb = TM == 2 ? mm >> 4 : 0;
  float v[NMAT];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) {
    float t = 0.f;
    if (live) {
#pragma unroll
      for (int w = 0; w < NW; ++w) t += red[w][mat * TM + tb][ln][r];
      if constexpr (FOLD) {
        // the second chunk of every slot: C[r + 8][mm + M]
        const int ln2 = acc_lane((oi & 7) + 8, mm + M);
        float t2 = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) t2 += red[w][mat * TM][ln2][r];
        t += t2;
      }
    }
    v[mat] = t;
  }
  if constexpr (NMAT == 1 && OUT_F32) {
    if (keys) {
      // Row-argmax mode: the fp32 output the epilogue would store (scale,
      // bias), its key, the maximum over the token's outputs in this
      // workgroup (consecutive threads: 8 folded, 16 otherwise, within one
      // wave), one key per token and workgroup.
      unsigned long long key = 0;
      if (live && has_out) {
        float out = v[0] * epi.s[0];
        if (pick_early(a.bias, g)) out += bf16_bits_to_f32(epi.bias);
        key = argmax_key(out, static_cast<uint32_t>(row0 + oi));
      }
      constexpr int G = FOLD ? 8 : 16;
#pragma unroll
      for (int off = 1; off < G; off <<= 1) {
        const uint32_t lo = __shfl_xor(static_cast<uint32_t>(key), off);
        const uint32_t hi = __shfl_xor(static_cast<uint32_t>(key >> 32), off);
        const unsigned long long other = (static_cast<unsigned long long>(hi) << 32) | lo;
        key = other > key ? other : key;
      }
      if (live && (idx & (G - 1)) == 0) keys[static_cast<int64_t>(blockIdx.x) * M + mm] = key;
      return;
    }
  }
  if (!live) return;
  if (NMAT == 1 && pairs) {
    // The two K halves of this tile meet in one 64-bit slot per output.
    // The first to arrive leaves (1, its partial); the second takes it,
    // empties the slot for the next call and finishes the output.  The data
    // travels inside the atomic, so no fence or wait is needed, and the sum
    // does not depend on the arrival order (fp32 addition is commutative).
    // System scope: the two workgroups run on different XCDs, and the
    // exchange is then performed beyond their L2s.
    unsigned long long* slot = pairs + static_cast<int64_t>(tile) * (256 * TM) + idx;
    const unsigned long long prev = __hip_atomic_exchange(slot, (1ull << 32) | __float_as_uint(v[0]), __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_SYSTEM);
    if (prev >> 32) {
      __hip_atomic_exchange(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      v[0] += __uint_as_float(static_cast<uint32_t>(prev));
      if (has_out) epilogue<NMAT, OUT_F32>(a, g, row0 + oi, mm, N, v, epi);
    }
  } else if (splits > 1) {
    float* mine = partials + (static_cast<int64_t>(tile) * splits + s) * (NMAT * 256 * TM);
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) mine[mat * 256 * TM + idx] = v[mat];
  } else if (has_out) {
    epilogue<NMAT, OUT_F32>(a, g, row0 + oi, mm, N, v, epi);
  }
}

// Sums the split partial tiles of each 16-row tile in split order, then runs
// the epilogue.  One 256-thread workgroup per tile (16 rows x up to 32 tokens).
template <int NMAT, bool OUT_F32>
__global__ __launch_bounds__(256) void skinny_reduce_kernel(GroupArgs a, int M, int splits,
                                                            const float* __restrict__ partials) {
  const int tile = blockIdx.x;
  const int g = (NMAT == 2) ? 0 : member_of(a, tile);
  const int N = pick_early(a.n, g);
  const int row0 = (tile - pick_early(a.unit_begin, g)) * 16;
  // outputs per tile and matrix: 16 rows x 16 tokens per 16-token block
  const int slots = 256 * ((M + 15) >> 4);
  const float* base = partials + static_cast<int64_t>(tile) * splits * (NMAT * slots);
  for (int idx = threadIdx.x; idx < M * 16; idx += 256) {
    const int mm = idx >> 4, i = idx & 15;
    if (row0 + i >= N) continue;
    float v[NMAT];
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) {
      float t = 0.f;
      for (int sp = 0; sp < splits; ++sp) t += base[(sp * NMAT + mat) * slots + idx];
      v[mat] = t;
    }
    epilogue<NMAT, OUT_F32>(a, g, row0 + i, mm, N, v, epilogue_load<NMAT>(a, g, row0 + i, mm, N,
                                         reinterpret_cast<const uint16_t*>(pick_early(a.scale, g) + row0 + i)));
  }
}

// Launches one skinny_kernel instance (and records it for pgs_last_plan:
// this function's pretty name spells out the instance's template arguments).
template <int NW, int U, int NB, int NMAT, bool OUT_F32, bool K64, bool FOLD, int XM, bool NORM, int TM = 1>
int launch_instance(Problem& p, const SkinnyPlan& plan, hipStream_t st) {
  const int64_t grid = static_cast<int64_t>(plan.tiles) * (FOLD ? 2 : plan.splits);
  unsigned long long* pairs = plan.pair ? p.pairs : nullptr;
  note_launch(__PRETTY_FUNCTION__, grid, plan.splits, plan.splits > 1 && !plan.pair ? "skinny_reduce_kernel" : nullptr);
  hipLaunchKernelGGL((skinny_kernel<NW, U, NB, NMAT, OUT_F32, K64, FOLD, XM, NORM, TM>), dim3(static_cast<unsigned>(grid)),
                     dim3(64 * NW), 0, st, p.x, p.args, p.m, p.k, plan.splits, p.partials, pairs, p.norm_w, p.eps,
                     p.keys);
  return check_launch("w8a16 skinny kernel");
}

template <int NW, int U, int NB, int NMAT, bool OUT_F32, bool FOLD>
int launch_kernel(Problem& p, const SkinnyPlan& plan, hipStream_t st) {
  if constexpr (NB > 0 && !OUT_F32) {
    // rms_norm applied to the staged activations
    if (p.norm_w) {
      if (p.k % 64 != 0 || p.m > 4 || plan.splits != 1 || plan.pair)
        return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16 skinny: the fused norm needs m <= 4 and one K range");
      constexpr int S = FOLD ? 2 : 1;
      if (p.m == 1) return launch_instance<NW, U, NB, NMAT, OUT_F32, true, FOLD, 1, true>(p, plan, st);
      if (p.m == 2) return launch_instance<NW, U, NB, NMAT, OUT_F32, true, FOLD, 2, true>(p, plan, st);
      if constexpr (skinny_lds_bytes(NW, U, NB, NMAT, S, 4, true) <= kLdsLimit)
        return launch_instance<NW, U, NB, NMAT, OUT_F32, true, FOLD, 4, true>(p, plan, st);
      return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16 skinny: the fused norm's staging exceeds LDS");
    }
  }
  if (p.norm_w) return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16 skinny: the fused norm needs a bf16 output");
  // 17..32 tokens: two token blocks, unfolded, on shapes of >= 8 waves whose
  // loads fit the registers (two batches per wave, or the looping kernel)
  if (p.m > 16) {
    if constexpr (!FOLD && NW >= 8 && (NB == 2 || NB == 0)) {
      if (p.m > 32 || plan.tm != 2)
        return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16 skinny: m=%d with %d token blocks", p.m, plan.tm);
      if (p.k % 64 == 0) return launch_instance<NW, U, NB, NMAT, OUT_F32, true, false, 0, false, 2>(p, plan, st);
      return launch_instance<NW, U, 0, NMAT, OUT_F32, false, false, 0, false, 2>(p, plan, st);
    } else {
      return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16 skinny: no two-block kernel for this launch shape (m=%d)", p.m);
    }
  }
  // Up to four tokens in a folded launch stage their activations through
  // LDS (measured at one token: down_proj 6.56 -> 6.27 us, q|k|v 3.55 ->
  // 3.38, o_proj 2.97 -> 3.03; at four tokens down_proj 7.24 -> 6.85).  An
  // unfolded single matrix stages them at 3..8 tokens, where a lane's direct
  // loads would repeat the last token in the idle columns (lm_head
  // [151936, 2048] at 4 tokens 54.8 -> 48.1 us, at 8: 63.2 -> 56.1;
  // 11008 x 2048 at 8: 7.6 -> 6.8; q|k|v at 8: 4.05 -> 3.82; down_proj's
  // paired halves at 8: 8.2 -> 7.4); at 1..2 tokens the folded launch is
  // faster, and the SwiGLU pair keeps direct loads (staged: 9.3 -> 9.5 us).
  if constexpr (NB > 0 && FOLD) {
    if (p.k % 64 == 0 && p.m <= 4) {
      if (p.m == 1) return launch_instance<NW, U, NB, NMAT, OUT_F32, true, FOLD, 1, false>(p, plan, st);
      if (p.m == 2) return launch_instance<NW, U, NB, NMAT, OUT_F32, true, FOLD, 2, false>(p, plan, st);
      return launch_instance<NW, U, NB, NMAT, OUT_F32, true, FOLD, 4, false>(p, plan, st);
    }
  }
  // 9..16 tokens (single matrices, unfolded, issue-once batches): the same
  // staging, one batch at a time.  A direct B load of 16 tokens touches 16
  // activation rows (16 cache lines per KiB); a staged load covers 8 rows x
  // 128 bytes.  Measured at 16 tokens: down_proj's paired halves 9.97 ->
  // 8.34 us, q|k|v 4.8 -> 4.1, o_proj's halves 4.4 -> 4.2; the SwiGLU pair
  // (each B fragment already feeds two MFMAs) 11.3 -> 11.4, so it keeps
  // direct loads.
  if constexpr (NB > 0 && !FOLD && NMAT == 1) {
    if (p.k % 64 == 0 && p.m > 8 && p.m <= 16) {
      if constexpr (skinny_lds_bytes(NW, U, NB, NMAT, 1, 16, false) <= kLdsLimit)
        return launch_instance<NW, U, NB, NMAT, OUT_F32, true, false, 16, false>(p, plan, st);
    }
  }
  if constexpr (NB > 0 && !FOLD && NMAT == 1) {
    if (p.k % 64 == 0 && p.m >= 3 && p.m <= 8) {
      if (p.m <= 4) {
        if constexpr (skinny_lds_bytes(NW, U, NB, NMAT, 1, 4, false) <= kLdsLimit)
          return launch_instance<NW, U, NB, NMAT, OUT_F32, true, false, 4, false>(p, plan, st);
      } else {
        if constexpr (skinny_lds_bytes(NW, U, NB, NMAT, 1, 8, false) <= kLdsLimit)
          return launch_instance<NW, U, NB, NMAT, OUT_F32, true, false, 8, false>(p, plan, st);
      }
    }
  }
  if (p.k % 64 == 0) return launch_instance<NW, U, NB, NMAT, OUT_F32, true, FOLD, 0, false>(p, plan, st);
  return launch_instance<NW, U, 0, NMAT, OUT_F32, false, FOLD, 0, false>(p, plan, st);
}

template <int NW, int U, int NB, int NMAT, bool OUT_F32>
int launch_cfg(Problem& p, const SkinnyPlan& plan, hipStream_t st) {
  if (plan.fold && (NMAT != 1 || plan.splits != 1 || plan.pair || p.m > 8))
    return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16 skinny: folded plan for m=%d, %d matrices", p.m, NMAT);
  // NB > 0: the waves' batches must cover a workgroup's whole K range
  const int chunks = (p.k + 63) / 64;
  const int per_wg = plan.fold ? (chunks + 1) / 2 : (chunks + plan.splits - 1) / plan.splits;
  if (NB > 0 && NB * U * NW < per_wg)
    return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16 skinny: plan covers %d of %d slots", NB * U * NW, per_wg);
  int rc;
  if constexpr (NMAT == 1)
    rc = plan.fold ? launch_kernel<NW, U, NB, NMAT, OUT_F32, true>(p, plan, st)
                   : launch_kernel<NW, U, NB, NMAT, OUT_F32, false>(p, plan, st);
  else
    rc = launch_kernel<NW, U, NB, NMAT, OUT_F32, false>(p, plan, st);
  if (rc || plan.splits == 1 || plan.pair) return rc;
  hipLaunchKernelGGL((skinny_reduce_kernel<NMAT, OUT_F32>), dim3(static_cast<unsigned>(plan.tiles)), dim3(256), 0, st,
                     p.args, p.m, plan.splits, p.partials);
  return check_launch("w8a16 skinny reduce kernel");
}

// Launch shapes (waves per workgroup, slots per batch, batches per wave);
// a workgroup covers NW * U * NB slots of 64 k (128 k folded).  Index
// kLoopShape: the looping kernel for longer ranges; kLoop8Shape: the same
// with 8 waves, for two token blocks.
struct SkinnyShape {
  int nw, u, nb;
};
constexpr SkinnyShape kSkinnyShapes[] = {{4, 2, 1}, {4, 2, 2}, {8, 2, 2},  {16, 2, 2},
                                         {16, 1, 6}, {16, 2, 4}, {16, 2, 0}, {8, 2, 0}};
constexpr int kLoopShape = 6, kLoop8Shape = 7;

template <int NMAT, bool OUT_F32>
int launch_shape(Problem& p, const SkinnyPlan& plan, hipStream_t st) {
  switch (plan.shape) {
    case 0: return launch_cfg<4, 2, 1, NMAT, OUT_F32>(p, plan, st);
    case 1: return launch_cfg<4, 2, 2, NMAT, OUT_F32>(p, plan, st);
    case 2: return launch_cfg<8, 2, 2, NMAT, OUT_F32>(p, plan, st);
    case 3: return launch_cfg<16, 2, 2, NMAT, OUT_F32>(p, plan, st);
    case 4: return launch_cfg<16, 1, 6, NMAT, OUT_F32>(p, plan, st);
    case kLoop8Shape: return launch_cfg<8, 2, 0, NMAT, OUT_F32>(p, plan, st);
    case 5:
      if constexpr (NMAT == 1) return launch_cfg<16, 2, 4, NMAT, OUT_F32>(p, plan, st);
      [[fallthrough]];
    default: return launch_cfg<16, 2, 0, NMAT, OUT_F32>(p, plan, st);
  }
}

// The SwiGLU pair at 14..16 tokens with a short K (K % 64 == 0, at most
// NW * CPW chunks): RT row tiles per workgroup instead of one.  With one
// tile per workgroup every workgroup loads the tokens' whole activation
// rows for its 16 rows, as many bytes as its weights, and at 16 tokens each
// of those loads touches 16 rows; here each activation fragment feeds the
// RT tiles' gate and up MFMAs, and RT = 3 gives ceil(688 / 3) = 230
// workgroups for an 11008-row pair, at most one per CU and at most 48 rows
// per CU as before.  Wave w takes chunks w * CPW .. w * CPW + CPW - 1 of
// every tile and issues all of its loads at once (one memory round trip);
// the waves' partial tiles are summed through LDS in wave order (a fixed
// order: reproducible), then each output thread applies silu(g s_g)(u s_u)
// (engine/model.py:188-189).  Measured on the 11008 x 2048 pair (graphs over
// 36 layers, us, one-tile plan -> this kernel): 16 tokens 11.56 -> 11.20,
// 15: 11.36 -> 11.24, 14: 11.15 -> 11.02, but 13: 11.0 -> 11.1, 12: 10.8 ->
// 10.9 and 9: 10.1 -> 10.5, hence 14..16 tokens; 8 waves x 4 chunks (11.9),
// four tiles per workgroup (11.9) and two (13.0) are slower at 16 tokens.
template <int RT, int NW, int CPW>
__global__ __launch_bounds__(64 * NW, 1) void pair_tiles_kernel(const uint16_t* __restrict__ x, GroupArgs a, int M,
                                                                int K, int tiles) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lrow = lane & 15, kgrp = lane >> 4;
  const int N = a.n[0];
  const int nchunks = K >> 6;
  const int t0 = blockIdx.x * RT;
  // one buffer resource per tile and matrix over the tile's whole block
  // row; a tile past the last reads zeros without touching memory
  __amdgpu_buffer_rsrc_t wres[RT][2];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int mat = 0; mat < 2; ++mat) {
      const bool ok = t0 + r < tiles;
      wres[r][mat] = make_rsrc(a.q[mat] + (ok ? static_cast<int64_t>(t0 + r) * nchunks * 1024 : 0),
                               ok ? static_cast<int64_t>(nchunks) * 1024 : 0);
    }
  const __amdgpu_buffer_rsrc_t xres = make_rsrc(x, static_cast<int64_t>(M) * K * 2);
  // B operand column lrow: token min(lrow, M - 1); this lane's 16 k of the chunk
  const int xoff = min(lrow, M - 1) * K * 2 + kgrp * 32;

  // output of this thread: tile er, token mm, tile row oi; its scales are
  // requested first, from a clamped (valid) row, so no branch waits for them
  const int idx = threadIdx.x;
  const int er = min(idx >> 8, RT - 1), mm = (idx >> 4) & 15, oi = idx & 15;
  const int row = (t0 + er) * 16 + oi;
  const bool has_out = idx < 256 * RT && mm < M && row < N;
  const int crow = min(row, N - 1);
  const float sg = a.scale[0][crow], su = a.scale[1][crow];

  u32x4 w[CPW][RT][2], xb[CPW][2];
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    const int c = wave * CPW + j;
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int mat = 0; mat < 2; ++mat)
        w[j][r][mat] = __builtin_amdgcn_raw_buffer_load_b128(wres[r][mat], lane * 16, c * 1024, kLoadNT);
    xb[j][0] = __builtin_amdgcn_raw_buffer_load_b128(xres, xoff, c * 128, 0);
    xb[j][1] = __builtin_amdgcn_raw_buffer_load_b128(xres, xoff + 16, c * 128, 0);
  }
  f32x4 acc[RT][2];
#pragma unroll
  for (int r = 0; r < RT; ++r) acc[r][0] = acc[r][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < CPW; ++j) {
    // a chunk past K reads zero weights; its activations (the next token's
    // row, or zeros) are masked too, so non-finite values cannot leak in
    const uint32_t mask = wave * CPW + j < nchunks ? 0xffffffffu : 0u;
    const bf16x8 b0 = __builtin_bit_cast(bf16x8, xb[j][0] & mask);
    const bf16x8 b1 = __builtin_bit_cast(bf16x8, xb[j][1] & mask);
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int mat = 0; mat < 2; ++mat) {
        acc[r][mat] = mfma16x16x32(i8x8_to_bf16x8(w[j][r][mat][0], w[j][r][mat][1]), b0, acc[r][mat]);
        acc[r][mat] = mfma16x16x32(i8x8_to_bf16x8(w[j][r][mat][2], w[j][r][mat][3]), b1, acc[r][mat]);
      }
  }
  __shared__ f32x4 part[NW][RT][2][64];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int mat = 0; mat < 2; ++mat) part[wave][r][mat][lane] = acc[r][mat];
  __syncthreads();
  if (has_out) {
    // output (row oi, token mm) of a 16x16 tile: lane acc_lane(oi, mm), register oi % 4
    const int ln = acc_lane(oi, mm), rg = oi & 3;
    float g = 0.f, u = 0.f;
#pragma unroll
    for (int wv = 0; wv < NW; ++wv) {
      g += part[wv][er][0][ln][rg];
      u += part[wv][er][1][ln][rg];
    }
    store_out<false>(a.y[0], static_cast<int64_t>(mm) * N + row, silu_f32(g * sg) * (u * su));
  }
}

constexpr int kPairRT = 3, kPairNW = 16, kPairCPW = 2;

// whether pair_tiles_kernel takes a SwiGLU pair launch
bool pair_tiles_fits(const Problem& p, const SkinnyPlan& plan) {
  return p.nmat == 2 && !p.out_f32 && !p.norm_w && plan.tm == 1 && plan.splits == 1 && p.m >= 14 && p.m <= 16 &&
         p.k % 64 == 0 && p.k / 64 <= kPairNW * kPairCPW;
}

template <int RT, int NW, int CPW>
int launch_pair_tiles(Problem& p, const SkinnyPlan& plan, hipStream_t st) {
  const int64_t grid = (static_cast<int64_t>(plan.tiles) + RT - 1) / RT;
  note_launch(__PRETTY_FUNCTION__, grid, 1, nullptr);
  hipLaunchKernelGGL((pair_tiles_kernel<RT, NW, CPW>), dim3(static_cast<unsigned>(grid)), dim3(64 * NW), 0, st,
                     p.x, p.args, p.m, p.k, plan.tiles);
  return check_launch("w8a16 pair tiles kernel");
}

}  // namespace

SkinnyPlan plan_skinny(int m, int k, int nmat, int tiles, bool can_split) {
  // Measured on MI355X inside HIP graphs that cycle > 512 MB of distinct
  // weights (decode shapes of a 2048-hidden model).  Every load of a
  // workgroup is issued at once when its range fits one of the fixed shapes;
  // fewer than 256 row tiles leave CUs idle.  A single matrix then folds
  // (8-row halves over the whole K, no combine) at up to 8 tokens, with two
  // limits: the folded workgroup reads every token's activations over the
  // whole K, so a long K folds at up to 4 tokens (down_proj: 6.6 vs 7.1 us
  // paired at one token, 7.2 vs 7.4 at 4, 9.1 vs 8.1 at 8) and 129..255
  // tiles, which fill the CUs unsplit, only at up to 2 (q|k|v at one token:
  // 3.55 vs 3.62 us, at 4: 3.83 vs 3.82); o_proj: 3.0 vs 3.4 us at one token,
  // 3.4 vs 4.0 at 8.  With 256 tiles or more (lm_head, a lone gate_proj) a
  // short K still folds at up to 2 tokens: the halves' two chunks per MFMA
  // and staged activations beat the unfolded launch (lm_head [151936, 2048]
  // at one token 47.1 vs 47.8 us staged unfolded, 52.0 unstaged; 11008 x
  // 2048 5.9 vs 6.1); from 3 tokens the unfolded launch with staged
  // activations is faster (lm_head at 3: 46.8 vs 50.2).  Past the fold, a single matrix splits K over two
  // workgroups when K is long or when at most 128 tiles meet several tokens
  // (o_proj at 16 tokens: 4.3 vs 4.8 us); otherwise a 32-chunk K is faster
  // unsplit, without the pair slot's round trip (q|k|v at 16 tokens: 4.7 vs
  // 5.4 us).  17..32 tokens (two token blocks): 8-wave workgroups (16 waves
  // are slower: o_proj at 32 tokens 6.4 vs 10.2 us), two batches per wave or
  // the looping kernel (down_proj 15.8 vs 17.5 us with 16 waves), K split in
  // pairs only for a long K (o_proj unsplit 6.4 vs 7.3 us paired; the slots
  // hold 128 tiles of 16 x 32 outputs).
  SkinnyPlan p{tiles, 1, false, kLoopShape, false, m > 16 ? 2 : 1};
  const int chunks = (k + 63) / 64;
  if (nmat == 1 && chunks >= 16 && m <= 8 &&
      ((tiles < 256 && (m <= 2 || (tiles <= 128 && (m <= 4 || chunks < 64)))) ||
       (tiles >= 256 && m <= 2 && chunks < 64))) {
    p.fold = true;
  } else if (can_split && tiles < 256) {
    if (nmat == 1 && chunks >= 16 && tiles * p.tm <= 256 &&
        (chunks >= 64 || (m > 4 && p.tm == 1 && tiles <= 128))) {
      p.splits = 2;  // K halves combined through pair slots
      p.pair = true;
    } else if (chunks >= 128) {
      p.splits = 2;  // SwiGLU pair: partial tiles and a reduce kernel
    }
  }
  const int per_wg = p.fold ? (chunks + 1) / 2 : (chunks + p.splits - 1) / p.splits;
  // (the SwiGLU pair stops at 96 chunks: 128 would not fit its registers)
  const int last = nmat == 2 ? 4 : 5;
  if (p.tm == 2) {
    const SkinnyShape& sh = kSkinnyShapes[2];
    p.shape = sh.nw * sh.u * sh.nb >= per_wg ? 2 : kLoop8Shape;
    return p;
  }
  for (int i = last; i >= 0; --i) {
    const SkinnyShape& sh = kSkinnyShapes[i];
    if (sh.nw * sh.u * sh.nb >= per_wg) p.shape = i;
  }
  return p;
}

bool skinny_norm_fusable(const SkinnyPlan& p, int m, int k, bool out_f32, int nmat) {
  if (out_f32 || m < 1 || m > 4 || k % 64 != 0 || p.splits != 1 || p.pair || p.shape == kLoopShape) return false;
  const SkinnyShape& sh = kSkinnyShapes[p.shape];
  return sh.nb > 0 && skinny_lds_bytes(sh.nw, sh.u, sh.nb, nmat, p.fold ? 2 : 1, m == 1 ? 1 : m == 2 ? 2 : 4, true) <=
                          kLdsLimit;
}

int64_t skinny_grid(const SkinnyPlan& p) { return static_cast<int64_t>(p.tiles) * (p.fold ? 2 : p.splits); }

size_t skinny_partial_bytes(const SkinnyPlan& p, int nmat) {
  return (p.splits > 1 && !p.pair) ? static_cast<size_t>(p.tiles) * p.splits * nmat * 256 * p.tm * sizeof(float) : 0;
}

int launch_skinny(Problem& p, const SkinnyPlan& plan, hipStream_t st) {
  if (p.m < 1 || p.m > 16 * plan.tm || plan.tm < 1 || plan.tm > 2)
    return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16 skinny: m=%d with %d token blocks", p.m, plan.tm);
  if (plan.pair && (!p.pairs || plan.tiles * 256 * plan.tm * sizeof(unsigned long long) > kPairBytes || p.nmat != 1))
    return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16 skinny: paired split without pair slots");
  if (plan.splits > 1 && !plan.pair && (!p.partials || p.partial_bytes < skinny_partial_bytes(plan, p.nmat)))
    return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16 skinny: split-K plan without a large enough workspace");
  if (pair_tiles_fits(p, plan)) return launch_pair_tiles<kPairRT, kPairNW, kPairCPW>(p, plan, st);
  if (p.nmat == 2) return launch_shape<2, false>(p, plan, st);
  return p.out_f32 ? launch_shape<1, true>(p, plan, st) : launch_shape<1, false>(p, plan, st);
}

}  // namespace pgs
