// One launch per attention gap of a decode step: everything a decoder layer
// runs between two attention calls (engine/model.py:184-190, then the next
// layer's :165-173):
//
//   x1  = residual + o_proj(attn)                       (:184)
//   h   = rms_norm(x1, post_attention_layernorm)        (:187)
//   act = silu(gate_proj(h)) * up_proj(h)               (:188-189)
//   x2  = x1 + down_proj(act)                           (:190)
//   h'  = rms_norm(x2, next input_layernorm)            (:166)
//   q, k, v = q|k|v_proj(h') (+ bias), RoPE of q and k  (:168-173)
//
// The four linears depend on each other through whole vectors (every output
// of one feeds every output of the next), so separate launches leave the
// HBM weight stream idle at each boundary: the launch gap, the first bytes'
// latency and the slowest workgroup's tail, four times per layer.  Here one
// persistent workgroup per CU streams its share of all four weight matrices
// through a ring of loads that keeps running across the dependencies, and
// the dependencies are met by exchanges through memory inside the launch.
//
// Roles inside a workgroup of 16 waves:
//  * 15 streaming waves own a fixed list of 1 KiB weight loads (packed tile
//    layout: whole 16-row blocks for gate|up; folded 8-row units elsewhere,
//    two 64-k chunks per MFMA as the skinny kernel's folded halves) over
//    the four stages.  A wave keeps span_ring
//    loads in flight, issuing the next load as soon as one is consumed, so
//    the next stage's weights arrive while the current dependency is being
//    met.  Its waits are on its own loads and on workgroup barriers only:
//    it never waits for memory that another workgroup writes, whose loads
//    would queue behind its weight loads (vector memory returns in order).
//  * 1 control wave holds no weight loads.  It sums the streaming waves'
//    partial tiles (fixed order), runs each stage's epilogue, publishes the
//    workgroup's outputs to an exchange buffer and gathers every
//    workgroup's outputs for the next stage.
//
// The exchange carries the data with its own validity: each 32-bit word is a
// bf16 value in the low half and a 16-bit tag in the high half, written and
// read at agent scope (sc1: coherent across the XCDs' L2 caches), so a
// reader needs no flag, counter or fence -- a word is valid once its tag is
// the launch's tag.  The tag comes from an epoch word in the workspace that
// workgroup 0 advances once every workgroup has read it (after the first
// exchange, which every workgroup contributes to), so a HIP graph that
// replays the launch gets a new tag every time.  Every word of the exchange
// buffers is rewritten by every launch, so a stale word holds the previous
// launch's tag, never the current one.
//
// Every wait is bounded: a gather that has not seen every tag after
// spin_limit polls writes an error word into the workspace, and the whole
// workgroup returns normally at its next barrier.  A launch that finds the
// error word set returns at once; the host reads the word
// (pgs_w8a16_decode_span_status) and must clear the workspace before its
// next use.
//
// Residency: the grid is one workgroup per CU (a launch of exactly the
// device's CU count, checked against the occupancy query) and nothing else
// may run on the device meanwhile, or a gather waits for a workgroup that
// cannot start; the bound above then ends the launch with an error.
#include <atomic>
#include <type_traits>

#include "pgs_linear.h"

// Stage timestamps (a tracing aid).  With a trace buffer set
// (pgs_w8a16_decode_span_trace), lane 0 of each workgroup's control wave
// writes s_memrealtime (a constant 100 MHz clock) at every stage boundary
// into slot (launch tag % slots) of the buffer, laid out [slots][256
// workgroups][16] u64: entries 0..12 the marks below, 13..15 the poll
// counts of the three gathers, as wave 0 saw them (it holds exchange
// pieces at every token count; the control wave holds none at one token).
// Without one, a mark is a uniform branch.
#define PGS_SPAN_MARK(i)                                                    \
  do {                                                                      \
    if (tracing && tid == kSpanSW * 64) trow[i] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#define PGS_SPAN_NOTE(i, v)                                   \
  do {                                                        \
    if (tracing && tid == kSpanSW * 64) trow[i] = (v);        \
  } while (0)
#define PGS_SPAN_POLLS(i, v)                                  \
  do {                                                        \
    if (tracing && tid == 0) trow[i] = (v);                   \
  } while (0)

namespace pgs {
namespace {

constexpr int kSpanG = 256;                       // workgroups: one per CU
constexpr int kSpanSW = 15;                       // streaming waves per workgroup
constexpr int kSpanThreads = 64 * (kSpanSW + 1);  // + one control wave
// Weight loads in flight per streaming wave.  Deeper is not better: a CU's
// vector memory requests are served in order, so every load queued when
// the control wave polls an exchange delays the poll; the ring only has to
// cover the memory latency at the CU's share of the bandwidth.
constexpr int kSpanRingDefault = 4;
// The waves that hold pieces of a normalising gather (x1, x2: 8 KiB per
// workgroup at one token) wait this many s_sleep units (64 clocks each)
// after the workgroup's own publish before their first poll: issued at once
// it misses the slowest publishers' words, and the second poll behind it
// comes a round trip later.  One poll at about the time the last words
// become visible needs no second in most workgroups, and reads the exchange
// once (per step 822-824 against 846 us with two polls 16 units apart; 20 /
// 24 / 32 units: 825 / 825 / 823 us; measured before the activation gather
// below took its form, with it 24 / 26 / 30 units are within 1-2 us of 28).
// The waves without pieces do not wait:
// they issue the next stage's first loads at once.
constexpr int kNormPollDelay = 28;
// From two tokens on every wave holds pieces and polls after a shorter
// delay (the chain at 2 / 3 / 4 tokens with 0 / 8 / 14 / 20 / 28 units:
// 926 / 922 / 919 / 921 / 931, 1040 / 1035 / 1031 / 1033 / 1041 and
// 1116 / 1116 / 1111 / 1114 / 1120 us).
constexpr int kNormPollDelayMulti = 14;
// The activation gather at one token (44 KiB per workgroup) likewise: its
// pieces in waves 0..10 (4 per thread), which poll first kActPollDelay
// units after the publish, while waves 11..15 issue down_proj's first loads
// at once (per step 807 against 825 us with the pieces in all 16 waves and
// an immediate poll; 640 / 768 / 832 holding threads: 809 / 811 / 822 us; a
// delay of 16 / 20 / 32 units: 810 / 808 / 814 us at 704 or 768 threads;
// either change alone gains nothing).  The same at two tokens (8 pieces
// per thread; the two-token chain 932 against 946 us); at three and four
// every wave holds pieces and polls at once.
constexpr int kActHolders = 704;
constexpr int kActPollDelay = 24;
constexpr int kSlot = 128;                        // exchange bytes per 8-row unit (8 rows x <= 4 tokens x 4 B)
constexpr int kHeader = 256;                      // workspace header: [0] epoch, [1] error word
constexpr int kSC1 = 16;                          // cache policy: sc1 (agent scope)
constexpr int kMinLds = 84 * 1024;                // > half the CU's LDS: one workgroup per CU

constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }
constexpr int cmax(int a, int b) { return a > b ? a : b; }
constexpr int cmin(int a, int b) { return a < b ? a : b; }

template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// The model dimensions a kernel instance is compiled for.
template <int H_, int I_, int NQ_, int NKV_, int HD_>
struct Dims {
  static constexpr int H = H_, I = I_, NQ = NQ_, NKV = NKV_, HD = HD_;
  static_assert(H % 128 == 0 && I % 128 == 0, "K ranges are whole 128-k fold slots");
  static_assert(NQ % HD == 0 && NKV % HD == 0 && HD % 16 == 0, "whole heads of whole 8-row unit pairs");
};
using Qwen25_3B = Dims<2048, 11008, 2048, 256, 128>;

// Stage geometry.  Stage 0: o_proj, 1: gate|up, 2: down_proj, 3: q|k|v.
// A unit is R = 16 / F rows of one matrix over its whole K, folded: F 64-k
// chunks per MFMA (A rows i of the tile's R-row group in chunk i / R, B
// columns t + M j for the tokens' chunk j), as the skinny kernel's folded
// halves; an item is one F*64-k slot of a unit (one 1 KiB load per matrix);
// the items of a workgroup's units are dealt to the streaming waves in
// contiguous runs of P.  gate|up: F = 1, whole 16-row units (2 or 3 per
// workgroup), so that every load is one contiguous packed block.  With
// 8-row units (F = 2) a load reads half of two blocks whose other halves
// another workgroup reads at another time, and the pair streams slower
// (per step 888 against 910 us; 4-row units, F = 4, reading half lines:
// 31 against 24.5 us per layer).  o_proj, down_proj and q|k|v: F = 2,
// 8-row units, since their 128 (o, down) block rows would leave half the
// CUs idle as whole units (and q|k|v pairs rows for RoPE).
template <class DM, int M>
struct Geo {
  static constexpr int H = DM::H, I = DM::I;
  // q and k heads in unit pairs (rows i and i + HD/2 of a head, for RoPE), v
  // units alone
  static constexpr int kQP = DM::NQ / 16, kKP = DM::NKV / 16, kVS = DM::NKV / 8;
  static constexpr int fold(int s) { return s == 1 ? 1 : 2; }
  static constexpr int rows(int s) { return 16 / fold(s); }
  static constexpr int units(int s) { return s == 1 ? I / rows(1) : s == 3 ? (DM::NQ + 2 * DM::NKV) / 8 : H / 8; }
  static constexpr int U(int s) { return s == 3 ? 2 : cdiv(units(s), kSpanG); }
  static constexpr int ipu(int s) { return (s == 2 ? I : H) / (64 * fold(s)); }
  static constexpr int kdim(int s) { return s == 2 ? I : H; }
  static constexpr int nl(int s) { return s == 1 ? 2 : 1; }
  static constexpr int P(int s) { return cdiv(U(s) * ipu(s), kSpanSW); }
  static constexpr int lb(int s) {
    int b = 0;
    for (int i = 0; i < s; ++i) b += P(i) * nl(i);
    return b;
  }
  static constexpr int kLoads = lb(4);
  static constexpr int stage_of(int li) { return li < lb(1) ? 0 : li < lb(2) ? 1 : li < lb(3) ? 2 : 3; }
  // B operand rows in LDS: [M][K + 64] bf16 (the pad staggers the tokens)
  static constexpr int ks(int s) { return kdim(s) + 64; }
  static constexpr int kBBytes = M * (cmax(H, I) + 64) * 2;
  static constexpr int kPartFloats = kSpanSW * 2 * 2 * 16 * M;  // room for 16-row units
  static constexpr int kOffB = 0;
  static constexpr int kOffLn = kOffB + kBBytes;  // two norm weights [H] bf16
  static constexpr int kOffPart = kOffLn + 2 * H * 2;
  static constexpr int kOffSsq = kOffPart + kPartFloats * 4;
  static constexpr int kOffFlag = kOffSsq + 16 * M * 4;
  static constexpr int kLds = cmax(kOffFlag + 32, kMinLds);
  static_assert(kLds <= 160 * 1024, "LDS of one workgroup");
  static_assert(P(0) <= ipu(0) && P(1) <= ipu(1) && P(2) <= ipu(2) && P(3) <= ipu(3),
                "a wave's run touches at most two units");
  static_assert(8 * M * 4 <= kSlot, "a unit's outputs fit its exchange slot");
  static_assert(fold(1) * M <= 16, "the folded token groups fit the MFMA's 16 columns");
};

// Kernel arguments (device pointers; see pgs_w8a16_decode_span).
struct SpanParams {
  const uint16_t* attn;
  const uint16_t* resid;
  uint16_t* x_out;
  const int8_t* qo;
  const float* so;
  const uint16_t* ln_post;
  const int8_t* qg;
  const float* sg;
  const int8_t* qu;
  const float* su;
  const int8_t* qd;
  const float* sd;
  const uint16_t* ln_next;  // null: no q|k|v stage (last layer)
  const int8_t* qkv[3];
  const float* sqkv[3];
  const uint16_t* bqkv[3];
  uint16_t* yqkv[3];
  const uint16_t* cos;  // null: no RoPE
  const uint16_t* sin;
  uint32_t* ws;
  float eps;
  int spin_limit;
  int force_giveup;
  unsigned long long* trace;  // null: no stage timestamps
  int trace_slots;
};

// Where a unit's weights are: its 16-row block row (whole K) and the byte
// offset of its rows inside a block.
struct URef {
  const int8_t* blk;
  int roff;
  bool ok;
};

// Unit lu (0 .. U-1) of workgroup wg in stage S.  q|k|v: workgroups
// [0, kQP) take a q pair (8 rows of a head's first half and their partners
// HD/2 rows on), [kQP, kQP + kKP) a k pair, then one v unit each.
template <class DM, int M, int S>
__device__ __forceinline__ URef unit_ref(const SpanParams& p, int wg, int lu, int mat, int* member, int* row0) {
  using G = Geo<DM, M>;
  URef u{nullptr, 0, false};
  if constexpr (S == 3) {
    constexpr int HO = DM::HD / 16, HU = DM::HD / 8;
    int mem = 0, unit = 0;
    bool ok = p.ln_next != nullptr;
    if (wg < G::kQP) {
      unit = (wg / HO) * HU + wg % HO + lu * HO;
    } else if (wg < G::kQP + G::kKP) {
      const int pr = wg - G::kQP;
      mem = 1;
      unit = (pr / HO) * HU + pr % HO + lu * HO;
    } else if (wg < G::kQP + G::kKP + G::kVS && lu == 0) {
      mem = 2;
      unit = wg - G::kQP - G::kKP;
    } else {
      ok = false;
    }
    const int8_t* q = pick_early(p.qkv, mem);
    if (member) *member = mem;
    if (row0) *row0 = unit * 8;
    u.blk = q + static_cast<int64_t>(unit >> 1) * (DM::H / 64) * 1024;
    u.roff = (unit & 1) * 128;
    u.ok = ok && q != nullptr;
  } else {
    const int g = wg + kSpanG * lu;
    const int8_t* q = S == 0 ? p.qo : S == 2 ? p.qd : (mat ? p.qu : p.qg);
    constexpr int kb = G::kdim(S) / 64;
    constexpr int R = G::rows(S), PER = 16 / R;  // units per 16-row tile
    if (row0) *row0 = g * R;
    u.blk = q + static_cast<int64_t>(g / PER) * kb * 1024;
    u.roff = (g % PER) * R * 16;
    u.ok = g < G::units(S);
  }
  return u;
}

__device__ __forceinline__ void barrier_lds() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Whether any thread of the workgroup has `pred` set; all threads call it
// and get the same answer.  (__syncthreads_or would also wait for every
// outstanding vector load, the streaming waves' ring included.)  Three LDS
// words in rotation, indexed by a workgroup-uniform sequence number `seq`
// that the caller increments per call: the word for call seq + 1 is cleared
// before this call's barrier, when every thread has read it (at call
// seq - 2) and passed call seq - 1's barrier; the kernel zeroes all three
// before its first call.
typedef __attribute__((address_space(3))) int lds_int;

__device__ __forceinline__ bool block_any(bool pred, int* words_generic, int& seq) {
  // (explicitly LDS: a generic access would be a flat one, which the
  // vector memory counter also tracks)
  lds_int* words = (lds_int*)words_generic;
  lds_int* w = words + seq % 3;
  if (__any(pred) && (threadIdx.x & 63) == 0) __hip_atomic_fetch_or(w, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  if (threadIdx.x == 0) __hip_atomic_store(words + (seq + 1) % 3, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  barrier_lds();
  const bool any = __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0;
  ++seq;
  return any;
}

__device__ __forceinline__ uint32_t ld_agent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float bf16r(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

// Gathers every unit's tagged outputs of one exchange buffer and builds the
// next stage's B operand from them (all waves of the workgroup).  Thread
// `tid` < HT polls pieces tid + HT i (16 bytes: four words of one unit's
// outputs of one token) into registers with agent-scope loads, the first
// poll DELAY s_sleep units after the workgroup's publish; a poll refetches
// only the pieces whose tags were stale, and the workgroup stops polling
// once no thread holds a stale piece.  A CU's vector memory requests are
// served in order, so a poll waits behind whatever the CU has queued; the
// waves without pieces issue the next stage's first loads at once.
// Then, NORM: rms_norm (engine/model.py:29-34) with the norm weight in LDS,
// r = 1 / sqrt(mean(x^2) + eps), h = bf16(w * bf16(x * r)), the sum of
// squares in a fixed order (per thread over its pieces, a wave butterfly,
// the 16 waves in order); otherwise the values as they are.  The B operand
// is [M][KS] bf16 in LDS.  Returns false (the same for every thread) after
// spin_limit polls.
template <int M, int K, int KS, bool NORM, int DELAY, int HT, bool EARLY, class OnPoll>
__device__ __forceinline__ bool gather_b(const uint32_t* xbuf, unsigned char* smem, int off_b, int off_ln,
                                         int off_ssq, int* any_words, int& seq, uint32_t want, int spin_limit,
                                         float eps, int& polls, OnPoll&& on_poll) {
  constexpr int NP = (K / 8) * 2 * M, NPT = cdiv(NP, HT);
  static_assert(HT % 64 == 0 && HT <= kSpanThreads, "pieces held by whole waves");
  static_assert(NPT <= 32, "one stale bit per piece");
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const __amdgpu_buffer_rsrc_t r = make_rsrc(xbuf, static_cast<int64_t>(K / 8) * kSlot);
  // piece i of this thread (NP: none): the first HT threads hold them
  auto piece = [&](int i) { return tid < HT ? cmin(tid + HT * i, NP) : NP; };
  auto piece_off = [&](int i) {
    const int pc = piece(i);
    return pc < NP ? (pc / (2 * M)) * kSlot + (pc % (2 * M)) * 16 : 0x7ffffff0;
  };
  auto fresh = [&](const u32x4& x) {
    return (x[0] >> 16) == want && (x[1] >> 16) == want && (x[2] >> 16) == want && (x[3] >> 16) == want;
  };
  // Each wave polls until its own pieces are fresh (a wave that holds
  // pieces waits DELAY s_sleep units before its first poll), and only then
  // issues (on_poll) the next stage's first loads: a wave's loads return in
  // order, so a poll issued behind its own weight loads would wait for
  // them.  EARLY: a holding wave issues them right behind its first poll
  // instead, which still returns first; only a second poll then waits
  // behind them (the normalising gathers at one token, where the median
  // workgroup polls once: per step 786-787 against 792-793 us; x1 alone
  // 791; the activation gather too: 810).  Then the workgroup-wide check
  // (which also makes a give-up uniform).
  u32x4 v[NPT];
  uint32_t stale = 0;
#pragma unroll
  for (int i = 0; i < NPT; ++i)
    if (piece(i) < NP) stale |= 1u << i;
  const bool holder = __any(stale != 0);
  if (holder) {
    if constexpr (DELAY > 0) __builtin_amdgcn_s_sleep(DELAY);
    for (int spin = 0;; ++spin) {
#pragma unroll
      for (int i = 0; i < NPT; ++i)
        if (stale & (1u << i)) v[i] = __builtin_amdgcn_raw_buffer_load_b128(r, piece_off(i), 0, kSC1);
      if constexpr (EARLY) {
        if (spin == 0) on_poll();
      }
#pragma unroll
      for (int i = 0; i < NPT; ++i)
        if ((stale & (1u << i)) && fresh(v[i])) stale &= ~(1u << i);
      polls = spin + 1;
      // (the next poll goes out as soon as this one is checked: each poll
      // waits for its own data, so the loop runs at one round trip per
      // poll; a sleep between polls measured 1-2 us per step slower)
      if (!__any(stale != 0) || spin >= spin_limit) break;
    }
  }
  if (!EARLY || !holder) on_poll();
  // piece pc: unit pc / 2M (rows 8 unit ..), token (pc % 2M) / 2, rows
  // 8 unit + 4 (pc % 2) + e for its words e = 0..3
  // NORM: each wave's sum of squares goes to LDS before the workgroup-wide
  // check, whose barrier then serves both (a give-up discards it)
  float* ssq = reinterpret_cast<float*>(smem + off_ssq);
  if constexpr (NORM) {
    float ss[M];
#pragma unroll
    for (int t = 0; t < M; ++t) ss[t] = 0.f;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      const int pc = piece(i);
      const int t = (pc % (2 * M)) / 2;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = bf16_bits_to_f32(v[i][e] & 0xffffu);
#pragma unroll
        for (int tt = 0; tt < M; ++tt)
          if (pc < NP && t == tt) ss[tt] += x * x;
      }
    }
#pragma unroll
    for (int t = 0; t < M; ++t) {
      float x = ss[t];
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) x += __shfl_xor(x, o);
      if (lane == 0) ssq[wave * M + t] = x;
    }
  }
  if (block_any(stale != 0, any_words, seq)) return false;
  float r_t[M];
  if constexpr (NORM) {
#pragma unroll
    for (int t = 0; t < M; ++t) {
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < 16; ++w) tot += ssq[w * M + t];
      r_t[t] = 1.0f / sqrtf(tot / static_cast<float>(K) + eps);
    }
  }
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    const int pc = piece(i);
    if (pc >= NP) continue;
    const int t = (pc % (2 * M)) / 2, n0 = (pc / (2 * M)) * 8 + (pc % 2) * 4;
    u32x2 out;
    if constexpr (NORM) {
      float rt = r_t[0];
#pragma unroll
      for (int tt = 1; tt < M; ++tt) rt = t == tt ? r_t[tt] : rt;
      const u32x2 w2 = *reinterpret_cast<const u32x2*>(smem + off_ln + n0 * 2);
      float h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t wb = (e & 1) ? (w2[e >> 1] >> 16) : (w2[e >> 1] & 0xffffu);
        h[e] = bf16_bits_to_f32(wb) * bf16r(bf16_bits_to_f32(v[i][e] & 0xffffu) * rt);
      }
      out = u32x2{pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3])};
    } else {
      out = u32x2{(v[i][0] & 0xffffu) | (v[i][1] << 16), (v[i][2] & 0xffffu) | (v[i][3] << 16)};
    }
    *reinterpret_cast<u32x2*>(smem + off_b + (t * KS + n0) * 2) = out;
  }
  return true;
}

template <class DM, int M, int RING = kSpanRingDefault>
__global__ __launch_bounds__(kSpanThreads, 1) void span_kernel(SpanParams p) {
  using G = Geo<DM, M>;
  constexpr int H = DM::H, I = DM::I;
  __shared__ __attribute__((aligned(16))) unsigned char smem[G::kLds];
  const int wg = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool control = wave == kSpanSW;
  const bool has_qkv = p.ln_next != nullptr;
  int* flag = reinterpret_cast<int*>(smem + G::kOffFlag);  // [0] abort, [1] the launch's tag, [4..6] block_any
  int any_seq = 0;
  float* part = reinterpret_cast<float*>(smem + G::kOffPart);
  uint32_t* const ws = p.ws;
  uint32_t* const x1x = ws + kHeader / 4;
  uint32_t* const actx = x1x + (H / 8) * (kSlot / 4);
  uint32_t* const x2x = actx + (I / 8) * (kSlot / 4);

  // ---- streaming-wave state -------------------------------------------
  const int lrow = lane & 15, kgrp = lane >> 4;
  // A operand (fold F, R = 16 / F rows): this lane's 16 bytes of a fold
  // slot, row lrow % R of the unit in chunk F j + lrow / R; B operand:
  // column lrow = token lrow % M of chunk F j + lrow / M (columns past F M
  // read token 0, unused)
  auto avoff = [&](int f) { return (lrow / (16 / f)) * 1024 + ((lrow % (16 / f)) + 16 * kgrp) * 16; };
  auto btok = [&](int f) { return lrow < f * M ? lrow % M : 0; };
  auto bsub = [&](int f) { return lrow < f * M ? lrow / M : 0; };
  constexpr int kSpanRing = RING;
  u32x4 ring[kSpanRing];
  f32x4 acc[2][2];

  auto issue = [&](auto LI) {
    constexpr int li = decltype(LI)::value;
    if constexpr (li < G::kLoads) {
      constexpr int S = G::stage_of(li);
      constexpr int it = (li - G::lb(S)) / G::nl(S), mat = (li - G::lb(S)) % G::nl(S);
      const int item = G::P(S) * wave + it;
      const int lu = item / G::ipu(S), slot = item - lu * G::ipu(S);
      const URef u = unit_ref<DM, M, S>(p, wg, lu, mat, nullptr, nullptr);
      // (the control wave issues the same loads with an empty range: no
      // memory access, but both roles then have the same loads in flight
      // where their code paths join, so the compiler's waits stay exact)
      const bool ok = !control && u.ok && item < G::U(S) * G::ipu(S);
      const __amdgpu_buffer_rsrc_t r = make_rsrc(ok ? u.blk : p.qo, ok ? (G::kdim(S) / 64) * 1024 : 0);
      constexpr int F = G::fold(S);
      ring[li % kSpanRing] =
          __builtin_amdgcn_raw_buffer_load_b128(r, avoff(F), uniform(slot * F * 1024 + u.roff), kLoadNT);
    }
  };
  // the first kSpanRing loads of stage S (the rest follow as its items are
  // consumed): issued right behind the gather that stage S waits for, so
  // that they stream in while the gather completes instead of delaying it
  auto prime = [&](auto SI) {
    constexpr int S = decltype(SI)::value;
    static_for<G::lb(S), cmin(G::lb(S) + kSpanRing, G::lb(S + 1))>(issue);
  };
  auto zero_acc = [&] {
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int m = 0; m < 2; ++m) acc[a][m] = f32x4{0.f, 0.f, 0.f, 0.f};
  };
  // the items of stage S: MFMAs on the ring's loads, each consumed load
  // replaced by the one kSpanRing further down the list
  auto run_stage = [&](auto SI) {
    constexpr int S = decltype(SI)::value;
    const int first = G::P(S) * wave;
    const int lu0 = first / G::ipu(S);
    constexpr int F = G::fold(S), R = G::rows(S);
    const unsigned char* bbase = smem + G::kOffB + (btok(F) * G::ks(S) + bsub(F) * 64 + 16 * kgrp) * 2;
    static_for<0, G::P(S)>([&](auto IT) {
      constexpr int it = decltype(IT)::value;
      const int item = first + it;
      const int lu = item / G::ipu(S), slot = item - lu * G::ipu(S);
      const bool ok = unit_ref<DM, M, S>(p, wg, lu, 0, nullptr, nullptr).ok && item < G::U(S) * G::ipu(S);
      if (ok) {
        const u32x4 b0 = *reinterpret_cast<const u32x4*>(bbase + slot * F * 128);
        const u32x4 b1 = *reinterpret_cast<const u32x4*>(bbase + slot * F * 128 + 16);
        const bf16x8 x0 = __builtin_bit_cast(bf16x8, b0), x1 = __builtin_bit_cast(bf16x8, b1);
        const bool second = lu != lu0;
        static_for<0, G::nl(S)>([&](auto MT) {
          constexpr int mat = decltype(MT)::value;
          const u32x4 w = ring[(G::lb(S) + it * G::nl(S) + mat) % kSpanRing];
          const bf16x8 a0 = i8x8_to_bf16x8(w[0], w[1]), a1 = i8x8_to_bf16x8(w[2], w[3]);
          if (second) {
            acc[1][mat] = mfma16x16x32(a0, x0, acc[1][mat]);
            acc[1][mat] = mfma16x16x32(a1, x1, acc[1][mat]);
          } else {
            acc[0][mat] = mfma16x16x32(a0, x0, acc[0][mat]);
            acc[0][mat] = mfma16x16x32(a1, x1, acc[0][mat]);
          }
        });
      }
      static_for<0, G::nl(S)>([&](auto MT) {
        constexpr int nxt = G::lb(S) + it * G::nl(S) + decltype(MT)::value + kSpanRing;
        if constexpr (nxt < G::lb(S + 1)) issue(std::integral_constant<int, nxt>{});
      });
    });
    // partial tiles: output (token t, row r) of a folded unit is
    // sum_s C[r + R s][t + M s] (s < F, in order); C[i][j] sits in lane
    // 16 (i / 4) + j, register i % 4.  F = 1: lanes t, 16 + t, 32 + t and
    // 48 + t hold rows 0-3 .. 12-15, no partners; F = 2: lanes t and 16 + t
    // hold rows 0-3 and 4-7, partners 32 + M lanes on; F = 4: lane t holds
    // rows 0-3, partners 16 + M, 2 (16 + M), 3 (16 + M) lanes on.
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int mat = 0; mat < G::nl(S); ++mat) {
        f32x4 v = acc[a][mat];
        constexpr int step = F == 2 ? 32 + M : 16 + M;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float x = v[i];
#pragma unroll
          for (int sft = 1; sft < F; ++sft) x += __shfl_down(v[i], sft * step);
          v[i] = x;
        }
        const int t = lane & 15;
        if (lane < 16 * (R / 4) && t < M) {
          float* dst = part + ((wave * 2 + a) * 2 + mat) * (16 * M) + t * R + (lane >> 4) * 4;
#pragma unroll
          for (int i = 0; i < 4; ++i) dst[i] = v[i];
        }
      }
    zero_acc();
  };

  // ---- control-wave state -------------------------------------------------
  // outputs per lane: o / down: (t, r) = (idx / 8, idx % 8) of this
  // workgroup's unit; gate|up: idx = (lu, t, r); q|k|v: (t, r) of the unit
  // (pair)
  // gate|up outputs of this workgroup: idx = (lu, t, r), r < R1 rows
  constexpr int R1 = G::rows(1);
  constexpr int NO = cdiv(8 * M, 64), NG = cdiv(G::U(1) * R1 * M, 64);
  static_assert(NO == 1, "one o/down output per control lane");
  uint32_t tag = 0;
  float so_r = 0.f, sd_r = 0.f, res_r = 0.f, x1_r = 0.f;
  float sg_r[NG], su_r[NG];
  // q|k|v epilogue operands as loaded (raw bits: converted where used)
  uint32_t sq_b[2] = {0u, 0u};
  uint16_t bq_b[2] = {0, 0}, cs_b[4] = {0, 0, 0, 0};
  bool bq_on[2] = {false, false};
  int qmem = 0, qrow[2] = {0, 0};

  // reduces unit lu's partial tiles of stage S for output (t, r), matrix mat
  // (a unit's items span at most cdiv(IPU, P) + 1 waves: all of their
  // partials are read before the first add, in a loop of that fixed length,
  // since a bound that depends on the lane would serialise the LDS reads;
  // the sum is the same, in wave order)
  auto reduce = [&](auto SI, int lu, int mat, int t, int r) {
    constexpr int S = decltype(SI)::value;
    constexpr int P = G::P(S), IPU = G::ipu(S), KMAX = cdiv(IPU, P) + 1;
    const int s_lo = lu * IPU / P, s_hi = cmin(kSpanSW - 1, ((lu + 1) * IPU - 1) / P);
    float pv[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      const int s = cmin(s_lo + k, kSpanSW - 1);
      const int a = cmin(cmax(lu - (P * s) / IPU, 0), 1);
      pv[k] = part[((s * 2 + a) * 2 + mat) * (16 * M) + t * G::rows(S) + r];
    }
    float v = 0.f;
#pragma unroll
    for (int k = 0; k < KMAX; ++k)
      if (s_lo + k <= s_hi) v += pv[k];
    return v;
  };
  auto abort_now = [&] {
    if (flag[0]) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      return true;
    }
    return false;
  };

  // The q|k|v epilogue operands (scales, bias, RoPE cos/sin), used only at
  // the launch's end.  The control wave requests them once the x1 gather is
  // done, when nothing of its own is in flight, and they have landed long
  // before its next wait: loaded in the prologue they make the workgroups
  // with q|k|v units publish x1 last.  The loads are unconditional -- an
  // absent operand reads a valid stand-in address -- so that the number of
  // loads in flight is the same on every path, and their raw bits stay in
  // registers until the epilogue, so that nothing waits for them earlier.
  auto load_qkv_operands = [&] {
    const int t = cmin(lane / 8, M - 1), r = lane % 8;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      int mem = 0, row0 = 0;
      const URef u = unit_ref<DM, M, 3>(p, wg, j, 0, &mem, &row0);
      qrow[j] = row0 + r;
      if (j == 0) qmem = mem;
      const bool ok = has_qkv && u.ok;
      const uint16_t* b = ok ? pick_early(p.bqkv, mem) : nullptr;
      const float* sptr = ok ? pick_early(p.sqkv, mem) + row0 + r : p.so + r;
      const uint16_t* bptr = b ? b + row0 + r : p.resid + r;
      sq_b[j] = __builtin_bit_cast(uint32_t, *sptr);
      bq_b[j] = *bptr;
      bq_on[j] = b != nullptr;
    }
    constexpr int HD = DM::HD;
    const bool rope = has_qkv && p.cos && qmem < 2;
    const int i = qrow[0] % HD;  // < HD / 2: the pair's first row
    const int64_t base = static_cast<int64_t>(t) * HD;
    const uint16_t* cp = rope ? p.cos + base + i : p.resid;
    const uint16_t* sp = rope ? p.sin + base + i : p.resid;
    cs_b[0] = cp[0];
    cs_b[1] = sp[0];
    cs_b[2] = cp[HD / 2];
    cs_b[3] = sp[HD / 2];
  };

  const bool tracing = p.trace != nullptr;
  const unsigned long long t_start = tracing ? __builtin_amdgcn_s_memrealtime() : 0ull;
  unsigned long long* trow = p.trace;  // this workgroup's row, once the tag is known
  // ================= prologue =================
  // The control wave's operand loads go out first, then (after a barrier)
  // the streaming waves' o_proj weight loads: the CU serves its vector
  // memory requests in order, and the workgroup waits for the operands
  // before o_proj can start (per step 790 against 804 us with both issued
  // together, 802 with the weights first).  The deeper weight stream starts
  // only behind the gathers, whose polls must not queue behind it.
  constexpr int PC = M * H / 8, NA = cdiv(PC, 64), NL = cdiv(H / 8, 64);
  u32x4 attn_v[NA], lnp_v[NL], lnn_v[NL];
  uint32_t ep = 0, err = 0;
  if (control) {
    ep = ld_agent(ws);
    err = ld_agent(ws + 1);
    // o_proj's B operand (the attention output) and the two norm weights
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int pc = cmin(lane + 64 * i, PC - 1);
      attn_v[i] = ld16(p.attn + static_cast<int64_t>(pc / (H / 8)) * H + 8 * (pc % (H / 8)));
    }
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int pc = cmin(lane + 64 * i, H / 8 - 1);
      lnp_v[i] = ld16(p.ln_post + 8 * pc);
      lnn_v[i] = ld16((has_qkv ? p.ln_next : p.ln_post) + 8 * pc);
    }
    // epilogue operands
    {
      const int t = cmin(lane / 8, M - 1), r = lane % 8, row = cmin(8 * wg + r, H - 1);
      so_r = p.so[row];
      sd_r = p.sd[row];
      res_r = bf16_bits_to_f32(p.resid[static_cast<int64_t>(t) * H + row]);
    }
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const int idx = lane + 64 * i;
      const int lu = idx / (R1 * M), r = idx % R1;
      const int g = cmin(wg + kSpanG * lu, I / R1 - 1);
      sg_r[i] = p.sg[R1 * g + r];
      su_r[i] = p.su[R1 * g + r];
    }
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  if (!control) {
    zero_acc();
    prime(std::integral_constant<int, 0>{});
  }
  if (control) {
    tag = ep % 65535u + 1u;
    if (lane == 0) {
      flag[0] = err != 0;
      flag[1] = static_cast<int>(tag);
      flag[4] = flag[5] = flag[6] = 0;
    }
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int pc = lane + 64 * i;
      if (pc < PC)
        *reinterpret_cast<u32x4*>(smem + G::kOffB + ((pc / (H / 8)) * G::ks(0) + 8 * (pc % (H / 8))) * 2) = attn_v[i];
    }
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int pc = lane + 64 * i;
      if (pc < H / 8) {
        *reinterpret_cast<u32x4*>(smem + G::kOffLn + pc * 16) = lnp_v[i];
        *reinterpret_cast<u32x4*>(smem + G::kOffLn + H * 2 + pc * 16) = lnn_v[i];
      }
    }
    __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0)
    // the epilogue operands have arrived: redefining them here (an empty
    // asm) tells the compiler so, which keeps it from waiting for loads
    // issued later wherever they are used
    asm volatile("" : "+v"(so_r), "+v"(sd_r), "+v"(res_r));
#pragma unroll
    for (int i = 0; i < NG; ++i) asm volatile("" : "+v"(sg_r[i]), "+v"(su_r[i]));
  }
  barrier_lds();
  if (abort_now()) return;
  if (tracing) trow = p.trace + (static_cast<int64_t>(static_cast<uint32_t>(flag[1]) % p.trace_slots) * kSpanG + wg) * 16;
  PGS_SPAN_NOTE(0, t_start);
  PGS_SPAN_MARK(1);

  // ================= stage 0: o_proj + residual =================
  const uint32_t ltag = static_cast<uint32_t>(flag[1]);  // every wave's copy of the tag
  int polls = 0;
  // the whole workgroup gave up waiting: the error word, then out
  auto give_up = [&] {
    if (tid == 0) st_agent(ws + 1, 1u);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  };
  if (!control) run_stage(std::integral_constant<int, 0>{});
  barrier_lds();
  PGS_SPAN_MARK(2);
  if (control) {
    const int t = lane / 8, r = lane % 8;
    if (lane < 8 * M && wg < H / 8) {
      const float v = reduce(std::integral_constant<int, 0>{}, 0, 0, t, r) * so_r;
      x1_r = bf16r(bf16r(v) + res_r);  // engine/model.py:184: residual + bf16(linear)
      st_agent(x1x + wg * (kSlot / 4) + t * 8 + r, (ltag << 16) | f32_to_bf16_bits(x1_r));
    }
    PGS_SPAN_MARK(3);
  }
  barrier_lds();
  if (!gather_b<M, H, G::ks(1), true, M == 1 ? kNormPollDelay : kNormPollDelayMulti, kSpanThreads, M == 1>(x1x, smem, G::kOffB, G::kOffLn, G::kOffSsq, flag + 4, any_seq,
                                      p.force_giveup ? ltag % 65535u + 1u : ltag, p.spin_limit, p.eps, polls, [&] {
                                        prime(std::integral_constant<int, 1>{});
                                      })) {
    give_up();
    return;
  }
  if (control) load_qkv_operands();
  // every workgroup has read the epoch (it published with its tag)
  if (wg == 0 && tid == 0) st_agent(ws, ltag);
  PGS_SPAN_POLLS(13, polls);
  barrier_lds();
  PGS_SPAN_MARK(4);

  // ================= stage 1: gate|up, SwiGLU =================
  if (!control) run_stage(std::integral_constant<int, 1>{});
  barrier_lds();
  PGS_SPAN_MARK(5);
  if (control) {
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const int idx = lane + 64 * i;
      const int lu = idx / (R1 * M), t = (idx / R1) % M, r = idx % R1;
      const int g = wg + kSpanG * lu;
      if (lu < G::U(1) && g < I / R1) {
        const float gv = reduce(std::integral_constant<int, 1>{}, lu, 0, t, r) * sg_r[i];
        const float uv = reduce(std::integral_constant<int, 1>{}, lu, 1, t, r) * su_r[i];
        const float a = silu_f32(gv) * uv;
        // row R1 g + r lives in the 8-row exchange slot of its rows
        const int row = R1 * g + r;
        st_agent(actx + (row >> 3) * (kSlot / 4) + t * 8 + (row & 7), (ltag << 16) | f32_to_bf16_bits(a));
      }
    }
    PGS_SPAN_MARK(6);
  }
  barrier_lds();
  if (!gather_b<M, I, G::ks(2), false, M <= 2 ? kActPollDelay : 0, M <= 2 ? kActHolders : kSpanThreads, false>(actx, smem, G::kOffB, G::kOffLn, G::kOffSsq, flag + 4, any_seq, ltag,
                                       p.spin_limit, p.eps, polls, [&] {
        prime(std::integral_constant<int, 2>{});
      })) {
    give_up();
    return;
  }
  PGS_SPAN_POLLS(14, polls);
  barrier_lds();
  PGS_SPAN_MARK(7);

  // ================= stage 2: down_proj + residual =================
  if (!control) run_stage(std::integral_constant<int, 2>{});
  barrier_lds();
  PGS_SPAN_MARK(8);
  if (control) {
    const int t = lane / 8, r = lane % 8;
    if (lane < 8 * M && wg < H / 8) {
      const float v = reduce(std::integral_constant<int, 2>{}, 0, 0, t, r) * sd_r;
      const float x2 = bf16r(bf16r(v) + x1_r);  // engine/model.py:190
      const uint16_t bits = f32_to_bf16_bits(x2);
      p.x_out[static_cast<int64_t>(t) * H + 8 * wg + r] = bits;
      if (has_qkv) st_agent(x2x + wg * (kSlot / 4) + t * 8 + r, (ltag << 16) | bits);
    }
    PGS_SPAN_MARK(9);
  }
  if (!has_qkv) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }
  barrier_lds();
  if (!gather_b<M, H, G::ks(3), true, M == 1 ? kNormPollDelay : kNormPollDelayMulti, kSpanThreads, M == 1>(x2x, smem, G::kOffB, G::kOffLn + H * 2, G::kOffSsq, flag + 4, any_seq,
                                      ltag, p.spin_limit, p.eps, polls, [&] {
                                        prime(std::integral_constant<int, 3>{});
                                      })) {
    give_up();
    return;
  }
  PGS_SPAN_POLLS(15, polls);
  barrier_lds();
  PGS_SPAN_MARK(10);

  // ================= stage 3: q|k|v (+ bias), RoPE =================
  if (!control) run_stage(std::integral_constant<int, 3>{});
  barrier_lds();
  PGS_SPAN_MARK(11);
  if (control && lane < 8 * M) {
    const int t = lane / 8, r = lane % 8;
    int mem = 0, row0 = 0;
    const URef u0 = unit_ref<DM, M, 3>(p, wg, 0, 0, &mem, &row0);
    if (u0.ok) {
      uint16_t* y = pick_early(p.yqkv, mem);
      const int n = mem == 0 ? DM::NQ : DM::NKV;
      // (the empty asm makes the loaded bits opaque up to here: the compiler
      // would otherwise convert them, and wait for the loads, where they
      // were issued)
      asm volatile("" : "+v"(sq_b[0]), "+v"(sq_b[1]), "+v"(bq_b[0]), "+v"(bq_b[1]), "+v"(cs_b[0]), "+v"(cs_b[1]),
                   "+v"(cs_b[2]), "+v"(cs_b[3]));
      float sq_r[2], bq_r[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        sq_r[j] = __builtin_bit_cast(float, sq_b[j]);
        bq_r[j] = bq_on[j] ? bf16_bits_to_f32(bq_b[j]) : 0.f;
      }
      const float y0 = bf16r(reduce(std::integral_constant<int, 3>{}, 0, 0, t, r) * sq_r[0] + bq_r[0]);
      if (mem < 2) {
        const float y1 = bf16r(reduce(std::integral_constant<int, 3>{}, 1, 0, t, r) * sq_r[1] + bq_r[1]);
        float o0 = y0, o1 = y1;
        if (p.cos) {
          float cs_r[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) cs_r[c] = bf16_bits_to_f32(cs_b[c]);
          // engine/model.py:53-56 with rotate_half (:37-39), the reference's roundings
          o0 = bf16r(bf16r(y0 * cs_r[0]) + bf16r(-y1 * cs_r[1]));
          o1 = bf16r(bf16r(y1 * cs_r[2]) + bf16r(y0 * cs_r[3]));
        }
        y[static_cast<int64_t>(t) * n + qrow[0]] = f32_to_bf16_bits(o0);
        y[static_cast<int64_t>(t) * n + qrow[1]] = f32_to_bf16_bits(o1);
      } else {
        y[static_cast<int64_t>(t) * n + qrow[0]] = f32_to_bf16_bits(y0);
      }
    }
  }
  PGS_SPAN_MARK(12);
}

// device CU counts, checked once per device (0 = not yet)
std::atomic<int> g_cus[kMaxDevices];

template <class DM, int M>
int launch_span(const SpanParams& p, hipStream_t st, int dev) {
  int cus = g_cus[dev].load(std::memory_order_relaxed);
  if (cus == 0) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
      (void)hipGetLastError();
      return fail(PGS_ERR_NO_DEVICE, "pgs_w8a16_decode_span: cannot query device %d", dev);
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, span_kernel<DM, M>, kSpanThreads, 0) != hipSuccess) {
      (void)hipGetLastError();
      per_cu = 0;
    }
    // one resident workgroup per CU, and exactly kSpanG CUs
    cus = (per_cu == 1 && prop.multiProcessorCount == kSpanG) ? prop.multiProcessorCount : -1;
    g_cus[dev].store(cus, std::memory_order_relaxed);
  }
  if (cus != kSpanG)
    return fail(PGS_ERR_INVALID_ARGUMENT,
                "pgs_w8a16_decode_span: the persistent launch needs %d CUs holding one workgroup each", kSpanG);
  note_launch(__PRETTY_FUNCTION__, kSpanG, 1);
  hipLaunchKernelGGL((span_kernel<DM, M>), dim3(kSpanG), dim3(kSpanThreads), 0, st, p);
  return check_launch("w8a16 decode span kernel");
}

int g_spin_limit = 1 << 18;
int g_force_giveup = 0;
unsigned long long* g_trace = nullptr;
int g_trace_slots = 0;

}  // namespace
}  // namespace pgs

using namespace pgs;

extern "C" size_t pgs_w8a16_decode_span_workspace_bytes(int64_t m, int64_t hidden, int64_t inter) {
  if (m < 1 || m > 4 || hidden <= 0 || inter <= 0 || hidden % 8 || inter % 8) return 0;
  return static_cast<size_t>(kHeader) + static_cast<size_t>(2 * hidden / 8 + inter / 8) * kSlot;
}

extern "C" int pgs_w8a16_decode_span_supported(int64_t m, int64_t hidden, int64_t inter, int64_t nq, int64_t nkv,
                                                int64_t head_dim) {
  return (m >= 1 && m <= 4 && hidden == Qwen25_3B::H && inter == Qwen25_3B::I && nq == Qwen25_3B::NQ &&
          nkv == Qwen25_3B::NKV && head_dim == Qwen25_3B::HD)
             ? 1
             : 0;
}

extern "C" int pgs_w8a16_decode_span_test_hooks(int spin_limit, int force_giveup) {
  if (spin_limit < 0) return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_w8a16_decode_span_test_hooks: negative spin limit");
  g_spin_limit = spin_limit == 0 ? (1 << 18) : spin_limit;
  g_force_giveup = force_giveup ? 1 : 0;
  return PGS_OK;
}

extern "C" int pgs_w8a16_decode_span_trace(void* buffer, size_t bytes) {
  constexpr size_t kSlotBytes = static_cast<size_t>(kSpanG) * 16 * sizeof(unsigned long long);
  if (!buffer) {
    g_trace = nullptr;
    g_trace_slots = 0;
    return PGS_OK;
  }
  if (!aligned(buffer, 8) || bytes < kSlotBytes)
    return fail(PGS_ERR_INVALID_ARGUMENT, "pgs_w8a16_decode_span_trace: need an 8-byte aligned buffer of at least %zu bytes",
                kSlotBytes);
  const size_t slots = bytes / kSlotBytes;
  g_trace = static_cast<unsigned long long*>(buffer);
  g_trace_slots = static_cast<int>(slots > 65535 ? 65535 : slots);
  return PGS_OK;
}

extern "C" int pgs_w8a16_decode_span_status(void* workspace, int reset, void* stream) {
  const char* fn = "pgs_w8a16_decode_span_status";
  if (!workspace) return fail(PGS_ERR_INVALID_ARGUMENT, "%s: null workspace", fn);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (int rc = require_device(fn, st)) return rc;
  uint32_t hdr[2] = {0, 0};
  if (hipMemcpyAsync(hdr, workspace, sizeof(hdr), hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess) {
    hipError_t e = hipGetLastError();
    return fail(PGS_ERR_LAUNCH, "%s: reading the workspace header failed: %s", fn, hipGetErrorString(e));
  }
  if (hdr[1] == 0) return PGS_OK;
  if (reset) {
    // the caller passes the size it allocated; the header and exchange
    // buffers start zero again (a kernel fill)
    if (int rc = fill_zero(workspace, static_cast<int64_t>(kHeader) + 2 * (Qwen25_3B::H / 8) * kSlot +
                                          (Qwen25_3B::I / 8) * kSlot, st))
      return rc;
  }
  return fail(PGS_ERR_TIMEOUT, "%s: a decode span launch gave up waiting for another workgroup's outputs", fn);
}

extern "C" int pgs_w8a16_decode_span(const void* attn, const void* residual, void* x_out, const pgs_span_weights* w,
                                     const pgs_span_next* next, float eps, int64_t m, int64_t hidden, int64_t inter,
                                     void* workspace, size_t workspace_bytes_, void* stream) {
  const char* fn = "pgs_w8a16_decode_span";
  if (!w || !attn || !residual || !x_out || !workspace)
    return fail(PGS_ERR_INVALID_ARGUMENT, "%s: null pointer argument", fn);
  const int64_t nq = next ? next->q.n : Qwen25_3B::NQ, nkv = next ? next->k.n : Qwen25_3B::NKV;
  const int64_t hd = next ? next->head_dim : Qwen25_3B::HD;
  if (!pgs_w8a16_decode_span_supported(m, hidden, inter, nq, nkv, hd))
    return fail(PGS_ERR_INVALID_ARGUMENT,
                "%s: no compiled configuration for m=%lld hidden=%lld inter=%lld q=%lld kv=%lld head_dim=%lld "
                "(pgs_w8a16_decode_span_supported)",
                fn, (long long)m, (long long)hidden, (long long)inter, (long long)nq, (long long)nkv, (long long)hd);
  if (next && next->v.n != nkv) return fail(PGS_ERR_INVALID_ARGUMENT, "%s: k and v sizes differ", fn);
  if (workspace_bytes_ < pgs_w8a16_decode_span_workspace_bytes(m, hidden, inter))
    return fail(PGS_ERR_INVALID_ARGUMENT, "%s: workspace of %zu bytes, %zu needed", fn, workspace_bytes_,
                pgs_w8a16_decode_span_workspace_bytes(m, hidden, inter));
  const void* need16[] = {attn, residual, w->qp_o, w->qp_gate, w->qp_up, w->qp_down, w->ln_post};
  for (const void* q : need16)
    if (!q || !aligned(q, 16)) return fail(PGS_ERR_MISALIGNED, "%s: weights, norm weights and activations need 16-byte alignment", fn);
  if (!w->s_o || !w->s_gate || !w->s_up || !w->s_down || !aligned(x_out, 2) || !aligned(workspace, 256))
    return fail(PGS_ERR_INVALID_ARGUMENT, "%s: null scale, misaligned output or workspace", fn);
  SpanParams p{};
  p.attn = static_cast<const uint16_t*>(attn);
  p.resid = static_cast<const uint16_t*>(residual);
  p.x_out = static_cast<uint16_t*>(x_out);
  p.qo = w->qp_o;
  p.so = w->s_o;
  p.ln_post = static_cast<const uint16_t*>(w->ln_post);
  p.qg = w->qp_gate;
  p.sg = w->s_gate;
  p.qu = w->qp_up;
  p.su = w->s_up;
  p.qd = w->qp_down;
  p.sd = w->s_down;
  if (next) {
    const pgs_linear_out* o[3] = {&next->q, &next->k, &next->v};
    if (!next->ln_in || !aligned(next->ln_in, 16))
      return fail(PGS_ERR_MISALIGNED, "%s: the next layer's norm weight must be 16-byte aligned", fn);
    if ((next->cos == nullptr) != (next->sin == nullptr))
      return fail(PGS_ERR_INVALID_ARGUMENT, "%s: cos and sin go together", fn);
    p.ln_next = static_cast<const uint16_t*>(next->ln_in);
    for (int j = 0; j < 3; ++j) {
      if (!o[j]->qp || !o[j]->scale || !o[j]->y || !aligned(o[j]->qp, 16) || !aligned(o[j]->y, 2))
        return fail(PGS_ERR_INVALID_ARGUMENT, "%s: q/k/v output %d lacks a weight, scale or output", fn, j);
      p.qkv[j] = o[j]->qp;
      p.sqkv[j] = o[j]->scale;
      p.bqkv[j] = static_cast<const uint16_t*>(o[j]->bias);
      p.yqkv[j] = static_cast<uint16_t*>(o[j]->y);
    }
    p.cos = static_cast<const uint16_t*>(next->cos);
    p.sin = static_cast<const uint16_t*>(next->sin);
  }
  p.ws = static_cast<uint32_t*>(workspace);
  p.eps = eps;
  p.spin_limit = g_spin_limit;
  p.force_giveup = g_force_giveup;
  p.trace = g_trace;
  p.trace_slots = g_trace_slots;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (int rc = require_device(fn, st)) return rc;
  int dev = -1;
  if (int rc = stream_device(st, &dev)) return rc;
  if (m == 1) return launch_span<Qwen25_3B, 1>(p, st, dev);
  if (m == 2) return launch_span<Qwen25_3B, 2>(p, st, dev);
  if (m == 3) return launch_span<Qwen25_3B, 3>(p, st, dev);
  return launch_span<Qwen25_3B, 4>(p, st, dev);
}
