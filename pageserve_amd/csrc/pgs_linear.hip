// C entry points of the W8A16 linear path: argument checks, the launch plan
// (skinny kernel for m <= 32, tile GEMM above) and the split-K workspace.
//
// Replaces the reference's per-call "dequantize to a dense weight, then GEMM"
// (engine/quantization.py:26-27 via engine/model.py:25-26 feeding F.linear at
// engine/model.py:168-170, 184, 188-190 and 193).  The int8 weight is read
// once from HBM and widened to bf16 in registers (exact: |q| <= 127); the
// products accumulate in fp32 on the matrix cores; the per-row scale (and
// bias) is applied once per output in the epilogue.
#include "pgs_linear.h"

namespace pgs {
namespace {

constexpr int kSkinnyMaxM = 32;

struct Plan {
  bool skinny;
  SkinnyPlan sk;
  GemmPlan gm;
};

Plan make_plan(int m, int k, int nmat, const int32_t* n, int members, bool can_split) {
  Plan p{};
  p.skinny = m <= kSkinnyMaxM;
  if (p.skinny) {
    int tiles = 0;
    for (int i = 0; i < members; ++i) tiles += (n[i] + 15) / 16;
    p.sk = plan_skinny(m, k, nmat, tiles, can_split);
  } else {
    p.gm = plan_gemm(m, k, nmat, n, members, can_split);
  }
  return p;
}

size_t partial_bytes(const Plan& p, int nmat) {
  return p.skinny ? skinny_partial_bytes(p.sk, nmat) : gemm_partial_bytes(p.gm, nmat);
}

// [pair slots][partials]: the slot region comes first whenever a workspace
// is used at all, so the same buffer serves every call shape.
size_t workspace_bytes(const Plan& p, int nmat) {
  const size_t part = partial_bytes(p, nmat);
  const bool pairs = p.skinny && p.sk.pair;
  return (part || pairs) ? kPairBytes + part : 0;
}

// Offset of the normalised activations in the workspace of a fused-norm
// call that cannot normalise inside the linear kernel: after the linear's own
// workspace, 256-byte aligned, and never inside the pair slots, which a later
// call on the same workspace expects to find empty even when this call's plan
// uses none.
size_t norm_offset(size_t linear_bytes) {
  return (std::max(linear_bytes, kPairBytes) + 255) & ~static_cast<size_t>(255);
}

int run(Problem& p, void* workspace, size_t ws_bytes, hipStream_t st) {
  if (int rc = require_device("w8a16 linear", st)) return rc;
  const int members = (p.nmat == 2) ? 1 : p.args.n_outs;
  const Plan plan = make_plan(p.m, p.k, p.nmat, p.args.n, members, workspace != nullptr);
  const size_t need = workspace_bytes(plan, p.nmat);
  if (p.norm_w && !(plan.skinny && skinny_norm_fusable(plan.sk, p.m, p.k, p.out_f32, p.nmat) && aligned(p.norm_w, 16))) {
    // rms_norm as its own kernel into the workspace, then the plain linear
    const size_t off = norm_offset(need), bytes = static_cast<size_t>(p.m) * p.k * 2;
    if (!workspace || ws_bytes < off + bytes)
      return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16 (rms_norm fused): workspace of %zu bytes, %zu needed", ws_bytes,
                  off + bytes);
    void* h = static_cast<char*>(workspace) + off;
    int rc = pgs_rmsnorm(p.x, p.norm_w, p.eps, h, p.m, p.k, st);
    if (rc) return rc;
    p.x = static_cast<const uint16_t*>(h);
    p.norm_w = nullptr;
    ws_bytes = off;
  }
  if (need > ws_bytes)
    return fail(PGS_ERR_INVALID_ARGUMENT, "w8a16: workspace of %zu bytes is smaller than the %zu this call needs",
                ws_bytes, need);
  if (need) {
    if (!aligned(workspace, 256)) return fail(PGS_ERR_MISALIGNED, "w8a16: workspace must be 256-byte aligned");
    p.pairs = reinterpret_cast<unsigned long long*>(workspace);
    p.partials = reinterpret_cast<float*>(reinterpret_cast<char*>(workspace) + kPairBytes);
    p.partial_bytes = ws_bytes - kPairBytes;
  }
  if (plan.skinny) {
    int tiles = 0;
    for (int i = 0; i < members; ++i) {
      p.args.unit_begin[i] = tiles;
      tiles += (p.args.n[i] + 15) / 16;
    }
    for (int i = members; i <= PGS_MAX_GROUP; ++i) p.args.unit_begin[i] = tiles;
    return launch_skinny(p, plan.sk, st);
  }
  return launch_gemm(p, plan.gm, st);
}

int check_common(const char* fn, const void* x, int64_t m, int64_t k) {
  if (m < 0 || k < 0)
    return fail(PGS_ERR_INVALID_ARGUMENT, "%s: negative size m=%lld k=%lld", fn, (long long)m, (long long)k);
  if (m > 0x7fffffff) return fail(PGS_ERR_INVALID_ARGUMENT, "%s: size too large", fn);
  // (32-bit buffer offsets inside the kernels)
  if (k > kMaxK) return fail(PGS_ERR_INVALID_ARGUMENT, "%s: in_features k=%lld above %d", fn, (long long)k, kMaxK);
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

extern "C" size_t pgs_w8a16_workspace_bytes(int64_t m, const int64_t* n, int n_outs, int64_t k, int swiglu) {
  if (m <= 0 || k <= 0 || !n || n_outs < 1 || n_outs > PGS_MAX_GROUP || m > 0x7fffffff || k > 0x7fffffff) return 0;
  int32_t nn[PGS_MAX_GROUP];
  int members = 0;
  for (int i = 0; i < (swiglu ? 1 : n_outs); ++i) {
    if (n[i] < 0 || n[i] > 0x7fffffff) return 0;
    if (n[i] > 0) nn[members++] = static_cast<int32_t>(n[i]);
  }
  if (members == 0) return 0;
  const int nmat = swiglu ? 2 : 1;
  return workspace_bytes(make_plan(static_cast<int>(m), static_cast<int>(k), nmat, nn, members, true), nmat);
}

extern "C" size_t pgs_w8a16_rmsnorm_workspace_bytes(int64_t m, const int64_t* n, int n_outs, int64_t k, int swiglu) {
  if (m <= 0 || k <= 0 || m > 0x7fffffff || k > 0x7fffffff) return 0;
  const size_t linear = pgs_w8a16_workspace_bytes(m, n, n_outs, k, swiglu);
  return norm_offset(linear) + static_cast<size_t>(m) * static_cast<size_t>(k) * 2;
}

namespace {

// q/k/v-style group of linears on the same activations; res (null or one
// bf16 [m, n] residual per output) is added in the epilogue.
int check_norm(const char* fn, const void* w, float eps, int64_t m, int64_t k) {
  if (m > 0 && k > 0 && !w) return fail(PGS_ERR_INVALID_ARGUMENT, "%s: null norm weight", fn);
  if (!aligned(w, 2)) return fail(PGS_ERR_MISALIGNED, "%s: norm weight misaligned", fn);
  if (!(eps >= 0.f)) return fail(PGS_ERR_INVALID_ARGUMENT, "%s: eps must be >= 0", fn);
  return PGS_OK;
}

int linear_group_impl(const char* fn, const void* x, const pgs_linear_out* outs, const void* const* res, int n_outs,
                      int y_dtype, int64_t m, int64_t k, void* workspace, size_t workspace_bytes_, void* stream,
                      const void* norm_w = nullptr, float eps = 0.f) {
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
  p.norm_w = static_cast<const uint16_t*>(norm_w);
  p.eps = eps;
  int used = 0;
  for (int i = 0; i < n_outs; ++i) {
    rc = check_member(fn, outs[i].qp, outs[i].scale, outs[i].bias, outs[i].y, outs[i].n, m, k);
    if (rc) return rc;
    if (res && outs[i].n > 0 && m > 0 && !res[i])
      return fail(PGS_ERR_INVALID_ARGUMENT, "%s: null residual pointer", fn);
    if (res && !aligned(res[i], 2)) return fail(PGS_ERR_MISALIGNED, "%s: residual misaligned", fn);
    if (outs[i].n == 0) continue;
    p.args.q[used] = outs[i].qp;
    p.args.scale[used] = outs[i].scale;
    p.args.bias[used] = reinterpret_cast<const uint16_t*>(outs[i].bias);
    p.args.y[used] = outs[i].y;
    p.args.res[used] = res ? reinterpret_cast<const uint16_t*>(res[i]) : nullptr;
    p.args.n[used] = static_cast<int32_t>(outs[i].n);
    ++used;
  }
  if (m == 0 || used == 0) return PGS_OK;
  if (k == 0) return fail(PGS_ERR_INVALID_ARGUMENT, "%s: in_features k=0 is not supported", fn);
  p.args.n_outs = used;
  for (int i = used; i < PGS_MAX_GROUP; ++i) {
    p.args.q[i] = p.args.q[0];
    p.args.scale[i] = p.args.scale[0];
    p.args.bias[i] = nullptr;
    p.args.y[i] = p.args.y[0];
    p.args.res[i] = nullptr;
    p.args.n[i] = 0;
  }
  return run(p, workspace, workspace_bytes_, reinterpret_cast<hipStream_t>(stream));
}

}  // namespace

namespace pgs {
int linear_call(const char* fn, const void* x, const pgs_linear_out* outs, int n_outs, int y_dtype, int64_t m,
                int64_t k, void* workspace, size_t workspace_bytes_, void* stream) {
  return linear_group_impl(fn, x, outs, nullptr, n_outs, y_dtype, m, k, workspace, workspace_bytes_, stream);
}
}  // namespace pgs

extern "C" int pgs_w8a16_linear_group(const void* x, const pgs_linear_out* outs, int n_outs, int y_dtype,
                                      int64_t m, int64_t k, void* workspace, size_t workspace_bytes_,
                                      void* stream) {
  return linear_group_impl("pgs_w8a16_linear_group", x, outs, nullptr, n_outs, y_dtype, m, k, workspace,
                           workspace_bytes_, stream);
}

extern "C" int pgs_w8a16_linear(const void* x, const int8_t* q, const float* scale, const void* bias, void* y,
                                int y_dtype, int64_t m, int64_t n, int64_t k, void* workspace,
                                size_t workspace_bytes_, void* stream) {
  pgs_linear_out o{q, scale, bias, y, n};
  return linear_group_impl("pgs_w8a16_linear", x, &o, nullptr, 1, y_dtype, m, k, workspace, workspace_bytes_, stream);
}

extern "C" int pgs_w8a16_linear_residual(const void* x, const int8_t* q, const float* scale, const void* bias,
                                         const void* residual, void* y, int y_dtype, int64_t m, int64_t n, int64_t k,
                                         void* workspace, size_t workspace_bytes_, void* stream) {
  pgs_linear_out o{q, scale, bias, y, n};
  const void* res[1] = {residual};
  return linear_group_impl("pgs_w8a16_linear_residual", x, &o, res, 1, y_dtype, m, k, workspace, workspace_bytes_,
                           stream);
}

namespace {

int swiglu_impl(const char* fn, const void* x, const int8_t* q_gate, const float* s_gate, const int8_t* q_up,
                const float* s_up, void* act, int64_t m, int64_t n, int64_t k, void* workspace,
                size_t workspace_bytes_, void* stream, const void* norm_w, float eps) {
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
  for (int i = 0; i < PGS_MAX_GROUP; ++i) {
    p.args.q[i] = q_gate;
    p.args.scale[i] = s_gate;
    p.args.bias[i] = nullptr;
    p.args.y[i] = act;
    p.args.n[i] = 0;
  }
  p.args.q[1] = q_up;
  p.args.scale[1] = s_up;
  p.args.n[0] = static_cast<int32_t>(n);
  p.args.n[1] = static_cast<int32_t>(n);
  p.norm_w = static_cast<const uint16_t*>(norm_w);
  p.eps = eps;
  return run(p, workspace, workspace_bytes_, reinterpret_cast<hipStream_t>(stream));
}

}  // namespace

extern "C" int pgs_w8a16_swiglu(const void* x, const int8_t* q_gate, const float* s_gate, const int8_t* q_up,
                                const float* s_up, void* act, int64_t m, int64_t n, int64_t k, void* workspace,
                                size_t workspace_bytes_, void* stream) {
  return swiglu_impl("pgs_w8a16_swiglu", x, q_gate, s_gate, q_up, s_up, act, m, n, k, workspace, workspace_bytes_,
                     stream, nullptr, 0.f);
}

extern "C" int pgs_w8a16_rmsnorm_linear_group(const void* x, const void* norm_weight, float eps,
                                              const pgs_linear_out* outs, int n_outs, int y_dtype, int64_t m,
                                              int64_t k, void* workspace, size_t workspace_bytes_, void* stream) {
  const char* fn = "pgs_w8a16_rmsnorm_linear_group";
  int rc = check_norm(fn, norm_weight, eps, m, k);
  if (rc) return rc;
  return linear_group_impl(fn, x, outs, nullptr, n_outs, y_dtype, m, k, workspace, workspace_bytes_, stream,
                           norm_weight, eps);
}

extern "C" int pgs_w8a16_rmsnorm_swiglu(const void* x, const void* norm_weight, float eps, const int8_t* q_gate,
                                        const float* s_gate, const int8_t* q_up, const float* s_up, void* act,
                                        int64_t m, int64_t n, int64_t k, void* workspace, size_t workspace_bytes_,
                                        void* stream) {
  const char* fn = "pgs_w8a16_rmsnorm_swiglu";
  int rc = check_norm(fn, norm_weight, eps, m, k);
  if (rc) return rc;
  return swiglu_impl(fn, x, q_gate, s_gate, q_up, s_up, act, m, n, k, workspace, workspace_bytes_, stream,
                     norm_weight, eps);
}

// ---------------------------------------------------------------------------
// Row argmax of the logits (the greedy next token), without writing them
// ---------------------------------------------------------------------------

namespace pgs {
namespace {

constexpr int kArgmaxMaxM = kSkinnyMaxM;

// One workgroup per token: the maximum of the launch's per-workgroup keys
// (exact and order-free), decoded to the row and its logit.  Each thread
// keeps four loads in flight (a lm_head launch leaves ~19000 keys per token).
constexpr int kArgmaxThreads = 1024;
__global__ __launch_bounds__(kArgmaxThreads) void argmax_reduce_kernel(const unsigned long long* __restrict__ keys,
                                                                       int groups, int M, int64_t* __restrict__ idx,
                                                                       float* __restrict__ vmax) {
  const int mm = blockIdx.x;
  unsigned long long best[4] = {0, 0, 0, 0};
  for (int b0 = threadIdx.x; b0 < groups; b0 += 4 * kArgmaxThreads) {
    unsigned long long k[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int b = b0 + i * kArgmaxThreads;
      k[i] = b < groups ? keys[static_cast<int64_t>(b) * M + mm] : 0ull;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) best[i] = k[i] > best[i] ? k[i] : best[i];
  }
  unsigned long long bb = best[0];
#pragma unroll
  for (int i = 1; i < 4; ++i) bb = best[i] > bb ? best[i] : bb;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t lo = __shfl_xor(static_cast<uint32_t>(bb), off);
    const uint32_t hi = __shfl_xor(static_cast<uint32_t>(bb >> 32), off);
    const unsigned long long other = (static_cast<unsigned long long>(hi) << 32) | lo;
    bb = other > bb ? other : bb;
  }
  __shared__ unsigned long long part[kArgmaxThreads / 64];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = bb;
  __syncthreads();
  if (threadIdx.x != 0) return;
  unsigned long long best_all = part[0];
#pragma unroll
  for (int w = 1; w < kArgmaxThreads / 64; ++w) best_all = part[w] > best_all ? part[w] : best_all;
  const unsigned long long best0 = best_all;
  idx[mm] = static_cast<int64_t>(argmax_key_row(best0));
  if (vmax) vmax[mm] = argmax_key_value(best0);
}

// the argmax call's plan: the fp32 linear's skinny plan without a K split
SkinnyPlan argmax_plan(int m, int n, int k) { return plan_skinny(m, k, 1, (n + 15) / 16, false); }

}  // namespace
}  // namespace pgs

extern "C" size_t pgs_w8a16_argmax_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (m < 1 || m > kArgmaxMaxM || n < 1 || n > 0x7fffffff || k < 1 || k > kMaxK) return 0;
  const SkinnyPlan sp = argmax_plan(static_cast<int>(m), static_cast<int>(n), static_cast<int>(k));
  return static_cast<size_t>(skinny_grid(sp)) * static_cast<size_t>(m) * sizeof(unsigned long long);
}

extern "C" int pgs_w8a16_linear_argmax(const void* x, const int8_t* q, const float* scale, const void* bias,
                                       int64_t* idx, float* vmax, int64_t m, int64_t n, int64_t k, void* workspace,
                                       size_t workspace_bytes_, void* stream) {
  const char* fn = "pgs_w8a16_linear_argmax";
  int rc = check_common(fn, x, m, k);
  if (rc) return rc;
  if (m < 1 || m > kArgmaxMaxM)
    return fail(PGS_ERR_INVALID_ARGUMENT, "%s: m=%lld rows; 1..%d are supported (pass the rows whose argmax is needed)",
                fn, (long long)m, kArgmaxMaxM);
  if (n < 1 || k < 1) return fail(PGS_ERR_INVALID_ARGUMENT, "%s: n=%lld, k=%lld must be positive", fn, (long long)n,
                                  (long long)k);
  rc = check_member(fn, q, scale, bias, idx, n, m, k);
  if (rc) return rc;
  if (!aligned(idx, 8) || !aligned(vmax, 4)) return fail(PGS_ERR_MISALIGNED, "%s: idx / vmax misaligned", fn);
  const size_t need = pgs_w8a16_argmax_workspace_bytes(m, n, k);
  if (!workspace || workspace_bytes_ < need)
    return fail(PGS_ERR_INVALID_ARGUMENT, "%s: workspace of %zu bytes, %zu needed", fn, workspace_bytes_, need);
  if (!aligned(workspace, 8)) return fail(PGS_ERR_MISALIGNED, "%s: workspace must be 8-byte aligned", fn);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if ((rc = require_device(fn, st))) return rc;
  Problem p{};
  p.x = reinterpret_cast<const uint16_t*>(x);
  p.m = static_cast<int>(m);
  p.k = static_cast<int>(k);
  p.nmat = 1;
  p.out_f32 = true;
  p.keys = static_cast<unsigned long long*>(workspace);
  p.args.n_outs = 1;
  for (int i = 0; i < PGS_MAX_GROUP; ++i) {
    p.args.q[i] = q;
    p.args.scale[i] = scale;
    p.args.bias[i] = i == 0 ? reinterpret_cast<const uint16_t*>(bias) : nullptr;
    p.args.y[i] = workspace;  // (not written in this mode)
    p.args.res[i] = nullptr;
    p.args.n[i] = i == 0 ? static_cast<int32_t>(n) : 0;
    p.args.unit_begin[i] = 0;
  }
  const SkinnyPlan sp = argmax_plan(p.m, static_cast<int>(n), p.k);
  for (int i = 1; i <= PGS_MAX_GROUP; ++i) p.args.unit_begin[i] = sp.tiles;
  if ((rc = launch_skinny(p, sp, st))) return rc;
  const int64_t groups = skinny_grid(sp);
  hipLaunchKernelGGL(argmax_reduce_kernel, dim3(static_cast<unsigned>(m)), dim3(kArgmaxThreads), 0, st,
                     static_cast<const unsigned long long*>(workspace), static_cast<int>(groups), p.m, idx, vmax);
  return check_launch("w8a16 argmax reduce kernel");
}
