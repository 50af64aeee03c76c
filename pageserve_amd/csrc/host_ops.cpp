// Host fast path of the linear entry points for PyTorch callers.
//
// pageserve_amd/quantization.py's linear / linear_group / swiglu (and their
// rms_norm and residual forms) run once per projection per token step; the
// reference calls them through F.linear from a runner thread
// (engine/model.py:168-190, engine/runner.py:79).  This module does their
// argument checks, output allocation, device and stream selection and the
// C-ABI call (include/pageserve_amd.h) in C++, so that an eager call costs a
// few microseconds of host time: the same work in Python with ctypes cost
// 10-20 us per call, more than the decode kernels themselves.  It computes
// nothing itself; every result comes from the gfx950 kernels.  Error
// messages and exception types are those of the Python wrappers (ValueError,
// TypeError, RuntimeError).
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/extension.h>

#include <string>
#include <vector>

#include "pageserve_amd.h"

namespace {

using Opt = c10::optional<at::Tensor>;

[[noreturn]] void value_error(const std::string& s) { throw pybind11::value_error(s); }
[[noreturn]] void type_error(const std::string& s) { throw pybind11::type_error(s); }

std::string dev_str(const at::Device& d) { return d.str(); }

void check_rc(int rc, const char* what) {
  if (rc == PGS_OK) return;
  std::string msg = std::string(what) + ": " + pgs_error_string(rc) + ": " + pgs_last_error();
  if (rc == PGS_ERR_INVALID_ARGUMENT || rc == PGS_ERR_MISALIGNED) value_error(msg);
  throw std::runtime_error(msg);
}

// contiguous, data pointer aligned to `align` bytes (copies only if needed)
at::Tensor aligned(const at::Tensor& t, uintptr_t align) {
  at::Tensor c = t.is_contiguous() ? t : t.contiguous();
  if (c.numel() && reinterpret_cast<uintptr_t>(c.data_ptr()) % align) c = c.clone();
  return c;
}

void* ptr(const at::Tensor& t) { return t.numel() ? t.data_ptr() : nullptr; }

// x: bf16 [..., k] on `dev` -> contiguous 16-byte aligned [m, k]
at::Tensor check_x(const at::Tensor& x, int64_t k, const at::Device& dev, const char* what) {
  if (x.device() != dev)
    value_error(std::string(what) + ": input on " + dev_str(x.device()) + " but weight on " + dev_str(dev));
  if (x.scalar_type() != at::kBFloat16)
    type_error(std::string(what) + ": the W8A16 kernels take bf16 activations, got " +
               std::string(c10::toString(x.scalar_type())));
  if (x.dim() < 1 || x.size(-1) != k)
    value_error(std::string(what) + ": input has " + std::to_string(x.dim() ? x.size(-1) : 0) +
                " features, weight expects " + std::to_string(k));
  // (a 2-D input is used as it is: each view op costs a few hundred ns of
  // host time per call)
  return aligned(x.dim() == 2 ? x : x.reshape({-1, k}), 16);
}

std::vector<int64_t> out_shape(const at::Tensor& x, int64_t n) {
  std::vector<int64_t> s(x.sizes().begin(), x.sizes().end() - 1);
  s.push_back(n);
  return s;
}

at::Tensor check_bias(const Opt& b, int64_t n, const at::Device& dev, const char* what) {
  if (!b.has_value() || !b->defined()) return at::Tensor();
  const at::Tensor& t = *b;
  if (t.device() != dev || t.scalar_type() != at::kBFloat16 || t.numel() != n)
    value_error(std::string(what) + ": bias must be a bf16 [" + std::to_string(n) + "] tensor on " + dev_str(dev));
  return aligned(t.dim() == 1 ? t : t.reshape({n}), 2);
}

at::Tensor check_norm(const Opt& w, int64_t k, const at::Device& dev, const char* what) {
  const at::Tensor& t = *w;
  if (t.scalar_type() != at::kBFloat16 || t.numel() != k || t.device() != dev)
    value_error(std::string(what) + ": norm weight must be a bf16 [" + std::to_string(k) + "] tensor on " +
                dev_str(dev));
  return aligned(t.reshape({k}), 16);
}

// One or more projections of the same input (linear, linear_group, and with
// a single member the residual / out forms; norm_w: rms_norm fused in front).
std::vector<at::Tensor> linear(const at::Tensor& x, const std::vector<at::Tensor>& qps,
                               const std::vector<at::Tensor>& scales, const std::vector<Opt>& biases,
                               const std::vector<int64_t>& ns, int64_t k, bool out_f32, const Opt& residual,
                               const Opt& out, const Opt& norm_w, double eps, int64_t ws_ptr, int64_t ws_bytes) {
  const size_t g = qps.size();
  if (g < 1 || g > PGS_MAX_GROUP || scales.size() != g || biases.size() != g || ns.size() != g)
    value_error("linear_group takes 1.." + std::to_string(PGS_MAX_GROUP) + " weights");
  const at::Device dev = qps[0].device();
  const char* what = "linear";
  at::Tensor x2 = check_x(x, k, dev, what);
  const int64_t m = x2.size(0);
  at::Tensor nw;
  if (norm_w.has_value()) nw = check_norm(norm_w, k, dev, "rmsnorm_linear_group");
  const auto odt = out_f32 ? at::kFloat : at::kBFloat16;
  pgs_linear_out outs[PGS_MAX_GROUP];
  std::vector<at::Tensor> ys;
  ys.reserve(g);
  at::Tensor bias_keep[PGS_MAX_GROUP];
  at::Tensor res;
  // a group's outputs are contiguous pieces of one allocation (one call into
  // the caching allocator instead of one per member), each starting on a
  // 64-element boundary (the kernels' vector stores want aligned rows)
  auto piece = [&](size_t i) { return (m * ns[i] + 63) / 64 * 64; };
  at::Tensor flat;
  if (g > 1) {
    int64_t total = 0;
    for (size_t i = 0; i < g; ++i) total += piece(i);
    flat = at::empty({total}, x2.options().dtype(odt));
  }
  int64_t off = 0;
  for (size_t i = 0; i < g; ++i) {
    const int64_t n = ns[i];
    bias_keep[i] = check_bias(biases[i], n, dev, what);
    at::Tensor y;
    if (g > 1) {
      y = flat.as_strided({m, n}, {n, 1}, off);  // (a fresh allocation: storage offset 0)
      off += piece(i);
    } else if (out.has_value()) {
      const at::Tensor& o = *out;
      if (o.device() != dev || o.scalar_type() != odt || o.numel() != m * n || !o.is_contiguous())
        value_error("linear: out must be a contiguous " + std::string(c10::toString(odt)) + " tensor of " +
                    std::to_string(m * n) + " elements on " + dev_str(dev));
      y = o.view({m, n});
    } else {
      y = at::empty({m, n}, x2.options().dtype(odt));
    }
    outs[i] = pgs_linear_out{static_cast<const int8_t*>(ptr(qps[i])), static_cast<const float*>(ptr(scales[i])),
                             bias_keep[i].defined() ? bias_keep[i].data_ptr() : nullptr, ptr(y), n};
    ys.push_back(y);
  }
  if (residual.has_value()) {
    const at::Tensor& r = *residual;
    const int64_t n = ns[0];
    if (r.device() != dev || r.scalar_type() != at::kBFloat16 || r.dim() < 1 || r.size(-1) != n || r.numel() != m * n)
      value_error("linear: residual must be a bf16 [..., " + std::to_string(n) + "] tensor with " + std::to_string(m) +
                  " rows on " + dev_str(dev));
    res = r.reshape({m, n});
    if (!res.is_contiguous()) res = res.contiguous();
  }
  at::hip::HIPGuardMasqueradingAsCUDA guard(dev);
  void* st = at::hip::getCurrentHIPStreamMasqueradingAsCUDA(dev.index()).stream();
  void* ws = reinterpret_cast<void*>(static_cast<uintptr_t>(ws_ptr));
  const int ydt = out_f32 ? PGS_DTYPE_F32 : PGS_DTYPE_BF16;
  int rc;
  if (nw.defined())
    rc = pgs_w8a16_rmsnorm_linear_group(ptr(x2), nw.data_ptr(), static_cast<float>(eps), outs, static_cast<int>(g), ydt,
                                        m, k, ws, static_cast<size_t>(ws_bytes), st);
  else if (res.defined() || out.has_value())
    rc = pgs_w8a16_linear_residual(ptr(x2), outs[0].qp, outs[0].scale, outs[0].bias, res.defined() ? ptr(res) : nullptr,
                                   outs[0].y, ydt, m, ns[0], k, ws, static_cast<size_t>(ws_bytes), st);
  else
    rc = pgs_w8a16_linear_group(ptr(x2), outs, static_cast<int>(g), ydt, m, k, ws, static_cast<size_t>(ws_bytes), st);
  check_rc(rc, "w8a16 linear");
  if (x.dim() != 2)
    for (size_t i = 0; i < g; ++i) ys[i] = ys[i].view(out_shape(x, ns[i]));
  return ys;
}

// One projection (linear and its residual / out forms): the group path
// without the four one-element lists a Python caller would build.
at::Tensor linear1(const at::Tensor& x, const at::Tensor& qp, const at::Tensor& scale, const Opt& bias, int64_t n,
                   int64_t k, bool out_f32, const Opt& residual, const Opt& out, int64_t ws_ptr, int64_t ws_bytes) {
  return linear(x, {qp}, {scale}, {bias}, {n}, k, out_f32, residual, out, c10::nullopt, 0.0, ws_ptr, ws_bytes)[0];
}

// gate / up / silu(gate) * up in one launch (norm_w: rms_norm fused in front)
at::Tensor swiglu(const at::Tensor& x, const at::Tensor& qg, const at::Tensor& sg, const at::Tensor& qu,
                  const at::Tensor& su, int64_t n, int64_t k, const Opt& norm_w, double eps, int64_t ws_ptr,
                  int64_t ws_bytes) {
  const at::Device dev = qg.device();
  at::Tensor x2 = check_x(x, k, dev, "swiglu");
  const int64_t m = x2.size(0);
  at::Tensor nw;
  if (norm_w.has_value()) nw = check_norm(norm_w, k, dev, "rmsnorm_swiglu");
  at::Tensor act = at::empty({m, n}, x2.options());
  at::hip::HIPGuardMasqueradingAsCUDA guard(dev);
  void* st = at::hip::getCurrentHIPStreamMasqueradingAsCUDA(dev.index()).stream();
  void* ws = reinterpret_cast<void*>(static_cast<uintptr_t>(ws_ptr));
  int rc;
  if (nw.defined())
    rc = pgs_w8a16_rmsnorm_swiglu(ptr(x2), nw.data_ptr(), static_cast<float>(eps), static_cast<const int8_t*>(ptr(qg)),
                                  static_cast<const float*>(ptr(sg)), static_cast<const int8_t*>(ptr(qu)),
                                  static_cast<const float*>(ptr(su)), ptr(act), m, n, k, ws,
                                  static_cast<size_t>(ws_bytes), st);
  else
    rc = pgs_w8a16_swiglu(ptr(x2), static_cast<const int8_t*>(ptr(qg)), static_cast<const float*>(ptr(sg)),
                          static_cast<const int8_t*>(ptr(qu)), static_cast<const float*>(ptr(su)), ptr(act), m, n, k,
                          ws, static_cast<size_t>(ws_bytes), st);
  check_rc(rc, "w8a16 swiglu");
  return x.dim() == 2 ? act : act.view(out_shape(x, n));
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, mod) {
  mod.doc() = "C++ host path of pageserve_amd's linear entry points (calls the gfx950 C ABI)";
  mod.def("abi_version", &pgs_abi_version);
  mod.def("linear", &linear, "one or more W8A16 projections of the same input");
  mod.def("linear1", &linear1, "one W8A16 projection");
  mod.def("swiglu", &swiglu, "fused gate/up/silu*up");
}
