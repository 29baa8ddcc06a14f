// torch.optim's foreach path and the per-tensor optimizer primitives on the
// PrivateUse1 device: _foreach_{mul,add,div}_ (Scalar / ScalarList / List),
// _foreach_lerp_, _foreach_addcmul_, _foreach_addcdiv_, _foreach_maximum_ /
// minimum_, _foreach_sqrt, and lerp / addcmul / addcdiv / maximum / minimum
// (reference: csrc/ops/optimizer_primitives.cpp:162-202, which registers the
// per-tensor ops; its foreach lists fall to ATen's per-tensor loops).  Every
// list is one multi-tensor launch through mx_foreach_f32.  FP32 device
// tensors only; a strided operand runs on a contiguous device copy (written
// back for outputs), other dtypes or devices go to the CPU and are counted.
#include <ATen/ExpandUtils.h>
#include <ATen/MemoryOverlap.h>
#include <ATen/native/Resize.h>
#include <c10/core/DeviceGuard.h>
#include <torch/library.h>

#include <vector>

#include "common.h"

namespace tvk {
namespace {

bool f32_dev(const at::Tensor& t) { return is_vk(t) && t.scalar_type() == at::kFloat && !t.is_neg() && !t.is_conj(); }

// One list op: out[i] = f(a[i], b[i], c[i], scalar[i]).  `outs` may be `a`
// (in place).  Returns false (nothing done) when an operand is not an FP32
// device tensor of the output's shape.
bool run_lists(int op, const std::vector<at::Tensor>& outs, const std::vector<at::Tensor>& a,
               const std::vector<at::Tensor>& b, const std::vector<at::Tensor>& c,
               const std::vector<double>& scalars) {
  const size_t n = outs.size();
  if (n == 0) return true;
  for (size_t i = 0; i < n; ++i) {
    const auto& o = outs[i];
    if (!f32_dev(o) || !f32_dev(a[i]) || a[i].sizes() != o.sizes() || a[i].device() != outs[0].device()) return false;
    if (!b.empty() && (!f32_dev(b[i]) || b[i].sizes() != o.sizes() || b[i].device() != o.device())) return false;
    if (!c.empty() && (!f32_dev(c[i]) || c[i].sizes() != o.sizes() || c[i].device() != o.device())) return false;
  }
  c10::DeviceGuard guard(outs[0].device());
  std::vector<at::Tensor> keep;  // contiguous copies alive until the launch is queued
  std::vector<std::pair<at::Tensor, at::Tensor>> write_back;
  std::vector<mx_foreach_tensor> ent(n);
  auto dense = [&](const at::Tensor& t) -> const float* {
    if (t.is_contiguous()) return t.data_ptr<float>();
    keep.push_back(t.contiguous());
    return keep.back().data_ptr<float>();
  };
  for (size_t i = 0; i < n; ++i) {
    const at::Tensor& o = outs[i];
    at::assert_no_internal_overlap(o);
    const bool in_place = o.is_same(a[i]);
    float* out;
    const float* pa;
    if (o.is_contiguous()) {
      out = o.data_ptr<float>();
      pa = in_place ? out : dense(a[i]);
    } else {
      at::Tensor tmp = in_place ? o.contiguous() : at::empty(o.sizes(), o.options());
      write_back.emplace_back(o, tmp);
      out = tmp.data_ptr<float>();
      pa = in_place ? out : dense(a[i]);
    }
    ent[i] = mx_foreach_tensor{out, pa, b.empty() ? nullptr : dense(b[i]), c.empty() ? nullptr : dense(c[i]),
                               o.numel(), scalars.size() == 1 ? scalars[0] : scalars[i]};
  }
  int64_t launches = 0;
  TVK_MX(mx_foreach_f32(op, ent.data(), int64_t(n), &launches, current_stream()));
  counters().kernel_launches += uint64_t(launches);
  for (auto& wb : write_back) wb.first.copy_(wb.second);
  return true;
}

std::vector<at::Tensor> vec(at::TensorList l) { return std::vector<at::Tensor>(l.begin(), l.end()); }

std::vector<double> doubles(at::ArrayRef<at::Scalar> s) {
  std::vector<double> d;
  for (const auto& v : s) d.push_back(v.toDouble());
  return d;
}

void check_lists(const char* name, at::TensorList self, std::initializer_list<size_t> others) {
  for (size_t n : others)
    TORCH_CHECK(n == self.size(), name, ": tensor lists must have the same length, got ", self.size(), " and ", n);
}

// Host loop over the CPU kernels for lists the device path does not take.
template <class F>
void host_loop(const char* name, size_t n, F&& f) {
  note_cpu_fallback(name);
  for (size_t i = 0; i < n; ++i) f(i);
}

at::Tensor cpu(const at::Tensor& t) { return t.cpu(); }

// ----------------------------------------------------------------- _foreach
void foreach_mul_scalar_(at::TensorList self, const at::Scalar& s) {
  auto v = vec(self);
  if (run_lists(MX_FOREACH_MUL_SCALAR, v, v, {}, {}, {s.toDouble()})) return;
  host_loop("_foreach_mul_.Scalar", v.size(), [&](size_t i) { v[i].copy_(cpu(v[i]).mul(s)); });
}

void foreach_mul_scalarlist_(at::TensorList self, at::ArrayRef<at::Scalar> s) {
  check_lists("_foreach_mul_", self, {s.size()});
  auto v = vec(self);
  if (run_lists(MX_FOREACH_MUL_SCALAR, v, v, {}, {}, doubles(s))) return;
  host_loop("_foreach_mul_.ScalarList", v.size(), [&](size_t i) { v[i].copy_(cpu(v[i]).mul(s[i])); });
}

std::vector<at::Tensor> foreach_mul_scalar(at::TensorList self, const at::Scalar& s) {
  std::vector<at::Tensor> out;
  for (const auto& t : self) out.push_back(at::empty(t.sizes(), t.options().memory_format(at::MemoryFormat::Contiguous)));
  if (run_lists(MX_FOREACH_MUL_SCALAR, out, vec(self), {}, {}, {s.toDouble()})) return out;
  host_loop("_foreach_mul.Scalar", out.size(), [&](size_t i) { out[i] = cpu(self[i]).mul(s).to(self[i].device()); });
  return out;
}

void foreach_div_scalar_(at::TensorList self, const at::Scalar& s) {
  auto v = vec(self);
  if (run_lists(MX_FOREACH_DIV_SCALAR, v, v, {}, {}, {s.toDouble()})) return;
  host_loop("_foreach_div_.Scalar", v.size(), [&](size_t i) { v[i].copy_(cpu(v[i]).div(s)); });
}

void foreach_div_scalarlist_(at::TensorList self, at::ArrayRef<at::Scalar> s) {
  check_lists("_foreach_div_", self, {s.size()});
  auto v = vec(self);
  if (run_lists(MX_FOREACH_DIV_SCALAR, v, v, {}, {}, doubles(s))) return;
  host_loop("_foreach_div_.ScalarList", v.size(), [&](size_t i) { v[i].copy_(cpu(v[i]).div(s[i])); });
}

void foreach_add_scalarlist_(at::TensorList self, at::ArrayRef<at::Scalar> s) {
  check_lists("_foreach_add_", self, {s.size()});
  auto v = vec(self);
  if (run_lists(MX_FOREACH_ADD_SCALAR, v, v, {}, {}, doubles(s))) return;
  host_loop("_foreach_add_.ScalarList", v.size(), [&](size_t i) { v[i].copy_(cpu(v[i]).add(s[i])); });
}

void foreach_add_list_(at::TensorList self, at::TensorList other, const at::Scalar& alpha) {
  check_lists("_foreach_add_", self, {other.size()});
  auto v = vec(self);
  if (run_lists(MX_FOREACH_ADD_LIST, v, v, vec(other), {}, {alpha.toDouble()})) return;
  host_loop("_foreach_add_.List", v.size(), [&](size_t i) { v[i].copy_(cpu(v[i]).add(cpu(other[i]), alpha)); });
}

std::vector<at::Tensor> foreach_add_list(at::TensorList self, at::TensorList other, const at::Scalar& alpha) {
  check_lists("_foreach_add", self, {other.size()});
  std::vector<at::Tensor> out;
  for (const auto& t : self) out.push_back(at::empty(t.sizes(), t.options().memory_format(at::MemoryFormat::Contiguous)));
  if (run_lists(MX_FOREACH_ADD_LIST, out, vec(self), vec(other), {}, {alpha.toDouble()})) return out;
  host_loop("_foreach_add.List", out.size(),
            [&](size_t i) { out[i] = cpu(self[i]).add(cpu(other[i]), alpha).to(self[i].device()); });
  return out;
}

void foreach_lerp_scalar_(at::TensorList self, at::TensorList end, const at::Scalar& w) {
  check_lists("_foreach_lerp_", self, {end.size()});
  auto v = vec(self);
  if (run_lists(MX_FOREACH_LERP_SCALAR, v, v, vec(end), {}, {w.toDouble()})) return;
  host_loop("_foreach_lerp_.Scalar", v.size(), [&](size_t i) { v[i].copy_(cpu(v[i]).lerp(cpu(end[i]), w)); });
}

void foreach_lerp_list_(at::TensorList self, at::TensorList end, at::TensorList w) {
  check_lists("_foreach_lerp_", self, {end.size(), w.size()});
  auto v = vec(self);
  if (run_lists(MX_FOREACH_LERP_TENSOR, v, v, vec(end), vec(w), {0.0})) return;
  host_loop("_foreach_lerp_.List", v.size(), [&](size_t i) { v[i].copy_(cpu(v[i]).lerp(cpu(end[i]), cpu(w[i]))); });
}

void foreach_addcmul_scalar_(at::TensorList self, at::TensorList t1, at::TensorList t2, const at::Scalar& value) {
  check_lists("_foreach_addcmul_", self, {t1.size(), t2.size()});
  auto v = vec(self);
  if (run_lists(MX_FOREACH_ADDCMUL, v, v, vec(t1), vec(t2), {value.toDouble()})) return;
  host_loop("_foreach_addcmul_.Scalar", v.size(),
            [&](size_t i) { v[i].copy_(cpu(v[i]).addcmul(cpu(t1[i]), cpu(t2[i]), value)); });
}

void foreach_addcmul_scalarlist_(at::TensorList self, at::TensorList t1, at::TensorList t2,
                                 at::ArrayRef<at::Scalar> s) {
  check_lists("_foreach_addcmul_", self, {t1.size(), t2.size(), s.size()});
  auto v = vec(self);
  if (run_lists(MX_FOREACH_ADDCMUL, v, v, vec(t1), vec(t2), doubles(s))) return;
  host_loop("_foreach_addcmul_.ScalarList", v.size(),
            [&](size_t i) { v[i].copy_(cpu(v[i]).addcmul(cpu(t1[i]), cpu(t2[i]), s[i])); });
}

void foreach_addcdiv_scalar_(at::TensorList self, at::TensorList t1, at::TensorList t2, const at::Scalar& value) {
  check_lists("_foreach_addcdiv_", self, {t1.size(), t2.size()});
  auto v = vec(self);
  if (run_lists(MX_FOREACH_ADDCDIV, v, v, vec(t1), vec(t2), {value.toDouble()})) return;
  host_loop("_foreach_addcdiv_.Scalar", v.size(),
            [&](size_t i) { v[i].copy_(cpu(v[i]).addcdiv(cpu(t1[i]), cpu(t2[i]), value)); });
}

void foreach_addcdiv_scalarlist_(at::TensorList self, at::TensorList t1, at::TensorList t2,
                                 at::ArrayRef<at::Scalar> s) {
  check_lists("_foreach_addcdiv_", self, {t1.size(), t2.size(), s.size()});
  auto v = vec(self);
  if (run_lists(MX_FOREACH_ADDCDIV, v, v, vec(t1), vec(t2), doubles(s))) return;
  host_loop("_foreach_addcdiv_.ScalarList", v.size(),
            [&](size_t i) { v[i].copy_(cpu(v[i]).addcdiv(cpu(t1[i]), cpu(t2[i]), s[i])); });
}

void foreach_maximum_list_(at::TensorList self, at::TensorList other) {
  check_lists("_foreach_maximum_", self, {other.size()});
  auto v = vec(self);
  if (run_lists(MX_FOREACH_MAXIMUM, v, v, vec(other), {}, {0.0})) return;
  host_loop("_foreach_maximum_.List", v.size(), [&](size_t i) { v[i].copy_(at::maximum(cpu(v[i]), cpu(other[i]))); });
}

void foreach_minimum_list_(at::TensorList self, at::TensorList other) {
  check_lists("_foreach_minimum_", self, {other.size()});
  auto v = vec(self);
  if (run_lists(MX_FOREACH_MINIMUM, v, v, vec(other), {}, {0.0})) return;
  host_loop("_foreach_minimum_.List", v.size(), [&](size_t i) { v[i].copy_(at::minimum(cpu(v[i]), cpu(other[i]))); });
}

std::vector<at::Tensor> foreach_sqrt(at::TensorList self) {
  std::vector<at::Tensor> out;
  for (const auto& t : self) out.push_back(at::empty(t.sizes(), t.options().memory_format(at::MemoryFormat::Contiguous)));
  if (run_lists(MX_FOREACH_SQRT, out, vec(self), {}, {}, {0.0})) return out;
  host_loop("_foreach_sqrt", out.size(), [&](size_t i) { out[i] = cpu(self[i]).sqrt().to(self[i].device()); });
  return out;
}

void foreach_sqrt_(at::TensorList self) {
  auto v = vec(self);
  if (run_lists(MX_FOREACH_SQRT, v, v, {}, {}, {0.0})) return;
  host_loop("_foreach_sqrt_", v.size(), [&](size_t i) { v[i].copy_(cpu(v[i]).sqrt()); });
}

// ------------------------------------------------------------- per tensor
// a (op) b (op) c with torch's broadcasting, into a fresh output; a list of
// one through the same kernel.
at::Tensor pointwise(const char* name, int op, const at::Tensor& a, const at::Tensor& b, const at::Tensor& c,
                     double s) {
  const bool ok = f32_dev(a) && f32_dev(b) && (!c.defined() || f32_dev(c)) && a.device() == b.device() &&
                  (!c.defined() || c.device() == a.device());
  TORCH_CHECK(ok || !(is_vk(a) && is_vk(b)) || a.scalar_type() != at::kFloat || b.scalar_type() != at::kFloat ||
                  (c.defined() && c.scalar_type() != at::kFloat) || a.device() == b.device(),
              name, ": expected all tensors on the same device");
  at::DimVector shape = at::infer_size_dimvector(a.sizes(), b.sizes());
  if (c.defined()) shape = at::infer_size_dimvector(shape, c.sizes());
  if (!ok) return at::Tensor();
  c10::DeviceGuard guard(a.device());
  at::Tensor out = at::empty(shape, a.options().memory_format(at::MemoryFormat::Contiguous));
  run_lists(op, {out}, {a.expand(shape)}, {b.expand(shape)}, c.defined() ? std::vector<at::Tensor>{c.expand(shape)}
                                                                         : std::vector<at::Tensor>{},
            {s});
  return out;
}

at::Tensor& into(at::Tensor& out, const at::Tensor& r) {
  TORCH_CHECK(out.device() == r.device() && out.scalar_type() == r.scalar_type(), "output device / dtype mismatch");
  at::native::resize_output(out, r.sizes());
  return out.copy_(r);
}

at::Tensor& in_place(at::Tensor& self, const at::Tensor& r) {
  TORCH_CHECK(r.sizes() == self.sizes(), "output with shape ", self.sizes(), " doesn't match the broadcast shape ",
              r.sizes());
  return self.copy_(r);
}

at::Tensor lerp_scalar(const at::Tensor& a, const at::Tensor& e, const at::Scalar& w) {
  at::Tensor r = pointwise("lerp", MX_FOREACH_LERP_SCALAR, a, e, at::Tensor(), w.toDouble());
  if (r.defined()) return r;
  note_cpu_fallback("lerp.Scalar");
  return at::lerp(cpu(a), cpu(e), w).to(a.device());
}

at::Tensor lerp_tensor(const at::Tensor& a, const at::Tensor& e, const at::Tensor& w) {
  at::Tensor r = pointwise("lerp", MX_FOREACH_LERP_TENSOR, a, e, w, 0.0);
  if (r.defined()) return r;
  note_cpu_fallback("lerp.Tensor");
  return at::lerp(cpu(a), cpu(e), cpu(w)).to(a.device());
}

at::Tensor addcmul_vk(const at::Tensor& a, const at::Tensor& t1, const at::Tensor& t2, const at::Scalar& v) {
  at::Tensor r = pointwise("addcmul", MX_FOREACH_ADDCMUL, a, t1, t2, v.toDouble());
  if (r.defined()) return r;
  note_cpu_fallback("addcmul");
  return at::addcmul(cpu(a), cpu(t1), cpu(t2), v).to(a.device());
}

at::Tensor addcdiv_vk(const at::Tensor& a, const at::Tensor& t1, const at::Tensor& t2, const at::Scalar& v) {
  at::Tensor r = pointwise("addcdiv", MX_FOREACH_ADDCDIV, a, t1, t2, v.toDouble());
  if (r.defined()) return r;
  note_cpu_fallback("addcdiv");
  return at::addcdiv(cpu(a), cpu(t1), cpu(t2), v).to(a.device());
}

at::Tensor maximum_vk(const at::Tensor& a, const at::Tensor& b) {
  at::Tensor r = pointwise("maximum", MX_FOREACH_MAXIMUM, a, b, at::Tensor(), 0.0);
  if (r.defined()) return r;
  note_cpu_fallback("maximum");
  return at::maximum(a.device().is_cpu() ? a : cpu(a), b.device().is_cpu() ? b : cpu(b))
      .to(is_vk(a) ? a.device() : b.device());
}

at::Tensor minimum_vk(const at::Tensor& a, const at::Tensor& b) {
  at::Tensor r = pointwise("minimum", MX_FOREACH_MINIMUM, a, b, at::Tensor(), 0.0);
  if (r.defined()) return r;
  note_cpu_fallback("minimum");
  return at::minimum(a.device().is_cpu() ? a : cpu(a), b.device().is_cpu() ? b : cpu(b))
      .to(is_vk(a) ? a.device() : b.device());
}

at::Tensor& lerp_scalar_out(const at::Tensor& a, const at::Tensor& e, const at::Scalar& w, at::Tensor& out) {
  return into(out, lerp_scalar(a, e, w));
}
at::Tensor& lerp_tensor_out(const at::Tensor& a, const at::Tensor& e, const at::Tensor& w, at::Tensor& out) {
  return into(out, lerp_tensor(a, e, w));
}
at::Tensor& lerp_scalar_(at::Tensor& a, const at::Tensor& e, const at::Scalar& w) {
  return in_place(a, lerp_scalar(a, e, w));
}
at::Tensor& lerp_tensor_(at::Tensor& a, const at::Tensor& e, const at::Tensor& w) {
  return in_place(a, lerp_tensor(a, e, w));
}
at::Tensor& addcmul_out(const at::Tensor& a, const at::Tensor& t1, const at::Tensor& t2, const at::Scalar& v,
                        at::Tensor& out) {
  return into(out, addcmul_vk(a, t1, t2, v));
}
at::Tensor& addcmul_(at::Tensor& a, const at::Tensor& t1, const at::Tensor& t2, const at::Scalar& v) {
  return in_place(a, addcmul_vk(a, t1, t2, v));
}
at::Tensor& addcdiv_out(const at::Tensor& a, const at::Tensor& t1, const at::Tensor& t2, const at::Scalar& v,
                        at::Tensor& out) {
  return into(out, addcdiv_vk(a, t1, t2, v));
}
at::Tensor& addcdiv_(at::Tensor& a, const at::Tensor& t1, const at::Tensor& t2, const at::Scalar& v) {
  return in_place(a, addcdiv_vk(a, t1, t2, v));
}
at::Tensor& maximum_out(const at::Tensor& a, const at::Tensor& b, at::Tensor& out) { return into(out, maximum_vk(a, b)); }
at::Tensor& minimum_out(const at::Tensor& a, const at::Tensor& b, at::Tensor& out) { return into(out, minimum_vk(a, b)); }

}  // namespace
}  // namespace tvk

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("_foreach_mul_.Scalar", TORCH_FN(tvk::foreach_mul_scalar_));
  m.impl("_foreach_mul_.ScalarList", TORCH_FN(tvk::foreach_mul_scalarlist_));
  m.impl("_foreach_mul.Scalar", TORCH_FN(tvk::foreach_mul_scalar));
  m.impl("_foreach_div_.Scalar", TORCH_FN(tvk::foreach_div_scalar_));
  m.impl("_foreach_div_.ScalarList", TORCH_FN(tvk::foreach_div_scalarlist_));
  m.impl("_foreach_add_.ScalarList", TORCH_FN(tvk::foreach_add_scalarlist_));
  m.impl("_foreach_add_.List", TORCH_FN(tvk::foreach_add_list_));
  m.impl("_foreach_add.List", TORCH_FN(tvk::foreach_add_list));
  m.impl("_foreach_lerp_.Scalar", TORCH_FN(tvk::foreach_lerp_scalar_));
  m.impl("_foreach_lerp_.List", TORCH_FN(tvk::foreach_lerp_list_));
  m.impl("_foreach_addcmul_.Scalar", TORCH_FN(tvk::foreach_addcmul_scalar_));
  m.impl("_foreach_addcmul_.ScalarList", TORCH_FN(tvk::foreach_addcmul_scalarlist_));
  m.impl("_foreach_addcdiv_.Scalar", TORCH_FN(tvk::foreach_addcdiv_scalar_));
  m.impl("_foreach_addcdiv_.ScalarList", TORCH_FN(tvk::foreach_addcdiv_scalarlist_));
  m.impl("_foreach_maximum_.List", TORCH_FN(tvk::foreach_maximum_list_));
  m.impl("_foreach_minimum_.List", TORCH_FN(tvk::foreach_minimum_list_));
  m.impl("_foreach_sqrt", TORCH_FN(tvk::foreach_sqrt));
  m.impl("_foreach_sqrt_", TORCH_FN(tvk::foreach_sqrt_));
  m.impl("lerp.Scalar", TORCH_FN(tvk::lerp_scalar));
  m.impl("lerp.Tensor", TORCH_FN(tvk::lerp_tensor));
  m.impl("lerp.Scalar_out", TORCH_FN(tvk::lerp_scalar_out));
  m.impl("lerp.Tensor_out", TORCH_FN(tvk::lerp_tensor_out));
  m.impl("lerp_.Scalar", TORCH_FN(tvk::lerp_scalar_));
  m.impl("lerp_.Tensor", TORCH_FN(tvk::lerp_tensor_));
  m.impl("addcmul", TORCH_FN(tvk::addcmul_vk));
  m.impl("addcmul.out", TORCH_FN(tvk::addcmul_out));
  m.impl("addcmul_", TORCH_FN(tvk::addcmul_));
  m.impl("addcdiv", TORCH_FN(tvk::addcdiv_vk));
  m.impl("addcdiv.out", TORCH_FN(tvk::addcdiv_out));
  m.impl("addcdiv_", TORCH_FN(tvk::addcdiv_));
  m.impl("maximum", TORCH_FN(tvk::maximum_vk));
  m.impl("maximum.out", TORCH_FN(tvk::maximum_out));
  m.impl("minimum", TORCH_FN(tvk::minimum_vk));
  m.impl("minimum.out", TORCH_FN(tvk::minimum_out));
}
