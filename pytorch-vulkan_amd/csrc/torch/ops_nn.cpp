// Normalisation, activation, resampling, softmax, loss and concatenation
// operators of the C3/C4 training steps on the PrivateUse1 device:
//   native_group_norm(+_backward)      csrc/ops/group_norm.cpp:73-160
//   native_batch_norm(+_backward) and
//   the _native_batch_norm_legit forms csrc/ops/batch_norm.cpp:21-125
//   silu / silu_backward               csrc/ops/diffusion_unary.cpp:143-166
//   relu / threshold_backward          csrc/ops/mm.cpp:475-495, :1096-1097
//   upsample_nearest2d(+_backward)     csrc/ops/upsample.cpp:33-62
//   _softmax / _softmax_backward_data  csrc/ops/mm.cpp:1100,
//                                      csrc/ops/softmax_axis_backward.cpp:11-43
//   mse_loss(+_backward)               csrc/ops/loss_primitives.cpp:349-364
//   cat                                csrc/ops/cat.cpp:8-64
// FP32 operands are packed to contiguous tensors on the device (the
// reference's packed()) and run through the C ABI; other dtypes go to the CPU
// and are counted as fallbacks, as the reference does.
#include <ATen/MemoryOverlap.h>
#include <ATen/WrapDimUtils.h>
#include <ATen/native/Resize.h>
#include <c10/core/DeviceGuard.h>
#include <torch/library.h>

#include <array>
#include <optional>
#include <tuple>
#include <vector>

#include "common.h"

namespace tvk {
namespace {

using OptT = std::optional<at::Tensor>;

bool present(const OptT& t) { return t.has_value() && t->defined(); }

bool f32_dev(const at::Tensor& t) { return is_vk(t) && t.scalar_type() == at::kFloat && !t.is_neg() && !t.is_conj(); }

// Contiguous FP32 device operand (a copy when the view is strided or offset
// from a 16-byte boundary is fine: the kernels check alignment themselves).
at::Tensor packed(const at::Tensor& t) { return t.is_contiguous() ? t : t.contiguous(); }

const float* cptr(const at::Tensor& t) { return t.defined() ? t.data_ptr<float>() : nullptr; }

OptT to_cpu(const OptT& t) { return present(t) ? OptT(t->cpu()) : OptT(); }
at::Tensor to_dev(const at::Tensor& t, const at::Device& d) { return t.defined() ? t.to(d) : t; }

void launched(int n = 1) { counters().kernel_launches += uint64_t(n); }

// ---------------------------------------------------------------- GroupNorm
std::tuple<at::Tensor, at::Tensor, at::Tensor> native_group_norm_vk(const at::Tensor& x, const OptT& weight,
                                                                 const OptT& bias, c10::SymInt N_, c10::SymInt C_,
                                                                 c10::SymInt HxW_, int64_t group, double eps) {
  const int64_t n = N_.expect_int(), c = C_.expect_int(), hw = HxW_.expect_int();
  TORCH_CHECK(group > 0 && n >= 0 && c > 0 && c % group == 0,
              "native_group_norm: invalid batch, channel, group or spatial dimensions");
  TORCH_CHECK(!present(weight) || weight->numel() == c, "native_group_norm: weight must have C elements");
  TORCH_CHECK(!present(bias) || bias->numel() == c, "native_group_norm: bias must have C elements");
  const bool ok = f32_dev(x) && hw > 0 && n * c * hw == x.numel() && (!present(weight) || f32_dev(*weight)) &&
                  (!present(bias) || f32_dev(*bias));
  if (!ok) {
    note_cpu_fallback("native_group_norm (non-FP32 / empty plane)");
    auto r = at::native_group_norm(x.cpu(), to_cpu(weight), to_cpu(bias), n, c, hw, group, eps);
    return {to_dev(std::get<0>(r), x.device()), to_dev(std::get<1>(r), x.device()), to_dev(std::get<2>(r), x.device())};
  }
  c10::DeviceGuard guard(x.device());
  at::Tensor xc = packed(x);
  at::Tensor wc = present(weight) ? packed(*weight) : at::Tensor();
  at::Tensor bc = present(bias) ? packed(*bias) : at::Tensor();
  at::Tensor y = at::empty(x.sizes(), x.options().memory_format(at::MemoryFormat::Contiguous));
  at::Tensor mean = at::empty({n, group}, x.options());
  at::Tensor rstd = at::empty({n, group}, x.options());
  if (n == 0) return {y, mean, rstd};
  TVK_MX(mx_group_norm_forward(xc.data_ptr<float>(), cptr(wc), cptr(bc), n, c, hw, group, float(eps),
                               y.data_ptr<float>(), mean.data_ptr<float>(), rstd.data_ptr<float>(),
                               current_stream()));
  launched(3);
  return {y, mean, rstd};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> native_group_norm_backward_vk(
    const at::Tensor& dy, const at::Tensor& x, const at::Tensor& mean, const at::Tensor& rstd, const OptT& weight,
    c10::SymInt N_, c10::SymInt C_, c10::SymInt HxW_, int64_t group, std::array<bool, 3> mask) {
  const int64_t n = N_.expect_int(), c = C_.expect_int(), hw = HxW_.expect_int();
  TORCH_CHECK(group > 0 && n >= 0 && c > 0 && c % group == 0, "native_group_norm_backward: invalid geometry");
  TORCH_CHECK(dy.sizes() == x.sizes() && mean.numel() == n * group && rstd.numel() == n * group,
              "native_group_norm_backward: input and saved statistic shape mismatch");
  TORCH_CHECK(!present(weight) || weight->numel() == c, "native_group_norm_backward: invalid gamma");
  const bool ok = f32_dev(dy) && f32_dev(x) && f32_dev(mean) && f32_dev(rstd) && hw > 0 &&
                  (!present(weight) || f32_dev(*weight));
  if (!ok) {
    note_cpu_fallback("native_group_norm_backward (non-FP32 / empty plane)");
    auto r = at::native_group_norm_backward(dy.cpu(), x.cpu(), mean.cpu(), rstd.cpu(), to_cpu(weight), n, c, hw,
                                            group, mask);
    return {to_dev(std::get<0>(r), x.device()), to_dev(std::get<1>(r), x.device()), to_dev(std::get<2>(r), x.device())};
  }
  c10::DeviceGuard guard(x.device());
  at::Tensor dx, dw, db;
  if (mask[0]) dx = at::empty(x.sizes(), x.options().memory_format(at::MemoryFormat::Contiguous));
  if (mask[1]) dw = at::empty({c}, x.options());
  if (mask[2]) db = at::empty({c}, x.options());
  if (!mask[0] && !mask[1] && !mask[2]) return {dx, dw, db};
  at::Tensor dyc = packed(dy), xc = packed(x), mc = packed(mean), rc = packed(rstd);
  at::Tensor wc = present(weight) ? packed(*weight) : at::Tensor();
  TVK_MX(mx_group_norm_backward(dyc.data_ptr<float>(), xc.data_ptr<float>(), mc.data_ptr<float>(),
                                rc.data_ptr<float>(), cptr(wc), n, c, hw, group,
                                mask[0] ? dx.data_ptr<float>() : nullptr, mask[1] ? dw.data_ptr<float>() : nullptr,
                                mask[2] ? db.data_ptr<float>() : nullptr, current_stream()));
  launched(4);
  return {dx, dw, db};
}

// ---------------------------------------------------------------- BatchNorm
std::tuple<at::Tensor, at::Tensor, at::Tensor> batch_norm_impl(const at::Tensor& x, const OptT& weight,
                                                               const OptT& bias, const OptT& running_mean,
                                                               const OptT& running_var, bool training,
                                                               double momentum, double eps) {
  TORCH_CHECK(x.dim() >= 2, "Vulkan BatchNorm requires an input of rank 2 or more");
  const int64_t n = x.size(0), c = x.size(1);
  TORCH_CHECK(training || (present(running_mean) && present(running_var)),
              "Vulkan BatchNorm evaluation requires running statistics");
  for (const OptT* t : {&weight, &bias, &running_mean, &running_var})
    TORCH_CHECK(!present(*t) || ((*t)->dim() == 1 && (*t)->numel() == c), "Vulkan BatchNorm expects a channel vector");
  bool ok = f32_dev(x) && x.numel() > 0;
  for (const OptT* t : {&weight, &bias, &running_mean, &running_var}) ok = ok && (!present(*t) || f32_dev(**t));
  if (!ok) {
    note_cpu_fallback("native_batch_norm (non-FP32 / empty)");
    OptT rm = to_cpu(running_mean), rv = to_cpu(running_var);
    auto r = at::native_batch_norm(x.cpu(), to_cpu(weight), to_cpu(bias), rm, rv, training, momentum, eps);
    if (present(running_mean)) const_cast<at::Tensor&>(*running_mean).copy_(*rm);
    if (present(running_var)) const_cast<at::Tensor&>(*running_var).copy_(*rv);
    return {to_dev(std::get<0>(r), x.device()), to_dev(std::get<1>(r), x.device()), to_dev(std::get<2>(r), x.device())};
  }
  c10::DeviceGuard guard(x.device());
  const int64_t hw = x.numel() / (n * c);
  at::Tensor xc = packed(x);
  at::Tensor wc = present(weight) ? packed(*weight) : at::Tensor();
  at::Tensor bc = present(bias) ? packed(*bias) : at::Tensor();
  at::Tensor y = at::empty(x.sizes(), x.options().memory_format(at::MemoryFormat::Contiguous));
  at::Tensor save_mean = at::empty({training ? c : 0}, x.options());
  at::Tensor save_inv = at::empty({training ? c : 0}, x.options());
  float* rm = present(running_mean) ? storage_f32(*running_mean) + running_mean->storage_offset() : nullptr;
  float* rv = present(running_var) ? storage_f32(*running_var) + running_var->storage_offset() : nullptr;
  TVK_MX(mx_batch_norm_forward(xc.data_ptr<float>(), cptr(wc), cptr(bc), rm,
                               present(running_mean) ? running_mean->stride(0) : 0, rv,
                               present(running_var) ? running_var->stride(0) : 0, n, c, hw, training ? 1 : 0,
                               float(momentum), float(eps), y.data_ptr<float>(),
                               training ? save_mean.data_ptr<float>() : nullptr,
                               training ? save_inv.data_ptr<float>() : nullptr, current_stream()));
  launched(training ? 3 : 2);
  return {y, save_mean, save_inv};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> native_batch_norm_vk(const at::Tensor& x, const OptT& weight,
                                                                 const OptT& bias, const OptT& running_mean,
                                                                 const OptT& running_var, bool training,
                                                                 double momentum, double eps) {
  return batch_norm_impl(x, weight, bias, running_mean, running_var, training, momentum, eps);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> batch_norm_legit(const at::Tensor& x, const OptT& weight,
                                                                const OptT& bias, at::Tensor& running_mean,
                                                                at::Tensor& running_var, bool training,
                                                                double momentum, double eps) {
  return batch_norm_impl(x, weight, bias, running_mean, running_var, training, momentum, eps);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> batch_norm_legit_no_stats(const at::Tensor& x, const OptT& weight,
                                                                         const OptT& bias, bool training,
                                                                         double momentum, double eps) {
  return batch_norm_impl(x, weight, bias, std::nullopt, std::nullopt, training, momentum, eps);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> batch_norm_legit_no_training(const at::Tensor& x, const OptT& weight,
                                                                            const OptT& bias,
                                                                            const at::Tensor& running_mean,
                                                                            const at::Tensor& running_var,
                                                                            double momentum, double eps) {
  return batch_norm_impl(x, weight, bias, running_mean, running_var, false, momentum, eps);
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> native_batch_norm_backward_vk(
    const at::Tensor& dy, const at::Tensor& x, const OptT& weight, const OptT& running_mean, const OptT& running_var,
    const OptT& save_mean, const OptT& save_invstd, bool train, double eps, std::array<bool, 3> mask) {
  TORCH_CHECK(x.dim() >= 2 && dy.sizes() == x.sizes(), "Vulkan BatchNorm gradient shape mismatch");
  const int64_t n = x.size(0), c = x.size(1);
  const OptT& mean = train ? save_mean : running_mean;
  const OptT& inv = train ? save_invstd : running_var;
  TORCH_CHECK(present(mean) && present(inv), "Vulkan BatchNorm backward requires statistics");
  TORCH_CHECK(mean->numel() == c && inv->numel() == c && (!present(weight) || weight->numel() == c),
              "Vulkan BatchNorm expects channel vectors");
  const bool ok = f32_dev(dy) && f32_dev(x) && x.numel() > 0 && f32_dev(*mean) && f32_dev(*inv) &&
                  (!present(weight) || f32_dev(*weight));
  if (!ok) {
    note_cpu_fallback("native_batch_norm_backward (non-FP32 / empty)");
    auto r = at::native_batch_norm_backward(dy.cpu(), x.cpu(), to_cpu(weight), to_cpu(running_mean),
                                            to_cpu(running_var), to_cpu(save_mean), to_cpu(save_invstd), train, eps,
                                            mask);
    return {to_dev(std::get<0>(r), x.device()), to_dev(std::get<1>(r), x.device()), to_dev(std::get<2>(r), x.device())};
  }
  c10::DeviceGuard guard(x.device());
  at::Tensor dx, dw, db;
  if (mask[0]) dx = at::empty(x.sizes(), x.options().memory_format(at::MemoryFormat::Contiguous));
  if (mask[1]) dw = at::empty({c}, x.options());
  if (mask[2]) db = at::empty({c}, x.options());
  if (!mask[0] && !mask[1] && !mask[2]) return {dx, dw, db};
  const int64_t hw = x.numel() / (n * c);
  at::Tensor dyc = packed(dy), xc = packed(x), mc = packed(*mean), ic = packed(*inv);
  at::Tensor wc = present(weight) ? packed(*weight) : at::Tensor();
  TVK_MX(mx_batch_norm_backward(dyc.data_ptr<float>(), xc.data_ptr<float>(), cptr(wc), mc.data_ptr<float>(),
                                ic.data_ptr<float>(), n, c, hw, train ? 1 : 0, float(eps),
                                mask[0] ? dx.data_ptr<float>() : nullptr, mask[1] ? dw.data_ptr<float>() : nullptr,
                                mask[2] ? db.data_ptr<float>() : nullptr, current_stream()));
  launched(mask[0] ? 3 : 2);
  return {dx, dw, db};
}

// ---------------------------------------------------------------- pointwise
at::Tensor unary(const at::Tensor& x, int op) {
  c10::DeviceGuard guard(x.device());
  at::Tensor xc = packed(x);
  at::Tensor y = at::empty(x.sizes(), x.options().memory_format(at::MemoryFormat::Contiguous));
  TVK_MX(mx_unary_f32(op, xc.data_ptr<float>(), y.data_ptr<float>(), y.numel(), current_stream()));
  launched();
  return y;
}

at::Tensor silu_vk(const at::Tensor& x) {
  if (!f32_dev(x)) {
    note_cpu_fallback("silu (non-FP32)");
    return at::silu(x.cpu()).to(x.device());
  }
  return unary(x, MX_UNARY_SILU);
}

at::Tensor& silu_out(const at::Tensor& x, at::Tensor& out) {
  at::Tensor r = silu_vk(x);
  at::native::resize_output(out, r.sizes());
  return out.copy_(r);
}

at::Tensor& silu_(at::Tensor& x) {
  if (f32_dev(x) && x.is_contiguous()) {
    c10::DeviceGuard guard(x.device());
    TVK_MX(mx_unary_f32(MX_UNARY_SILU, x.data_ptr<float>(), x.data_ptr<float>(), x.numel(), current_stream()));
    launched();
    return x;
  }
  return x.copy_(silu_vk(x));
}

at::Tensor silu_backward_vk(const at::Tensor& dy, const at::Tensor& x) {
  if (!f32_dev(dy) || !f32_dev(x)) {
    note_cpu_fallback("silu_backward (non-FP32)");
    return at::silu_backward(dy.cpu(), x.cpu()).to(x.device());
  }
  TORCH_CHECK(dy.sizes() == x.sizes(), "silu_backward: gradient / input shape mismatch");
  c10::DeviceGuard guard(x.device());
  at::Tensor dyc = packed(dy), xc = packed(x);
  at::Tensor dx = at::empty(x.sizes(), x.options().memory_format(at::MemoryFormat::Contiguous));
  TVK_MX(mx_unary_backward_f32(MX_UNARY_SILU_GRAD, dyc.data_ptr<float>(), xc.data_ptr<float>(), 0.f,
                               dx.data_ptr<float>(), dx.numel(), current_stream()));
  launched();
  return dx;
}

at::Tensor& silu_backward_out(const at::Tensor& dy, const at::Tensor& x, at::Tensor& out) {
  at::Tensor r = silu_backward_vk(dy, x);
  at::native::resize_output(out, r.sizes());
  return out.copy_(r);
}

at::Tensor relu_vk(const at::Tensor& x) {
  if (!f32_dev(x)) {
    note_cpu_fallback("relu (non-FP32)");
    return at::relu(x.cpu()).to(x.device());
  }
  return unary(x, MX_UNARY_RELU);
}

at::Tensor& relu_(at::Tensor& x) {
  if (f32_dev(x) && x.is_contiguous()) {
    c10::DeviceGuard guard(x.device());
    TVK_MX(mx_unary_f32(MX_UNARY_RELU, x.data_ptr<float>(), x.data_ptr<float>(), x.numel(), current_stream()));
    launched();
    return x;
  }
  return x.copy_(relu_vk(x));
}

at::Tensor threshold_backward_vk(const at::Tensor& dy, const at::Tensor& x, const at::Scalar& threshold) {
  if (!f32_dev(dy) || !f32_dev(x)) {
    note_cpu_fallback("threshold_backward (non-FP32)");
    return at::threshold_backward(dy.cpu(), x.cpu(), threshold).to(x.device());
  }
  TORCH_CHECK(dy.sizes() == x.sizes(), "threshold_backward requires identical gradient/output shapes");
  c10::DeviceGuard guard(x.device());
  at::Tensor dyc = packed(dy), xc = packed(x);
  at::Tensor dx = at::empty(x.sizes(), x.options().memory_format(at::MemoryFormat::Contiguous));
  TVK_MX(mx_unary_backward_f32(MX_UNARY_THRESHOLD_GRAD, dyc.data_ptr<float>(), xc.data_ptr<float>(),
                               threshold.toFloat(), dx.data_ptr<float>(), dx.numel(), current_stream()));
  launched();
  return dx;
}

// ----------------------------------------------------------- nearest resize
at::Tensor upsample_nearest2d_vk(const at::Tensor& x, c10::SymIntArrayRef size, std::optional<double> sh,
                              std::optional<double> sw) {
  TORCH_CHECK(x.dim() == 4 && size.size() == 2, "Vulkan nearest2d requires rank 4 input and two output sizes");
  const int64_t oh = size[0].expect_int(), ow = size[1].expect_int();
  TORCH_CHECK(x.size(1) > 0 && x.size(2) > 0 && x.size(3) > 0 && oh > 0 && ow > 0,
              "Vulkan nearest2d requires positive channels and spatial dimensions");
  if (!f32_dev(x)) {
    note_cpu_fallback("upsample_nearest2d (non-FP32)");
    return at::upsample_nearest2d(x.cpu(), {oh, ow}, sh, sw).to(x.device());
  }
  c10::DeviceGuard guard(x.device());
  at::Tensor y = at::empty({x.size(0), x.size(1), oh, ow}, x.options());
  if (y.numel() == 0) return y;
  at::Tensor xc = packed(x);
  TVK_MX(mx_upsample_nearest2d(xc.data_ptr<float>(), x.size(0) * x.size(1), x.size(2), x.size(3), oh, ow,
                               sh.value_or(0.0), sw.value_or(0.0), y.data_ptr<float>(), current_stream()));
  launched();
  return y;
}

at::Tensor upsample_nearest2d_backward_vk(const at::Tensor& dy, c10::SymIntArrayRef size, c10::SymIntArrayRef input_size,
                                       std::optional<double> sh, std::optional<double> sw) {
  TORCH_CHECK(size.size() == 2 && input_size.size() == 4, "Vulkan nearest2d backward: bad sizes");
  std::vector<int64_t> in;
  for (const auto& d : input_size) in.push_back(d.expect_int());
  const int64_t oh = size[0].expect_int(), ow = size[1].expect_int();
  TORCH_CHECK(dy.dim() == 4 && dy.size(0) == in[0] && dy.size(1) == in[1] && dy.size(2) == oh && dy.size(3) == ow,
              "Vulkan nearest2d gradient shape mismatch");
  TORCH_CHECK(in[1] > 0 && in[2] > 0 && in[3] > 0 && oh > 0 && ow > 0,
              "Vulkan nearest2d requires positive channels and spatial dimensions");
  if (!f32_dev(dy)) {
    note_cpu_fallback("upsample_nearest2d_backward (non-FP32)");
    return at::upsample_nearest2d_backward(dy.cpu(), {oh, ow}, in, sh, sw).to(dy.device());
  }
  c10::DeviceGuard guard(dy.device());
  at::Tensor dx = at::empty(in, dy.options());
  if (dx.numel() == 0) return dx;
  at::Tensor dyc = packed(dy);
  TVK_MX(mx_upsample_nearest2d_backward(dyc.data_ptr<float>(), in[0] * in[1], in[2], in[3], oh, ow,
                                        sh.value_or(0.0), sw.value_or(0.0), dx.data_ptr<float>(), current_stream()));
  launched();
  return dx;
}

// ------------------------------------------------------------------ softmax
void axis_split(const at::Tensor& t, int64_t dim, int64_t& outer, int64_t& axis, int64_t& inner) {
  outer = 1;
  inner = 1;
  axis = t.dim() ? t.size(dim) : 1;
  for (int64_t d = 0; d < t.dim(); ++d) {
    if (d < dim) outer *= t.size(d);
    if (d > dim) inner *= t.size(d);
  }
}

at::Tensor softmax_vk(const at::Tensor& x, int64_t dim, bool half_to_float) {
  const int64_t d = at::maybe_wrap_dim(dim, x.dim());
  if (!f32_dev(x) || half_to_float) {
    note_cpu_fallback("_softmax (non-FP32)");
    return at::_softmax(x.cpu(), dim, half_to_float).to(x.device());
  }
  c10::DeviceGuard guard(x.device());
  at::Tensor y = at::empty(x.sizes(), x.options().memory_format(at::MemoryFormat::Contiguous));
  if (y.numel() == 0) return y;
  at::Tensor xc = packed(x);
  int64_t outer, axis, inner;
  axis_split(xc, d, outer, axis, inner);
  TVK_MX(mx_softmax_f32(xc.data_ptr<float>(), outer, axis, inner, y.data_ptr<float>(), current_stream()));
  launched();
  return y;
}

at::Tensor softmax_backward_data_vk(const at::Tensor& dy, const at::Tensor& y, int64_t dim, at::ScalarType input_dtype) {
  TORCH_CHECK(dy.sizes() == y.sizes() && dy.device() == y.device(),
              "Vulkan softmax backward: grad/output shape or device mismatch");
  const int64_t d = at::maybe_wrap_dim(dim, y.dim());
  if (!f32_dev(dy) || !f32_dev(y) || input_dtype != at::kFloat) {
    note_cpu_fallback("_softmax_backward_data (non-FP32)");
    return at::_softmax_backward_data(dy.cpu(), y.cpu(), dim, input_dtype).to(y.device());
  }
  c10::DeviceGuard guard(y.device());
  at::Tensor dx = at::empty(y.sizes(), y.options().memory_format(at::MemoryFormat::Contiguous));
  if (dx.numel() == 0) return dx;
  at::Tensor dyc = packed(dy), yc = packed(y);
  int64_t outer, axis, inner;
  axis_split(yc, d, outer, axis, inner);
  TVK_MX(mx_softmax_backward_f32(dyc.data_ptr<float>(), yc.data_ptr<float>(), outer, axis, inner,
                                 dx.data_ptr<float>(), current_stream()));
  launched();
  return dx;
}

// ------------------------------------------------------------------ MSE loss
at::Tensor mse_loss_vk(const at::Tensor& x, const at::Tensor& target, int64_t reduction) {
  TORCH_CHECK(reduction >= 0 && reduction <= 2, "mse_loss: invalid reduction");
  if (!f32_dev(x) || !f32_dev(target) || x.device() != target.device()) {
    note_cpu_fallback("mse_loss (non-FP32)");
    return at::mse_loss(x.cpu(), target.cpu(), reduction).to(x.device());
  }
  c10::DeviceGuard guard(x.device());
  const auto shape = at::infer_size(x.sizes(), target.sizes());
  at::Tensor xc = packed(x.expand(shape)), tc = packed(target.expand(shape));
  const int64_t count = xc.numel();
  at::Tensor out = reduction == 0 ? at::empty(shape, x.options()) : at::empty({}, x.options());
  TVK_MX(mx_mse_loss_f32(xc.data_ptr<float>(), tc.data_ptr<float>(), count, int(reduction), out.data_ptr<float>(),
                         current_stream()));
  launched(reduction == 0 ? 1 : 2);
  return out;
}

at::Tensor mse_loss_backward_vk(const at::Tensor& dy, const at::Tensor& x, const at::Tensor& target,
                             int64_t reduction) {
  TORCH_CHECK(reduction >= 0 && reduction <= 2, "mse_loss_backward: invalid reduction");
  if (!f32_dev(dy) || !f32_dev(x) || !f32_dev(target)) {
    note_cpu_fallback("mse_loss_backward (non-FP32)");
    return at::mse_loss_backward(dy.cpu(), x.cpu(), target.cpu(), reduction).to(x.device());
  }
  c10::DeviceGuard guard(x.device());
  const auto shape = at::infer_size(x.sizes(), target.sizes());
  at::Tensor xc = packed(x.expand(shape)), tc = packed(target.expand(shape));
  at::Tensor g = reduction == 0 ? packed(dy.expand(shape)) : packed(dy);
  TORCH_CHECK(reduction == 0 || g.numel() == 1, "mse_loss_backward: reduced loss needs a scalar gradient");
  at::Tensor dx = at::empty(shape, x.options());
  TVK_MX(mx_mse_loss_backward_f32(g.data_ptr<float>(), xc.data_ptr<float>(), tc.data_ptr<float>(), xc.numel(),
                                  int(reduction), dx.data_ptr<float>(), current_stream()));
  launched();
  return dx;
}

at::Tensor& mse_loss_out(const at::Tensor& x, const at::Tensor& target, int64_t reduction, at::Tensor& out) {
  at::Tensor r = mse_loss_vk(x, target, reduction);
  at::native::resize_output(out, r.sizes());
  return out.copy_(r);
}

// ---------------------------------------------------------------------- cat
at::Tensor cat_vk(const at::ITensorListRef& list, int64_t dim) {
  std::vector<at::Tensor> ts(list.begin(), list.end());
  TORCH_CHECK(!ts.empty(), "torch.cat(): expected a non-empty list of Tensors");
  const at::Device dev = ts[0].device();
  bool same = true;
  at::ScalarType dtype = ts[0].scalar_type();
  for (const auto& t : ts) {
    TORCH_CHECK(t.device() == dev, "Expected all tensors to be on the same device");
    same = same && t.scalar_type() == dtype && !t.is_neg() && !t.is_conj();
  }
  if (!same || ts[0].is_complex()) {
    note_cpu_fallback("cat (mixed dtypes)");
    std::vector<at::Tensor> cpu;
    for (const auto& t : ts) cpu.push_back(t.cpu());
    return at::cat(cpu, dim).to(dev);
  }
  // Legacy rule: 1-D empty tensors are skipped whatever the other shapes are.
  auto skipped = [](const at::Tensor& t) { return t.dim() == 1 && t.numel() == 0; };
  const at::Tensor* ref = &ts[0];
  for (const auto& t : ts)
    if (!skipped(t)) {
      ref = &t;
      break;
    }
  TORCH_CHECK(ref->dim() > 0, "zero-dimensional tensor cannot be concatenated");
  const int64_t d = at::maybe_wrap_dim(dim, ref->dim());
  std::vector<int64_t> shape(ref->sizes().begin(), ref->sizes().end());
  shape[size_t(d)] = 0;
  for (const auto& t : ts) {
    if (skipped(t)) continue;
    TORCH_CHECK(t.dim() == ref->dim(), "Tensors must have same number of dimensions");
    for (int64_t k = 0; k < t.dim(); ++k)
      TORCH_CHECK(k == d || t.size(k) == ref->size(k), "Sizes of tensors must match except in dimension ", d);
    shape[size_t(d)] += t.size(d);
  }
  c10::DeviceGuard guard(dev);
  at::Tensor out = at::empty(shape, ref->options().memory_format(at::MemoryFormat::Contiguous));
  if (out.numel() == 0) return out;
  int64_t outer = 1, inner = 1;
  for (int64_t k = 0; k < d; ++k) outer *= shape[size_t(k)];
  for (int64_t k = d + 1; k < int64_t(shape.size()); ++k) inner *= shape[size_t(k)];
  const int64_t item = int64_t(out.element_size());
  const int64_t dst_pitch = shape[size_t(d)] * inner * item;
  int64_t offset = 0;
  for (const auto& t : ts) {
    if (skipped(t)) continue;
    if (t.numel() > 0) {
      at::assert_no_partial_overlap(out, t);
      at::Tensor tc = packed(t);
      const int64_t row = t.size(d) * inner * item;
      TVK_MX(mx_copy_rows(static_cast<char*>(out.data_ptr()) + offset * inner * item, dst_pitch, tc.data_ptr(), row,
                          row, outer, current_stream()));
      launched();
    }
    offset += t.size(d);
  }
  return out;
}

}  // namespace
}  // namespace tvk

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("native_group_norm", TORCH_FN(tvk::native_group_norm_vk));
  m.impl("native_group_norm_backward", TORCH_FN(tvk::native_group_norm_backward_vk));
  m.impl("native_batch_norm", TORCH_FN(tvk::native_batch_norm_vk));
  m.impl("_native_batch_norm_legit", TORCH_FN(tvk::batch_norm_legit));
  m.impl("_native_batch_norm_legit.no_stats", TORCH_FN(tvk::batch_norm_legit_no_stats));
  m.impl("_native_batch_norm_legit_no_training", TORCH_FN(tvk::batch_norm_legit_no_training));
  m.impl("native_batch_norm_backward", TORCH_FN(tvk::native_batch_norm_backward_vk));
  m.impl("silu", TORCH_FN(tvk::silu_vk));
  m.impl("silu_", TORCH_FN(tvk::silu_));
  m.impl("silu.out", TORCH_FN(tvk::silu_out));
  m.impl("silu_backward", TORCH_FN(tvk::silu_backward_vk));
  m.impl("silu_backward.grad_input", TORCH_FN(tvk::silu_backward_out));
  m.impl("relu", TORCH_FN(tvk::relu_vk));
  m.impl("relu_", TORCH_FN(tvk::relu_));
  m.impl("threshold_backward", TORCH_FN(tvk::threshold_backward_vk));
  m.impl("upsample_nearest2d", TORCH_FN(tvk::upsample_nearest2d_vk));
  m.impl("upsample_nearest2d_backward", TORCH_FN(tvk::upsample_nearest2d_backward_vk));
  m.impl("_softmax", TORCH_FN(tvk::softmax_vk));
  m.impl("_softmax_backward_data", TORCH_FN(tvk::softmax_backward_data_vk));
  m.impl("mse_loss", TORCH_FN(tvk::mse_loss_vk));
  m.impl("mse_loss.out", TORCH_FN(tvk::mse_loss_out));
  m.impl("mse_loss_backward", TORCH_FN(tvk::mse_loss_backward_vk));
  m.impl("cat", TORCH_FN(tvk::cat_vk));
}
