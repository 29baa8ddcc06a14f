// Fused AdamW operators for the PrivateUse1 device.
//
// Keeps the reference's custom schemas exactly (torch_vulkan::adamw_step_,
// adamw_step_batch_, adamw_amsgrad_step_batch_; csrc/ops/adamw.cpp:306-324)
// and adds aten::_fused_adamw_ (+ .tensor_lr) so that
// torch.optim.AdamW(fused=True) on "vulkan" parameters runs on the device
// instead of the reference's CPU fallback.  All tensors of a call go to one
// mx_adamw_step, which issues a single launch unless entries alias.
#include <c10/core/DeviceGuard.h>
#include <torch/library.h>

#include <vector>

#include "common.h"

namespace tvk {
namespace {

float* f32_ptr(const at::Tensor& t, const char* what, size_t i) {
  TORCH_CHECK(is_vk(t), "fused AdamW requires Vulkan tensors (", what, " ", i, ")");
  TORCH_CHECK(t.scalar_type() == at::kFloat && t.is_contiguous(),
              "fused AdamW requires contiguous float32 tensors (", what, " ", i, ")");
  return const_cast<at::Tensor&>(t).data_ptr<float>();
}

struct Lists {
  at::TensorList params, grads, m, v;
  std::optional<at::TensorList> vmax;
};

void run(const Lists& l, double lr, double beta1, double beta2, double eps, double weight_decay,
         const std::vector<int64_t>* host_steps, at::TensorList dev_steps, bool maximize,
         const at::Tensor* lr_dev, const std::optional<at::Tensor>& grad_scale,
         const std::optional<at::Tensor>& found_inf) {
  const size_t n = l.params.size();
  TORCH_CHECK(l.grads.size() == n && l.m.size() == n && l.v.size() == n && (!l.vmax || l.vmax->size() == n) &&
                  (host_steps ? host_steps->size() == n : dev_steps.size() == n),
              "fused AdamW batch: all parameter/gradient/moment/step lists must match");
  TORCH_CHECK(lr >= 0 && beta1 >= 0 && beta1 < 1 && beta2 >= 0 && beta2 < 1 && eps >= 0 && weight_decay >= 0,
              "fused AdamW batch: invalid hyperparameters");
  if (n == 0) return;
  c10::DeviceGuard guard(l.params[0].device());
  std::vector<mx_adamw_tensor> tab(n);
  for (size_t i = 0; i < n; ++i) {
    const at::Tensor& p = l.params[i];
    TORCH_CHECK(p.sizes() == l.grads[i].sizes() && p.sizes() == l.m[i].sizes() && p.sizes() == l.v[i].sizes() &&
                    (!l.vmax || p.sizes() == (*l.vmax)[i].sizes()),
                "fused AdamW batch: incompatible tensor shapes at ", i);
    TORCH_CHECK(p.device() == l.params[0].device(), "fused AdamW batch: tensors on different devices");
    mx_adamw_tensor& e = tab[i];
    e.numel = p.numel();
    if (host_steps) {
      e.step = (*host_steps)[i];
      TORCH_CHECK(e.step >= 1, "fused AdamW batch: step must be positive");
    } else {
      const at::Tensor& st = dev_steps[i];
      TORCH_CHECK(is_vk(st) && st.scalar_type() == at::kFloat && st.numel() == 1,
                  "_fused_adamw_: state_steps must be float32 scalars on the device");
      e.step_dev = st.data_ptr<float>();
    }
    if (e.numel == 0) continue;
    e.param = f32_ptr(p, "param", i);
    e.grad = f32_ptr(l.grads[i], "grad", i);
    e.exp_avg = f32_ptr(l.m[i], "exp_avg", i);
    e.exp_avg_sq = f32_ptr(l.v[i], "exp_avg_sq", i);
    if (l.vmax) e.max_exp_avg_sq = f32_ptr((*l.vmax)[i], "max_exp_avg_sq", i);
  }
  mx_adamw_hparams hp{};
  hp.lr = lr;
  hp.beta1 = beta1;
  hp.beta2 = beta2;
  hp.eps = eps;
  hp.weight_decay = weight_decay;
  hp.amsgrad = l.vmax ? 1 : 0;
  hp.maximize = maximize ? 1 : 0;
  at::Tensor lr_t, gs_t, fi_t;
  if (lr_dev) {
    lr_t = lr_dev->to(l.params[0].device(), at::kFloat);
    hp.lr_dev = lr_t.data_ptr<float>();
  }
  if (grad_scale && grad_scale->defined()) {
    gs_t = grad_scale->to(l.params[0].device(), at::kFloat);
    hp.grad_scale = gs_t.data_ptr<float>();
  }
  if (found_inf && found_inf->defined()) {
    fi_t = found_inf->to(l.params[0].device(), at::kFloat);
    hp.found_inf = fi_t.data_ptr<float>();
  }
  int64_t launches = 0;
  GpuTimer timer(gpu_timing_enabled() ? (l.vmax ? "adamw_kernel<amsgrad>" : "adamw_kernel") : "");
  TVK_MX(mx_adamw_step(tab.data(), int64_t(n), &hp, &launches, current_stream()));
  counters().kernel_launches += uint64_t(launches);
  counters().adamw_launches += uint64_t(launches);
}

void adamw_step_(const at::Tensor& param, const at::Tensor& grad, const at::Tensor& exp_avg,
                 const at::Tensor& exp_avg_sq, double lr, double beta1, double beta2, double eps,
                 double weight_decay, int64_t step) {
  TORCH_CHECK(param.defined() && grad.defined() && exp_avg.defined() && exp_avg_sq.defined(),
              "fused AdamW: all four tensors must be defined");
  TORCH_CHECK(param.sizes() == grad.sizes() && param.sizes() == exp_avg.sizes() && param.sizes() == exp_avg_sq.sizes(),
              "fused AdamW: parameter, gradient and moments must have identical shapes");
  TORCH_CHECK(step >= 1, "fused AdamW: step must be positive");
  std::vector<at::Tensor> p{param}, g{grad}, m{exp_avg}, v{exp_avg_sq};
  std::vector<int64_t> steps{step};
  run({p, g, m, v, std::nullopt}, lr, beta1, beta2, eps, weight_decay, &steps, {}, false, nullptr, std::nullopt,
      std::nullopt);
}

void adamw_step_batch_(at::TensorList params, at::TensorList grads, at::TensorList exp_avgs,
                       at::TensorList exp_avg_sqs, double lr, double beta1, double beta2, double eps,
                       double weight_decay, at::IntArrayRef steps) {
  std::vector<int64_t> st(steps.begin(), steps.end());
  TORCH_CHECK(st.size() == params.size(), "fused AdamW batch: all parameter/gradient/moment/step lists must match");
  run({params, grads, exp_avgs, exp_avg_sqs, std::nullopt}, lr, beta1, beta2, eps, weight_decay, &st, {}, false,
      nullptr, std::nullopt, std::nullopt);
}

void adamw_amsgrad_step_batch_(at::TensorList params, at::TensorList grads, at::TensorList exp_avgs,
                               at::TensorList exp_avg_sqs, at::TensorList max_exp_avg_sqs, double lr, double beta1,
                               double beta2, double eps, double weight_decay, at::IntArrayRef steps) {
  std::vector<int64_t> st(steps.begin(), steps.end());
  TORCH_CHECK(st.size() == params.size(), "fused AdamW batch: all parameter/gradient/moment/step lists must match");
  run({params, grads, exp_avgs, exp_avg_sqs, max_exp_avg_sqs}, lr, beta1, beta2, eps, weight_decay, &st, {}, false,
      nullptr, std::nullopt, std::nullopt);
}

void fused_adamw_(at::TensorList self, at::TensorList grads, at::TensorList exp_avgs, at::TensorList exp_avg_sqs,
                  at::TensorList max_exp_avg_sqs, at::TensorList state_steps, double lr, double beta1, double beta2,
                  double weight_decay, double eps, bool amsgrad, bool maximize,
                  const std::optional<at::Tensor>& grad_scale, const std::optional<at::Tensor>& found_inf) {
  std::optional<at::TensorList> vmax;
  if (amsgrad) vmax = max_exp_avg_sqs;
  run({self, grads, exp_avgs, exp_avg_sqs, vmax}, lr, beta1, beta2, eps, weight_decay, nullptr, state_steps, maximize,
      nullptr, grad_scale, found_inf);
}

void fused_adamw_tensor_lr_(at::TensorList self, at::TensorList grads, at::TensorList exp_avgs,
                            at::TensorList exp_avg_sqs, at::TensorList max_exp_avg_sqs, at::TensorList state_steps,
                            const at::Tensor& lr, double beta1, double beta2, double weight_decay, double eps,
                            bool amsgrad, bool maximize, const std::optional<at::Tensor>& grad_scale,
                            const std::optional<at::Tensor>& found_inf) {
  std::optional<at::TensorList> vmax;
  if (amsgrad) vmax = max_exp_avg_sqs;
  run({self, grads, exp_avgs, exp_avg_sqs, vmax}, 0.0, beta1, beta2, eps, weight_decay, nullptr, state_steps,
      maximize, &lr, grad_scale, found_inf);
}

}  // namespace
}  // namespace tvk

TORCH_LIBRARY(torch_vulkan, m) {
  m.def(
      "adamw_step_(Tensor(a!) param, Tensor grad, Tensor(b!) exp_avg, Tensor(c!) exp_avg_sq, float lr, float beta1, "
      "float beta2, float eps, float weight_decay, int step) -> ()");
  m.def(
      "adamw_step_batch_(Tensor(a!)[] params, Tensor[] grads, Tensor(b!)[] exp_avgs, Tensor(c!)[] exp_avg_sqs, "
      "float lr, float beta1, float beta2, float eps, float weight_decay, int[] steps) -> ()");
  m.def(
      "adamw_amsgrad_step_batch_(Tensor(a!)[] params, Tensor[] grads, Tensor(b!)[] exp_avgs, Tensor(c!)[] "
      "exp_avg_sqs, Tensor(d!)[] max_exp_avg_sqs, float lr, float beta1, float beta2, float eps, float "
      "weight_decay, int[] steps) -> ()");
}

TORCH_LIBRARY_IMPL(torch_vulkan, PrivateUse1, m) {
  m.impl("adamw_step_", TORCH_FN(tvk::adamw_step_));
  m.impl("adamw_step_batch_", TORCH_FN(tvk::adamw_step_batch_));
  m.impl("adamw_amsgrad_step_batch_", TORCH_FN(tvk::adamw_amsgrad_step_batch_));
}

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("_fused_adamw_", TORCH_FN(tvk::fused_adamw_));
  m.impl("_fused_adamw_.tensor_lr", TORCH_FN(tvk::fused_adamw_tensor_lr_));
}
