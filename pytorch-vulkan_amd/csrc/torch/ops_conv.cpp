// aten::convolution_overrideable / convolution_backward_overrideable for the
// PrivateUse1 device (reference: csrc/ops/convolution.cpp:641-702).
//
// Operands are packed to contiguous NCHW FP32 on the device (the reference's
// packed(), csrc/ops/convolution.cpp:62-99), the algorithm is chosen by the
// library's planner unless forced through the reference's environment knobs
// (read on every call, as csrc/ops/convolution.cpp:402-422 does), and each
// phase runs as one or two MFMA launches.  Transposed, non-2D and non-FP32
// convolutions are outside this backend and run on the CPU (counted).
#include <c10/core/DeviceGuard.h>
#include <torch/library.h>

#include <cstdlib>
#include <cstring>
#include <string>

#include "common.h"

namespace tvk {
namespace {

const char* algo_name(int algo) {
  switch (algo) {
    case MX_CONV_ALGO_DIRECT: return "direct";
    case MX_CONV_ALGO_IMPLICIT_GEMM: return "implicit_gemm";
    case MX_CONV_ALGO_WINOGRAD: return "winograd_f2";
    case MX_CONV_ALGO_REDUCE: return "reduce";
    case MX_CONV_ALGO_DEPTHWISE: return "depthwise";
    default: return "auto";
  }
}

std::string env_or(const char* name, const char* dflt) {
  const char* v = std::getenv(name);
  return (v && *v) ? std::string(v) : std::string(dflt);
}

// Forward algorithm from TORCH_VULKAN_CONV_ALGO (auto/direct/tiled/depthwise/winograd).
int forward_algo() {
  const std::string a = env_or("TORCH_VULKAN_CONV_ALGO", "auto");
  if (a == "auto") return MX_CONV_ALGO_AUTO;
  if (a == "direct") return MX_CONV_ALGO_DIRECT;
  if (a == "depthwise") return MX_CONV_ALGO_DEPTHWISE;
  if (a == "tiled" || a == "implicit_gemm") return MX_CONV_ALGO_IMPLICIT_GEMM;
  if (a == "winograd") return MX_CONV_ALGO_WINOGRAD;
  TORCH_CHECK(false, "TORCH_VULKAN_CONV_ALGO has an invalid algorithm (forward: auto/direct/tiled/depthwise/winograd)");
}

// Backward algorithm from TORCH_VULKAN_CONV_BACKWARD_ALGO (auto/direct/optimized,
// plus this build's winograd: F(2x2,3x3) input and weight gradients for the
// layers they apply to, the optimized kernels everywhere else).
int backward_algo(const mx_conv2d_desc& d, int phase) {
  const std::string a = env_or("TORCH_VULKAN_CONV_BACKWARD_ALGO", "auto");
  if (a == "auto") return MX_CONV_ALGO_AUTO;
  if (a == "direct") return MX_CONV_ALGO_DIRECT;
  const int optimized = phase == MX_CONV_DBIAS ? MX_CONV_ALGO_REDUCE : MX_CONV_ALGO_IMPLICIT_GEMM;
  if (a == "optimized") return optimized;
  if (a == "winograd") {
    int algo = 0;
    if (phase != MX_CONV_DBIAS && mx_conv2d_select(&d, phase, MX_CONV_ALGO_WINOGRAD, &algo) == MX_OK)
      return MX_CONV_ALGO_WINOGRAD;
    return optimized;
  }
  TORCH_CHECK(false,
              "TORCH_VULKAN_CONV_BACKWARD_ALGO has an invalid algorithm (backward: auto/direct/optimized/winograd)");
}

mx_conv2d_desc make_desc(const at::Tensor& input, const at::Tensor& weight, at::IntArrayRef stride,
                         at::IntArrayRef padding, at::IntArrayRef dilation, at::IntArrayRef output_padding,
                         int64_t groups) {
  TORCH_CHECK(input.dim() == 4 && weight.dim() == 4, "Vulkan convolution supports NCHW tensors only");
  TORCH_CHECK(stride.size() == 2 && padding.size() == 2 && dilation.size() == 2 && output_padding.size() == 2,
              "Vulkan convolution requires two spatial dimensions");
  TORCH_CHECK(output_padding[0] == 0 && output_padding[1] == 0,
              "Vulkan convolution: output_padding requires transposed convolution");
  mx_conv2d_desc d{};
  d.n = input.size(0);
  d.cin = input.size(1);
  d.h = input.size(2);
  d.w = input.size(3);
  d.cout = weight.size(0);
  d.kh = weight.size(2);
  d.kw = weight.size(3);
  d.sh = stride[0];
  d.sw = stride[1];
  d.ph = padding[0];
  d.pw = padding[1];
  d.dh = dilation[0];
  d.dw = dilation[1];
  d.groups = groups;
  TORCH_CHECK(groups > 0 && weight.size(1) * groups == d.cin, "Vulkan convolution: invalid shapes or parameters");
  TVK_MX(mx_conv2d_check(&d));
  return d;
}

// Contiguous FP32 device operand (one strided-copy launch for views).
at::Tensor packed(const at::Tensor& t) {
  TORCH_CHECK(is_vk(t) && t.scalar_type() == at::kFloat, "Vulkan convolution requires FP32 Vulkan tensors");
  at::Tensor r = t.resolve_neg();
  return r.is_contiguous() ? r : r.contiguous();
}

bool native_conv(const at::Tensor& input, const at::Tensor& weight, bool transposed) {
  return !transposed && input.dim() == 4 && weight.dim() == 4 && input.scalar_type() == at::kFloat &&
         weight.scalar_type() == at::kFloat && is_vk(input) && is_vk(weight);
}

// Name a gpu_timing_stats() entry: the main kernel of the call.
std::string kernel_label(const mx_conv2d_desc& d, int phase, int algo) {
  if (!gpu_timing_enabled()) return {};
  char buf[128];
  return mx_conv2d_kernel_name(&d, phase, algo, buf, sizeof buf) == MX_OK ? std::string(buf) : "conv2d";
}

int choose(const mx_conv2d_desc& d, int phase, int requested) {
  int algo = 0;
  TVK_MX(mx_conv2d_select(&d, phase, requested, &algo));
  static const char* phases[] = {"forward", "dinput", "dweight", "dbias"};
  count_selection(std::string("selected_") + phases[phase] + "_" + algo_name(algo));
  return algo;
}

at::Tensor convolution_overrideable(const at::Tensor& input, const at::Tensor& weight,
                                    const std::optional<at::Tensor>& bias, at::IntArrayRef stride,
                                    at::IntArrayRef padding, at::IntArrayRef dilation, bool transposed,
                                    at::IntArrayRef output_padding, int64_t groups) {
  if (!native_conv(input, weight, transposed)) {
    note_cpu_fallback("convolution_overrideable (transposed / non-2D / non-FP32)");
    std::optional<at::Tensor> b;
    if (bias && bias->defined()) b = bias->cpu();
    return at::convolution(input.cpu(), weight.cpu(), b, stride, padding, dilation, transposed, output_padding,
                           groups)
        .to(input.device());
  }
  c10::DeviceGuard guard(input.device());
  const mx_conv2d_desc d = make_desc(input, weight, stride, padding, dilation, output_padding, groups);
  const at::Tensor x = packed(input), w = packed(weight);
  at::Tensor b;
  if (bias && bias->defined()) {
    TORCH_CHECK(bias->numel() == d.cout && bias->scalar_type() == at::kFloat,
                "Vulkan convolution: bias shape/dtype mismatch");
    b = packed(*bias);
  }
  at::Tensor y = at::empty({d.n, d.cout, d.oh, d.ow}, input.options().memory_format(at::MemoryFormat::Contiguous));
  const int algo = choose(d, MX_CONV_FORWARD, forward_algo());
  GpuTimer timer(kernel_label(d, MX_CONV_FORWARD, algo));
  TVK_MX(mx_conv2d_forward(&d, x.data_ptr<float>(), w.data_ptr<float>(), b.defined() ? b.data_ptr<float>() : nullptr,
                           y.data_ptr<float>(), algo, current_stream()));
  counters().kernel_launches++;
  return y;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> backward_phases(const mx_conv2d_desc& d, const at::Tensor& dy,
                                                               const at::Tensor& input, const at::Tensor& weight,
                                                               std::array<bool, 3> output_mask, int ax, int aw);

std::tuple<at::Tensor, at::Tensor, at::Tensor> convolution_backward_overrideable(
    const at::Tensor& grad_output, const at::Tensor& input, const at::Tensor& weight, at::IntArrayRef stride,
    at::IntArrayRef padding, at::IntArrayRef dilation, bool transposed, at::IntArrayRef output_padding,
    int64_t groups, std::array<bool, 3> output_mask) {
  if (!native_conv(input, weight, transposed)) {
    note_cpu_fallback("convolution_backward_overrideable (transposed / non-2D / non-FP32)");
    std::vector<int64_t> bias_sizes = {weight.size(transposed ? 1 : 0) * (transposed ? groups : 1)};
    auto r = at::convolution_backward(grad_output.cpu(), input.cpu(), weight.cpu(), bias_sizes, stride, padding,
                                      dilation, transposed, output_padding, groups, output_mask);
    auto dev = [&](const at::Tensor& t) { return t.defined() ? t.to(input.device()) : t; };
    return {dev(std::get<0>(r)), dev(std::get<1>(r)), dev(std::get<2>(r))};
  }
  c10::DeviceGuard guard(input.device());
  const mx_conv2d_desc d = make_desc(input, weight, stride, padding, dilation, output_padding, groups);
  TORCH_CHECK(grad_output.dim() == 4 && grad_output.size(0) == d.n && grad_output.size(1) == d.cout &&
                  grad_output.size(2) == d.oh && grad_output.size(3) == d.ow,
              "Vulkan convolution backward: output gradient shape mismatch");
  const at::Tensor dy = packed(grad_output);
  at::Tensor dx, dw, db;
  auto opts = input.options().memory_format(at::MemoryFormat::Contiguous);
  if (output_mask[0] && output_mask[1]) {
    // Both gradients in one library call (convolution_backward's dispatch of
    // Input, Weight and Bias, csrc/ops/convolution.cpp:667-697): where both
    // take the fused Winograd paths the library runs them as one launch.
    const int ax = choose(d, MX_CONV_DINPUT, backward_algo(d, MX_CONV_DINPUT));
    const int aw = choose(d, MX_CONV_DWEIGHT, backward_algo(d, MX_CONV_DWEIGHT));
    if (ax == MX_CONV_ALGO_WINOGRAD && aw == MX_CONV_ALGO_WINOGRAD) {
      dx = at::empty(input.sizes(), opts);
      dw = at::empty(weight.sizes(), weight.options().memory_format(at::MemoryFormat::Contiguous));
      if (output_mask[2]) {
        db = at::empty({d.cout}, weight.options());
        count_selection("selected_dbias_fused_dweight");
      }
      const at::Tensor x = packed(input), w = packed(weight);
      GpuTimer timer(kernel_label(d, MX_CONV_DWEIGHT, aw));
      TVK_MX(mx_conv2d_backward(&d, x.data_ptr<float>(), w.data_ptr<float>(), dy.data_ptr<float>(),
                                dx.data_ptr<float>(), dw.data_ptr<float>(), db.defined() ? db.data_ptr<float>() : nullptr,
                                ax, aw, current_stream()));
      counters().kernel_launches++;
      return {dx, dw, db};
    }
    return backward_phases(d, dy, input, weight, output_mask, ax, aw);
  }
  return backward_phases(d, dy, input, weight, output_mask, -1, -1);
}

// The requested gradients one library call each.  ax / aw: algorithms
// already chosen (and counted) for dInput / dWeight, or -1.
std::tuple<at::Tensor, at::Tensor, at::Tensor> backward_phases(const mx_conv2d_desc& d, const at::Tensor& dy,
                                                               const at::Tensor& input, const at::Tensor& weight,
                                                               std::array<bool, 3> output_mask, int ax, int aw) {
  at::Tensor dx, dw, db;
  auto opts = input.options().memory_format(at::MemoryFormat::Contiguous);
  if (output_mask[0]) {
    dx = at::empty(input.sizes(), opts);
    const at::Tensor w = packed(weight);
    const int algo = ax >= 0 ? ax : choose(d, MX_CONV_DINPUT, backward_algo(d, MX_CONV_DINPUT));
    GpuTimer timer(kernel_label(d, MX_CONV_DINPUT, algo));
    TVK_MX(mx_conv2d_backward_input(&d, dy.data_ptr<float>(), w.data_ptr<float>(), dx.data_ptr<float>(), algo,
                                    current_stream()));
    counters().kernel_launches++;
  }
  if (output_mask[2]) db = at::empty({d.cout}, weight.options());
  if (output_mask[1]) {
    dw = at::empty(weight.sizes(), weight.options().memory_format(at::MemoryFormat::Contiguous));
    const at::Tensor x = packed(input);
    const int algo = aw >= 0 ? aw : choose(d, MX_CONV_DWEIGHT, backward_algo(d, MX_CONV_DWEIGHT));
    // dBias rides on the dWeight launch when both are requested.
    float* dbp = nullptr;
    if (output_mask[2]) {
      dbp = db.data_ptr<float>();
      count_selection(std::string("selected_dbias_") + (algo == MX_CONV_ALGO_IMPLICIT_GEMM ? "fused_dweight" : "reduce"));
    }
    if (algo == MX_CONV_ALGO_IMPLICIT_GEMM) {
      // Split plan counters under the reference's names
      // (tests/test_conv_dispatch.py:274-284).
      mx_conv2d_plan_info plan{};
      TVK_MX(mx_conv2d_plan(&d, MX_CONV_DWEIGHT, algo, output_mask[2] ? 1 : 0, &plan));
      count_selection("dweight_tiled_dispatches");
      count_selection("dweight_tiled_split_count_total", uint64_t(plan.splits));
      count_selection("dweight_tiled_split_span_total", uint64_t(plan.span));
      count_selection("dweight_tiled_workspace_bytes_total", uint64_t(plan.workspace_bytes));
    }
    GpuTimer timer(kernel_label(d, MX_CONV_DWEIGHT, algo));
    TVK_MX(mx_conv2d_backward_weight(&d, x.data_ptr<float>(), dy.data_ptr<float>(), dw.data_ptr<float>(), dbp, algo,
                                     current_stream()));
    counters().kernel_launches++;
  } else if (output_mask[2]) {
    const int algo = choose(d, MX_CONV_DBIAS, backward_algo(d, MX_CONV_DBIAS));
    GpuTimer timer(kernel_label(d, MX_CONV_DBIAS, algo));
    TVK_MX(mx_conv2d_backward_bias(&d, dy.data_ptr<float>(), db.data_ptr<float>(), current_stream()));
    counters().kernel_launches++;
  }
  return {dx, dw, db};
}

}  // namespace
}  // namespace tvk

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("convolution_overrideable", TORCH_FN(tvk::convolution_overrideable));
  m.impl("convolution_backward_overrideable", TORCH_FN(tvk::convolution_backward_overrideable));
}
