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

#include <algorithm>
#include <array>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <mutex>
#include <sstream>
#include <string>
#include <unordered_map>
#include <vector>

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

// Algorithmic FLOPs of one phase (2 per multiply-add of the direct
// convolution, whatever algorithm runs); dBias counts none.
double conv_flops(const mx_conv2d_desc& d, int phase) {
  if (phase == MX_CONV_DBIAS) return 0.0;
  return 2.0 * double(d.n) * double(d.cout) * double(d.oh) * double(d.ow) * double(d.cin / d.groups) *
         double(d.kh) * double(d.kw);
}

// FLOPs the phase's kernels execute: Winograd F(2x2,3x3) multiplies 16
// transformed values per 2x2 tile and channel pair where the direct
// convolution takes 36 products (the tiles of the input gradient cover the
// input, the others the output); the transforms are not counted.
double conv_exec_flops(const mx_conv2d_desc& d, int phase, int algo) {
  if (algo != MX_CONV_ALGO_WINOGRAD || phase == MX_CONV_DBIAS) return conv_flops(d, phase);
  const int64_t th = phase == MX_CONV_DINPUT ? (d.h + 1) / 2 : (d.oh + 1) / 2;
  const int64_t tw = phase == MX_CONV_DINPUT ? (d.w + 1) / 2 : (d.ow + 1) / 2;
  return 2.0 * 16.0 * double(d.n) * double(th) * double(tw) * double(d.cout) * double(d.cin / d.groups);
}

const char* const kPhaseNames[] = {"forward", "dinput", "dweight", "dbias"};

// TORCH_VULKAN_CONV_TILE as the caller set it ("" for unset / auto).  The
// library validates the name and maps it onto its tile menu; the counters
// record the reference's candidate name (csrc/ops/convolution.cpp:182).
std::string tile_knob_name() {
  const std::string t = env_or("TORCH_VULKAN_CONV_TILE", "auto");
  return t == "auto" ? std::string() : t;
}

// TORCH_VULKAN_CONV_AUTOTUNE, validated on every call as the reference's
// controls() does (csrc/ops/convolution.cpp:415-418): "0", "1" or unset.
bool autotune_requested() {
  const std::string v = env_or("TORCH_VULKAN_CONV_AUTOTUNE", "0");
  TORCH_CHECK(v == "0" || v == "1", "TORCH_VULKAN_CONV_AUTOTUNE must be 0 or 1");
  return v == "1";
}

// ---------------------------------------------------------------- autotune
// Plan cache of TORCH_VULKAN_CONV_AUTOTUNE=1 (csrc/ops/convolution.cpp:
// 523-639): per (device, phase, descriptor, workspace budget, dBias) the
// algorithm measured fastest, at most kMaxConvPlans entries evicted first in
// first out.  The candidates are this build's algorithms for the phase
// (direct, implicit GEMM, Winograd, reduce, depthwise, each where it applies);
// the implicit GEMM's tile and K split come from the library's fitted planner.
// Timing follows the reference: every candidate runs once, then five rounds in
// rotating order, each run bracketed by stream synchronisations on the host
// clock; a candidate replaces the heuristic's choice only if its median is 5%
// faster.  The direct kernel is not timed for convolutions above 8e6
// multiply-adds unless the heuristic chose it.
constexpr size_t kMaxConvPlans = 256;
std::mutex g_plan_mu;
std::unordered_map<std::string, int> g_plans;
std::deque<std::string> g_plan_fifo;

std::string plan_key(const mx_conv2d_desc& d, int phase, bool with_bias) {
  int dev = 0;
  TVK_MX(mx_get_device(&dev));
  const char* v = std::getenv("TORCH_VULKAN_CONV_WORKSPACE_MB");
  std::ostringstream key;
  key << dev << ':' << phase << ':' << (v ? v : "default") << ':' << with_bias;
  for (int64_t f : {d.n, d.cin, d.h, d.w, d.cout, d.kh, d.kw, d.sh, d.sw, d.ph, d.pw, d.dh, d.dw, d.groups})
    key << ':' << f;
  return key.str();
}

template <class Run>
int tune(const mx_conv2d_desc& d, int phase, int heuristic, bool with_bias, const Run& run) {
  const auto t0 = std::chrono::steady_clock::now();
  auto lookup_ns = [&] {
    return uint64_t(std::chrono::duration_cast<std::chrono::nanoseconds>(std::chrono::steady_clock::now() - t0)
                        .count());
  };
  const std::string key = plan_key(d, phase, with_bias);
  {
    std::lock_guard<std::mutex> lock(g_plan_mu);
    auto it = g_plans.find(key);
    if (it != g_plans.end()) {
      count_selection("hits");
      record_hotpath("algo_hit", lookup_ns());
      return it->second;
    }
  }
  count_selection("misses");
  record_hotpath("algo_miss", lookup_ns());
  std::vector<int> shortlist;
  const double work = double(d.n) * d.cout * d.oh * d.ow * double(d.cin / d.groups) * d.kh * d.kw;
  for (int a : {MX_CONV_ALGO_DIRECT, MX_CONV_ALGO_IMPLICIT_GEMM, MX_CONV_ALGO_WINOGRAD, MX_CONV_ALGO_REDUCE,
                MX_CONV_ALGO_DEPTHWISE}) {
    int got = 0;
    if (mx_conv2d_select(&d, phase, a, &got) != MX_OK || got != a) continue;
    if (a == MX_CONV_ALGO_DIRECT && work > 8e6 && a != heuristic) continue;
    shortlist.push_back(a);
  }
  if (std::find(shortlist.begin(), shortlist.end(), heuristic) == shortlist.end()) shortlist.push_back(heuristic);
  void* stream = current_stream();
  auto trial = [&](int a) {
    run(a);
    TVK_MX(mx_stream_synchronize(stream));
  };
  TVK_MX(mx_stream_synchronize(stream));
  for (int a : shortlist) trial(a);
  const size_t n = shortlist.size();
  std::vector<std::array<double, 5>> samples(n);
  for (int rep = 0; rep < 5; ++rep)
    for (size_t j = 0; j < n; ++j) {
      const size_t i = (j + rep) % n;
      const auto t0 = std::chrono::steady_clock::now();
      trial(shortlist[i]);
      samples[i][rep] = std::chrono::duration<double, std::nano>(std::chrono::steady_clock::now() - t0).count();
    }
  for (auto& s : samples) std::sort(s.begin(), s.end());
  const size_t inc = std::find(shortlist.begin(), shortlist.end(), heuristic) - shortlist.begin();
  int selected = heuristic;
  double best = samples[inc][2];
  for (size_t i = 0; i < n; ++i)
    if (samples[i][2] < best * 0.95) {
      best = samples[i][2];
      selected = shortlist[i];
    }
  count_selection("tunes");
  count_selection("candidates_timed", n);
  for (int a : shortlist)
    count_selection(std::string("candidates_timed_") + kPhaseNames[phase] + "_" + algo_name(a));
  std::lock_guard<std::mutex> lock(g_plan_mu);
  if (!g_plans.count(key)) {
    if (g_plans.size() >= kMaxConvPlans) {
      g_plans.erase(g_plan_fifo.front());
      g_plan_fifo.pop_front();
      count_selection("evictions");
    }
    g_plan_fifo.push_back(key);
  }
  g_plans[key] = selected;
  return selected;
}

// The algorithm of one phase: the requested one (AUTO resolved by the
// library's heuristic), or under TORCH_VULKAN_CONV_AUTOTUNE=1 with nothing
// forced the cached / measured fastest (`run` launches the phase with a given
// algorithm into its real outputs).  Counted as selected_<phase>_<algorithm>,
// and selected_<phase>_tiled_<name> when a forced tile shapes the implicit GEMM.
template <class Run>
int choose(const mx_conv2d_desc& d, int phase, int requested, bool with_bias, const Run& run) {
  const bool tune_it = autotune_requested();
  const std::string tile = tile_knob_name();
  int algo = 0;
  TVK_MX(mx_conv2d_select(&d, phase, requested, &algo));
  // dBias has one kernel per library call (mx_conv2d_backward_bias picks it).
  if (tune_it && requested == MX_CONV_ALGO_AUTO && tile.empty() && phase != MX_CONV_DBIAS)
    algo = tune(d, phase, algo, with_bias, run);
  count_selection(std::string("selected_") + kPhaseNames[phase] + "_" + algo_name(algo));
  if (algo == MX_CONV_ALGO_IMPLICIT_GEMM && !tile.empty()) {
    // A fixed-3x3 name on another filter size falls back to the base tile.
    const bool fixed3x3 = tile == "register3" || tile == "register3_hoist";
    const bool fits = !fixed3x3 || (d.kh == 3 && d.kw == 3);
    count_selection(std::string("selected_") + kPhaseNames[phase] + "_tiled_" + (fits ? tile : "base"));
  }
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
  const float* bp = b.defined() ? b.data_ptr<float>() : nullptr;
  auto run = [&](int a) {
    TVK_MX(mx_conv2d_forward(&d, x.data_ptr<float>(), w.data_ptr<float>(), bp, y.data_ptr<float>(), a,
                             current_stream()));
  };
  const int algo = choose(d, MX_CONV_FORWARD, forward_algo(), b.defined(), run);
  GpuTimer timer(kernel_label(d, MX_CONV_FORWARD, algo), conv_flops(d, MX_CONV_FORWARD),
                 conv_exec_flops(d, MX_CONV_FORWARD, algo));
  run(algo);
  counters().kernel_launches++;
  return y;
}

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
  at::Tensor dx, dw, db, x, w;
  if (output_mask[0]) {
    dx = at::empty(input.sizes(), input.options().memory_format(at::MemoryFormat::Contiguous));
    w = packed(weight);
  }
  if (output_mask[1]) {
    dw = at::empty(weight.sizes(), weight.options().memory_format(at::MemoryFormat::Contiguous));
    x = packed(input);
  }
  if (output_mask[2]) db = at::empty({d.cout}, weight.options());
  // dBias rides on the dWeight launch when both are requested.
  float* const dbw = output_mask[1] && output_mask[2] ? db.data_ptr<float>() : nullptr;
  auto run_dx = [&](int a) {
    TVK_MX(mx_conv2d_backward_input(&d, dy.data_ptr<float>(), w.data_ptr<float>(), dx.data_ptr<float>(), a,
                                    current_stream()));
  };
  auto run_dw = [&](int a) {
    TVK_MX(mx_conv2d_backward_weight(&d, x.data_ptr<float>(), dy.data_ptr<float>(), dw.data_ptr<float>(), dbw, a,
                                     current_stream()));
  };
  // Each requested gradient is chosen (and, under autotune, measured) on its
  // own, as the reference dispatches Input, Weight and Bias
  // (csrc/ops/convolution.cpp:684-695).
  const int ax = output_mask[0] ? choose(d, MX_CONV_DINPUT, backward_algo(d, MX_CONV_DINPUT), false, run_dx) : -1;
  const int aw = output_mask[1] ? choose(d, MX_CONV_DWEIGHT, backward_algo(d, MX_CONV_DWEIGHT), dbw, run_dw) : -1;
  if (output_mask[2] && output_mask[1]) {
    // The implicit-GEMM and Winograd weight gradients compute dBias in
    // their own launch; the direct and reduce kernels add a reduction.
    const bool fused = aw == MX_CONV_ALGO_IMPLICIT_GEMM || aw == MX_CONV_ALGO_WINOGRAD;
    count_selection(std::string("selected_dbias_") + (fused ? "fused_dweight" : "reduce"));
  }
  if (aw == MX_CONV_ALGO_IMPLICIT_GEMM) {
    // Split plan counters under the reference's names
    // (tests/test_conv_dispatch.py:274-284).
    mx_conv2d_plan_info plan{};
    TVK_MX(mx_conv2d_plan(&d, MX_CONV_DWEIGHT, aw, dbw ? 1 : 0, &plan));
    count_selection("dweight_tiled_dispatches");
    count_selection("dweight_tiled_split_count_total", uint64_t(plan.splits));
    count_selection("dweight_tiled_split_span_total", uint64_t(plan.span));
    count_selection("dweight_tiled_workspace_bytes_total", uint64_t(plan.workspace_bytes));
  }
  int one = 0;
  if (output_mask[0] && output_mask[1]) TVK_MX(mx_conv2d_backward_one_launch(&d, ax, aw, dbw ? 1 : 0, &one));
  if (one) {
    // Both Winograd gradients (and dBias) in one launch
    // (convolution_backward's dispatch of Input, Weight and Bias,
    // csrc/ops/convolution.cpp:667-697).
    GpuTimer timer(gpu_timing_enabled() ? "wino_bwd_kernel" : "",
                   conv_flops(d, MX_CONV_DINPUT) + conv_flops(d, MX_CONV_DWEIGHT),
                   conv_exec_flops(d, MX_CONV_DINPUT, ax) + conv_exec_flops(d, MX_CONV_DWEIGHT, aw));
    TVK_MX(mx_conv2d_backward(&d, x.data_ptr<float>(), w.data_ptr<float>(), dy.data_ptr<float>(),
                              dx.data_ptr<float>(), dw.data_ptr<float>(), dbw, ax, aw, current_stream()));
    counters().kernel_launches++;
    return {dx, dw, db};
  }
  if (output_mask[0]) {
    GpuTimer timer(kernel_label(d, MX_CONV_DINPUT, ax), conv_flops(d, MX_CONV_DINPUT),
                   conv_exec_flops(d, MX_CONV_DINPUT, ax));
    run_dx(ax);
    counters().kernel_launches++;
  }
  if (output_mask[1]) {
    GpuTimer timer(kernel_label(d, MX_CONV_DWEIGHT, aw), conv_flops(d, MX_CONV_DWEIGHT),
                   conv_exec_flops(d, MX_CONV_DWEIGHT, aw));
    run_dw(aw);
    counters().kernel_launches++;
  } else if (output_mask[2]) {
    auto run_db = [&](int a) {
      (void)a;
      TVK_MX(mx_conv2d_backward_bias(&d, dy.data_ptr<float>(), db.data_ptr<float>(), current_stream()));
    };
    const int algo = choose(d, MX_CONV_DBIAS, backward_algo(d, MX_CONV_DBIAS), true, run_db);
    GpuTimer timer(kernel_label(d, MX_CONV_DBIAS, algo));
    run_db(algo);
    counters().kernel_launches++;
  }
  return {dx, dw, db};
}

}  // namespace

size_t conv_plan_cache_entries() {
  std::lock_guard<std::mutex> lock(g_plan_mu);
  return g_plans.size();
}

void clear_conv_plan_cache() {
  std::lock_guard<std::mutex> lock(g_plan_mu);
  g_plans.clear();
  g_plan_fifo.clear();
}

}  // namespace tvk

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("convolution_overrideable", TORCH_FN(tvk::convolution_overrideable));
  m.impl("convolution_backward_overrideable", TORCH_FN(tvk::convolution_backward_overrideable));
}
