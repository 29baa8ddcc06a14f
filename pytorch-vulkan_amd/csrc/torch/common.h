// Shared helpers of the PrivateUse1 ("vulkan") operator surface.  Everything
// device-side goes through the C ABI in include/mx.h; this layer only maps
// ATen tensors (sizes, strides, storage offsets) onto it.
#pragma once

#include <ATen/ATen.h>
#include <c10/core/Stream.h>
#include <torch/library.h>

#include <atomic>
#include <cstdint>
#include <map>
#include <mutex>
#include <string>

#include "mx.h"

namespace tvk {

// Raises c10::Error (Python RuntimeError) carrying the library's message.
#define TVK_MX(call)                                                                    \
  do {                                                                                  \
    int tvk_rc_ = (call);                                                               \
    TORCH_CHECK(tvk_rc_ == MX_OK, mx_last_error()[0] ? mx_last_error() : #call " failed", \
                " (status ", tvk_rc_, ")");                                             \
  } while (0)

int cur_dev();
// Current HIP stream (as void*) of the current PrivateUse1 device / thread.
void* current_stream();
// Stream object for c10 stream ids.
void* stream_for_id(c10::DeviceIndex device, c10::StreamId id);
int stream_pool_size(int device);

c10::Allocator* allocator();

// Execution counters (execution_stats()).
struct Counters {
  std::atomic<uint64_t> cpu_fallback_calls{0};
  std::atomic<uint64_t> host_reads{0};
  std::atomic<uint64_t> kernel_launches{0};
  std::atomic<uint64_t> adamw_launches{0};
  std::atomic<uint64_t> async_copies{0};  // non_blocking copies to / from page-locked host memory
};

// Asynchronous host copies whose host storage is still held (completed ones
// are released first).
size_t pending_host_copies();
Counters& counters();

// Conv algorithm selections (conv_dispatch_stats()).
void count_selection(const std::string& key, uint64_t n = 1);
std::map<std::string, uint64_t> selection_stats();
void clear_selection_stats();
// The autotune plan cache of the convolution ops (TORCH_VULKAN_CONV_AUTOTUNE=1).
size_t conv_plan_cache_entries();
void clear_conv_plan_cache();

// Host fallback bookkeeping: increments the counter, honours
// TORCH_VULKAN_FORBID_CPU_FALLBACK and TORCH_VULKAN_TRACE_FALLBACK.
void note_cpu_fallback(const char* what);

// Opt-in GPU timing of the hot-path ops (TORCH_VULKAN_PROFILE_TIMESTAMPS=1,
// the reference's knob, csrc/vulkan_context.cpp:368-404): a scope records a
// HIP event pair on the current stream around the op's launches under `name`
// (the kernel the op runs); gpu_timing_stats() waits for the pairs and sums
// them per name.  When the knob is off a scope costs one getenv.
bool gpu_timing_enabled();

// Host hot-path timers (TORCH_VULKAN_PROFILE_HOST_HOTPATH=1, read once, the
// reference's knob, csrc/vulkan_context.cpp:29-58): cumulative nanoseconds and
// counts under the reference's keys.  `key` is "enqueue" (host time of one
// op's library calls), "algo_hit" / "algo_miss" (autotune plan-cache
// lookups) or "allocator" (with `fresh` and `bytes`).
bool host_hotpath_enabled();
void record_hotpath(const char* key, uint64_t nanos, bool fresh = false, size_t bytes = 0);
std::map<std::string, uint64_t> hotpath_stats();

// Times the ops of its scope on the current stream with two HIP events when
// TORCH_VULKAN_PROFILE_TIMESTAMPS=1 (an empty name times nothing).  `flops`
// is the scope's algorithmic work (2 per multiply-add of the direct
// convolution / GEMM) and `executed_flops` the multiply-adds its kernels run
// (fewer for Winograd; negative: the same as `flops`), both summed per name.
class GpuTimer {
 public:
  explicit GpuTimer(std::string name, double flops = 0.0, double executed_flops = -1.0);
  ~GpuTimer();
  GpuTimer(const GpuTimer&) = delete;
  GpuTimer& operator=(const GpuTimer&) = delete;

 private:
  std::string name_;
  void* start_ = nullptr;
  void* stream_ = nullptr;
  double host_t0_ = 0;
  double flops_ = 0, exec_flops_ = 0;
  int64_t hot_t0_ = -1;  // steady-clock ns when host hot-path timing is on
};
struct GpuTiming {
  uint64_t samples = 0;
  double shader_ms = 0, host_eval_ms = 0, flops = 0, executed_flops = 0;
};
std::map<std::string, GpuTiming> gpu_timing_stats();
void reset_gpu_timing_stats();

inline bool is_vk(const at::Tensor& t) { return t.defined() && t.device().type() == c10::DeviceType::PrivateUse1; }

// Base pointer of the tensor's storage (element offsets are passed separately).
inline float* storage_f32(const at::Tensor& t) {
  return static_cast<float*>(t.storage().mutable_data());
}

}  // namespace tvk
