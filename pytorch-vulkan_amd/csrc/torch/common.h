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

// Host fallback bookkeeping: increments the counter, honours
// TORCH_VULKAN_FORBID_CPU_FALLBACK and TORCH_VULKAN_TRACE_FALLBACK.
void note_cpu_fallback(const char* what);

inline bool is_vk(const at::Tensor& t) { return t.defined() && t.device().type() == c10::DeviceType::PrivateUse1; }

// Base pointer of the tensor's storage (element offsets are passed separately).
inline float* storage_f32(const at::Tensor& t) {
  return static_cast<float*>(t.storage().mutable_data());
}

}  // namespace tvk
