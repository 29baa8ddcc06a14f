// Tensor plumbing for the PrivateUse1 device: factories, copies, views,
// resize, scalar read, fill, add and sum.  Mirrors the subset the reference
// registers so tensors can live on the device at all
// (csrc/ops/mm.cpp:480-700, :940-992, :1089-1121; csrc/ops/reduce.cpp:24-35;
// csrc/ops/loss_primitives.cpp:374-375), implemented on the HIP C ABI.
#include <ATen/EmptyTensor.h>
#include <ATen/InferSize.h>
#include <ATen/ExpandUtils.h>
#include <ATen/MemoryOverlap.h>
#include <ATen/NativeFunctions.h>
#include <ATen/TensorUtils.h>
#include <ATen/native/Resize.h>
#include <c10/core/DeviceGuard.h>
#include <torch/library.h>

#include <cstring>
#include <deque>
#include <mutex>
#include <vector>

#include "common.h"

namespace tvk {

void resize_vk_storage(c10::StorageImpl* impl, size_t bytes);

namespace {

c10::DispatchKeySet vk_keys() { return c10::DispatchKeySet(c10::DispatchKey::PrivateUse1); }

void check_device(const std::optional<at::Device>& device) {
  if (!device) return;
  TORCH_CHECK(device->type() == c10::DeviceType::PrivateUse1, "vulkan factory got device ", *device);
}

at::Tensor empty_memory_format(at::IntArrayRef size, std::optional<at::ScalarType> dtype,
                               std::optional<at::Layout> layout, std::optional<at::Device> device,
                               std::optional<bool> pin_memory, std::optional<at::MemoryFormat> memory_format) {
  check_device(device);
  TORCH_CHECK(layout.value_or(at::kStrided) == at::kStrided, "vulkan empty requires strided layout");
  TORCH_CHECK(!pin_memory.value_or(false), "vulkan empty does not support pinned memory");
  c10::OptionalDeviceGuard guard(device);
  return at::detail::empty_generic(size, allocator(), vk_keys(), c10::dtype_or_default(dtype), memory_format);
}

at::Tensor empty_strided(at::IntArrayRef size, at::IntArrayRef stride, std::optional<at::ScalarType> dtype,
                         std::optional<at::Layout> layout, std::optional<at::Device> device,
                         std::optional<bool> pin_memory) {
  check_device(device);
  TORCH_CHECK(layout.value_or(at::kStrided) == at::kStrided, "vulkan empty_strided requires strided layout");
  TORCH_CHECK(!pin_memory.value_or(false), "vulkan empty_strided does not support pinned memory");
  c10::OptionalDeviceGuard guard(device);
  return at::detail::empty_strided_generic(size, stride, allocator(), vk_keys(), c10::dtype_or_default(dtype));
}

// Device-to-device copy of equally-typed tensors of equal shape.
void d2d_copy(const at::Tensor& dst, const at::Tensor& src) {
  c10::DeviceGuard guard(dst.device());
  const int64_t n = dst.numel();
  if (n == 0) return;
  const size_t item = dst.element_size();
  if (dst.is_contiguous() && src.is_contiguous()) {
    TVK_MX(mx_memcpy(dst.data_ptr(), src.data_ptr(), size_t(n) * item, MX_COPY_D2D, current_stream()));
    counters().kernel_launches++;
    return;
  }
  const int nd = int(dst.dim());
  TORCH_CHECK(nd <= 8, "vulkan strided copy supports at most 8 dimensions");
  std::vector<int64_t> sizes(dst.sizes().begin(), dst.sizes().end());
  std::vector<int64_t> ds(dst.strides().begin(), dst.strides().end());
  std::vector<int64_t> ss(src.strides().begin(), src.strides().end());
  TORCH_CHECK(item == 1 || item == 2 || item == 4 || item == 8 || item == 16, "vulkan copy: element size ", item);
  TVK_MX(mx_copy_strided(dst.storage().mutable_data(), src.storage().data(), nd, sizes.data(), ds.data(),
                         ss.data(), dst.storage_offset(), src.storage_offset(), int(item), current_stream()));
  counters().kernel_launches++;
}

// ----------------------------------------------------- non_blocking copies
// A non_blocking copy between the device and page-locked host memory is
// queued on the current stream and returns at once (the reference has no
// pinned memory and always waits).  The host storage is held here until an
// event recorded after the copy has completed, so freeing the host tensor
// right after the call cannot hand its pages to another allocation while the
// copy still reads or writes them.
struct PendingHost {
  void* event;
  c10::Storage storage;
};
std::mutex g_pending_mu;
std::deque<PendingHost> g_pending;   // in issue order
std::vector<void*> g_event_pool;     // completed events, reused

void reap_pending_locked() {
  while (!g_pending.empty()) {
    int done = 0;
    TVK_MX(mx_event_query(g_pending.front().event, &done));
    if (!done) break;
    g_event_pool.push_back(g_pending.front().event);
    g_pending.pop_front();
  }
}

bool host_pinned(const at::Tensor& t) {
  int pinned = 0;
  TVK_MX(mx_host_is_pinned(t.data_ptr(), &pinned));
  return pinned != 0;
}

void copy_async(void* dst, const void* src, size_t bytes, int kind, const c10::Storage& host) {
  std::lock_guard<std::mutex> lock(g_pending_mu);
  reap_pending_locked();
  void* stream = current_stream();
  TVK_MX(mx_memcpy_async(dst, src, bytes, kind, stream));
  void* ev = nullptr;
  if (!g_event_pool.empty()) {
    ev = g_event_pool.back();
    g_event_pool.pop_back();
  } else {
    TVK_MX(mx_event_create(&ev, 0));
  }
  TVK_MX(mx_event_record(ev, stream));
  g_pending.push_back({ev, host});
  counters().async_copies++;
}

}  // namespace

size_t pending_host_copies() {
  std::lock_guard<std::mutex> lock(g_pending_mu);
  reap_pending_locked();
  return g_pending.size();
}

namespace {

at::Tensor& copy_impl(at::Tensor& self, const at::Tensor& src, bool non_blocking) {
  TORCH_CHECK(self.defined() && src.defined(), "copy_: undefined tensor");
  if (self.numel() == 0) return self;
  if (self.is_same(src)) return self;
  const at::Tensor s = src.sizes().equals(self.sizes()) ? src : src.expand(self.sizes());
  if (is_vk(self) && is_vk(s)) {
    if (self.scalar_type() != s.scalar_type() || s.is_neg() || s.is_conj()) {
      // Casts between dtypes go through the host (not part of the hot path).
      note_cpu_fallback("copy_ (dtype cast on device)");
      at::Tensor host = s.cpu().to(self.scalar_type());
      return copy_impl(self, host, non_blocking);
    }
    if (self.storage().is_alias_of(s.storage()) && self.storage_offset() == s.storage_offset() &&
        self.strides().equals(s.strides()))
      return self;
    at::assert_no_internal_overlap(self);
    at::assert_no_partial_overlap(self, s);
    if (self.storage().is_alias_of(s.storage())) {
      // Overlapping source: stage through a fresh buffer.
      at::Tensor tmp = at::empty(s.sizes(), s.options());
      d2d_copy(tmp, s);
      d2d_copy(self, tmp);
    } else {
      d2d_copy(self, s);
    }
    return self;
  }
  if (is_vk(self)) {  // host -> device
    c10::DeviceGuard guard(self.device());
    at::Tensor host = s.to(self.scalar_type()).contiguous();
    if (host.is_neg()) host = host.resolve_neg();
    if (host.is_conj()) host = host.resolve_conj();
    if (self.is_contiguous()) {
      if (non_blocking && host_pinned(host))
        copy_async(self.data_ptr(), host.data_ptr(), host.nbytes(), MX_COPY_H2D, host.storage());
      else
        TVK_MX(mx_memcpy(self.data_ptr(), host.data_ptr(), host.nbytes(), MX_COPY_H2D, current_stream()));
    } else {
      at::Tensor tmp = at::empty(self.sizes(), self.options().memory_format(at::MemoryFormat::Contiguous));
      TVK_MX(mx_memcpy(tmp.data_ptr(), host.data_ptr(), host.nbytes(), MX_COPY_H2D, current_stream()));
      d2d_copy(self, tmp);
    }
    return self;
  }
  // device -> host
  TORCH_CHECK(is_vk(s), "copy_: expected a vulkan tensor on one side");
  c10::DeviceGuard guard(s.device());
  at::Tensor dense = s.is_contiguous() ? s : s.contiguous();
  if (non_blocking && self.is_contiguous() && self.scalar_type() == dense.scalar_type() && !self.is_neg() &&
      !self.is_conj() && host_pinned(self)) {
    copy_async(self.data_ptr(), dense.data_ptr(), self.nbytes(), MX_COPY_D2H, self.storage());
    counters().host_reads++;
    return self;
  }
  at::Tensor host = at::empty(dense.sizes(), dense.options().device(at::kCPU));
  TVK_MX(mx_memcpy(host.data_ptr(), dense.data_ptr(), host.nbytes(), MX_COPY_D2H, current_stream()));
  counters().host_reads++;
  self.copy_(host, non_blocking);
  return self;
}

at::Tensor copy_from(const at::Tensor& self, const at::Tensor& dst, bool non_blocking) {
  at::Tensor d = dst;
  copy_impl(d, self, non_blocking);
  return dst;
}

at::Tensor copy_from_and_resize(const at::Tensor& self, const at::Tensor& dst) {
  TORCH_CHECK(self.scalar_type() == dst.scalar_type(), "vulkan _copy_from_and_resize: dtype mismatch");
  at::Tensor d = dst;
  if (!d.sizes().equals(self.sizes())) d.resize_(self.sizes());
  copy_impl(d, self, false);
  return dst;
}

at::Tensor& copy_(at::Tensor& self, const at::Tensor& src, bool non_blocking) {
  return copy_impl(self, src, non_blocking);
}

at::Tensor alias_view(const at::Tensor& self, at::IntArrayRef sizes, at::IntArrayRef strides, int64_t offset) {
  auto impl = c10::make_intrusive<c10::TensorImpl>(c10::TensorImpl::VIEW, c10::Storage(self.storage()),
                                                   self.key_set(), self.dtype());
  at::Tensor out(std::move(impl));
  at::native::setStrided(out, sizes, strides, offset);
  return out;
}

at::Tensor view(const at::Tensor& self, at::IntArrayRef size) {
  auto shape = at::infer_size_dv(size, self.numel());
  auto strides = at::detail::computeStride(self.sizes(), self.strides(), shape);
  TORCH_CHECK(strides.has_value(),
              "view size is not compatible with input tensor's size and stride (at least one dimension spans "
              "across two contiguous subspaces). Use .reshape(...) instead.");
  return alias_view(self, shape, *strides, self.storage_offset());
}

at::Tensor as_strided(const at::Tensor& self, at::IntArrayRef size, at::IntArrayRef stride,
                      std::optional<int64_t> storage_offset) {
  return alias_view(self, size, stride, storage_offset.value_or(self.storage_offset()));
}

at::Tensor reshape_alias(const at::Tensor& self, at::IntArrayRef size, at::IntArrayRef stride) {
  return alias_view(self, size, stride, self.storage_offset());
}

const at::Tensor& resize_(const at::Tensor& self, at::IntArrayRef size, std::optional<at::MemoryFormat> fmt) {
  TORCH_CHECK(!fmt || *fmt != at::MemoryFormat::Preserve, "resize_ does not support preserve memory format");
  for (auto v : size) TORCH_CHECK(v >= 0, "negative resize dimension");
  auto* impl = self.unsafeGetTensorImpl();
  impl->set_sizes_contiguous(size);
  const size_t need = (size_t(self.storage_offset()) + size_t(c10::multiply_integers(size))) * self.element_size();
  if (need > self.storage().nbytes()) {
    c10::DeviceGuard guard(self.device());
    resize_vk_storage(self.storage().unsafeGetStorageImpl(), need);
  }
  if (fmt) impl->empty_tensor_restride(*fmt);
  return self;
}

// set_ onto an existing device storage (metadata only: the tensor then
// aliases `source` at `offset` with the given sizes and strides, contiguous
// when `stride` is empty).  copy.deepcopy of a device tensor reaches it after
// cloning the storage, as torch.optim checkpoints do.  The view must fit the
// storage, as for any other device: the storage is not grown here.
at::Tensor& set_storage_offset(at::Tensor& self, c10::Storage source, int64_t offset, at::IntArrayRef size,
                               at::IntArrayRef stride) {
  TORCH_CHECK(source.device().type() == c10::DeviceType::PrivateUse1 || source.nbytes() == 0,
              "set_: expected a vulkan storage, got one on ", source.device());
  TORCH_CHECK(offset >= 0, "set_: negative storage offset");
  TORCH_CHECK(stride.empty() || stride.size() == size.size(), "set_: ", size.size(), " sizes but ", stride.size(),
              " strides");
  int64_t last = offset;  // one past the largest element index the view reaches
  bool empty = false;
  for (size_t i = 0; i < size.size(); ++i) {
    TORCH_CHECK(size[i] >= 0, "set_: negative size");
    if (size[i] == 0) empty = true;
  }
  if (!empty) {
    if (stride.empty()) {
      last += c10::multiply_integers(size);
    } else {
      for (size_t i = 0; i < size.size(); ++i) last += (size[i] - 1) * stride[i];
      last += 1;
    }
    TORCH_CHECK(size_t(last) * self.element_size() <= source.nbytes(), "set_: a view of ", last,
                " elements does not fit a storage of ", source.nbytes(), " bytes");
  }
  auto* impl = self.unsafeGetTensorImpl();
  impl->set_storage_keep_dtype(std::move(source));
  if (stride.empty())
    impl->set_sizes_contiguous(size);
  else
    impl->set_sizes_and_strides(size, stride);
  impl->set_storage_offset(offset);
  return self;
}

at::Tensor& set_storage(at::Tensor& self, c10::Storage source) {
  const int64_t n = int64_t(source.nbytes() / self.element_size());
  return set_storage_offset(self, std::move(source), 0, {n}, {});
}

at::Scalar local_scalar_dense(const at::Tensor& self) {
  TORCH_CHECK(self.numel() == 1, "a Tensor with ", self.numel(), " elements cannot be converted to Scalar");
  c10::DeviceGuard guard(self.device());
  at::Tensor host = at::empty({}, self.options().device(at::kCPU));
  TVK_MX(mx_memcpy(host.data_ptr(), self.data_ptr(), self.element_size(), MX_COPY_D2H, current_stream()));
  counters().host_reads++;
  return at::_local_scalar_dense(host);
}

at::Tensor& fill_scalar(at::Tensor& self, const at::Scalar& value) {
  if (self.numel() == 0) return self;
  c10::DeviceGuard guard(self.device());
  const size_t item = self.element_size();
  if (item > 8 || self.is_neg() || self.is_conj()) {
    note_cpu_fallback("fill_ (unsupported dtype)");
    at::Tensor host = at::empty(self.sizes(), self.options().device(at::kCPU)).fill_(value);
    return copy_impl(self, host, false);
  }
  at::Tensor scalar = at::scalar_tensor(value, at::TensorOptions().dtype(self.scalar_type()));
  uint64_t pattern = 0;
  std::memcpy(&pattern, scalar.data_ptr(), item);
  if (self.is_non_overlapping_and_dense()) {
    // A dense tensor occupies exactly numel consecutive elements from its
    // lowest-addressed element (which is at storage_offset for non-negative strides).
    TVK_MX(mx_fill(self.data_ptr(), self.numel(), int(item), pattern, current_stream()));
  } else {
    at::Tensor tmp = at::empty(self.sizes(), self.options().memory_format(at::MemoryFormat::Contiguous));
    TVK_MX(mx_fill(tmp.data_ptr(), tmp.numel(), int(item), pattern, current_stream()));
    d2d_copy(self, tmp);
  }
  counters().kernel_launches++;
  return self;
}

at::Tensor& zero_(at::Tensor& self) { return fill_scalar(self, 0); }

bool is_host_scalar(const at::Tensor& t) { return t.device().is_cpu() && t.dim() == 0; }

// A 0-dim CPU operand (a Python number arrives as a wrapped double) joins an
// FP32 device tensor on the device when the result stays FP32.
bool f32_with_host_scalar(const at::Tensor& dev_t, const at::Tensor& oth) {
  return dev_t.scalar_type() == at::kFloat && is_host_scalar(oth) && !oth.is_complex() &&
         at::result_type(dev_t, oth) == at::kFloat;
}

at::Tensor add_tensor(const at::Tensor& self, const at::Tensor& other, const at::Scalar& alpha) {
  const bool f32 = (self.scalar_type() == at::kFloat && other.scalar_type() == at::kFloat) ||
                   f32_with_host_scalar(self, other);
  if (f32 && is_vk(self) && !self.is_neg() && (is_host_scalar(other) || (is_vk(other) && !other.is_neg()))) {
    c10::DeviceGuard guard(self.device());
    if (is_host_scalar(other)) {
      at::Tensor a = self.contiguous();
      at::Tensor out = at::empty(self.sizes(), self.options().memory_format(at::MemoryFormat::Contiguous));
      const float v = alpha.toFloat() * other.item<float>();
      TVK_MX(mx_add_f32(out.data_ptr<float>(), a.data_ptr<float>(), nullptr, v, a.numel(), current_stream()));
      counters().kernel_launches++;
      return out;
    }
    const auto shape = at::infer_size(self.sizes(), other.sizes());
    at::Tensor a = self.expand(shape).contiguous();
    at::Tensor b = other.expand(shape).contiguous();
    at::Tensor out = at::empty(shape, self.options().memory_format(at::MemoryFormat::Contiguous));
    TVK_MX(mx_add_f32(out.data_ptr<float>(), a.data_ptr<float>(), b.data_ptr<float>(), alpha.toFloat(), out.numel(),
                      current_stream()));
    counters().kernel_launches++;
    return out;
  }
  note_cpu_fallback("add.Tensor");
  at::Tensor r = at::add(self.cpu(), other.device().is_cpu() ? other : other.cpu(), alpha);
  return r.to(self.device());
}

at::Tensor mul_tensor(const at::Tensor& self, const at::Tensor& other) {
  const at::Tensor& dev_t = is_vk(self) ? self : other;
  const at::Tensor& oth = is_vk(self) ? other : self;
  const bool f32 = (self.scalar_type() == at::kFloat && other.scalar_type() == at::kFloat) ||
                   f32_with_host_scalar(dev_t, oth);
  if (f32 && is_vk(dev_t) && !dev_t.is_neg() && (is_host_scalar(oth) || (is_vk(oth) && !oth.is_neg()))) {
    c10::DeviceGuard guard(dev_t.device());
    if (is_host_scalar(oth)) {
      at::Tensor a = dev_t.contiguous();
      at::Tensor out = at::empty(dev_t.sizes(), dev_t.options().memory_format(at::MemoryFormat::Contiguous));
      TVK_MX(mx_scale_f32(out.data_ptr<float>(), a.data_ptr<float>(), oth.item<float>(), a.numel(), current_stream()));
      counters().kernel_launches++;
      return out;
    }
    const auto shape = at::infer_size(self.sizes(), other.sizes());
    at::Tensor a = self.expand(shape).contiguous();
    at::Tensor b = other.expand(shape).contiguous();
    at::Tensor out = at::empty(shape, self.options().memory_format(at::MemoryFormat::Contiguous));
    TVK_MX(mx_mul_f32(out.data_ptr<float>(), a.data_ptr<float>(), b.data_ptr<float>(), out.numel(), current_stream()));
    counters().kernel_launches++;
    return out;
  }
  note_cpu_fallback("mul.Tensor");
  at::Tensor r = at::mul(self.device().is_cpu() ? self : self.cpu(), other.device().is_cpu() ? other : other.cpu());
  return r.to(dev_t.device());
}

at::Tensor mul_scalar(const at::Tensor& self, const at::Scalar& other) {
  return mul_tensor(self, at::scalar_tensor(other, at::TensorOptions().dtype(self.scalar_type())));
}

at::Tensor& add_inplace(at::Tensor& self, const at::Tensor& other, const at::Scalar& alpha) {
  at::Tensor r = add_tensor(self, other, alpha);
  TORCH_CHECK(r.sizes().equals(self.sizes()), "output with shape ", self.sizes(),
              " doesn't match the broadcast shape ", r.sizes());
  return copy_impl(self, r, false);
}

at::Tensor sum_dims(const at::Tensor& self, at::OptionalIntArrayRef dim_opt, bool keepdim,
                    std::optional<at::ScalarType> dtype) {
  const bool ok = is_vk(self) && self.scalar_type() == at::kFloat && (!dtype || *dtype == at::kFloat) &&
                  !self.is_neg();
  if (!ok) {
    note_cpu_fallback("sum.dim_IntList");
    return at::sum(self.cpu(), dim_opt, keepdim, dtype).to(self.device());
  }
  c10::DeviceGuard guard(self.device());
  const int64_t nd = self.dim();
  std::vector<bool> red(size_t(std::max<int64_t>(nd, 1)), false);
  if (!dim_opt.has_value() || dim_opt->empty()) {
    for (int64_t d = 0; d < nd; ++d) red[size_t(d)] = true;
  } else {
    for (int64_t d : *dim_opt) red[size_t(c10::maybe_wrap_dim(d, std::max<int64_t>(nd, 1)))] = true;
  }
  std::vector<int64_t> out_shape, keep_shape;
  for (int64_t d = 0; d < nd; ++d) {
    if (red[size_t(d)]) {
      keep_shape.push_back(1);
    } else {
      keep_shape.push_back(self.size(d));
      out_shape.push_back(self.size(d));
    }
  }
  at::Tensor cur = self.contiguous();
  std::vector<int64_t> cur_shape(cur.sizes().begin(), cur.sizes().end());
  // Reduce one maximal run of adjacent reduced axes at a time, last run first.
  for (int64_t d = nd - 1; d >= 0;) {
    if (!red[size_t(d)]) {
      --d;
      continue;
    }
    int64_t lo = d;
    while (lo - 1 >= 0 && red[size_t(lo - 1)]) --lo;
    int64_t outer = 1, reduce = 1, inner = 1;
    for (int64_t k = 0; k < lo; ++k) outer *= cur_shape[size_t(k)];
    for (int64_t k = lo; k <= d; ++k) reduce *= cur_shape[size_t(k)];
    for (int64_t k = d + 1; k < nd; ++k) inner *= cur_shape[size_t(k)];
    std::vector<int64_t> next_shape = cur_shape;
    for (int64_t k = lo; k <= d; ++k) next_shape[size_t(k)] = 1;
    at::Tensor next = at::empty(next_shape, cur.options());
    if (outer > 65535) {
      // The kernel's row grid is 16-bit: fold the outer rows into chunks.
      for (int64_t o0 = 0; o0 < outer; o0 += 65535) {
        const int64_t oc = std::min<int64_t>(65535, outer - o0);
        TVK_MX(mx_sum_f32(next.data_ptr<float>() + o0 * inner, cur.data_ptr<float>() + o0 * reduce * inner, oc,
                          reduce, inner, current_stream()));
      }
    } else {
      TVK_MX(mx_sum_f32(next.data_ptr<float>(), cur.data_ptr<float>(), outer, reduce, inner, current_stream()));
    }
    counters().kernel_launches++;
    cur = next;
    cur_shape = next_shape;
    d = lo - 1;
  }
  if (nd == 0) return cur.clone();
  return keepdim ? cur.view(keep_shape) : cur.view(out_shape);
}

at::Tensor sum_all(const at::Tensor& self, std::optional<at::ScalarType> dtype) {
  return sum_dims(self, std::nullopt, false, dtype);
}

void foreach_add_scalar(at::TensorList self, const at::Scalar& scalar) {
  bool fused = !self.empty();
  for (const auto& t : self)
    fused = fused && is_vk(t) && t.scalar_type() == at::kFloat && t.is_contiguous() && t.device() == self[0].device();
  if (!fused) {
    for (const auto& t : self) const_cast<at::Tensor&>(t).add_(scalar);
    return;
  }
  c10::DeviceGuard guard(self[0].device());
  std::vector<float*> ptrs;
  std::vector<int64_t> numels;
  for (const auto& t : self) {
    ptrs.push_back(const_cast<at::Tensor&>(t).data_ptr<float>());
    numels.push_back(t.numel());
  }
  TVK_MX(mx_foreach_add_scalar_f32(ptrs.data(), numels.data(), int64_t(ptrs.size()), scalar.toFloat(),
                                   current_stream()));
  counters().kernel_launches++;
}

// Tensor.record_stream: the storage's block is not reused until the work
// queued on `s` at the time the tensor is freed has completed.
void record_stream_vk(at::Tensor& self, at::Stream s) {
  TORCH_CHECK(s.device_type() == c10::DeviceType::PrivateUse1, "record_stream: expected a vulkan stream, got ",
              s.device_type());
  void* base = self.storage().mutable_data();
  if (base) TVK_MX(mx_record_stream(base, stream_for_id(s.device_index(), s.id())));
}

}  // namespace
}  // namespace tvk

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("record_stream", TORCH_FN(tvk::record_stream_vk));
  m.impl("empty.memory_format", TORCH_FN(tvk::empty_memory_format));
  m.impl("empty_strided", TORCH_FN(tvk::empty_strided));
  m.impl("_copy_from", TORCH_FN(tvk::copy_from));
  m.impl("_copy_from_and_resize", TORCH_FN(tvk::copy_from_and_resize));
  m.impl("copy_", TORCH_FN(tvk::copy_));
  m.impl("view", TORCH_FN(tvk::view));
  m.impl("as_strided", TORCH_FN(tvk::as_strided));
  m.impl("_reshape_alias", TORCH_FN(tvk::reshape_alias));
  m.impl("resize_", TORCH_FN(tvk::resize_));
  m.impl("set_.source_Storage_storage_offset", TORCH_FN(tvk::set_storage_offset));
  m.impl("set_.source_Storage", TORCH_FN(tvk::set_storage));
  m.impl("_local_scalar_dense", TORCH_FN(tvk::local_scalar_dense));
  m.impl("fill_.Scalar", TORCH_FN(tvk::fill_scalar));
  m.impl("zero_", TORCH_FN(tvk::zero_));
  m.impl("add.Tensor", TORCH_FN(tvk::add_tensor));
  m.impl("add_.Tensor", TORCH_FN(tvk::add_inplace));
  m.impl("mul.Tensor", TORCH_FN(tvk::mul_tensor));
  m.impl("mul.Scalar", TORCH_FN(tvk::mul_scalar));
  m.impl("sum.dim_IntList", TORCH_FN(tvk::sum_dims));
  m.impl("sum", TORCH_FN(tvk::sum_all));
  m.impl("_foreach_add_.Scalar", TORCH_FN(tvk::foreach_add_scalar));
}
