// mm / mm.out / addmm / bmm / bmm.out / baddbmm / addbmm (+ out= and in-place
// forms) for the PrivateUse1 device on the MFMA GEMM of the C ABI
// (mx_gemm_f32).
//
// Reference counterparts: mm_impl / mm_out csrc/ops/mm.cpp:244-383,
// vulkan_addmm / addmm_bias_vulkan csrc/ops/mm.cpp:835-917, bmm_impl /
// bmm_out csrc/ops/bmm.cpp:16-110.  Differences by design: views with a
// storage offset are consumed in place (the reference packs them), and no
// FP32 view ever routes to the CPU.
#include <ATen/ExpandUtils.h>
#include <ATen/MemoryOverlap.h>
#include <ATen/native/Resize.h>
#include <c10/core/DeviceGuard.h>
#include <torch/library.h>

#include <cstdlib>
#include <cstring>

#include "common.h"

namespace tvk {
namespace {

bool gemm_native(const at::Tensor& t) {
  return is_vk(t) && t.scalar_type() == at::kFloat && !t.is_neg() && !t.is_conj();
}

// TORCH_VULKAN_MM_KERNEL for mm / addmm (csrc/ops/mm.cpp:299-307, :851-854):
// "register" keeps the tile choice among the large register-blocked tiles,
// "tiled" forces the small one; any other value (or none) lets the cost model
// choose, as the reference treats unknown values as automatic.
int mm_kernel_knob() {
  const char* k = std::getenv("TORCH_VULKAN_MM_KERNEL");
  if (k && std::strcmp(k, "register") == 0) return MX_GEMM_KERNEL_REGISTER;
  if (k && std::strcmp(k, "tiled") == 0) return MX_GEMM_KERNEL_TILED;
  return MX_GEMM_KERNEL_AUTO;
}

// C[b] (+)= alpha * A[b] B[b] + beta * bias into a contiguous `out`.
void run_gemm(const at::Tensor& a, const at::Tensor& b, at::Tensor& out, int64_t batch, const at::Tensor* bias,
              float alpha, float beta, int kernel = MX_GEMM_KERNEL_AUTO) {
  const bool batched = a.dim() == 3;
  const int64_t M = a.size(batched ? 1 : 0), K = a.size(batched ? 2 : 1), N = b.size(batched ? 2 : 1);
  mx_gemm_desc d{};
  d.batch = batch;
  d.m = M;
  d.n = N;
  d.k = K;
  d.a_offset = a.storage_offset();
  d.a_stride_b = batched ? a.stride(0) : 0;
  d.a_stride_m = a.stride(batched ? 1 : 0);
  d.a_stride_k = a.stride(batched ? 2 : 1);
  d.b_offset = b.storage_offset();
  d.b_stride_b = batched ? b.stride(0) : 0;
  d.b_stride_k = b.stride(batched ? 1 : 0);
  d.b_stride_n = b.stride(batched ? 2 : 1);
  d.c_offset = out.storage_offset();
  d.c_stride_b = batched ? out.stride(0) : 0;
  d.ldc = out.stride(batched ? 1 : 0);
  d.alpha = alpha;
  d.beta = beta;
  d.kernel = kernel;
  d.bias_kind = MX_BIAS_NONE;
  const float* bias_ptr = nullptr;
  if (bias && bias->defined() && beta != 0.f) {
    if (bias->dim() == 1 && bias->size(0) == N) {
      d.bias_kind = MX_BIAS_COL;  // one row for every batch
      d.bias_stride_n = bias->stride(0);
    } else {
      // Anything broadcastable to [M, N] (or [batch, M, N]); broadcast dims get stride 0.
      const at::Tensor e = batched ? bias->expand({batch, M, N}) : bias->expand({M, N});
      d.bias_kind = MX_BIAS_MATRIX;
      d.bias_stride_m = e.stride(-2);
      d.bias_stride_n = e.stride(-1);
      d.bias_stride_b = batched ? e.stride(0) : 0;
    }
    d.bias_offset = bias->storage_offset();
    bias_ptr = static_cast<const float*>(bias->storage().data());
  }
  std::string label;
  if (gpu_timing_enabled()) {
    char buf[128];
    label = mx_gemm_variant(&d, static_cast<const float*>(a.storage().data()),
                            static_cast<const float*>(b.storage().data()), buf, sizeof buf) == MX_OK
                ? std::string(buf) : "gemm";
  }
  GpuTimer timer(label, 2.0 * double(d.batch) * double(d.m) * double(d.n) * double(d.k));
  TVK_MX(mx_gemm_f32(&d, static_cast<const float*>(a.storage().data()), static_cast<const float*>(b.storage().data()),
                     bias_ptr, static_cast<float*>(out.storage().mutable_data()), current_stream()));
  counters().kernel_launches++;
}

at::Tensor mm_impl(const at::Tensor& self, const at::Tensor& mat2, at::Tensor* destination) {
  TORCH_CHECK(self.dim() == 2 && mat2.dim() == 2, "mm: inputs must be 2D");
  TORCH_CHECK(self.size(1) == mat2.size(0), "mm: dimension mismatch (", self.sizes(), " x ", mat2.sizes(), ")");
  TORCH_CHECK(self.scalar_type() == mat2.scalar_type(), "mm: expected both matrices to have the same dtype");
  TORCH_CHECK(self.device() == mat2.device(), "mm: expected both matrices on the same vulkan device");
  if (!gemm_native(self) || !gemm_native(mat2)) {
    if (self.scalar_type() == at::kFloat) return mm_impl(self.resolve_neg().resolve_conj(), mat2.resolve_neg(), destination);
    note_cpu_fallback("mm (non-FP32)");
    at::Tensor r = at::mm(self.cpu(), mat2.cpu()).to(self.device());
    if (destination) {
      destination->copy_(r);
      return *destination;
    }
    return r;
  }
  c10::DeviceGuard guard(self.device());
  const int64_t M = self.size(0), N = mat2.size(1);
  at::Tensor out = destination ? *destination : at::empty({M, N}, self.options());
  if (M == 0 || N == 0) return out;
  run_gemm(self, mat2, out, 1, nullptr, 1.f, 0.f, mm_kernel_knob());
  return out;
}

at::Tensor mm(const at::Tensor& self, const at::Tensor& mat2) { return mm_impl(self, mat2, nullptr); }

at::Tensor& mm_out(const at::Tensor& self, const at::Tensor& mat2, at::Tensor& out) {
  TORCH_CHECK(out.device() == self.device() && self.device() == mat2.device(),
              "out tensor must be on the same device as the inputs");
  at::assert_no_internal_overlap(out);
  at::assert_no_partial_overlap(out, self);
  at::assert_no_partial_overlap(out, mat2);
  const bool aliases = out.storage().is_alias_of(self.storage()) || out.storage().is_alias_of(mat2.storage());
  const bool shape_ok = self.dim() == 2 && mat2.dim() == 2 && self.size(1) == mat2.size(0) &&
                        out.sizes().equals({self.size(0), mat2.size(1)});
  if (shape_ok && !aliases && out.scalar_type() == at::kFloat && out.stride(1) == 1 && !out.is_neg() &&
      !out.is_conj()) {
    mm_impl(self, mat2, &out);
    return out;
  }
  at::Tensor value = mm_impl(self, mat2, nullptr);
  TORCH_CHECK(c10::canCast(value.scalar_type(), out.scalar_type()),
              "result type cannot be cast to the desired output type");
  at::native::resize_output(out, value.sizes());
  out.copy_(value);
  return out;
}

at::Tensor addmm(const at::Tensor& self, const at::Tensor& mat1, const at::Tensor& mat2, const at::Scalar& beta,
                 const at::Scalar& alpha) {
  TORCH_CHECK(mat1.dim() == 2 && mat2.dim() == 2, "addmm: mat1 and mat2 must be matrices");
  TORCH_CHECK(mat1.size(1) == mat2.size(0), "addmm: matrix shapes cannot be multiplied (", mat1.sizes(), " and ",
              mat2.sizes(), ")");
  TORCH_CHECK(self.device() == mat1.device() && self.device() == mat2.device(),
              "addmm: all tensors must be on the same device");
  TORCH_CHECK(self.scalar_type() == mat1.scalar_type() && self.scalar_type() == mat2.scalar_type(),
              "addmm: all tensors must have the same dtype");
  const std::vector<int64_t> shape = {mat1.size(0), mat2.size(1)};
  const at::Tensor bias = self.expand(shape);  // validates broadcasting even when beta == 0
  if (!gemm_native(self) || !gemm_native(mat1) || !gemm_native(mat2)) {
    note_cpu_fallback("addmm (non-FP32)");
    return at::addmm(self.cpu(), mat1.cpu(), mat2.cpu(), beta, alpha).to(self.device());
  }
  c10::DeviceGuard guard(self.device());
  // TORCH_VULKAN_FUSE_ADDMM=0 (csrc/ops/mm.cpp:900-916): no bias epilogue,
  // out = mm, scaled by alpha unless it is 1, plus beta * bias unless beta is
  // 0 (so a NaN bias is still ignored at beta == 0).
  const char* fuse = std::getenv("TORCH_VULKAN_FUSE_ADDMM");
  if (fuse && std::strcmp(fuse, "0") == 0 && shape[0] > 0 && shape[1] > 0 && mat1.size(1) > 0) {
    at::Tensor product = mm_impl(mat1, mat2, nullptr);
    if (alpha.toFloat() != 1.0f) product = product.mul(alpha);
    if (beta.toFloat() == 0.0f) return product;
    return product.add(bias, beta);
  }
  at::Tensor out = at::empty(shape, mat1.options());
  if (shape[0] == 0 || shape[1] == 0) return out;
  const at::Tensor bias_arg = self.dim() == 1 && self.size(0) == shape[1] ? self : bias;
  run_gemm(mat1, mat2, out, 1, &bias_arg, alpha.toFloat(), beta.toFloat(), mm_kernel_knob());
  return out;
}

at::Tensor bmm_impl(const at::Tensor& a, const at::Tensor& b, at::Tensor* destination) {
  TORCH_CHECK(a.device() == b.device() && a.dim() == 3 && b.dim() == 3 && a.size(0) == b.size(0) &&
                  a.size(2) == b.size(1),
              "Vulkan bmm: expected matching batch dimensions and contraction size");
  TORCH_CHECK(a.scalar_type() == b.scalar_type(), "Vulkan bmm: dtype mismatch");
  if (!gemm_native(a) || !gemm_native(b)) {
    if (a.scalar_type() == at::kFloat) return bmm_impl(a.resolve_neg().resolve_conj(), b.resolve_neg(), destination);
    note_cpu_fallback("bmm (non-FP32)");
    at::Tensor r = at::bmm(a.cpu(), b.cpu()).to(a.device());
    if (destination) {
      destination->copy_(r);
      return *destination;
    }
    return r;
  }
  c10::DeviceGuard guard(a.device());
  const int64_t batch = a.size(0), m = a.size(1), n = b.size(2);
  at::Tensor out = destination ? *destination : at::empty({batch, m, n}, a.options());
  if (batch == 0 || m == 0 || n == 0) return out;
  run_gemm(a, b, out, batch, nullptr, 1.f, 0.f);
  return out;
}

at::Tensor bmm(const at::Tensor& a, const at::Tensor& b) { return bmm_impl(a, b, nullptr); }

at::Tensor& bmm_out(const at::Tensor& a, const at::Tensor& b, at::Tensor& out) {
  TORCH_CHECK(out.device() == a.device() && a.device() == b.device(),
              "out tensor must be on the same device as the inputs");
  at::assert_no_internal_overlap(out);
  at::assert_no_partial_overlap(out, a);
  at::assert_no_partial_overlap(out, b);
  const bool aliases = out.storage().is_alias_of(a.storage()) || out.storage().is_alias_of(b.storage());
  const bool right = a.dim() == 3 && b.dim() == 3 && a.size(0) == b.size(0) && a.size(2) == b.size(1) &&
                     out.sizes().equals({a.size(0), a.size(1), b.size(2)});
  if (right && !aliases && out.scalar_type() == at::kFloat && out.stride(2) == 1 && !out.is_neg() &&
      !out.is_conj()) {
    bmm_impl(a, b, &out);
    return out;
  }
  at::Tensor value = bmm_impl(a, b, nullptr);
  TORCH_CHECK(c10::canCast(value.scalar_type(), out.scalar_type()),
              "result type cannot be cast to the desired output type");
  at::native::resize_output(out, value.sizes());
  out.copy_(value);
  return out;
}

// baddbmm: out[b] = beta * self[b] + alpha * batch1[b] x batch2[b], self
// broadcast to the product shape; beta == 0 ignores self (NaN included), as
// baddbmm_native (csrc/ops/tensor_selection.cpp:92) and torch.  One launch:
// the product and the scaled bias are combined in the GEMM epilogue.
at::Tensor baddbmm(const at::Tensor& self, const at::Tensor& batch1, const at::Tensor& batch2, const at::Scalar& beta,
                   const at::Scalar& alpha) {
  TORCH_CHECK(batch1.dim() == 3 && batch2.dim() == 3, "baddbmm: batch1 and batch2 must be 3-D tensors");
  TORCH_CHECK(batch1.size(0) == batch2.size(0) && batch1.size(2) == batch2.size(1),
              "baddbmm: expected matching batch dimensions and contraction size, got ", batch1.sizes(), " and ",
              batch2.sizes());
  TORCH_CHECK(self.device() == batch1.device() && self.device() == batch2.device(),
              "baddbmm: all tensors must be on the same device");
  TORCH_CHECK(self.scalar_type() == batch1.scalar_type() && self.scalar_type() == batch2.scalar_type(),
              "baddbmm: all tensors must have the same dtype");
  const std::vector<int64_t> shape = {batch1.size(0), batch1.size(1), batch2.size(2)};
  const at::Tensor bias = self.expand(shape);  // broadcast check even when beta == 0
  if (!gemm_native(self) || !gemm_native(batch1) || !gemm_native(batch2)) {
    note_cpu_fallback("baddbmm (non-FP32)");
    return at::baddbmm(self.cpu(), batch1.cpu(), batch2.cpu(), beta, alpha).to(self.device());
  }
  c10::DeviceGuard guard(self.device());
  at::Tensor out = at::empty(shape, batch1.options());
  if (out.numel() == 0) return out;
  const at::Tensor bias_arg = self.dim() == 1 && self.size(0) == shape[2] ? self : bias;
  run_gemm(batch1, batch2, out, shape[0], &bias_arg, alpha.toFloat(), beta.toFloat());
  return out;
}

// addbmm: out = beta * self + alpha * sum_b batch1[b] x batch2[b]
// (addbmm_general, csrc/ops/tensor_selection.cpp:102).  The batch sum is
// accumulated in the output: the first GEMM stores beta * self + alpha * P0,
// each later one adds alpha * Pb with the output as its own bias (every
// element is read and written by the same thread), in batch order.
at::Tensor addbmm(const at::Tensor& self, const at::Tensor& batch1, const at::Tensor& batch2, const at::Scalar& beta,
                  const at::Scalar& alpha) {
  TORCH_CHECK(batch1.dim() == 3 && batch2.dim() == 3 && batch1.size(0) == batch2.size(0),
              "addbmm expects matching batches");
  TORCH_CHECK(batch1.size(2) == batch2.size(1), "addbmm: contraction sizes differ, got ", batch1.sizes(), " and ",
              batch2.sizes());
  TORCH_CHECK(self.device() == batch1.device() && self.device() == batch2.device(),
              "addbmm: all tensors must be on the same device");
  TORCH_CHECK(self.scalar_type() == batch1.scalar_type() && self.scalar_type() == batch2.scalar_type(),
              "addbmm: all tensors must have the same dtype");
  const std::vector<int64_t> shape = {batch1.size(1), batch2.size(2)};
  const at::Tensor bias = self.expand(shape);
  if (!gemm_native(self) || !gemm_native(batch1) || !gemm_native(batch2)) {
    note_cpu_fallback("addbmm (non-FP32)");
    return at::addbmm(self.cpu(), batch1.cpu(), batch2.cpu(), beta, alpha).to(self.device());
  }
  c10::DeviceGuard guard(self.device());
  at::Tensor out = at::empty(shape, batch1.options());
  if (out.numel() == 0) return out;
  const float a = alpha.toFloat(), b = beta.toFloat();
  if (batch1.size(0) == 0) {  // empty sum
    if (b == 0.f) return out.zero_();
    return out.copy_(at::mul(bias, beta));
  }
  const at::Tensor bias_arg = self.dim() == 1 && self.size(0) == shape[1] ? self : bias;
  run_gemm(batch1.select(0, 0), batch2.select(0, 0), out, 1, &bias_arg, a, b);
  for (int64_t i = 1; i < batch1.size(0); ++i) run_gemm(batch1.select(0, i), batch2.select(0, i), out, 1, &out, a, 1.f);
  return out;
}

// out= and in-place forms: compute, then resize/copy into the destination.
template <at::Tensor (*F)(const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Scalar&,
                          const at::Scalar&)>
at::Tensor& into_out(const at::Tensor& self, const at::Tensor& b1, const at::Tensor& b2, const at::Scalar& beta,
                     const at::Scalar& alpha, at::Tensor& out) {
  at::Tensor value = F(self, b1, b2, beta, alpha);
  TORCH_CHECK(c10::canCast(value.scalar_type(), out.scalar_type()),
              "result type cannot be cast to the desired output type");
  at::native::resize_output(out, value.sizes());
  out.copy_(value);
  return out;
}

template <at::Tensor (*F)(const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Scalar&,
                          const at::Scalar&)>
at::Tensor& in_place(at::Tensor& self, const at::Tensor& b1, const at::Tensor& b2, const at::Scalar& beta,
                     const at::Scalar& alpha) {
  at::Tensor value = F(self, b1, b2, beta, alpha);
  TORCH_CHECK(value.sizes().equals(self.sizes()), "in-place result of shape ", value.sizes(),
              " does not match self of shape ", self.sizes());
  self.copy_(value);
  return self;
}

}  // namespace
}  // namespace tvk

TORCH_LIBRARY_IMPL(aten, PrivateUse1, m) {
  m.impl("baddbmm", TORCH_FN(tvk::baddbmm));
  m.impl("baddbmm.out", TORCH_FN(tvk::into_out<tvk::baddbmm>));
  m.impl("baddbmm_", TORCH_FN(tvk::in_place<tvk::baddbmm>));
  m.impl("addbmm", TORCH_FN(tvk::addbmm));
  m.impl("addbmm.out", TORCH_FN(tvk::into_out<tvk::addbmm>));
  m.impl("addbmm_", TORCH_FN(tvk::in_place<tvk::addbmm>));
  m.impl("mm", TORCH_FN(tvk::mm));
  m.impl("mm.out", TORCH_FN(tvk::mm_out));
  m.impl("addmm", TORCH_FN(tvk::addmm));
  m.impl("bmm", TORCH_FN(tvk::bmm));
  m.impl("bmm.out", TORCH_FN(tvk::bmm_out));
}
