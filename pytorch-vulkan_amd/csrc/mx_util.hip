// Layout and elementwise plumbing kernels behind the operator surface:
// fill_/zero_, strided copy (view packing, conv2d_pack.comp:12-22), add,
// scale, the middle-axis sum used for Linear bias gradients
// (sum.dim_IntList, csrc/ops/reduce.cpp:24-35) and the one-launch
// _foreach_add_ on optimizer step counters.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <vector>

#include "mx_internal.hpp"

namespace mx {
namespace {

int grid_for(int64_t total, int per_thread = 1) {
  const int64_t threads = (total + per_thread - 1) / per_thread;
  return int(std::max<int64_t>(1, std::min<int64_t>((threads + 255) / 256, int64_t(cu_count()) * 16)));
}

template <class T>
__global__ void fill_kernel(T* dst, int64_t n, T value) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    dst[i] = value;
}

// 16-byte stores of a repeated 16-byte pattern (the host checks alignment
// and that the byte count is a multiple of 16).
__global__ void fill16_kernel(uint4* dst, int64_t n16, uint4 value) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += int64_t(gridDim.x) * blockDim.x)
    dst[i] = value;
}

struct StridedDesc {
  int ndim;
  int64_t sizes[8];
  int64_t dst_strides[8];
  int64_t src_strides[8];
  int64_t dst_offset, src_offset, total;
};

template <class T>
__global__ void copy_strided_kernel(T* __restrict__ dst, const T* __restrict__ src, StridedDesc d) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < d.total;
       i += int64_t(gridDim.x) * blockDim.x) {
    int64_t rem = i, so = d.src_offset, dof = d.dst_offset;
    for (int k = d.ndim - 1; k >= 0; --k) {
      const int64_t idx = rem % d.sizes[k];
      rem /= d.sizes[k];
      so += idx * d.src_strides[k];
      dof += idx * d.dst_strides[k];
    }
    dst[dof] = src[so];
  }
}

__global__ void add_kernel(float* out, const float* a, const float* b, float alpha, int64_t n) {
#pragma clang fp contract(off)
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    out[i] = b ? a[i] + alpha * b[i] : a[i] + alpha;
}

__global__ void scale_kernel(float* out, const float* a, float s, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    out[i] = a[i] * s;
}

__global__ void mul_kernel(float* out, const float* a, const float* b, int64_t n) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    out[i] = a[i] * b[i];
}

// out/partial[split][o][i] = sum over r in the split's range of src[o][r][i].
__global__ void sum_mid_kernel(float* out, const float* src, int64_t outer, int64_t reduce, int64_t inner,
                               int64_t span) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t o = blockIdx.y;
  const int64_t split = blockIdx.z;
  if (i >= inner) return;
  const int64_t r0 = split * span, r1 = min(reduce, r0 + span);
  const float* p = src + (o * reduce) * inner + i;
  float acc = 0.f;
  for (int64_t r = r0; r < r1; ++r) acc += p[r * inner];
  out[(split * outer + o) * inner + i] = acc;
}

// inner == 1: one workgroup per (outer row, split), strided sums + LDS tree.
__global__ __launch_bounds__(256) void sum_last_kernel(float* out, const float* src, int64_t outer, int64_t reduce,
                                                       int64_t span) {
  __shared__ float part[256];
  const int64_t o = blockIdx.x;
  const int64_t split = blockIdx.y;
  const int64_t r0 = split * span, r1 = min(reduce, r0 + span);
  const float* p = src + o * reduce;
  float acc = 0.f;
  for (int64_t r = r0 + threadIdx.x; r < r1; r += 256) acc += p[r];
  part[threadIdx.x] = acc;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (int(threadIdx.x) < s) part[threadIdx.x] += part[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[split * outer + o] = part[0];
}

// out[j] = sum over splits of partial[split][j], in split order.
__global__ void sum_splits_kernel(float* out, const float* partial, int64_t n, int64_t splits) {
  for (int64_t j = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; j < n; j += int64_t(gridDim.x) * blockDim.x) {
    float acc = 0.f;
    for (int64_t s = 0; s < splits; ++s) acc += partial[s * n + j];
    out[j] = acc;
  }
}

struct ForeachEntry {
  float* ptr;
  int64_t numel;
};

__global__ void foreach_add_kernel(const ForeachEntry* tab, int64_t count, float value) {
  for (int64_t t = blockIdx.x; t < count; t += gridDim.x) {
    const ForeachEntry e = tab[t];
    for (int64_t i = threadIdx.x; i < e.numel; i += blockDim.x) e.ptr[i] = e.ptr[i] + value;
  }
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" {

int mx_fill(void* dst, int64_t count, int elem_size, uint64_t pattern, void* stream) {
  MX_ABI_BEGIN
  MX_REQUIRE(count >= 0, MX_ERR_INVALID, "mx_fill: negative count");
  if (count == 0) return MX_OK;
  MX_REQUIRE(dst, MX_ERR_INVALID, "mx_fill: null destination");
  hipStream_t s = resolve_stream(stream);
  const int64_t bytes = count * elem_size;
  if ((reinterpret_cast<uintptr_t>(dst) & 15) == 0 && bytes % 16 == 0 &&
      (elem_size == 1 || elem_size == 2 || elem_size == 4 || elem_size == 8)) {
    uint64_t rep = pattern;  // the element pattern repeated over 8 bytes
    if (elem_size == 1) rep = (pattern & 0xFF) * 0x0101010101010101ull;
    if (elem_size == 2) rep = (pattern & 0xFFFF) * 0x0001000100010001ull;
    if (elem_size == 4) rep = (pattern & 0xFFFFFFFFull) * 0x0000000100000001ull;
    const uint4 v{uint32_t(rep), uint32_t(rep >> 32), uint32_t(rep), uint32_t(rep >> 32)};
    hipLaunchKernelGGL(fill16_kernel, dim3(grid_for(bytes / 16)), dim3(256), 0, s, static_cast<uint4*>(dst),
                       bytes / 16, v);
    MX_HIP(hipGetLastError());
    return MX_OK;
  }
  const dim3 grid(grid_for(count)), block(256);
  switch (elem_size) {
    case 1: hipLaunchKernelGGL(fill_kernel<uint8_t>, grid, block, 0, s, static_cast<uint8_t*>(dst), count, uint8_t(pattern)); break;
    case 2: hipLaunchKernelGGL(fill_kernel<uint16_t>, grid, block, 0, s, static_cast<uint16_t*>(dst), count, uint16_t(pattern)); break;
    case 4: hipLaunchKernelGGL(fill_kernel<uint32_t>, grid, block, 0, s, static_cast<uint32_t*>(dst), count, uint32_t(pattern)); break;
    case 8: hipLaunchKernelGGL(fill_kernel<uint64_t>, grid, block, 0, s, static_cast<uint64_t*>(dst), count, uint64_t(pattern)); break;
    default: return set_error(MX_ERR_INVALID, cat("mx_fill: unsupported element size ", elem_size));
  }
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

int mx_copy_strided(void* dst, const void* src, int ndim, const int64_t* sizes, const int64_t* dst_strides,
                    const int64_t* src_strides, int64_t dst_offset, int64_t src_offset, int elem_size,
                    void* stream) {
  MX_ABI_BEGIN
  MX_REQUIRE(ndim >= 0 && ndim <= 8, MX_ERR_INVALID, "mx_copy_strided: at most 8 dimensions");
  StridedDesc d{};
  d.ndim = ndim;
  d.total = 1;
  for (int k = 0; k < ndim; ++k) {
    MX_REQUIRE(sizes[k] >= 0, MX_ERR_INVALID, "mx_copy_strided: negative size");
    d.sizes[k] = sizes[k];
    d.dst_strides[k] = dst_strides[k];
    d.src_strides[k] = src_strides[k];
    d.total *= sizes[k];
  }
  d.dst_offset = dst_offset;
  d.src_offset = src_offset;
  if (d.total == 0) return MX_OK;
  MX_REQUIRE(dst && src, MX_ERR_INVALID, "mx_copy_strided: null pointer");
  hipStream_t s = resolve_stream(stream);
  const dim3 grid(grid_for(d.total)), block(256);
  switch (elem_size) {
    case 1: hipLaunchKernelGGL(copy_strided_kernel<uint8_t>, grid, block, 0, s, static_cast<uint8_t*>(dst), static_cast<const uint8_t*>(src), d); break;
    case 2: hipLaunchKernelGGL(copy_strided_kernel<uint16_t>, grid, block, 0, s, static_cast<uint16_t*>(dst), static_cast<const uint16_t*>(src), d); break;
    case 4: hipLaunchKernelGGL(copy_strided_kernel<uint32_t>, grid, block, 0, s, static_cast<uint32_t*>(dst), static_cast<const uint32_t*>(src), d); break;
    case 8: hipLaunchKernelGGL(copy_strided_kernel<uint64_t>, grid, block, 0, s, static_cast<uint64_t*>(dst), static_cast<const uint64_t*>(src), d); break;
    case 16: hipLaunchKernelGGL(copy_strided_kernel<uint4>, grid, block, 0, s, static_cast<uint4*>(dst), static_cast<const uint4*>(src), d); break;
    default: return set_error(MX_ERR_INVALID, cat("mx_copy_strided: unsupported element size ", elem_size));
  }
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

int mx_add_f32(float* out, const float* a, const float* b, float alpha, int64_t n, void* stream) {
  MX_ABI_BEGIN
  MX_REQUIRE(n >= 0, MX_ERR_INVALID, "mx_add_f32: negative size");
  if (n == 0) return MX_OK;
  hipStream_t s = resolve_stream(stream);
  hipLaunchKernelGGL(add_kernel, dim3(grid_for(n)), dim3(256), 0, s, out, a, b, alpha, n);
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

int mx_scale_f32(float* out, const float* a, float sc, int64_t n, void* stream) {
  MX_ABI_BEGIN
  MX_REQUIRE(n >= 0, MX_ERR_INVALID, "mx_scale_f32: negative size");
  if (n == 0) return MX_OK;
  hipStream_t s = resolve_stream(stream);
  hipLaunchKernelGGL(scale_kernel, dim3(grid_for(n)), dim3(256), 0, s, out, a, sc, n);
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

int mx_mul_f32(float* out, const float* a, const float* b, int64_t n, void* stream) {
  MX_ABI_BEGIN
  MX_REQUIRE(n >= 0, MX_ERR_INVALID, "mx_mul_f32: negative size");
  if (n == 0) return MX_OK;
  hipStream_t s = resolve_stream(stream);
  hipLaunchKernelGGL(mul_kernel, dim3(grid_for(n)), dim3(256), 0, s, out, a, b, n);
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

int mx_sum_f32(float* out, const float* src, int64_t outer, int64_t reduce, int64_t inner, void* stream) {
  MX_ABI_BEGIN
  MX_REQUIRE(outer >= 0 && reduce >= 0 && inner >= 0, MX_ERR_INVALID, "mx_sum_f32: negative size");
  if (outer == 0 || inner == 0) return MX_OK;
  hipStream_t s = resolve_stream(stream);
  if (reduce == 0) return mx_fill(out, outer * inner, 4, 0, stream);
  MX_REQUIRE(outer <= 65535, MX_ERR_INVALID, "mx_sum_f32: outer extent above 65535");
  const int64_t target = int64_t(cu_count()) * 4;
  if (inner == 1) {
    int64_t splits = std::max<int64_t>(1, std::min<int64_t>(target / std::max<int64_t>(outer, 1), reduce / 4096));
    splits = std::min<int64_t>(splits, 65535);
    const int64_t span = (reduce + splits - 1) / splits;
    splits = (reduce + span - 1) / span;
    if (splits == 1) {
      hipLaunchKernelGGL(sum_last_kernel, dim3(unsigned(outer), 1), dim3(256), 0, s, out, src, outer, reduce, span);
      MX_HIP(hipGetLastError());
      return MX_OK;
    }
    Scratch part;
    MX_TRY(part.alloc(size_t(splits * outer) * 4, s));
    hipLaunchKernelGGL(sum_last_kernel, dim3(unsigned(outer), unsigned(splits)), dim3(256), 0, s, part.as<float>(),
                       src, outer, reduce, span);
    MX_HIP(hipGetLastError());
    hipLaunchKernelGGL(sum_splits_kernel, dim3(grid_for(outer)), dim3(256), 0, s, out, part.as<float>(), outer, splits);
    MX_HIP(hipGetLastError());
    return MX_OK;
  }
  const int64_t xblocks = (inner + 255) / 256;
  int64_t splits = std::max<int64_t>(1, std::min<int64_t>(target / std::max<int64_t>(xblocks * outer, 1), reduce / 64));
  splits = std::min<int64_t>(splits, 65535);
  const int64_t span = (reduce + splits - 1) / splits;
  splits = (reduce + span - 1) / span;
  MX_REQUIRE(xblocks <= INT32_MAX, MX_ERR_INVALID, "mx_sum_f32: inner extent too large");
  if (splits == 1) {
    hipLaunchKernelGGL(sum_mid_kernel, dim3(unsigned(xblocks), unsigned(outer), 1), dim3(256), 0, s, out, src, outer,
                       reduce, inner, span);
    MX_HIP(hipGetLastError());
    return MX_OK;
  }
  Scratch part;
  MX_TRY(part.alloc(size_t(splits * outer * inner) * 4, s));
  hipLaunchKernelGGL(sum_mid_kernel, dim3(unsigned(xblocks), unsigned(outer), unsigned(splits)), dim3(256), 0, s,
                     part.as<float>(), src, outer, reduce, inner, span);
  MX_HIP(hipGetLastError());
  hipLaunchKernelGGL(sum_splits_kernel, dim3(grid_for(outer * inner)), dim3(256), 0, s, out, part.as<float>(),
                     outer * inner, splits);
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

int mx_foreach_add_scalar_f32(float* const* ptrs, const int64_t* numels, int64_t count, float value, void* stream) {
  MX_ABI_BEGIN
  MX_REQUIRE(count >= 0, MX_ERR_INVALID, "mx_foreach_add_scalar_f32: negative count");
  if (count == 0) return MX_OK;
  hipStream_t s = resolve_stream(stream);
  std::vector<ForeachEntry> tab(static_cast<size_t>(count));
  for (int64_t i = 0; i < count; ++i) tab[size_t(i)] = {ptrs[i], numels[i]};
  Scratch dtab;
  MX_TRY(upload(tab.data(), tab.size() * sizeof(ForeachEntry), s, dtab));
  hipLaunchKernelGGL(foreach_add_kernel, dim3(unsigned(std::min<int64_t>(count, 4096))), dim3(64), 0, s,
                     dtab.as<ForeachEntry>(), count, value);
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

}  // extern "C"
