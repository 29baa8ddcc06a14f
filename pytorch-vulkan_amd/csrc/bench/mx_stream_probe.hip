// Measurement probes for bench.py.  HBM streams: the access patterns of the multi-tensor
// AdamW kernel (mx_adamw.hip) with trivial arithmetic, so the benchmark can
// report AdamW against what the same pattern reaches on the same GPU in the
// same run.  Measurement infrastructure only: not part of the drop-in C ABI
// (include/mx.h) and not used by the operator surface.
//
//   int mxp_stream(int kind, float* const* bufs, int64_t n, int per_cu, void* stream)
//
//   kind 0  copy:       bufs[1][i] = bufs[0][i]                      (1 read, 1 write)
//   kind 1  read:       sum of bufs[0..3][i], one value per workgroup (4 reads)
//   kind 2  AdamW mix:  bufs[0], bufs[2], bufs[3] updated in place from
//                       themselves and bufs[1]                        (4 reads, 3 writes)
//   kind 3  AdamW math: kind 2's streams with AdamW's per-element update
//                       (two divisions and a square root, fixed
//                       hyperparameters), next chunk's loads issued before
//                       this chunk's stores                           (4 reads, 3 writes)
//
//   int mxp_mfma_chain(int shape, const float* in, float* out, int blocks, int iters,
//                      unsigned long long* clk, void* stream)
//
//   Register-only chains of FP32 MFMAs (shape 0: v_mfma_f32_32x32x2f32 on
//   four accumulators, shape 1: v_mfma_f32_16x16x4f32 on sixteen), operands
//   read once from `in` (real data or zeros), iters x 131072 FLOPs per wave.
//   Each workgroup records its cycle-counter and 100 MHz real-time-counter
//   spans in clk[2b], clk[2b + 1], which give the engine clock it ran at.
//
// n must be a multiple of 4096 (one chunk); buffers 16-byte aligned.  Chunks
// of 4096 elements are dealt round-robin to per_cu * CUs workgroups, a thread
// issues all its 128-bit loads of a chunk before any arithmetic, and every
// access is non-temporal -- the AdamW kernel's scheme.  Returns 0, or the HIP
// error code.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kVec = 4;                 // float4 per stream per thread per chunk
constexpr int kChunk = 256 * 4 * kVec;  // elements per chunk

__global__ __launch_bounds__(256) void copy_kernel(const float* __restrict__ a, float* __restrict__ b,
                                                   int64_t chunks) {
  for (int64_t ch = blockIdx.x; ch < chunks; ch += gridDim.x) {
    const int64_t base = ch * kChunk + int64_t(threadIdx.x) * 4;
    f32x4 v[kVec];
#pragma unroll
    for (int u = 0; u < kVec; ++u) v[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(a + base + u * 1024));
#pragma unroll
    for (int u = 0; u < kVec; ++u) __builtin_nontemporal_store(v[u], reinterpret_cast<f32x4*>(b + base + u * 1024));
  }
}

__global__ __launch_bounds__(256) void read_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                   const float* __restrict__ c, const float* __restrict__ d,
                                                   float* __restrict__ out, int64_t chunks) {
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  for (int64_t ch = blockIdx.x; ch < chunks; ch += gridDim.x) {
    const int64_t base = ch * kChunk + int64_t(threadIdx.x) * 4;
    f32x4 v[4 * kVec];
#pragma unroll
    for (int u = 0; u < kVec; ++u) {
      const int64_t i = base + u * 1024;
      v[4 * u + 0] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(a + i));
      v[4 * u + 1] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(b + i));
      v[4 * u + 2] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(c + i));
      v[4 * u + 3] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(d + i));
    }
#pragma unroll
    for (int q = 0; q < 4 * kVec; ++q) s += v[q];
  }
  // One store per workgroup keeps the loads live.
  __shared__ float part[256];
  part[threadIdx.x] = s[0] + s[1] + s[2] + s[3];
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int i = 0; i < 256; ++i) t += part[i];
    out[blockIdx.x] = t;
  }
}

__global__ __launch_bounds__(256) void mix_kernel(float* __restrict__ p, const float* __restrict__ g,
                                                  float* __restrict__ m, float* __restrict__ v, int64_t chunks) {
  for (int64_t ch = blockIdx.x; ch < chunks; ch += gridDim.x) {
    const int64_t base = ch * kChunk + int64_t(threadIdx.x) * 4;
    f32x4 P[kVec], G[kVec], M[kVec], V[kVec];
#pragma unroll
    for (int u = 0; u < kVec; ++u) {
      const int64_t i = base + u * 1024;
      P[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + i));
      G[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(g + i));
      M[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(m + i));
      V[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(v + i));
    }
#pragma unroll
    for (int u = 0; u < kVec; ++u) {
      M[u] = M[u] * 0.5f + G[u];
      V[u] = V[u] * 0.5f + G[u];
      P[u] = P[u] * 0.5f + M[u] - V[u];
    }
#pragma unroll
    for (int u = 0; u < kVec; ++u) {
      const int64_t i = base + u * 1024;
      __builtin_nontemporal_store(P[u], reinterpret_cast<f32x4*>(p + i));
      __builtin_nontemporal_store(M[u], reinterpret_cast<f32x4*>(m + i));
      __builtin_nontemporal_store(V[u], reinterpret_cast<f32x4*>(v + i));
    }
  }
}


// AdamW's update (mx_adamw.hip, no AMSGrad, host step) with fixed
// coefficients, contraction off as there.
__device__ __forceinline__ void adam_update(float& p, float g, float& m, float& v) {
#pragma clang fp contract(off)
  p = p * 0.99999f;
  m = fmaf(0.1f, g - m, m);
  v = v * 0.999f;
  v = v + (0.001f * g) * g;
  const float denom = sqrtf(v) / 0.0316f + 1e-8f;
  p = p + (-0.01f * m) / denom;
}

__global__ __launch_bounds__(256) void math_kernel(float* __restrict__ p, const float* __restrict__ g,
                                                   float* __restrict__ m, float* __restrict__ v, int64_t chunks) {
  int64_t ch = blockIdx.x;
  if (ch >= chunks) return;
  f32x4 P[kVec], G[kVec], M[kVec], V[kVec];
  auto load = [&](int64_t c) {
    const int64_t base = c * kChunk + int64_t(threadIdx.x) * 4;
#pragma unroll
    for (int u = 0; u < kVec; ++u) {
      const int64_t i = base + u * 1024;
      P[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + i));
      G[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(g + i));
      M[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(m + i));
      V[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(v + i));
    }
  };
  load(ch);
  for (; ch < chunks; ch += gridDim.x) {
    f32x4 P2[kVec], M2[kVec], V2[kVec];
#pragma unroll
    for (int u = 0; u < kVec; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float pp = P[u][j], mm = M[u][j], vv = V[u][j];
        adam_update(pp, G[u][j], mm, vv);
        P2[u][j] = pp;
        M2[u][j] = mm;
        V2[u][j] = vv;
      }
    if (ch + gridDim.x < chunks) load(ch + gridDim.x);
    const int64_t base = ch * kChunk + int64_t(threadIdx.x) * 4;
#pragma unroll
    for (int u = 0; u < kVec; ++u) {
      const int64_t i = base + u * 1024;
      __builtin_nontemporal_store(P2[u], reinterpret_cast<f32x4*>(p + i));
      __builtin_nontemporal_store(M2[u], reinterpret_cast<f32x4*>(m + i));
      __builtin_nontemporal_store(V2[u], reinterpret_cast<f32x4*>(v + i));
    }
  }
}

// The 4-read / 3-write in-place mix with its memory schedule as parameters:
// VEC float4 per stream per thread per chunk (chunk = 1024 * VEC elements,
// bytes in flight per thread = 64 * VEC), PREFETCH issues the next chunk's
// loads before this chunk's stores, CONTIG gives each workgroup one
// contiguous run of chunks instead of dealing them round-robin.
template <int VEC, bool PREFETCH, bool CONTIG>
__global__ __launch_bounds__(256) void mix_sweep_kernel(float* __restrict__ p, const float* __restrict__ g,
                                                        float* __restrict__ m, float* __restrict__ v,
                                                        int64_t chunks) {
  constexpr int64_t CH = 1024 * VEC;
  const int64_t per = (chunks + gridDim.x - 1) / gridDim.x;
  const int64_t first = CONTIG ? int64_t(blockIdx.x) * per : blockIdx.x;
  const int64_t last = CONTIG ? std::min<int64_t>(chunks, first + per) : chunks;
  const int64_t step = CONTIG ? 1 : gridDim.x;
  f32x4 P[VEC], G[VEC], M[VEC], V[VEC];
  auto load = [&](int64_t c) {
    const int64_t base = c * CH + int64_t(threadIdx.x) * 4;
#pragma unroll
    for (int u = 0; u < VEC; ++u) {
      const int64_t i = base + u * 1024;
      P[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p + i));
      G[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(g + i));
      M[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(m + i));
      V[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(v + i));
    }
  };
  if (first >= last) return;
  if (PREFETCH) load(first);
  for (int64_t ch = first; ch < last; ch += step) {
    if (!PREFETCH) load(ch);
    f32x4 P2[VEC], M2[VEC], V2[VEC];
#pragma unroll
    for (int u = 0; u < VEC; ++u) {
      M2[u] = M[u] * 0.5f + G[u];
      V2[u] = V[u] * 0.5f + G[u];
      P2[u] = P[u] * 0.5f + M2[u] - V2[u];
    }
    if (PREFETCH && ch + step < last) load(ch + step);
    const int64_t base = ch * CH + int64_t(threadIdx.x) * 4;
#pragma unroll
    for (int u = 0; u < VEC; ++u) {
      const int64_t i = base + u * 1024;
      __builtin_nontemporal_store(P2[u], reinterpret_cast<f32x4*>(p + i));
      __builtin_nontemporal_store(M2[u], reinterpret_cast<f32x4*>(m + i));
      __builtin_nontemporal_store(V2[u], reinterpret_cast<f32x4*>(v + i));
    }
  }
}

template <int VEC, bool PREFETCH, bool CONTIG>
void launch_sweep(float* const* b, int64_t n, unsigned grid, hipStream_t s) {
  hipLaunchKernelGGL((mix_sweep_kernel<VEC, PREFETCH, CONTIG>), dim3(grid), dim3(256), 0, s, b[0], b[1], b[2], b[3],
                     n / (1024 * VEC));
}

template <int VEC>
void launch_sweep_v(int prefetch, int contig, float* const* b, int64_t n, unsigned grid, hipStream_t s) {
  if (prefetch && contig) launch_sweep<VEC, true, true>(b, n, grid, s);
  else if (prefetch) launch_sweep<VEC, true, false>(b, n, grid, s);
  else if (contig) launch_sweep<VEC, false, true>(b, n, grid, s);
  else launch_sweep<VEC, false, false>(b, n, grid, s);
}

}  // namespace

// The 4-read / 3-write mix under one memory schedule (mix_sweep_kernel): vec
// in {1, 2, 4, 8}, prefetch / contig 0 or 1, per_cu workgroups per CU.  n must
// be a multiple of 8192.
extern "C" int mxp_mix_sweep(int vec, int prefetch, int contig, float* const* bufs, int64_t n, int per_cu,
                             void* stream) {
  if (n <= 0 || n % 8192 != 0 || per_cu <= 0) return int(hipErrorInvalidValue);
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return int(e);
  const unsigned grid = unsigned(std::min<int64_t>(n / (1024 * vec), int64_t(cus) * per_cu));
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (vec) {
    case 1: launch_sweep_v<1>(prefetch, contig, bufs, n, grid, s); break;
    case 2: launch_sweep_v<2>(prefetch, contig, bufs, n, grid, s); break;
    case 4: launch_sweep_v<4>(prefetch, contig, bufs, n, grid, s); break;
    case 8: launch_sweep_v<8>(prefetch, contig, bufs, n, grid, s); break;
    default: return int(hipErrorInvalidValue);
  }
  return int(hipGetLastError());
}

namespace {
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int SHAPE>
__global__ __launch_bounds__(256) void mfma_chain_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                          int iters, unsigned long long* __restrict__ clk) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  float a[8], b[8];
  for (int i = 0; i < 8; ++i) {
    a[i] = in[(t * 16 + i) & 1048575];
    b[i] = in[(t * 16 + 8 + i) & 1048575];
  }
  const uint64_t c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  float s = 0.f;
  if constexpr (SHAPE == 0) {
    f32x16 acc[4];
    for (int j = 0; j < 4; ++j) acc[j] = f32x16{0.f};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int q = 0; q < 8; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[q], b[(q + j) & 7], acc[j], 0, 0, 0);
    }
    for (int j = 0; j < 4; ++j)
      for (int v = 0; v < 16; ++v) s += acc[j][v];
  } else {
    f32x4 acc[16];
    for (int j = 0; j < 16; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < 16; ++j)
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[(q + j) & 7], b[(q * 3 + j) & 7], acc[j], 0, 0, 0);
    }
    for (int j = 0; j < 16; ++j)
      for (int v = 0; v < 4; ++v) s += acc[j][v];
  }
  const uint64_t c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  out[t] = s;
  if (threadIdx.x == 0) {
    clk[2 * blockIdx.x] = c1 - c0;
    clk[2 * blockIdx.x + 1] = r1 - r0;
  }
}
}  // namespace

extern "C" int mxp_mfma_chain(int shape, const float* in, float* out, int blocks, int iters,
                              unsigned long long* clk, void* stream) {
  if (blocks <= 0 || iters <= 0 || shape < 0 || shape > 1) return int(hipErrorInvalidValue);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (shape == 0)
    hipLaunchKernelGGL(mfma_chain_kernel<0>, dim3(blocks), dim3(256), 0, s, in, out, iters, clk);
  else
    hipLaunchKernelGGL(mfma_chain_kernel<1>, dim3(blocks), dim3(256), 0, s, in, out, iters, clk);
  return int(hipGetLastError());
}

extern "C" int mxp_stream(int kind, float* const* bufs, int64_t n, int per_cu, void* stream) {
  if (n <= 0 || n % kChunk != 0 || per_cu <= 0 || kind < 0 || kind > 3) return int(hipErrorInvalidValue);
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return int(e);
  const int64_t chunks = n / kChunk;
  const unsigned grid = unsigned(std::min<int64_t>(chunks, int64_t(cus) * per_cu));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (kind == 0)
    hipLaunchKernelGGL(copy_kernel, dim3(grid), dim3(256), 0, s, bufs[0], bufs[1], chunks);
  else if (kind == 1)
    hipLaunchKernelGGL(read_kernel, dim3(grid), dim3(256), 0, s, bufs[0], bufs[1], bufs[2], bufs[3], bufs[4], chunks);
  else if (kind == 2)
    hipLaunchKernelGGL(mix_kernel, dim3(grid), dim3(256), 0, s, bufs[0], bufs[1], bufs[2], bufs[3], chunks);
  else
    hipLaunchKernelGGL(math_kernel, dim3(grid), dim3(256), 0, s, bufs[0], bufs[1], bufs[2], bufs[3], chunks);
  return int(hipGetLastError());
}
