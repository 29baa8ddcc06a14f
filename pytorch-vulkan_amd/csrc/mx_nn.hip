// Normalisation, activation, resampling, softmax and loss kernels of the
// C3/C4 training steps (FP32, contiguous NCHW), all HBM-bound.
//
// Reference operators whose behaviour these follow (their CPU results are the
// parity target):
//   GroupNorm   csrc/ops/group_norm.cpp:73-153, group_norm_forward.comp,
//               group_norm_backward_input.comp, group_norm_backward_affine.comp
//   BatchNorm   csrc/ops/batch_norm.cpp:21-110, batch_norm_forward.comp,
//               batch_norm_backward.comp
//   SiLU        csrc/ops/diffusion_unary.cpp:42-57,143-151 (diffusion_unary*.comp op 0)
//   ReLU        csrc/ops/mm.cpp:475-495 (relu.comp, threshold_backward.comp)
//   nearest 2d  csrc/ops/upsample.cpp:7-56, upsample_nearest2d.comp
//   softmax     csrc/ops/mm.cpp:1100 (softmax_axis.comp),
//               csrc/ops/softmax_axis_backward.cpp:11-38
//   MSE loss    csrc/ops/loss_primitives.cpp:349-356
//   cat         csrc/ops/cat.cpp:8-58 (cat_copy.comp)
//
// GroupNorm runs one workgroup per (sample, group) when a group has at most
// 1024 channels (gn_fwd_fused_kernel / gn_bwd_fused_kernel); wider groups and
// BatchNorm share the row structure below.  The tensor is seen as rows
// r = n*C + c of HW contiguous elements.  Statistics are gathered per row by
// one wave (a centred two-pass over the row, so the second read comes from the
// cache), merged per group / channel with Chan's pairwise formula (exact for
// equal-size parts, no E[x^2]-E[x]^2 cancellation), and the merge writes a
// per-row coefficient table that a float4 elementwise pass applies.  The
// backward is the same: per-row sum(dy) and sum(dy*(x-mean)), a merge into
// per-row coefficients (dx = p*dy + k*(x-mean) + q) and the affine gradients,
// and the elementwise pass.  Every reduction has a fixed order, so results are
// bitwise reproducible run to run.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>

#include "mx_internal.hpp"

namespace mx {
namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / 64;

int grid_for(int64_t threads_needed) {
  return int(std::max<int64_t>(1, std::min<int64_t>((threads_needed + kThreads - 1) / kThreads,
                                                    int64_t(cu_count()) * 32)));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Lane 0's value in every lane (read through a scalar register: lane 0 is the
// first active lane wherever these reductions run, with the whole wave active).
__device__ __forceinline__ float lane0(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

// The value of lane l + o for a wave tree's step o: LDS permutes across
// the 16-lane rows (o = 32, 16), a DPP row shift inside them (o <= 8; a lane
// whose source lies past its row reads 0, and lane 0's tree never uses it).
template <int O>
__device__ __forceinline__ float lane_down(float v) {
  if constexpr (O >= 16) {
    return __shfl_down(v, O, 64);
  } else {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x100 + O, 0xf, 0xf, true));
  }
}

// Sum over the 64 lanes of a wave, the same value returned to every lane:
// lane 0's tree v[l] += v[l + o] for o = 32, 16, ..., 1, broadcast.
__device__ __forceinline__ float wave_sum(float v) {
  v += lane_down<32>(v);
  v += lane_down<16>(v);
  v += lane_down<8>(v);
  v += lane_down<4>(v);
  v += lane_down<2>(v);
  v += lane_down<1>(v);
  return lane0(v);
}

// Maximum over the 64 lanes (lane 0's tree, broadcast) with fmaxf, one
// v_max_f32 per step.  fmaxf drops a NaN operand; the softmax kernels, its
// only users, still give NaN for a row holding a NaN, since that element's
// exponential, the row sum and every quotient are NaN.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, lane_down<32>(v));
  v = fmaxf(v, lane_down<16>(v));
  v = fmaxf(v, lane_down<8>(v));
  v = fmaxf(v, lane_down<4>(v));
  v = fmaxf(v, lane_down<2>(v));
  v = fmaxf(v, lane_down<1>(v));
  return lane0(v);
}

// exp(d) for d <= 0 (or NaN), as the softmax forward needs it after taking
// the row maximum off.  Cody and Waite's split of the argument: d * log2(e)
// as a two-float product ph + pl (log2(e) split into its nearest float and the
// nearest float to the remainder, the low part of d * hi recovered exactly by
// an fma), n = rint(ph), exp(d) = 2^n * 2^((ph - n) + pl) with the hardware
// exp2 on the reduced argument (|.| <= 0.5) and ldexp.  The error is that of
// the exp2 plus half an ulp of the reduced argument, about 1 ulp.  No overflow
// branch (d never exceeds 0); below ln(2^-150), half the smallest subnormal,
// the result is 0 (also for d = -inf, where the reduction gives NaN).
__device__ __forceinline__ float exp_nonpos(float d) {
#pragma clang fp contract(off)
  constexpr float kLog2eHi = 1.44269502162933349609375f;   // float(log2 e)
  constexpr float kLog2eLo = 1.925963033500011079e-8f;     // float(log2 e - kLog2eHi)
  constexpr float kZeroBelow = -103.972076416015625f;      // float(ln 2^-150)
  const float ph = d * kLog2eHi;
  float pl = __builtin_fmaf(d, kLog2eHi, -ph);
  pl = __builtin_fmaf(d, kLog2eLo, pl);
  const float n = __builtin_rintf(ph);
  const float r = __builtin_ldexpf(__builtin_amdgcn_exp2f((ph - n) + pl), int(n));
  return d < kZeroBelow ? 0.f : r;
}

// 1 / s for a softmax row sum (s >= 1: the row maximum contributes
// exp(0) = 1; NaN for a NaN row): the hardware reciprocal refined by one
// Newton step, r + r (1 - s r), three instructions instead of the ten of an
// IEEE division.  The refined value is within an ulp of 1 / s.
__device__ __forceinline__ float recip_row_sum(float s) {
  const float r = __builtin_amdgcn_rcpf(s);
  return __builtin_fmaf(r, __builtin_fmaf(-s, r, 1.f), r);
}

// wave_sum / wave_max of R values at once: the same tree for each value, the
// R trees' cross-lane steps issued together so their latencies overlap.
template <int O, int R>
__device__ __forceinline__ void sum_step_n(float (&v)[R]) {
  float w[R];
#pragma unroll
  for (int k = 0; k < R; ++k) w[k] = lane_down<O>(v[k]);
#pragma unroll
  for (int k = 0; k < R; ++k) v[k] += w[k];
}

template <int O, int R>
__device__ __forceinline__ void max_step_n(float (&v)[R]) {
  float w[R];
#pragma unroll
  for (int k = 0; k < R; ++k) w[k] = lane_down<O>(v[k]);
#pragma unroll
  for (int k = 0; k < R; ++k) v[k] = fmaxf(v[k], w[k]);
}

template <int R>
__device__ __forceinline__ void wave_sum_n(float (&v)[R]) {
  sum_step_n<32>(v);
  sum_step_n<16>(v);
  sum_step_n<8>(v);
  sum_step_n<4>(v);
  sum_step_n<2>(v);
  sum_step_n<1>(v);
#pragma unroll
  for (int k = 0; k < R; ++k) v[k] = lane0(v[k]);
}

template <int R>
__device__ __forceinline__ void wave_max_n(float (&v)[R]) {
  max_step_n<32>(v);
  max_step_n<16>(v);
  max_step_n<8>(v);
  max_step_n<4>(v);
  max_step_n<2>(v);
  max_step_n<1>(v);
#pragma unroll
  for (int k = 0; k < R; ++k) v[k] = lane0(v[k]);
}

// ------------------------------------------------------------ row statistics
// mean_r and M2_r = sum (x - mean_r)^2 of each row of `hw` contiguous floats.
template <bool VEC>
__global__ __launch_bounds__(kThreads) void row_moments_kernel(const float* __restrict__ x, int64_t rows, int hw,
                                                               float* __restrict__ rmean, float* __restrict__ rm2) {
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* p = x + r * hw;
  float s = 0.f;
  if (VEC) {
    const float4* p4 = reinterpret_cast<const float4*>(p);
    for (int i = lane; i < hw / 4; i += 64) {
      const float4 v = p4[i];
      s += (v.x + v.y) + (v.z + v.w);
    }
  } else {
    for (int i = lane; i < hw; i += 64) s += p[i];
  }
  const float m = wave_sum(s) / float(hw);
  float q = 0.f;
  if (VEC) {
    const float4* p4 = reinterpret_cast<const float4*>(p);
    for (int i = lane; i < hw / 4; i += 64) {
      const float4 v = p4[i];
      const float a = v.x - m, b = v.y - m, c = v.z - m, d = v.w - m;
      q += (a * a + b * b) + (c * c + d * d);
    }
  } else {
    for (int i = lane; i < hw; i += 64) {
      const float a = p[i] - m;
      q += a * a;
    }
  }
  q = wave_sum(q);
  if (lane == 0) {
    rmean[r] = m;
    rm2[r] = q;
  }
}

// sum(dy) and sum(dy * (x - mean_s)) of each row; mean_s is the row's
// statistic: mean[(r / C) * stat_n + (r % C) / cpg] (GroupNorm: stat_n = G;
// BatchNorm: stat_n = 0, cpg = 1).
template <bool VEC>
__global__ __launch_bounds__(kThreads) void row_grad_kernel(const float* __restrict__ dy, const float* __restrict__ x,
                                                            const float* __restrict__ mean, int64_t rows, int hw,
                                                            int C, int stat_n, int cpg, float* __restrict__ sdy,
                                                            float* __restrict__ sdyx) {
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float mu = mean[(r / C) * stat_n + (r % C) / cpg];
  const float* pg = dy + r * hw;
  const float* px = x + r * hw;
  float a = 0.f, b = 0.f;
  if (VEC) {
    const float4* g4 = reinterpret_cast<const float4*>(pg);
    const float4* x4 = reinterpret_cast<const float4*>(px);
    for (int i = lane; i < hw / 4; i += 64) {
      const float4 g = g4[i], v = x4[i];
      a += (g.x + g.y) + (g.z + g.w);
      b += (g.x * (v.x - mu) + g.y * (v.y - mu)) + (g.z * (v.z - mu) + g.w * (v.w - mu));
    }
  } else {
    for (int i = lane; i < hw; i += 64) {
      const float g = pg[i];
      a += g;
      b += g * (px[i] - mu);
    }
  }
  a = wave_sum(a);
  b = wave_sum(b);
  if (lane == 0) {
    sdy[r] = a;
    sdyx[r] = b;
  }
}

// ---------------------------------------------------------------- GroupNorm
// One thread per (n, g): merge the group's cpg rows, write mean/rstd and the
// forward coefficients {mean, rstd*gamma_c, beta_c} of each row.
__global__ void gn_merge_kernel(const float* __restrict__ rmean, const float* __restrict__ rm2,
                                const float* __restrict__ gamma, const float* __restrict__ beta, int N, int C, int G,
                                int hw, float eps, float* __restrict__ mean, float* __restrict__ rstd,
                                float4* __restrict__ coef) {
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= int64_t(N) * G) return;
  const int n = int(t / G), g = int(t % G), cpg = C / G;
  const int64_t r0 = int64_t(n) * C + int64_t(g) * cpg;
  float s = 0.f;
  for (int i = 0; i < cpg; ++i) s += rmean[r0 + i];
  const float m = s / float(cpg);
  float m2 = 0.f, spread = 0.f;
  for (int i = 0; i < cpg; ++i) {
    const float d = rmean[r0 + i] - m;
    m2 += rm2[r0 + i];
    spread += d * d;
  }
  m2 += spread * float(hw);
  const float var = m2 / (float(cpg) * float(hw));
  const float inv = 1.f / sqrtf(var + eps);
  mean[t] = m;
  rstd[t] = inv;
  for (int i = 0; i < cpg; ++i) {
    const int c = g * cpg + i;
    coef[r0 + i] = make_float4(m, gamma ? inv * gamma[c] : inv, beta ? beta[c] : 0.f, 0.f);
  }
}

// One thread per (n, g): dx coefficients of the group's rows.
//   dx = rstd*(v - mean(v) - z*mean(v*z)),  v = gamma_c*dy,  z = (x-mean)*rstd
//      = p*dy + k*(x - mean) + q.
__global__ void gn_grad_merge_kernel(const float* __restrict__ sdy, const float* __restrict__ sdyx,
                                     const float* __restrict__ mean, const float* __restrict__ rstd,
                                     const float* __restrict__ gamma, int N, int C, int G, int hw,
                                     float4* __restrict__ coef) {
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= int64_t(N) * G) return;
  const int n = int(t / G), g = int(t % G), cpg = C / G;
  const int64_t r0 = int64_t(n) * C + int64_t(g) * cpg;
  const float inv = rstd[t], mu = mean[t];
  float sv = 0.f, svz = 0.f;
  for (int i = 0; i < cpg; ++i) {
    const float w = gamma ? gamma[g * cpg + i] : 1.f;
    sv += w * sdy[r0 + i];
    svz += w * sdyx[r0 + i];
  }
  svz *= inv;
  const float cnt = float(cpg) * float(hw);
  const float k = -inv * inv * (svz / cnt);
  const float q = -inv * (sv / cnt);
  for (int i = 0; i < cpg; ++i) {
    const float w = gamma ? gamma[g * cpg + i] : 1.f;
    coef[r0 + i] = make_float4(inv * w, k, q, mu);
  }
}

// One thread per channel: dgamma_c = sum_n sdyx[n,c]*rstd[n,g],
// dbeta_c = sum_n sdy[n,c], in n order.
__global__ void gn_affine_kernel(const float* __restrict__ sdy, const float* __restrict__ sdyx,
                                 const float* __restrict__ rstd, int N, int C, int G, float* __restrict__ dgamma,
                                 float* __restrict__ dbeta) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  const int g = c / (C / G);
  float dw = 0.f, db = 0.f;
  // Sixteen samples' loads go out before their sums (still added in n order):
  // one dependent load per sample would cost a memory round trip each.
  constexpr int kB = 16;
  int n = 0;
  for (; n + kB <= N; n += kB) {
    float a[kB], b[kB], r[kB];
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      const int64_t i = int64_t(n + j) * C + c;
      a[j] = sdyx[i];
      b[j] = sdy[i];
      r[j] = rstd[int64_t(n + j) * G + g];
    }
#pragma unroll
    for (int j = 0; j < kB; ++j) {
      dw += a[j] * r[j];
      db += b[j];
    }
  }
  for (; n < N; ++n) {
    const int64_t i = int64_t(n) * C + c;
    dw += sdyx[i] * rstd[int64_t(n) * G + g];
    db += sdy[i];
  }
  if (dgamma) dgamma[c] = dw;
  if (dbeta) dbeta[c] = db;
}

// One workgroup per (n, g) for the common GroupNorm shapes (at most
// kGnMaxCpg channels per group): the group's cpg*hw elements are contiguous,
// so the statistics, the normalisation and, in the backward, the per-channel
// sums all come from one block of memory that stays in L2 / the Infinity Cache
// between passes.  Forward is one launch, backward two (the second sums the
// per-sample affine partials over n).
constexpr int kGnMaxCpg = 1024;

// Sum of one value per thread over the block, the same result in every
// thread (fixed order: wave trees, then waves 0..3).
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float t = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return t;
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void gn_fwd_fused_kernel(const float* __restrict__ x,
                                                                const float* __restrict__ gamma,
                                                                const float* __restrict__ beta, int C, int G, int hw,
                                                                float eps, float* __restrict__ y,
                                                                float* __restrict__ mean, float* __restrict__ rstd) {
  __shared__ float red[kWavesPerBlock];
  const int ng = blockIdx.x;
  const int n = ng / G, g = ng - (ng / G) * G, cpg = C / G;
  const int count = cpg * hw;
  const int64_t base = (int64_t(n) * C + int64_t(g) * cpg) * hw;
  const float* p = x + base;
  float* q = y + base;
  float s = 0.f;
  if (VEC) {
    const float4* p4 = reinterpret_cast<const float4*>(p);
    for (int i = threadIdx.x; i < count / 4; i += kThreads) {
      const float4 v = p4[i];
      s += (v.x + v.y) + (v.z + v.w);
    }
  } else {
    for (int i = threadIdx.x; i < count; i += kThreads) s += p[i];
  }
  const float m = block_sum(s, red) / float(count);
  float sq = 0.f;
  if (VEC) {
    const float4* p4 = reinterpret_cast<const float4*>(p);
    for (int i = threadIdx.x; i < count / 4; i += kThreads) {
      const float4 v = p4[i];
      const float a = v.x - m, b = v.y - m, c = v.z - m, d = v.w - m;
      sq += (a * a + b * b) + (c * c + d * d);
    }
  } else {
    for (int i = threadIdx.x; i < count; i += kThreads) {
      const float a = p[i] - m;
      sq += a * a;
    }
  }
  const float inv = 1.f / sqrtf(block_sum(sq, red) / float(count) + eps);
  if (threadIdx.x == 0) {
    mean[ng] = m;
    rstd[ng] = inv;
  }
  const int c0 = g * cpg;
  if (VEC) {
    const float4* p4 = reinterpret_cast<const float4*>(p);
    float4* q4 = reinterpret_cast<float4*>(q);
    for (int i = threadIdx.x; i < count / 4; i += kThreads) {
      const int c = c0 + (4 * i) / hw;
      const float a = gamma ? inv * gamma[c] : inv, b = beta ? beta[c] : 0.f;
      const float4 v = p4[i];
      q4[i] = make_float4((v.x - m) * a + b, (v.y - m) * a + b, (v.z - m) * a + b, (v.w - m) * a + b);
    }
  } else {
    for (int i = threadIdx.x; i < count; i += kThreads) {
      const int c = c0 + i / hw;
      const float a = gamma ? inv * gamma[c] : inv, b = beta ? beta[c] : 0.f;
      q[i] = (p[i] - m) * a + b;
    }
  }
}

// Per (n, g): per-channel sum(dy) and sum(dy * (x - mean)) (waves over the
// group's channels, lanes over the channel's plane), written to the affine
// partials [n][c]; the group totals of v = gamma_c * dy and v * (x - mean) in
// channel order; then dx = p_c * dy + k * (x - mean) + q (see gn_grad_merge_kernel).
template <bool VEC>
__global__ __launch_bounds__(kThreads) void gn_bwd_fused_kernel(const float* __restrict__ dy,
                                                                const float* __restrict__ x,
                                                                const float* __restrict__ mean,
                                                                const float* __restrict__ rstd,
                                                                const float* __restrict__ gamma, int C, int G, int hw,
                                                                float* __restrict__ dx, float* __restrict__ part_dy,
                                                                float* __restrict__ part_dyx) {
  // No multiply-add contraction: the fused and register-resident kernels then
  // perform the same roundings in the same order whatever the compiler's
  // instruction scheduling, so their results are bit-identical.
#pragma clang fp contract(off)
  __shared__ float sdy[kGnMaxCpg], sdyx[kGnMaxCpg];
  __shared__ float tot[2];
  const int ng = blockIdx.x;
  const int n = ng / G, g = ng - (ng / G) * G, cpg = C / G;
  const int64_t base = (int64_t(n) * C + int64_t(g) * cpg) * hw;
  const float mu = mean[ng], inv = rstd[ng];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int ci = wave; ci < cpg; ci += kWavesPerBlock) {
    const float* pg = dy + base + int64_t(ci) * hw;
    const float* px = x + base + int64_t(ci) * hw;
    float a = 0.f, b = 0.f;
    if (VEC) {
      const float4* g4 = reinterpret_cast<const float4*>(pg);
      const float4* x4 = reinterpret_cast<const float4*>(px);
      for (int i = lane; i < hw / 4; i += 64) {
        const float4 gv = g4[i], v = x4[i];
        a += (gv.x + gv.y) + (gv.z + gv.w);
        b += (gv.x * (v.x - mu) + gv.y * (v.y - mu)) + (gv.z * (v.z - mu) + gv.w * (v.w - mu));
      }
    } else {
      for (int i = lane; i < hw; i += 64) {
        const float gv = pg[i];
        a += gv;
        b += gv * (px[i] - mu);
      }
    }
    a = wave_sum(a);
    b = wave_sum(b);
    if (lane == 0) {
      sdy[ci] = a;
      sdyx[ci] = b;
      const int64_t r = int64_t(n) * C + int64_t(g) * cpg + ci;
      part_dy[r] = a;
      part_dyx[r] = b;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float sv = 0.f, svx = 0.f;
    for (int ci = 0; ci < cpg; ++ci) {
      const float w = gamma ? gamma[g * cpg + ci] : 1.f;
      sv += w * sdy[ci];
      svx += w * sdyx[ci];
    }
    tot[0] = sv;
    tot[1] = svx;
  }
  __syncthreads();
  if (!dx) return;
  const int count = cpg * hw;
  const float cnt = float(count);
  const float k = -inv * inv * inv * (tot[1] / cnt);
  const float q = -inv * (tot[0] / cnt);
  const int c0 = g * cpg;
  if (VEC) {
    const float4* g4 = reinterpret_cast<const float4*>(dy + base);
    const float4* x4 = reinterpret_cast<const float4*>(x + base);
    float4* d4 = reinterpret_cast<float4*>(dx + base);
    for (int i = threadIdx.x; i < count / 4; i += kThreads) {
      const int c = c0 + (4 * i) / hw;
      const float pc = gamma ? inv * gamma[c] : inv;
      const float4 gv = g4[i], v = x4[i];
      d4[i] = make_float4(pc * gv.x + k * (v.x - mu) + q, pc * gv.y + k * (v.y - mu) + q,
                          pc * gv.z + k * (v.z - mu) + q, pc * gv.w + k * (v.w - mu) + q);
    }
  } else {
    for (int i = threadIdx.x; i < count; i += kThreads) {
      const int c = c0 + i / hw;
      const float pc = gamma ? inv * gamma[c] : inv;
      dx[base + i] = pc * dy[base + i] + k * (x[base + i] - mu) + q;
    }
  }
}

// Streaming variants of the two kernels above for 16-byte aligned groups
// whose bytes fit a buffer resource: each thread keeps a batch of float4
// loads in flight per pass (in the element-wise pass the next batch is
// loaded before the current one is stored), gamma / beta come from LDS, and
// masked lanes use an out-of-range buffer offset (the load reads 0, the
// store is dropped), so the stores form straight-line code.  Per thread the
// elements, the order of their sums and every expression are those of the
// loops above, so the results are bit-identical.
typedef float nn_f32x4 __attribute__((ext_vector_type(4)));
typedef int nn_i32x4 __attribute__((ext_vector_type(4)));
extern "C" __device__ nn_f32x4 mx_nn_buffer_load_v4f32(nn_i32x4 rsrc, int voffset, int soffset, int aux) __asm(
    "llvm.amdgcn.raw.buffer.load.v4f32");
extern "C" __device__ void mx_nn_buffer_store_v4f32(nn_f32x4 v, nn_i32x4 rsrc, int voffset, int soffset,
                                                    int aux) __asm("llvm.amdgcn.raw.buffer.store.v4f32");
constexpr int kGnBatch = 4;
constexpr int kNnOffNone = int(0x80000000u);

// Buffer resource over [base, base + bytes) (bytes < 2^31): raw addressing,
// 32-bit elements; an offset at or past the extent reads 0 / drops the store.
__device__ __forceinline__ nn_i32x4 nn_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  nn_i32x4 r;
  r.x = __builtin_amdgcn_readfirstlane(int(uint32_t(a)));
  r.y = __builtin_amdgcn_readfirstlane(int(uint32_t(a >> 32) & 0xFFFFu));
  r.z = __builtin_amdgcn_readfirstlane(int(bytes));
  r.w = 0x00020000;
  return r;
}

__global__ __launch_bounds__(kThreads) void gn_fwd_stream_kernel(const float* __restrict__ x,
                                                                 const float* __restrict__ gamma,
                                                                 const float* __restrict__ beta, int C, int G,
                                                                 int hw, float eps, float* __restrict__ y,
                                                                 float* __restrict__ mean,
                                                                 float* __restrict__ rstd) {
  __shared__ float red[kWavesPerBlock];
  __shared__ float saff[2 * kGnMaxCpg];
  const int ng = blockIdx.x;
  const int n = ng / G, g = ng - (ng / G) * G, cpg = C / G;
  const int count = cpg * hw, count4 = count / 4;
  const int64_t base = (int64_t(n) * C + int64_t(g) * cpg) * hw;
  const int c0 = g * cpg;
  const nn_i32x4 rx = nn_rsrc(x + base, uint32_t(count) * 4u);
  const nn_i32x4 ry = nn_rsrc(y + base, uint32_t(count) * 4u);
  for (int ci = threadIdx.x; ci < cpg; ci += kThreads) {
    saff[ci] = gamma ? gamma[c0 + ci] : 1.f;
    saff[kGnMaxCpg + ci] = beta ? beta[c0 + ci] : 0.f;
  }
  auto off = [&](int i) { return i < count4 ? 16 * i : kNnOffNone; };
  constexpr int kStep = kGnBatch * kThreads;
  float s = 0.f;
  for (int i0 = threadIdx.x; i0 < count4; i0 += kStep) {
    nn_f32x4 v[kGnBatch];
#pragma unroll
    for (int u = 0; u < kGnBatch; ++u) v[u] = mx_nn_buffer_load_v4f32(rx, off(i0 + u * kThreads), 0, 0);
#pragma unroll
    for (int u = 0; u < kGnBatch; ++u)
      if (i0 + u * kThreads < count4) s += (v[u].x + v[u].y) + (v[u].z + v[u].w);
  }
  const float m = block_sum(s, red) / float(count);
  float sq = 0.f;
  for (int i0 = threadIdx.x; i0 < count4; i0 += kStep) {
    nn_f32x4 v[kGnBatch];
#pragma unroll
    for (int u = 0; u < kGnBatch; ++u) v[u] = mx_nn_buffer_load_v4f32(rx, off(i0 + u * kThreads), 0, 0);
#pragma unroll
    for (int u = 0; u < kGnBatch; ++u) {
      if (i0 + u * kThreads < count4) {
        const float a = v[u].x - m, b = v[u].y - m, c = v[u].z - m, d = v[u].w - m;
        sq += (a * a + b * b) + (c * c + d * d);
      }
    }
  }
  const float inv = 1.f / sqrtf(block_sum(sq, red) / float(count) + eps);
  if (threadIdx.x == 0) {
    mean[ng] = m;
    rstd[ng] = inv;
  }
  nn_f32x4 cur[kGnBatch];
#pragma unroll
  for (int u = 0; u < kGnBatch; ++u) cur[u] = mx_nn_buffer_load_v4f32(rx, off(threadIdx.x + u * kThreads), 0, 0);
  for (int i0 = threadIdx.x; i0 < count4; i0 += kStep) {
    nn_f32x4 nxt[kGnBatch];
#pragma unroll
    for (int u = 0; u < kGnBatch; ++u) nxt[u] = mx_nn_buffer_load_v4f32(rx, off(i0 + kStep + u * kThreads), 0, 0);
#pragma unroll
    for (int u = 0; u < kGnBatch; ++u) {
      const int i = i0 + u * kThreads;
      const int cl = (4 * min(i, count4 - 1)) / hw;
      const float a = inv * saff[cl], b = saff[kGnMaxCpg + cl];  // gamma == 1 without one: inv * 1 == inv
      const nn_f32x4 v = cur[u];
      const nn_f32x4 o = {(v.x - m) * a + b, (v.y - m) * a + b, (v.z - m) * a + b, (v.w - m) * a + b};
      mx_nn_buffer_store_v4f32(o, ry, off(i), 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kGnBatch; ++u) cur[u] = nxt[u];
  }
}

__global__ __launch_bounds__(kThreads) void gn_bwd_stream_kernel(const float* __restrict__ dy,
                                                                 const float* __restrict__ x,
                                                                 const float* __restrict__ mean,
                                                                 const float* __restrict__ rstd,
                                                                 const float* __restrict__ gamma, int C, int G,
                                                                 int hw, float* __restrict__ dx,
                                                                 float* __restrict__ part_dy,
                                                                 float* __restrict__ part_dyx) {
#pragma clang fp contract(off)
  __shared__ float sdy[kGnMaxCpg], sdyx[kGnMaxCpg], sg[kGnMaxCpg];
  __shared__ float tot[2];
  const int ng = blockIdx.x;
  const int n = ng / G, g = ng - (ng / G) * G, cpg = C / G;
  const int count = cpg * hw, count4 = count / 4, hw4 = hw / 4;
  const int64_t base = (int64_t(n) * C + int64_t(g) * cpg) * hw;
  const float mu = mean[ng], inv = rstd[ng];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const nn_i32x4 rg = nn_rsrc(dy + base, uint32_t(count) * 4u);
  const nn_i32x4 rx = nn_rsrc(x + base, uint32_t(count) * 4u);
  for (int ci = threadIdx.x; ci < cpg; ci += kThreads) sg[ci] = gamma ? gamma[g * cpg + ci] : 1.f;
  for (int ci = wave; ci < cpg; ci += kWavesPerBlock) {
    float a = 0.f, b = 0.f;
    auto coff = [&](int i) { return i < hw4 ? 16 * (ci * hw4 + i) : kNnOffNone; };
    for (int i0 = lane; i0 < hw4; i0 += kGnBatch * 64) {
      nn_f32x4 gv[kGnBatch], xv[kGnBatch];
#pragma unroll
      for (int u = 0; u < kGnBatch; ++u) {
        gv[u] = mx_nn_buffer_load_v4f32(rg, coff(i0 + 64 * u), 0, 0);
        xv[u] = mx_nn_buffer_load_v4f32(rx, coff(i0 + 64 * u), 0, 0);
      }
#pragma unroll
      for (int u = 0; u < kGnBatch; ++u) {
        if (i0 + 64 * u < hw4) {
          const nn_f32x4 gg = gv[u], v = xv[u];
          a += (gg.x + gg.y) + (gg.z + gg.w);
          b += (gg.x * (v.x - mu) + gg.y * (v.y - mu)) + (gg.z * (v.z - mu) + gg.w * (v.w - mu));
        }
      }
    }
    a = wave_sum(a);
    b = wave_sum(b);
    if (lane == 0) {
      sdy[ci] = a;
      sdyx[ci] = b;
      const int64_t r = int64_t(n) * C + int64_t(g) * cpg + ci;
      part_dy[r] = a;
      part_dyx[r] = b;
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float sv = 0.f, svx = 0.f;
    for (int ci = 0; ci < cpg; ++ci) {
      const float w = sg[ci];
      sv += w * sdy[ci];
      svx += w * sdyx[ci];
    }
    tot[0] = sv;
    tot[1] = svx;
  }
  __syncthreads();
  if (!dx) return;
  const float cnt = float(count);
  const float k = -inv * inv * inv * (tot[1] / cnt);
  const float q = -inv * (tot[0] / cnt);
  const nn_i32x4 rd = nn_rsrc(dx + base, uint32_t(count) * 4u);
  auto off = [&](int i) { return i < count4 ? 16 * i : kNnOffNone; };
  constexpr int kStep = kGnBatch * kThreads;
  nn_f32x4 cg[kGnBatch], cx[kGnBatch];
#pragma unroll
  for (int u = 0; u < kGnBatch; ++u) {
    cg[u] = mx_nn_buffer_load_v4f32(rg, off(threadIdx.x + u * kThreads), 0, 0);
    cx[u] = mx_nn_buffer_load_v4f32(rx, off(threadIdx.x + u * kThreads), 0, 0);
  }
  for (int i0 = threadIdx.x; i0 < count4; i0 += kStep) {
    nn_f32x4 ng4[kGnBatch], nx4[kGnBatch];
#pragma unroll
    for (int u = 0; u < kGnBatch; ++u) {
      ng4[u] = mx_nn_buffer_load_v4f32(rg, off(i0 + kStep + u * kThreads), 0, 0);
      nx4[u] = mx_nn_buffer_load_v4f32(rx, off(i0 + kStep + u * kThreads), 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kGnBatch; ++u) {
      const int i = i0 + u * kThreads;
      const float pc = inv * sg[(4 * min(i, count4 - 1)) / hw];
      const nn_f32x4 gg = cg[u], v = cx[u];
      const nn_f32x4 o = {pc * gg.x + k * (v.x - mu) + q, pc * gg.y + k * (v.y - mu) + q,
                          pc * gg.z + k * (v.z - mu) + q, pc * gg.w + k * (v.w - mu) + q};
      mx_nn_buffer_store_v4f32(o, rd, off(i), 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kGnBatch; ++u) {
      cg[u] = ng4[u];
      cx[u] = nx4[u];
    }
  }
}

// Register-resident variants of the two kernels above for groups that fit a
// workgroup's registers (forward: at most 32 float4 per thread; backward: at
// most 16 per thread of 4 or 8 waves; 16-byte aligned planes): each element
// is read from HBM once instead of three times (forward) or twice
// (backward).  Every thread holds exactly the elements the multi-pass
// kernel's loops give it, in the same order, and each channel's backward sums
// are one wave's over the same lanes and elements, so the sums and the
// results are bit-identical to that kernel's.
template <int NPT>
__global__ __launch_bounds__(kThreads) void gn_fwd_regs_kernel(const float* __restrict__ x,
                                                               const float* __restrict__ gamma,
                                                               const float* __restrict__ beta, int C, int G, int hw,
                                                               float eps, float* __restrict__ y,
                                                               float* __restrict__ mean, float* __restrict__ rstd) {
  // Up to 16 float4 per thread, each element's gamma / beta ride in
  // registers; with 32 the group's gamma / beta go to LDS instead (the
  // registers hold the data).
  constexpr bool kLdsAffine = NPT > 16;
  __shared__ float red[kWavesPerBlock];
  __shared__ float saff[kLdsAffine ? 2 * kGnMaxCpg : 1];
  const int ng = blockIdx.x;
  const int n = ng / G, g = ng - (ng / G) * G, cpg = C / G;
  const int count = cpg * hw, count4 = count / 4;
  const int64_t base = (int64_t(n) * C + int64_t(g) * cpg) * hw;
  const float4* p4 = reinterpret_cast<const float4*>(x + base);
  const int c0 = g * cpg;
  float4 v[NPT];
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int i = threadIdx.x + kThreads * j;
    v[j] = i < count4 ? p4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  // The affine parameters of each element's channel, loaded with the data:
  // a load between the stores below would make each store wait for the
  // earlier ones (loads and stores share one counter).  The LDS copy is read
  // after block_sum's barriers.
  float ga[kLdsAffine ? 1 : NPT], be[kLdsAffine ? 1 : NPT];
  if constexpr (kLdsAffine) {
    for (int ci = threadIdx.x; ci < cpg; ci += kThreads) {
      saff[ci] = gamma ? gamma[c0 + ci] : 1.f;
      saff[kGnMaxCpg + ci] = beta ? beta[c0 + ci] : 0.f;
    }
  } else {
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      const int i = threadIdx.x + kThreads * j;
      const int c = c0 + (4 * min(i, count4 - 1)) / hw;
      ga[j] = gamma ? gamma[c] : 1.f;
      be[j] = beta ? beta[c] : 0.f;
    }
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NPT; ++j)
    if (threadIdx.x + kThreads * j < count4) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  const float m = block_sum(s, red) / float(count);
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    if (threadIdx.x + kThreads * j < count4) {
      const float a = v[j].x - m, b = v[j].y - m, c = v[j].z - m, d = v[j].w - m;
      sq += (a * a + b * b) + (c * c + d * d);
    }
  }
  const float inv = 1.f / sqrtf(block_sum(sq, red) / float(count) + eps);
  if (threadIdx.x == 0) {
    mean[ng] = m;
    rstd[ng] = inv;
  }
  float4* q4 = reinterpret_cast<float4*>(y + base);
#pragma unroll
  for (int j = 0; j < NPT; ++j) {
    const int i = threadIdx.x + kThreads * j;
    if (i >= count4) continue;
    float a, b;  // gamma == 1 without one: inv * 1 == inv exactly
    if constexpr (kLdsAffine) {
      const int cl = (4 * i) / hw;
      a = inv * saff[cl];
      b = saff[kGnMaxCpg + cl];
    } else {
      a = inv * ga[j];
      b = be[j];
    }
    q4[i] = make_float4((v[j].x - m) * a + b, (v[j].y - m) * a + b, (v[j].z - m) * a + b, (v[j].w - m) * a + b);
  }
}

// Backward: with W waves, wave w holds channels w, w + W, ... of the group
// and lanes the plane's float4 lane, lane + 64, ... (np of them per channel),
// for dy and x.  W = 8 takes groups that need more than 16 float4 per thread
// at 4 waves.  FULL: every one of a thread's NPT slots holds a valid float4
// (channels per group a multiple of W, planes a multiple of 256 floats, NPT
// equal to (cpg / W) * (hw / 256)), so loads and stores carry no per-slot
// condition and form straight-line code (a conditional store block makes the
// compiler wait for every earlier store at its entry).
template <int NPT, bool FULL, int W>
__global__ __launch_bounds__(64 * W) void gn_bwd_regs_kernel(const float* __restrict__ dy,
                                                               const float* __restrict__ x,
                                                               const float* __restrict__ mean,
                                                               const float* __restrict__ rstd,
                                                               const float* __restrict__ gamma, int C, int G, int hw,
                                                               float* __restrict__ dx, float* __restrict__ part_dy,
                                                               float* __restrict__ part_dyx) {
  // No multiply-add contraction: the fused and register-resident kernels then
  // perform the same roundings in the same order whatever the compiler's
  // instruction scheduling, so their results are bit-identical.
#pragma clang fp contract(off)
  __shared__ float sdy[kGnMaxCpg], sdyx[kGnMaxCpg], sg[kGnMaxCpg];
  __shared__ float tot[2];
  const int ng = blockIdx.x;
  const int n = ng / G, g = ng - (ng / G) * G, cpg = C / G;
  const int64_t base = (int64_t(n) * C + int64_t(g) * cpg) * hw;
  const float mu = mean[ng], inv = rstd[ng];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int hw4 = hw / 4, np = (hw4 + 63) / 64;
  const float4* g4 = reinterpret_cast<const float4*>(dy + base);
  const float4* x4 = reinterpret_cast<const float4*>(x + base);
  float4 gv[NPT], xv[NPT];
  // Element k of this thread: channel wave + 4 (k / np), plane float4 lane + 64 (k % np).
#pragma unroll
  for (int k = 0; k < NPT; ++k) {
    const int ci = wave + W * (k / np), i = lane + 64 * (k % np);
    const bool ok = FULL || (ci < cpg && i < hw4);
    gv[k] = ok ? g4[int64_t(ci) * hw4 + i] : make_float4(0.f, 0.f, 0.f, 0.f);
    xv[k] = ok ? x4[int64_t(ci) * hw4 + i] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  // The group's gamma (1 without one: inv * 1 == inv exactly) goes to LDS, so
  // the dx stores below have neither a global load nor a branch between them
  // (loads and stores share one counter: such a load would make each store
  // wait for the earlier ones).
  for (int ci = threadIdx.x; ci < cpg; ci += 64 * W) sg[ci] = gamma ? gamma[g * cpg + ci] : 1.f;
  for (int cb = 0; cb * W < cpg; ++cb) {
    const int ci = wave + W * cb;
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int k = 0; k < NPT; ++k) {
      if (k / np != cb || (!FULL && lane + 64 * (k % np) >= hw4)) continue;
      const float4 gg = gv[k], v = xv[k];
      a += (gg.x + gg.y) + (gg.z + gg.w);
      b += (gg.x * (v.x - mu) + gg.y * (v.y - mu)) + (gg.z * (v.z - mu) + gg.w * (v.w - mu));
    }
    if (FULL || ci < cpg) {
      a = wave_sum(a);
      b = wave_sum(b);
      if (lane == 0) {
        sdy[ci] = a;
        sdyx[ci] = b;
        const int64_t r = int64_t(n) * C + int64_t(g) * cpg + ci;
        part_dy[r] = a;
        part_dyx[r] = b;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float sv = 0.f, svx = 0.f;
    for (int ci = 0; ci < cpg; ++ci) {
      const float w = sg[ci];
      sv += w * sdy[ci];
      svx += w * sdyx[ci];
    }
    tot[0] = sv;
    tot[1] = svx;
  }
  __syncthreads();
  if (!dx) return;
  const float cnt = float(cpg * hw);
  const float kk = -inv * inv * inv * (tot[1] / cnt);
  const float q = -inv * (tot[0] / cnt);
  // Every dx value first (into gv), then the stores: each store reads its own
  // registers, so none waits for an earlier one to release its data.
#pragma unroll
  for (int k = 0; k < NPT; ++k) {
    const float pc = inv * sg[min(wave + W * (k / np), cpg - 1)];
    const float4 gg = gv[k], v = xv[k];
    gv[k] = make_float4(pc * gg.x + kk * (v.x - mu) + q, pc * gg.y + kk * (v.y - mu) + q,
                        pc * gg.z + kk * (v.z - mu) + q, pc * gg.w + kk * (v.w - mu) + q);
  }
  float4* d4 = reinterpret_cast<float4*>(dx + base);
#pragma unroll
  for (int k = 0; k < NPT; ++k) {
    const int ci = wave + W * (k / np), i = lane + 64 * (k % np);
    if (FULL || (ci < cpg && i < hw4)) d4[int64_t(ci) * hw4 + i] = gv[k];
  }
}

// ---------------------------------------------------------------- BatchNorm
// One thread per channel: merge the N rows of channel c.  Training: batch
// mean / inverse std (0 when var == eps == 0, as torch's InvStd) and the
// running-statistics update with the unbiased variance; evaluation: running
// statistics.  Writes the forward coefficients of every row of the channel.
__global__ void bn_merge_kernel(const float* __restrict__ rmean, const float* __restrict__ rm2,
                                const float* __restrict__ gamma, const float* __restrict__ beta,
                                float* __restrict__ run_mean, int64_t rm_stride, float* __restrict__ run_var,
                                int64_t rv_stride, int N, int C, int hw, int training, float momentum, float eps,
                                float* __restrict__ save_mean, float* __restrict__ save_inv,
                                float4* __restrict__ coef) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  float m, inv;
  if (training) {
    float s = 0.f;
    for (int n = 0; n < N; ++n) s += rmean[int64_t(n) * C + c];
    m = s / float(N);
    float m2 = 0.f, spread = 0.f;
    for (int n = 0; n < N; ++n) {
      const float d = rmean[int64_t(n) * C + c] - m;
      m2 += rm2[int64_t(n) * C + c];
      spread += d * d;
    }
    m2 += spread * float(hw);
    const float cnt = float(N) * float(hw);
    const float var = m2 / cnt;
    inv = (var == 0.f && eps == 0.f) ? 0.f : 1.f / sqrtf(var + eps);
    save_mean[c] = m;
    save_inv[c] = inv;
    if (run_mean) run_mean[c * rm_stride] = momentum * m + (1.f - momentum) * run_mean[c * rm_stride];
    if (run_var) run_var[c * rv_stride] = momentum * (m2 / (cnt - 1.f)) + (1.f - momentum) * run_var[c * rv_stride];
  } else {
    m = run_mean[c * rm_stride];
    inv = 1.f / sqrtf(run_var[c * rv_stride] + eps);
  }
  const float a = gamma ? inv * gamma[c] : inv, b = beta ? beta[c] : 0.f;
  for (int n = 0; n < N; ++n) coef[int64_t(n) * C + c] = make_float4(m, a, b, 0.f);
}

// One thread per channel: dx coefficients and the affine gradients.
//   training: dx = gamma*inv*(dy - S1/M - (x-mean)*inv^2*S2/M)
//   eval:     dx = gamma*inv*dy   (inv from the running variance)
__global__ void bn_grad_merge_kernel(const float* __restrict__ sdy, const float* __restrict__ sdyx,
                                     const float* __restrict__ mean, const float* __restrict__ inv_or_var,
                                     const float* __restrict__ gamma, int N, int C, int hw, int training, float eps,
                                     float* __restrict__ dgamma, float* __restrict__ dbeta,
                                     float4* __restrict__ coef) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  float s1 = 0.f, s2 = 0.f;
  for (int n = 0; n < N; ++n) {
    s1 += sdy[int64_t(n) * C + c];
    s2 += sdyx[int64_t(n) * C + c];
  }
  const float inv = training ? inv_or_var[c] : 1.f / sqrtf(inv_or_var[c] + eps);
  const float w = gamma ? gamma[c] : 1.f;
  const float cnt = float(N) * float(hw);
  if (dgamma) dgamma[c] = s2 * inv;
  if (dbeta) dbeta[c] = s1;
  if (!coef) return;
  const float p = w * inv;
  const float k = training ? -p * inv * inv * (s2 / cnt) : 0.f;
  const float q = training ? -p * (s1 / cnt) : 0.f;
  const float mu = mean[c];
  for (int n = 0; n < N; ++n) coef[int64_t(n) * C + c] = make_float4(p, k, q, mu);
}

// ------------------------------------------------------------- apply passes
// y = (x - c.x) * c.y + c.z with c = coef[element / hw].
template <bool VEC>
__global__ __launch_bounds__(kThreads) void norm_apply_kernel(const float* __restrict__ x,
                                                              const float4* __restrict__ coef, int64_t total, int hw,
                                                              float* __restrict__ y) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  if (VEC) {
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float4* y4 = reinterpret_cast<float4*>(y);
    const int hw4 = hw / 4;
    const bool narrow = total / 4 <= int64_t(UINT32_MAX);
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total / 4; i += stride) {
      const float4 c = coef[narrow ? int64_t(uint32_t(i) / uint32_t(hw4)) : i / hw4];
      const float4 v = x4[i];
      y4[i] = make_float4((v.x - c.x) * c.y + c.z, (v.y - c.x) * c.y + c.z, (v.z - c.x) * c.y + c.z,
                          (v.w - c.x) * c.y + c.z);
    }
  } else {
    const bool narrow = total <= int64_t(UINT32_MAX);
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
      const float4 c = coef[narrow ? int64_t(uint32_t(i) / uint32_t(hw)) : i / hw];
      y[i] = (x[i] - c.x) * c.y + c.z;
    }
  }
}

// dx = c.x*dy + c.y*(x - c.w) + c.z with c = coef[element / hw].
template <bool VEC>
__global__ __launch_bounds__(kThreads) void norm_grad_apply_kernel(const float* __restrict__ dy,
                                                                   const float* __restrict__ x,
                                                                   const float4* __restrict__ coef, int64_t total,
                                                                   int hw, float* __restrict__ dx) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  if (VEC) {
    const float4* g4 = reinterpret_cast<const float4*>(dy);
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float4* d4 = reinterpret_cast<float4*>(dx);
    const int hw4 = hw / 4;
    const bool narrow = total / 4 <= int64_t(UINT32_MAX);
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total / 4; i += stride) {
      const float4 c = coef[narrow ? int64_t(uint32_t(i) / uint32_t(hw4)) : i / hw4];
      const float4 g = g4[i], v = x4[i];
      d4[i] = make_float4(c.x * g.x + c.y * (v.x - c.w) + c.z, c.x * g.y + c.y * (v.y - c.w) + c.z,
                          c.x * g.z + c.y * (v.z - c.w) + c.z, c.x * g.w + c.y * (v.w - c.w) + c.z);
    }
  } else {
    const bool narrow = total <= int64_t(UINT32_MAX);
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
      const float4 c = coef[narrow ? int64_t(uint32_t(i) / uint32_t(hw)) : i / hw];
      dx[i] = c.x * dy[i] + c.y * (x[i] - c.w) + c.z;
    }
  }
}

// ---------------------------------------------------------------- pointwise
// SiLU and its derivative as torch's CPU kernels: x / (1 + exp(-x)) and
// dy * s * (1 + x * (1 - s)), s = 1 / (1 + exp(-x)).  ReLU keeps NaN (x <= 0
// is false for NaN); threshold_backward: x <= threshold ? 0 : dy.
enum UnaryOp { kSilu = 0, kRelu = 1 };
enum UnaryGradOp { kSiluGrad = 0, kThresholdGrad = 1 };

template <int OP>
__device__ __forceinline__ float unary(float v) {
  if (OP == kSilu) return v / (1.f + expf(-v));
  return v <= 0.f ? 0.f : v;
}

template <int OP>
__device__ __forceinline__ float unary_grad(float g, float v, float thr) {
  if (OP == kSiluGrad) {
    const float s = 1.f / (1.f + expf(-v));
    return g * (s * (1.f + v * (1.f - s)));
  }
  return v <= thr ? 0.f : g;
}

template <int OP>
__global__ __launch_bounds__(kThreads) void unary_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                         int64_t n) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  const int64_t n4 = (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15 ? 0 : n / 4;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
    const float4 v = reinterpret_cast<const float4*>(x)[i];
    reinterpret_cast<float4*>(y)[i] = make_float4(unary<OP>(v.x), unary<OP>(v.y), unary<OP>(v.z), unary<OP>(v.w));
  }
  for (int64_t i = n4 * 4 + int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    y[i] = unary<OP>(x[i]);
}

template <int OP>
__global__ __launch_bounds__(kThreads) void unary_grad_kernel(const float* __restrict__ dy,
                                                              const float* __restrict__ x, float thr,
                                                              float* __restrict__ dx, int64_t n) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  const uintptr_t bits =
      reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(dy) | reinterpret_cast<uintptr_t>(dx);
  const int64_t n4 = (bits & 15) ? 0 : n / 4;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
    const float4 g = reinterpret_cast<const float4*>(dy)[i];
    const float4 v = reinterpret_cast<const float4*>(x)[i];
    reinterpret_cast<float4*>(dx)[i] = make_float4(unary_grad<OP>(g.x, v.x, thr), unary_grad<OP>(g.y, v.y, thr),
                                                   unary_grad<OP>(g.z, v.z, thr), unary_grad<OP>(g.w, v.w, thr));
  }
  for (int64_t i = n4 * 4 + int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    dx[i] = unary_grad<OP>(dy[i], x[i], thr);
}

// ----------------------------------------------------------- nearest resize
// Source index of output index `o` as torch's CPU nearest_idx: identity for
// equal sizes, o >> 1 for exact doubling, else min(floor(o * scale), in - 1)
// in float with scale = 1/scale_factor or in/out.
struct NearestAxis {
  int in, out;
  float scale;
  int mode;  // 0 identity, 1 halving, 2 general
};

__device__ __forceinline__ int nearest_src(const NearestAxis& a, int o) {
  if (a.mode == 0) return o;
  if (a.mode == 1) return o >> 1;
  const int s = int(floorf(float(o) * a.scale));
  return s < a.in - 1 ? s : a.in - 1;
}

// First output index whose source index is >= target (sources are
// nondecreasing in the output index).
__device__ int nearest_lower_bound(const NearestAxis& a, int target) {
  if (target <= 0) return 0;
  if (target >= a.in) return a.out;
  if (a.mode == 0) return target;
  if (a.mode == 1) return 2 * target;
  int lo = 0, hi = a.out;
  while (lo < hi) {
    const int mid = lo + (hi - lo) / 2;
    if (nearest_src(a, mid) < target)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

__global__ __launch_bounds__(kThreads) void upsample_nearest_kernel(const float* __restrict__ x,
                                                                    float* __restrict__ y, int64_t planes,
                                                                    NearestAxis ah, NearestAxis aw) {
  const int64_t total = planes * ah.out * aw.out;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int ow = int(i % aw.out);
    const int64_t t = i / aw.out;
    const int oh = int(t % ah.out);
    const int64_t plane = t / ah.out;
    y[i] = x[(plane * ah.in + nearest_src(ah, oh)) * aw.in + nearest_src(aw, ow)];
  }
}

// dx[ih, iw] = sum of dy over the output pixels that read (ih, iw), in
// row-major output order (the order torch's CPU backward accumulates them).
__global__ __launch_bounds__(kThreads) void upsample_nearest_grad_kernel(const float* __restrict__ dy,
                                                                         float* __restrict__ dx, int64_t planes,
                                                                         NearestAxis ah, NearestAxis aw) {
  const int64_t total = planes * ah.in * aw.in;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int iw = int(i % aw.in);
    const int64_t t = i / aw.in;
    const int ih = int(t % ah.in);
    const int64_t plane = t / ah.in;
    const int hb = nearest_lower_bound(ah, ih), he = nearest_lower_bound(ah, ih + 1);
    const int wb = nearest_lower_bound(aw, iw), we = nearest_lower_bound(aw, iw + 1);
    const float* p = dy + plane * ah.out * aw.out;
    float s = 0.f;
    for (int oh = hb; oh < he; ++oh)
      for (int ow = wb; ow < we; ++ow) s += p[int64_t(oh) * aw.out + ow];
    dx[i] = s;
  }
}

// Exact 2x in both axes (iw even, 8-byte aligned x, 16-byte aligned y): a
// thread reads two neighbouring inputs (8 bytes) and writes their 2x2 blocks
// as two 16-byte rows.  32-bit indices (the host checks the sizes).
__global__ __launch_bounds__(kThreads) void upsample2x_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                              uint32_t rows, uint32_t half_w) {
  const uint32_t total = rows * half_w;
  for (uint32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < total; t += gridDim.x * blockDim.x) {
    const uint32_t row = t / half_w, j = t - row * half_w;  // row = plane * ih + input row
    const float2 a = reinterpret_cast<const float2*>(x)[t];
    const float4 v = make_float4(a.x, a.x, a.y, a.y);
    float4* out = reinterpret_cast<float4*>(y) + (2 * row) * half_w + j;
    out[0] = v;
    out[half_w] = v;
  }
}

// Its gradient: the 2x2 block of each input summed in row-major output order
// (((0 + d00) + d01) + d10) + d11, torch's CPU order.
__global__ __launch_bounds__(kThreads) void upsample2x_grad_kernel(const float* __restrict__ dy,
                                                                   float* __restrict__ dx, uint32_t rows,
                                                                   uint32_t half_w) {
  const uint32_t total = rows * half_w;
  for (uint32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < total; t += gridDim.x * blockDim.x) {
    const uint32_t row = t / half_w, j = t - row * half_w;
    const float4* in = reinterpret_cast<const float4*>(dy) + (2 * row) * half_w + j;
    const float4 r0 = in[0], r1 = in[half_w];
    // From a zero start, as the general kernel (a sum of negative zeros is +0).
    reinterpret_cast<float2*>(dx)[t] = make_float2((((0.f + r0.x) + r0.y) + r1.x) + r1.y,
                                                   (((0.f + r0.z) + r0.w) + r1.z) + r1.w);
  }
}

// ------------------------------------------------------------------ softmax
// Last axis (inner == 1): one wave per row.  y = exp(x - max) * (1 / sum).
__global__ __launch_bounds__(kThreads) void softmax_last_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                                int64_t rows, int len) {
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* p = x + r * len;
  float* q = y + r * len;
  float m = -std::numeric_limits<float>::infinity();
  for (int i = lane; i < len; i += 64) m = fmaxf(m, p[i]);
  m = wave_max(m);
  float s = 0.f;
  for (int i = lane; i < len; i += 64) s += exp_nonpos(p[i] - m);
  const float inv = recip_row_sum(wave_sum(s));
  for (int i = lane; i < len; i += 64) q[i] = exp_nonpos(p[i] - m) * inv;
}

// dx = y * (dy - sum(dy * y)) over the last axis, one wave per row.
__global__ __launch_bounds__(kThreads) void softmax_last_grad_kernel(const float* __restrict__ dy,
                                                                     const float* __restrict__ y,
                                                                     float* __restrict__ dx, int64_t rows, int len) {
  const int lane = threadIdx.x & 63;
  const int64_t r = int64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float* g = dy + r * len;
  const float* p = y + r * len;
  float s = 0.f;
  for (int i = lane; i < len; i += 64) s += g[i] * p[i];
  s = wave_sum(s);
  for (int i = lane; i < len; i += 64) dx[r * len + i] = p[i] * (g[i] - s);
}

// Rows of len % 4 == 0 floats (16-byte aligned), len <= 256 NV: each wave
// holds R consecutive rows in registers, lane l owning float4s l, l + 64, ...
// of every row; each element is read once and its exponential computed once.
// All R rows' loads are issued before the first reduction, so a wave keeps
// R * NV float4 per lane in flight (short rows would otherwise leave a wave
// waiting on one 16-byte load).  Per row the arithmetic and its order do not
// depend on R.
template <int NV, int R>
__global__ __launch_bounds__(kThreads) void softmax_rows_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                                int64_t rows, int len) {
  const int lane = threadIdx.x & 63;
  const int64_t r0 = (int64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6)) * R;
  if (r0 >= rows) return;
  const int n4 = len / 4;
  const float ninf = -std::numeric_limits<float>::infinity();
  float e[R][NV][4];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const float4* p = reinterpret_cast<const float4*>(x + (r0 + k) * len);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int i = lane + 64 * j;
      const float4 v = (r0 + k < rows && i < n4) ? p[i] : make_float4(ninf, ninf, ninf, ninf);
      e[k][j][0] = v.x;
      e[k][j][1] = v.y;
      e[k][j][2] = v.z;
      e[k][j][3] = v.w;
    }
  }
  // Rows past the end hold -inf (their results are never stored).
  float m[R], sum[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    m[k] = ninf;
#pragma unroll
    for (int j = 0; j < NV; ++j)
#pragma unroll
      for (int c = 0; c < 4; ++c) m[k] = fmaxf(m[k], e[k][j][c]);
  }
  wave_max_n<R>(m);
#pragma unroll
  for (int k = 0; k < R; ++k) {
    sum[k] = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const bool ok = lane + 64 * j < n4;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        e[k][j][c] = exp_nonpos(e[k][j][c] - m[k]);
        if (ok) sum[k] += e[k][j][c];
      }
    }
  }
  wave_sum_n<R>(sum);
#pragma unroll
  for (int k = 0; k < R; ++k) {
    if (r0 + k >= rows) break;
    const float inv = recip_row_sum(sum[k]);
    float4* q = reinterpret_cast<float4*>(y + (r0 + k) * len);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int i = lane + 64 * j;
      if (i < n4) q[i] = make_float4(e[k][j][0] * inv, e[k][j][1] * inv, e[k][j][2] * inv, e[k][j][3] * inv);
    }
  }
}

template <int NV, int R>
__global__ __launch_bounds__(kThreads) void softmax_rows_grad_kernel(const float* __restrict__ dy,
                                                                     const float* __restrict__ y,
                                                                     float* __restrict__ dx, int64_t rows, int len) {
  // No multiply-add contraction: the rounding of each product does not depend
  // on how the compiler schedules the R rows.
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int64_t r0 = (int64_t(blockIdx.x) * kWavesPerBlock + (threadIdx.x >> 6)) * R;
  if (r0 >= rows) return;
  const int n4 = len / 4;
  float4 gv[R][NV], pv[R][NV];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const float4* g4 = reinterpret_cast<const float4*>(dy + (r0 + k) * len);
    const float4* p4 = reinterpret_cast<const float4*>(y + (r0 + k) * len);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int i = lane + 64 * j;
      const bool ok = r0 + k < rows && i < n4;
      gv[k][j] = ok ? g4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      pv[k][j] = ok ? p4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  float sum[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    sum[k] = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      if (lane + 64 * j < n4) {
        const float4 g = gv[k][j], p = pv[k][j];
        sum[k] += ((g.x * p.x + g.y * p.y) + g.z * p.z) + g.w * p.w;
      }
    }
  }
  wave_sum_n<R>(sum);
#pragma unroll
  for (int k = 0; k < R; ++k) {
    if (r0 + k >= rows) break;
    const float s = sum[k];
    float4* d4 = reinterpret_cast<float4*>(dx + (r0 + k) * len);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int i = lane + 64 * j;
      if (i < n4)
        d4[i] = make_float4(pv[k][j].x * (gv[k][j].x - s), pv[k][j].y * (gv[k][j].y - s),
                            pv[k][j].z * (gv[k][j].z - s), pv[k][j].w * (gv[k][j].w - s));
    }
  }
}

// Axis with inner > 1: one thread per (outer, inner) column, loads coalesced
// across the inner index.
__global__ __launch_bounds__(kThreads) void softmax_inner_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                                 int64_t outer, int64_t axis, int64_t inner) {
  const int64_t cols = outer * inner;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t c = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; c < cols; c += stride) {
    const int64_t o = c / inner, in = c % inner;
    const float* p = x + o * axis * inner + in;
    float* q = y + o * axis * inner + in;
    float m = -std::numeric_limits<float>::infinity();
    for (int64_t a = 0; a < axis; ++a) m = fmaxf(m, p[a * inner]);
    float s = 0.f;
    for (int64_t a = 0; a < axis; ++a) s += exp_nonpos(p[a * inner] - m);
    const float inv = recip_row_sum(s);
    for (int64_t a = 0; a < axis; ++a) q[a * inner] = exp_nonpos(p[a * inner] - m) * inv;
  }
}

__global__ __launch_bounds__(kThreads) void softmax_inner_grad_kernel(const float* __restrict__ dy,
                                                                      const float* __restrict__ y,
                                                                      float* __restrict__ dx, int64_t outer,
                                                                      int64_t axis, int64_t inner) {
  const int64_t cols = outer * inner;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t c = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; c < cols; c += stride) {
    const int64_t base = (c / inner) * axis * inner + c % inner;
    float s = 0.f;
    for (int64_t a = 0; a < axis; ++a) s += dy[base + a * inner] * y[base + a * inner];
    for (int64_t a = 0; a < axis; ++a) dx[base + a * inner] = y[base + a * inner] * (dy[base + a * inner] - s);
  }
}

// ------------------------------------------------------------------ MSE loss
// Stage 1: per-block sums of (x - t)^2 over a fixed grid-stride partition.
__global__ __launch_bounds__(kThreads) void sq_diff_partial_kernel(const float* __restrict__ x,
                                                                   const float* __restrict__ t, int64_t n,
                                                                   float* __restrict__ partial) {
  __shared__ float part[kWavesPerBlock];
  float s = 0.f;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    const float d = x[i] - t[i];
    s += d * d;
  }
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) partial[blockIdx.x] = (part[0] + part[1]) + (part[2] + part[3]);
}

// Stage 2: one block sums the partials in a fixed order and scales.
__global__ __launch_bounds__(kThreads) void sum_partials_kernel(const float* __restrict__ partial, int count,
                                                                float scale, float* __restrict__ out) {
  __shared__ float part[kWavesPerBlock];
  float s = 0.f;
  for (int i = threadIdx.x; i < count; i += blockDim.x) s += partial[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) out[0] = ((part[0] + part[1]) + (part[2] + part[3])) * scale;
}

__global__ __launch_bounds__(kThreads) void sq_diff_kernel(const float* __restrict__ x, const float* __restrict__ t,
                                                           int64_t n, float* __restrict__ y) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    const float d = x[i] - t[i];
    y[i] = d * d;
  }
}

// dx = norm * (x - t) * dy  (dy a device scalar for mean/sum, elementwise for
// none), norm = 2/n for mean, else 2: torch's CPU mse_backward order.
__global__ __launch_bounds__(kThreads) void mse_grad_kernel(const float* __restrict__ dy, int dy_scalar,
                                                            const float* __restrict__ x,
                                                            const float* __restrict__ t, int64_t n, float norm,
                                                            float* __restrict__ dx) {
  const float g0 = dy_scalar ? dy[0] : 0.f;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x)
    dx[i] = norm * (x[i] - t[i]) * (dy_scalar ? g0 : dy[i]);
}

// --------------------------------------------------------------- row copies
// dst[row * dst_pitch + j] = src[row * src_pitch + j], j < row_elems: rows
// over grid y (strided past 65535), elements over grid x.
template <class T>
__global__ __launch_bounds__(kThreads) void copy_rows_kernel(T* __restrict__ dst, int64_t dst_pitch,
                                                             const T* __restrict__ src, int64_t src_pitch,
                                                             int64_t row_elems, int64_t rows) {
  for (int64_t r = blockIdx.y; r < rows; r += gridDim.y) {
    T* d = dst + r * dst_pitch;
    const T* p = src + r * src_pitch;
    for (int64_t j = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; j < row_elems; j += int64_t(gridDim.x) * blockDim.x)
      d[j] = p[j];
  }
}

template <class T>
void launch_copy_rows(void* dst, int64_t dst_pitch, const void* src, int64_t src_pitch, int64_t row_bytes,
                      int64_t rows, hipStream_t s) {
  const int64_t elems = row_bytes / int64_t(sizeof(T));
  const int64_t gy = std::min<int64_t>(rows, 65535);
  const int64_t want = std::max<int64_t>(1, int64_t(cu_count()) * 8 / gy);
  const int64_t gx = std::max<int64_t>(1, std::min<int64_t>((elems + kThreads - 1) / kThreads, want));
  hipLaunchKernelGGL(copy_rows_kernel<T>, dim3(unsigned(gx), unsigned(gy)), dim3(kThreads), 0, s, static_cast<T*>(dst),
                     dst_pitch / int64_t(sizeof(T)), static_cast<const T*>(src), src_pitch / int64_t(sizeof(T)), elems,
                     rows);
}

int launch_rows(int64_t rows) { return int((rows + kWavesPerBlock - 1) / kWavesPerBlock); }

// Smallest register-array size of {1, 2, 4, ..., cap} holding `need` float4
// per thread (0: more than cap).
int regs_for(int64_t need, int cap = 16) {
  for (int r = 1; r <= cap; r *= 2)
    if (need <= r) return r;
  return 0;
}

NearestAxis nearest_axis(int64_t in, int64_t out, double scale) {
  NearestAxis a{int(in), int(out), 0.f, 2};
  if (out == in)
    a.mode = 0;
  else if (out == 2 * in)
    a.mode = 1;
  else
    a.scale = scale > 0 ? float(1.0 / scale) : float(in) / float(out);
  return a;
}

}  // namespace
}  // namespace mx

using namespace mx;

namespace {

// Shapes the row kernels take: rows of hw elements, int32 per row and per
// table entry, at least one element.
int check_rows(const char* who, int64_t n, int64_t c, int64_t hw) {
  MX_REQUIRE(n >= 0 && c > 0 && hw > 0, MX_ERR_INVALID, who, ": invalid batch, channel or spatial size");
  MX_REQUIRE(c <= INT32_MAX && hw <= INT32_MAX && n <= INT32_MAX, MX_ERR_INVALID, who, ": size exceeds int32");
  MX_REQUIRE(n * c <= int64_t(INT32_MAX) * kWavesPerBlock, MX_ERR_INVALID, who, ": too many rows");
  return MX_OK;
}

}  // namespace

extern "C" {

int mx_group_norm_forward(const float* x, const float* gamma, const float* beta, int64_t n, int64_t c, int64_t hw,
                          int64_t groups, float eps, float* y, float* mean, float* rstd, void* stream) {
  MX_ABI_BEGIN
  MX_TRY(check_rows("mx_group_norm_forward", n, c, hw));
  MX_REQUIRE(groups > 0 && c % groups == 0, MX_ERR_INVALID,
             "mx_group_norm_forward: channels must be divisible by groups");
  if (n == 0) return MX_OK;
  MX_REQUIRE(x && y && mean && rstd, MX_ERR_INVALID, "mx_group_norm_forward: null tensor");
  hipStream_t s = resolve_stream(stream);
  const int64_t cpg64 = c / groups;
  if (cpg64 <= kGnMaxCpg && cpg64 * hw <= INT32_MAX && n * groups <= INT32_MAX) {
    const bool vec4 = hw % 4 == 0 && aligned16(x) && aligned16(y);
    const int npt = vec4 ? regs_for((cpg64 * hw / 4 + kThreads - 1) / kThreads, 32) : 0;
    const dim3 grid(unsigned(n * groups));
    const int C = int(c), G = int(groups), HW = int(hw);
    switch (npt) {
      case 1: hipLaunchKernelGGL(gn_fwd_regs_kernel<1>, grid, dim3(kThreads), 0, s, x, gamma, beta, C, G, HW, eps, y,
                                 mean, rstd); break;
      case 2: hipLaunchKernelGGL(gn_fwd_regs_kernel<2>, grid, dim3(kThreads), 0, s, x, gamma, beta, C, G, HW, eps, y,
                                 mean, rstd); break;
      case 4: hipLaunchKernelGGL(gn_fwd_regs_kernel<4>, grid, dim3(kThreads), 0, s, x, gamma, beta, C, G, HW, eps, y,
                                 mean, rstd); break;
      case 8: hipLaunchKernelGGL(gn_fwd_regs_kernel<8>, grid, dim3(kThreads), 0, s, x, gamma, beta, C, G, HW, eps, y,
                                 mean, rstd); break;
      case 16: hipLaunchKernelGGL(gn_fwd_regs_kernel<16>, grid, dim3(kThreads), 0, s, x, gamma, beta, C, G, HW, eps,
                                  y, mean, rstd); break;
      case 32: hipLaunchKernelGGL(gn_fwd_regs_kernel<32>, grid, dim3(kThreads), 0, s, x, gamma, beta, C, G, HW, eps,
                                  y, mean, rstd); break;
      default: break;
    }
    if (npt) {
      MX_HIP(hipGetLastError());
      return MX_OK;
    }
    if (vec4 && cpg64 * hw * 4 < (int64_t(1) << 31))
      hipLaunchKernelGGL(gn_fwd_stream_kernel, dim3(unsigned(n * groups)), dim3(kThreads), 0, s, x, gamma, beta,
                         int(c), int(groups), int(hw), eps, y, mean, rstd);
    else if (vec4)
      hipLaunchKernelGGL(gn_fwd_fused_kernel<true>, dim3(unsigned(n * groups)), dim3(kThreads), 0, s, x, gamma, beta,
                         int(c), int(groups), int(hw), eps, y, mean, rstd);
    else
      hipLaunchKernelGGL(gn_fwd_fused_kernel<false>, dim3(unsigned(n * groups)), dim3(kThreads), 0, s, x, gamma,
                         beta, int(c), int(groups), int(hw), eps, y, mean, rstd);
    MX_HIP(hipGetLastError());
    return MX_OK;
  }
  const int64_t rows = n * c;
  Scratch stats, coef;
  MX_TRY(stats.alloc(size_t(rows) * 2 * sizeof(float), s));
  MX_TRY(coef.alloc(size_t(rows) * sizeof(float4), s));
  float* rmean = stats.as<float>();
  float* rm2 = rmean + rows;
  const bool vec = hw % 4 == 0 && aligned16(x) && aligned16(y);
  if (vec)
    hipLaunchKernelGGL(row_moments_kernel<true>, dim3(launch_rows(rows)), dim3(kThreads), 0, s, x, rows, int(hw),
                       rmean, rm2);
  else
    hipLaunchKernelGGL(row_moments_kernel<false>, dim3(launch_rows(rows)), dim3(kThreads), 0, s, x, rows, int(hw),
                       rmean, rm2);
  MX_HIP(hipGetLastError());
  const int64_t ng = n * groups;
  hipLaunchKernelGGL(gn_merge_kernel, dim3(int((ng + 255) / 256)), dim3(256), 0, s, rmean, rm2, gamma, beta, int(n),
                     int(c), int(groups), int(hw), eps, mean, rstd, coef.as<float4>());
  MX_HIP(hipGetLastError());
  const int64_t total = rows * hw;
  if (vec)
    hipLaunchKernelGGL(norm_apply_kernel<true>, dim3(grid_for(total / 4)), dim3(kThreads), 0, s, x,
                       coef.as<const float4>(), total, int(hw), y);
  else
    hipLaunchKernelGGL(norm_apply_kernel<false>, dim3(grid_for(total)), dim3(kThreads), 0, s, x,
                       coef.as<const float4>(), total, int(hw), y);
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

int mx_group_norm_backward(const float* dy, const float* x, const float* mean, const float* rstd, const float* gamma,
                           int64_t n, int64_t c, int64_t hw, int64_t groups, float* dx, float* dgamma, float* dbeta,
                           void* stream) {
  MX_ABI_BEGIN
  MX_TRY(check_rows("mx_group_norm_backward", n, c, hw));
  MX_REQUIRE(groups > 0 && c % groups == 0, MX_ERR_INVALID,
             "mx_group_norm_backward: channels must be divisible by groups");
  hipStream_t s = resolve_stream(stream);
  if (n == 0) {
    // No samples: the affine gradients are zero sums.
    if (dgamma) MX_TRY(mx_fill(dgamma, c, 4, 0, stream));
    if (dbeta) MX_TRY(mx_fill(dbeta, c, 4, 0, stream));
    return MX_OK;
  }
  if (!dx && !dgamma && !dbeta) return MX_OK;
  MX_REQUIRE(dy && x && mean && rstd, MX_ERR_INVALID, "mx_group_norm_backward: null tensor");
  const int64_t rows = n * c;
  Scratch sums, coef;
  MX_TRY(sums.alloc(size_t(rows) * 2 * sizeof(float), s));
  float* sdy = sums.as<float>();
  float* sdyx = sdy + rows;
  const bool vec = hw % 4 == 0 && aligned16(x) && aligned16(dy) && (!dx || aligned16(dx));
  const int cpg = int(c / groups);
  if (cpg <= kGnMaxCpg && int64_t(cpg) * hw <= INT32_MAX && n * groups <= INT32_MAX) {
    // Float4 per thread at 4 waves; groups that need more than 16 take 8.
    const int64_t np = (hw / 4 + 63) / 64;
    int waves = kWavesPerBlock;
    int npt = vec ? regs_for(int64_t((cpg + waves - 1) / waves) * np) : 0;
    if (vec && !npt) {
      waves = 2 * kWavesPerBlock;
      npt = regs_for(int64_t((cpg + waves - 1) / waves) * np);
    }
    const dim3 grid(unsigned(n * groups));
    const int C = int(c), G = int(groups), HW = int(hw);
    const bool full = npt && cpg % waves == 0 && hw % 256 == 0 && int64_t(cpg / waves) * (hw / 256) == npt;
#define MX_GN_BWD(N, W)                                                                                             \
  do {                                                                                                             \
    if (full)                                                                                                      \
      hipLaunchKernelGGL((gn_bwd_regs_kernel<N, true, W>), grid, dim3(64 * W), 0, s, dy, x, mean, rstd, gamma, C,   \
                         G, HW, dx, sdy, sdyx);                                                                    \
    else                                                                                                           \
      hipLaunchKernelGGL((gn_bwd_regs_kernel<N, false, W>), grid, dim3(64 * W), 0, s, dy, x, mean, rstd, gamma, C,  \
                         G, HW, dx, sdy, sdyx);                                                                    \
  } while (0)
    switch (waves == kWavesPerBlock ? npt : 32 + npt) {
      case 1: MX_GN_BWD(1, 4); break;
      case 2: MX_GN_BWD(2, 4); break;
      case 4: MX_GN_BWD(4, 4); break;
      case 8: MX_GN_BWD(8, 4); break;
      case 16: MX_GN_BWD(16, 4); break;
      case 32 + 16: MX_GN_BWD(16, 8); break;
      default:
        if (vec && int64_t(cpg) * hw * 4 < (int64_t(1) << 31))
          hipLaunchKernelGGL(gn_bwd_stream_kernel, grid, dim3(kThreads), 0, s, dy, x, mean, rstd, gamma, C, G, HW,
                             dx, sdy, sdyx);
        else if (vec)
          hipLaunchKernelGGL(gn_bwd_fused_kernel<true>, grid, dim3(kThreads), 0, s, dy, x, mean, rstd, gamma, C, G, HW,
                             dx, sdy, sdyx);
        else
          hipLaunchKernelGGL(gn_bwd_fused_kernel<false>, grid, dim3(kThreads), 0, s, dy, x, mean, rstd, gamma, C, G,
                             HW, dx, sdy, sdyx);
    }
#undef MX_GN_BWD
    MX_HIP(hipGetLastError());
    if (dgamma || dbeta) {
      hipLaunchKernelGGL(gn_affine_kernel, dim3(int((c + 255) / 256)), dim3(256), 0, s, sdy, sdyx, rstd, int(n),
                         int(c), int(groups), dgamma, dbeta);
      MX_HIP(hipGetLastError());
    }
    return MX_OK;
  }
  if (vec)
    hipLaunchKernelGGL(row_grad_kernel<true>, dim3(launch_rows(rows)), dim3(kThreads), 0, s, dy, x, mean, rows,
                       int(hw), int(c), int(groups), cpg, sdy, sdyx);
  else
    hipLaunchKernelGGL(row_grad_kernel<false>, dim3(launch_rows(rows)), dim3(kThreads), 0, s, dy, x, mean, rows,
                       int(hw), int(c), int(groups), cpg, sdy, sdyx);
  MX_HIP(hipGetLastError());
  if (dgamma || dbeta) {
    hipLaunchKernelGGL(gn_affine_kernel, dim3(int((c + 255) / 256)), dim3(256), 0, s, sdy, sdyx, rstd, int(n),
                       int(c), int(groups), dgamma, dbeta);
    MX_HIP(hipGetLastError());
  }
  if (dx) {
    MX_TRY(coef.alloc(size_t(rows) * sizeof(float4), s));
    const int64_t ng = n * groups;
    hipLaunchKernelGGL(gn_grad_merge_kernel, dim3(int((ng + 255) / 256)), dim3(256), 0, s, sdy, sdyx, mean, rstd,
                       gamma, int(n), int(c), int(groups), int(hw), coef.as<float4>());
    MX_HIP(hipGetLastError());
    const int64_t total = rows * hw;
    if (vec)
      hipLaunchKernelGGL(norm_grad_apply_kernel<true>, dim3(grid_for(total / 4)), dim3(kThreads), 0, s, dy, x,
                         coef.as<const float4>(), total, int(hw), dx);
    else
      hipLaunchKernelGGL(norm_grad_apply_kernel<false>, dim3(grid_for(total)), dim3(kThreads), 0, s, dy, x,
                         coef.as<const float4>(), total, int(hw), dx);
    MX_HIP(hipGetLastError());
  }
  return MX_OK;
  MX_ABI_END
}

int mx_batch_norm_forward(const float* x, const float* gamma, const float* beta, float* running_mean,
                          int64_t rm_stride, float* running_var, int64_t rv_stride, int64_t n, int64_t c, int64_t hw,
                          int training, float momentum, float eps, float* y, float* save_mean, float* save_invstd,
                          void* stream) {
  MX_ABI_BEGIN
  MX_TRY(check_rows("mx_batch_norm_forward", n, c, hw));
  MX_REQUIRE(n > 0, MX_ERR_INVALID, "mx_batch_norm_forward: empty batch");
  MX_REQUIRE(x && y, MX_ERR_INVALID, "mx_batch_norm_forward: null tensor");
  MX_REQUIRE(training || (running_mean && running_var), MX_ERR_INVALID,
             "mx_batch_norm_forward: evaluation requires running statistics");
  MX_REQUIRE(!training || (save_mean && save_invstd), MX_ERR_INVALID,
             "mx_batch_norm_forward: training requires the saved-statistics outputs");
  hipStream_t s = resolve_stream(stream);
  const int64_t rows = n * c;
  Scratch stats, coef;
  MX_TRY(coef.alloc(size_t(rows) * sizeof(float4), s));
  const bool vec = hw % 4 == 0 && aligned16(x) && aligned16(y);
  float *rmean = nullptr, *rm2 = nullptr;
  if (training) {
    MX_TRY(stats.alloc(size_t(rows) * 2 * sizeof(float), s));
    rmean = stats.as<float>();
    rm2 = rmean + rows;
    if (vec)
      hipLaunchKernelGGL(row_moments_kernel<true>, dim3(launch_rows(rows)), dim3(kThreads), 0, s, x, rows, int(hw),
                         rmean, rm2);
    else
      hipLaunchKernelGGL(row_moments_kernel<false>, dim3(launch_rows(rows)), dim3(kThreads), 0, s, x, rows,
                         int(hw), rmean, rm2);
    MX_HIP(hipGetLastError());
  }
  hipLaunchKernelGGL(bn_merge_kernel, dim3(int((c + 255) / 256)), dim3(256), 0, s, rmean, rm2, gamma, beta,
                     running_mean, rm_stride, running_var, rv_stride, int(n), int(c), int(hw), training, momentum, eps,
                     save_mean, save_invstd, coef.as<float4>());
  MX_HIP(hipGetLastError());
  const int64_t total = rows * hw;
  if (vec)
    hipLaunchKernelGGL(norm_apply_kernel<true>, dim3(grid_for(total / 4)), dim3(kThreads), 0, s, x,
                       coef.as<const float4>(), total, int(hw), y);
  else
    hipLaunchKernelGGL(norm_apply_kernel<false>, dim3(grid_for(total)), dim3(kThreads), 0, s, x,
                       coef.as<const float4>(), total, int(hw), y);
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

int mx_batch_norm_backward(const float* dy, const float* x, const float* gamma, const float* mean,
                           const float* invstd_or_var, int64_t n, int64_t c, int64_t hw, int training, float eps,
                           float* dx, float* dgamma, float* dbeta, void* stream) {
  MX_ABI_BEGIN
  MX_TRY(check_rows("mx_batch_norm_backward", n, c, hw));
  MX_REQUIRE(n > 0, MX_ERR_INVALID, "mx_batch_norm_backward: empty batch");
  if (!dx && !dgamma && !dbeta) return MX_OK;
  MX_REQUIRE(dy && x && mean && invstd_or_var, MX_ERR_INVALID, "mx_batch_norm_backward: null tensor");
  hipStream_t s = resolve_stream(stream);
  const int64_t rows = n * c;
  Scratch sums, coef;
  MX_TRY(sums.alloc(size_t(rows) * 2 * sizeof(float), s));
  float* sdy = sums.as<float>();
  float* sdyx = sdy + rows;
  const bool vec = hw % 4 == 0 && aligned16(x) && aligned16(dy) && (!dx || aligned16(dx));
  if (vec)
    hipLaunchKernelGGL(row_grad_kernel<true>, dim3(launch_rows(rows)), dim3(kThreads), 0, s, dy, x, mean, rows,
                       int(hw), int(c), 0, 1, sdy, sdyx);
  else
    hipLaunchKernelGGL(row_grad_kernel<false>, dim3(launch_rows(rows)), dim3(kThreads), 0, s, dy, x, mean, rows,
                       int(hw), int(c), 0, 1, sdy, sdyx);
  MX_HIP(hipGetLastError());
  if (dx) MX_TRY(coef.alloc(size_t(rows) * sizeof(float4), s));
  hipLaunchKernelGGL(bn_grad_merge_kernel, dim3(int((c + 255) / 256)), dim3(256), 0, s, sdy, sdyx, mean,
                     invstd_or_var, gamma, int(n), int(c), int(hw), training, eps, dgamma, dbeta,
                     dx ? coef.as<float4>() : nullptr);
  MX_HIP(hipGetLastError());
  if (dx) {
    const int64_t total = rows * hw;
    if (vec)
      hipLaunchKernelGGL(norm_grad_apply_kernel<true>, dim3(grid_for(total / 4)), dim3(kThreads), 0, s, dy, x,
                         coef.as<const float4>(), total, int(hw), dx);
    else
      hipLaunchKernelGGL(norm_grad_apply_kernel<false>, dim3(grid_for(total)), dim3(kThreads), 0, s, dy, x,
                         coef.as<const float4>(), total, int(hw), dx);
    MX_HIP(hipGetLastError());
  }
  return MX_OK;
  MX_ABI_END
}

int mx_unary_f32(int op, const float* x, float* y, int64_t count, void* stream) {
  MX_ABI_BEGIN
  MX_REQUIRE(count >= 0, MX_ERR_INVALID, "mx_unary_f32: negative count");
  if (count == 0) return MX_OK;
  MX_REQUIRE(x && y, MX_ERR_INVALID, "mx_unary_f32: null tensor");
  hipStream_t s = resolve_stream(stream);
  const dim3 grid(grid_for((count + 3) / 4));
  switch (op) {
    case MX_UNARY_SILU: hipLaunchKernelGGL(unary_kernel<kSilu>, grid, dim3(kThreads), 0, s, x, y, count); break;
    case MX_UNARY_RELU: hipLaunchKernelGGL(unary_kernel<kRelu>, grid, dim3(kThreads), 0, s, x, y, count); break;
    default: return set_error(MX_ERR_INVALID, cat("mx_unary_f32: unknown op ", op));
  }
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

int mx_unary_backward_f32(int op, const float* dy, const float* x, float threshold, float* dx, int64_t count,
                          void* stream) {
  MX_ABI_BEGIN
  MX_REQUIRE(count >= 0, MX_ERR_INVALID, "mx_unary_backward_f32: negative count");
  if (count == 0) return MX_OK;
  MX_REQUIRE(dy && x && dx, MX_ERR_INVALID, "mx_unary_backward_f32: null tensor");
  hipStream_t s = resolve_stream(stream);
  const dim3 grid(grid_for((count + 3) / 4));
  switch (op) {
    case MX_UNARY_SILU_GRAD:
      hipLaunchKernelGGL(unary_grad_kernel<kSiluGrad>, grid, dim3(kThreads), 0, s, dy, x, threshold, dx, count);
      break;
    case MX_UNARY_THRESHOLD_GRAD:
      hipLaunchKernelGGL(unary_grad_kernel<kThresholdGrad>, grid, dim3(kThreads), 0, s, dy, x, threshold, dx, count);
      break;
    default: return set_error(MX_ERR_INVALID, cat("mx_unary_backward_f32: unknown op ", op));
  }
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

int mx_upsample_nearest2d(const float* x, int64_t planes, int64_t ih, int64_t iw, int64_t oh, int64_t ow,
                          double scale_h, double scale_w, float* y, void* stream) {
  MX_ABI_BEGIN
  MX_REQUIRE(planes >= 0 && ih > 0 && iw > 0 && oh > 0 && ow > 0, MX_ERR_INVALID,
             "mx_upsample_nearest2d: sizes must be positive");
  MX_REQUIRE(ih <= INT32_MAX && iw <= INT32_MAX && oh <= INT32_MAX && ow <= INT32_MAX, MX_ERR_INVALID,
             "mx_upsample_nearest2d: size exceeds int32");
  if (planes == 0) return MX_OK;
  MX_REQUIRE(x && y, MX_ERR_INVALID, "mx_upsample_nearest2d: null tensor");
  hipStream_t s = resolve_stream(stream);
  const NearestAxis ah = nearest_axis(ih, oh, scale_h), aw = nearest_axis(iw, ow, scale_w);
  if (ah.mode == 1 && aw.mode == 1 && iw % 2 == 0 && (reinterpret_cast<uintptr_t>(x) & 7) == 0 && aligned16(y) &&
      planes * oh * ow <= INT32_MAX) {
    const uint32_t rows = uint32_t(planes * ih), half_w = uint32_t(iw / 2);
    hipLaunchKernelGGL(upsample2x_kernel, dim3(grid_for(int64_t(rows) * half_w)), dim3(kThreads), 0, s, x, y, rows,
                       half_w);
    MX_HIP(hipGetLastError());
    return MX_OK;
  }
  hipLaunchKernelGGL(upsample_nearest_kernel, dim3(grid_for(planes * oh * ow)), dim3(kThreads), 0, s, x, y, planes,
                     ah, aw);
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

int mx_upsample_nearest2d_backward(const float* dy, int64_t planes, int64_t ih, int64_t iw, int64_t oh, int64_t ow,
                                   double scale_h, double scale_w, float* dx, void* stream) {
  MX_ABI_BEGIN
  MX_REQUIRE(planes >= 0 && ih > 0 && iw > 0 && oh > 0 && ow > 0, MX_ERR_INVALID,
             "mx_upsample_nearest2d_backward: sizes must be positive");
  MX_REQUIRE(ih <= INT32_MAX && iw <= INT32_MAX && oh <= INT32_MAX && ow <= INT32_MAX, MX_ERR_INVALID,
             "mx_upsample_nearest2d_backward: size exceeds int32");
  if (planes == 0) return MX_OK;
  MX_REQUIRE(dy && dx, MX_ERR_INVALID, "mx_upsample_nearest2d_backward: null tensor");
  hipStream_t s = resolve_stream(stream);
  const NearestAxis ah = nearest_axis(ih, oh, scale_h), aw = nearest_axis(iw, ow, scale_w);
  if (ah.mode == 1 && aw.mode == 1 && iw % 2 == 0 && aligned16(dy) && (reinterpret_cast<uintptr_t>(dx) & 7) == 0 &&
      planes * oh * ow <= INT32_MAX) {
    const uint32_t rows = uint32_t(planes * ih), half_w = uint32_t(iw / 2);
    hipLaunchKernelGGL(upsample2x_grad_kernel, dim3(grid_for(int64_t(rows) * half_w)), dim3(kThreads), 0, s, dy, dx,
                       rows, half_w);
    MX_HIP(hipGetLastError());
    return MX_OK;
  }
  hipLaunchKernelGGL(upsample_nearest_grad_kernel, dim3(grid_for(planes * ih * iw)), dim3(kThreads), 0, s, dy, dx,
                     planes, ah, aw);
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

int mx_softmax_f32(const float* x, int64_t outer, int64_t axis, int64_t inner, float* y, void* stream) {
  MX_ABI_BEGIN
  MX_REQUIRE(outer >= 0 && axis >= 0 && inner >= 0, MX_ERR_INVALID, "mx_softmax_f32: negative size");
  if (outer == 0 || axis == 0 || inner == 0) return MX_OK;
  MX_REQUIRE(x && y, MX_ERR_INVALID, "mx_softmax_f32: null tensor");
  hipStream_t s = resolve_stream(stream);
  if (inner == 1) {
    MX_REQUIRE(axis <= INT32_MAX && outer <= int64_t(INT32_MAX) * kWavesPerBlock, MX_ERR_INVALID,
               "mx_softmax_f32: size exceeds int32");
    const int nv = (axis % 4 == 0 && aligned16(x) && aligned16(y)) ? regs_for((axis / 4 + 63) / 64) : 0;
    // One row per wave: the forward's exponentials and two reductions per row
    // overlap best with other waves' memory traffic when the rows run in
    // several rounds of waves (measured against two and four rows per wave).
    const dim3 grid(launch_rows(outer));
    switch (nv) {
      case 1: hipLaunchKernelGGL((softmax_rows_kernel<1, 1>), grid, dim3(kThreads), 0, s, x, y, outer, int(axis));
        break;
      case 2: hipLaunchKernelGGL((softmax_rows_kernel<2, 1>), grid, dim3(kThreads), 0, s, x, y, outer, int(axis));
        break;
      case 4: hipLaunchKernelGGL((softmax_rows_kernel<4, 1>), grid, dim3(kThreads), 0, s, x, y, outer, int(axis));
        break;
      default: hipLaunchKernelGGL(softmax_last_kernel, grid, dim3(kThreads), 0, s, x, y, outer, int(axis));
    }
  } else {
    hipLaunchKernelGGL(softmax_inner_kernel, dim3(grid_for(outer * inner)), dim3(kThreads), 0, s, x, y, outer, axis,
                       inner);
  }
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

int mx_softmax_backward_f32(const float* dy, const float* y, int64_t outer, int64_t axis, int64_t inner, float* dx,
                            void* stream) {
  MX_ABI_BEGIN
  MX_REQUIRE(outer >= 0 && axis >= 0 && inner >= 0, MX_ERR_INVALID, "mx_softmax_backward_f32: negative size");
  if (outer == 0 || axis == 0 || inner == 0) return MX_OK;
  MX_REQUIRE(dy && y && dx, MX_ERR_INVALID, "mx_softmax_backward_f32: null tensor");
  hipStream_t s = resolve_stream(stream);
  if (inner == 1) {
    MX_REQUIRE(axis <= INT32_MAX && outer <= int64_t(INT32_MAX) * kWavesPerBlock, MX_ERR_INVALID,
               "mx_softmax_backward_f32: size exceeds int32");
    const int nv =
        (axis % 4 == 0 && aligned16(dy) && aligned16(y) && aligned16(dx)) ? regs_for((axis / 4 + 63) / 64) : 0;
    const dim3 grid(launch_rows(outer)), grid4(launch_rows((outer + 3) / 4)), grid2(launch_rows((outer + 1) / 2));
    switch (nv) {
      case 1: hipLaunchKernelGGL((softmax_rows_grad_kernel<1, 4>), grid4, dim3(kThreads), 0, s, dy, y, dx, outer,
                                 int(axis));
        break;
      case 2: hipLaunchKernelGGL((softmax_rows_grad_kernel<2, 2>), grid2, dim3(kThreads), 0, s, dy, y, dx, outer,
                                 int(axis));
        break;
      case 4: hipLaunchKernelGGL((softmax_rows_grad_kernel<4, 1>), grid, dim3(kThreads), 0, s, dy, y, dx, outer,
                                 int(axis));
        break;
      default:
        hipLaunchKernelGGL(softmax_last_grad_kernel, grid, dim3(kThreads), 0, s, dy, y, dx, outer, int(axis));
    }
  } else {
    hipLaunchKernelGGL(softmax_inner_grad_kernel, dim3(grid_for(outer * inner)), dim3(kThreads), 0, s, dy, y, dx,
                       outer, axis, inner);
  }
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

int mx_mse_loss_f32(const float* x, const float* t, int64_t count, int reduction, float* out, void* stream) {
  MX_ABI_BEGIN
  MX_REQUIRE(count >= 0, MX_ERR_INVALID, "mx_mse_loss_f32: negative count");
  MX_REQUIRE(reduction == MX_REDUCE_NONE || reduction == MX_REDUCE_MEAN || reduction == MX_REDUCE_SUM,
             MX_ERR_INVALID, "mx_mse_loss_f32: unknown reduction ", reduction);
  if (reduction == MX_REDUCE_NONE && count == 0) return MX_OK;
  MX_REQUIRE(out, MX_ERR_INVALID, "mx_mse_loss_f32: null output");
  hipStream_t s = resolve_stream(stream);
  if (reduction == MX_REDUCE_NONE) {
    MX_REQUIRE(x && t, MX_ERR_INVALID, "mx_mse_loss_f32: null tensor");
    hipLaunchKernelGGL(sq_diff_kernel, dim3(grid_for(count)), dim3(kThreads), 0, s, x, t, count, out);
    MX_HIP(hipGetLastError());
    return MX_OK;
  }
  if (count == 0) {
    // Mean of nothing is NaN, sum of nothing is 0 (torch's CPU results).
    const float v = reduction == MX_REDUCE_MEAN ? std::numeric_limits<float>::quiet_NaN() : 0.f;
    uint32_t bits;
    std::memcpy(&bits, &v, 4);
    return mx_fill(out, 1, 4, bits, stream);
  }
  MX_REQUIRE(x && t, MX_ERR_INVALID, "mx_mse_loss_f32: null tensor");
  // A fixed number of partials for a given count, so the sum order is fixed.
  const int blocks = int(std::min<int64_t>((count + kThreads - 1) / kThreads, 1024));
  Scratch partial;
  MX_TRY(partial.alloc(size_t(blocks) * sizeof(float), s));
  hipLaunchKernelGGL(sq_diff_partial_kernel, dim3(blocks), dim3(kThreads), 0, s, x, t, count, partial.as<float>());
  MX_HIP(hipGetLastError());
  const float scale = reduction == MX_REDUCE_MEAN ? float(1.0 / double(count)) : 1.f;
  hipLaunchKernelGGL(sum_partials_kernel, dim3(1), dim3(kThreads), 0, s, partial.as<const float>(), blocks, scale,
                     out);
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

int mx_mse_loss_backward_f32(const float* dy, const float* x, const float* t, int64_t count, int reduction,
                             float* dx, void* stream) {
  MX_ABI_BEGIN
  MX_REQUIRE(count >= 0, MX_ERR_INVALID, "mx_mse_loss_backward_f32: negative count");
  MX_REQUIRE(reduction == MX_REDUCE_NONE || reduction == MX_REDUCE_MEAN || reduction == MX_REDUCE_SUM,
             MX_ERR_INVALID, "mx_mse_loss_backward_f32: unknown reduction ", reduction);
  if (count == 0) return MX_OK;
  MX_REQUIRE(dy && x && t && dx, MX_ERR_INVALID, "mx_mse_loss_backward_f32: null tensor");
  hipStream_t s = resolve_stream(stream);
  const float norm = reduction == MX_REDUCE_MEAN ? float(2.0 / double(count)) : 2.f;
  hipLaunchKernelGGL(mse_grad_kernel, dim3(grid_for(count)), dim3(kThreads), 0, s, dy,
                     reduction == MX_REDUCE_NONE ? 0 : 1, x, t, count, norm, dx);
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

int mx_copy_rows(void* dst, int64_t dst_pitch, const void* src, int64_t src_pitch, int64_t row_bytes, int64_t rows,
                 void* stream) {
  MX_ABI_BEGIN
  MX_REQUIRE(rows >= 0 && row_bytes >= 0 && dst_pitch >= row_bytes && src_pitch >= row_bytes, MX_ERR_INVALID,
             "mx_copy_rows: invalid pitches");
  if (rows == 0 || row_bytes == 0) return MX_OK;
  MX_REQUIRE(dst && src, MX_ERR_INVALID, "mx_copy_rows: null pointer");
  hipStream_t s = resolve_stream(stream);
  const uintptr_t bits = reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src) |
                         uintptr_t(dst_pitch) | uintptr_t(src_pitch) | uintptr_t(row_bytes);
  if ((bits & 15) == 0)
    launch_copy_rows<float4>(dst, dst_pitch, src, src_pitch, row_bytes, rows, s);
  else if ((bits & 3) == 0)
    launch_copy_rows<uint32_t>(dst, dst_pitch, src, src_pitch, row_bytes, rows, s);
  else
    launch_copy_rows<uint8_t>(dst, dst_pitch, src, src_pitch, row_bytes, rows, s);
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

}  // extern "C"
