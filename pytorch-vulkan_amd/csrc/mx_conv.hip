// FP32 NCHW Conv2D on gfx950: validation, algorithm planner, implicit-GEMM
// forward / dInput / dWeight(+dBias) on FP32 MFMA, direct kernels and the
// dBias reduction.
//
// Reference behaviour followed (mistrjirka/Pytorch-vulkan):
//   validation + output shape  csrc/ops/convolution.cpp:101-156
//   candidate menu / heuristic csrc/ops/convolution.cpp:357-482
//   dWeight split-K plan       csrc/ops/convolution.cpp:204-238
//   forward implicit GEMM      csrc/shaders/conv2d_tiled_body.glsl:1-87
//   dInput implicit GEMM       csrc/shaders/conv2d_backward_input_tiled_body.glsl:1-95
//   dWeight split + finalize   conv2d_backward_weight_tiled_body.glsl:1-71,
//                              conv2d_backward_weight_finalize.comp:9-18
//   direct kernels             conv2d_forward.comp:11-43, conv2d_backward_input.comp:10-47,
//                              conv2d_backward_weight.comp:10-41
//   dBias                      conv2d_backward_bias_reduce.comp:10-24
//
// GEMM views (per group g):
//   forward : C[co, pos]        = W[co, (ci,kh,kw)]  x im2col(x)[(ci,kh,kw), pos]
//   dInput  : C[ci, ipos]       = W^T[ci, (co,kh,kw)] x gather(dy)[(co,kh,kw), ipos]
//   dWeight : C[co, (ci,kh,kw)] = dy[co, pos]        x im2col(x)^T[pos, (ci,kh,kw)]
// The dWeight K dimension (all N*OH*OW positions) is split across workgroups;
// partial tiles are summed in fixed split order by the last workgroup to
// finish each tile (an atomic arrival counter), so the result is
// deterministic and no separate finalize launch is needed.  dBias rides on
// the dy operand already streamed by the dWeight tiles of column 0.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstring>
#include <string>

#include "mfma_core.hpp"
#include "mx_internal.hpp"

namespace mx {
namespace {

using namespace mfma;

struct ConvArgs {
  const float* x;
  const float* w;
  const float* bias;
  const float* dy;
  float* out;
  float* db;
  int N, Cin, H, W, Cout, KH, KW, OH, OW, sh, sw, ph, pw, dh, dw, G;
  int Cin_g, Cout_g, KK, HW, OHOW;
  int M, Ncols, K;
  int tiles_m, tiles_n, splits, kps;
  float* ws;
  float* ws_db;
  unsigned* counters;
};

// ------------------------------------------------------------------ loaders
// Forward B operand: rows = output positions (img, oh, ow), k = (ci, kh, kw).
// Consecutive lanes take consecutive positions (coalesced along ow).
template <int ROWS, int BK>
struct Im2colLoader {
  static constexpr int EPT = ROWS * BK / kThreads;
  static_assert(ROWS <= kThreads && EPT >= 1, "Im2colLoader tiling");
  float v[EPT];
  const float* xg;
  int ih0, iw0, ks, k;
  bool ok;
  int K, KK, KH, KW, dh, dw, H, W, HW;
  __device__ void init(const ConvArgs& p, int col0, int g) {
    const int tid = threadIdx.x;
    const int r = tid % ROWS;
    ks = (tid / ROWS) * EPT;
    const int pos = col0 + r;
    ok = pos < p.Ncols;
    const int pp = ok ? pos : 0;
    const int img = pp / p.OHOW;
    const int q = pp - img * p.OHOW;
    const int oh = q / p.OW;
    const int ow = q - oh * p.OW;
    ih0 = oh * p.sh - p.ph;
    iw0 = ow * p.sw - p.pw;
    xg = p.x + (int64_t(img) * p.Cin + int64_t(g) * p.Cin_g) * p.HW;
    K = p.K;
    KK = p.KK;
    KH = p.KH;
    KW = p.KW;
    dh = p.dh;
    dw = p.dw;
    H = p.H;
    W = p.W;
    HW = p.HW;
    k = 0;
  }
  __device__ __forceinline__ void load() {
    const int kb = k + ks;
    int ci = kb / KK;
    const int rem = kb - ci * KK;
    int kh = rem / KW;
    int kw = rem - kh * KW;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const int ih = ih0 + kh * dh, iw = iw0 + kw * dw;
      const bool valid = ok && (kb + e) < K && unsigned(ih) < unsigned(H) && unsigned(iw) < unsigned(W);
      v[e] = valid ? xg[ci * HW + ih * W + iw] : 0.f;
      if (++kw == KW) {
        kw = 0;
        if (++kh == KH) {
          kh = 0;
          ++ci;
        }
      }
    }
    k += BK;
  }
  __device__ __forceinline__ void store(float* lds) const {
    constexpr int LDK = BK + 4;
    const int tid = threadIdx.x;
    float* dst = lds + (tid % ROWS) * LDK + ks;
    if constexpr (EPT % 4 == 0) {
#pragma unroll
      for (int e = 0; e < EPT; e += 4)
        *reinterpret_cast<f32x4*>(dst + e) = f32x4{v[e], v[e + 1], v[e + 2], v[e + 3]};
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e) dst[e] = v[e];
    }
  }
};

// dInput A operand: rows = ci, k = (co, kh, kw); element w[g*Cout_g+co][ci][kh][kw].
template <int ROWS, int BK>
struct WeightTLoader {
  static constexpr int RPP = kThreads / BK;
  static constexpr int PASSES = ROWS / RPP;
  static_assert(PASSES >= 1 && ROWS % RPP == 0, "WeightTLoader tiling");
  float v[PASSES];
  int roff[PASSES];
  bool ok[PASSES];
  const float* wg;
  int k, kk, K, KK, CKK;
  __device__ void init(const ConvArgs& p, int row0, int g) {
    const int tid = threadIdx.x;
    kk = tid % BK;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      const int ci = row0 + tid / BK + q * RPP;
      ok[q] = ci < p.Cin_g;
      roff[q] = ok[q] ? ci * p.KK : 0;
    }
    wg = p.w + int64_t(g) * p.Cout_g * p.Cin_g * p.KK;
    K = p.K;
    KK = p.KK;
    CKK = p.Cin_g * p.KK;
    k = 0;
  }
  __device__ __forceinline__ void load() {
    const int kx = k + kk;
    const bool kin = kx < K;
    const int co = kx / KK;
    const int base = co * CKK + (kx - co * KK);
#pragma unroll
    for (int q = 0; q < PASSES; ++q) v[q] = (ok[q] && kin) ? wg[base + roff[q]] : 0.f;
    k += BK;
  }
  __device__ __forceinline__ void store(float* lds) const {
    constexpr int LDK = BK + 4;
    const int tid = threadIdx.x;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) lds[(tid / BK + q * RPP) * LDK + kk] = v[q];
  }
};

// dInput B operand: rows = input positions (img, ih, iw), k = (co, kh, kw);
// element dy[img][co][oh][ow] with oh*sh = ih + ph - kh*dh (no zero insertion).
template <int ROWS, int BK, bool UNIT>
struct DyGatherLoader {
  static constexpr int EPT = ROWS * BK / kThreads;
  static_assert(ROWS <= kThreads && EPT >= 1, "DyGatherLoader tiling");
  float v[EPT];
  const float* dyg;
  int ihp, iwp, ks, k;
  bool ok;
  int K, KK, KH, KW, dh, dw, sh, sw, OH, OW, OHOW;
  __device__ void init(const ConvArgs& p, int col0, int g) {
    const int tid = threadIdx.x;
    const int r = tid % ROWS;
    ks = (tid / ROWS) * EPT;
    const int pos = col0 + r;
    ok = pos < p.Ncols;
    const int pp = ok ? pos : 0;
    const int img = pp / p.HW;
    const int q = pp - img * p.HW;
    const int ih = q / p.W;
    const int iw = q - ih * p.W;
    ihp = ih + p.ph;
    iwp = iw + p.pw;
    dyg = p.dy + (int64_t(img) * p.Cout + int64_t(g) * p.Cout_g) * p.OHOW;
    K = p.K;
    KK = p.KK;
    KH = p.KH;
    KW = p.KW;
    dh = p.dh;
    dw = p.dw;
    sh = p.sh;
    sw = p.sw;
    OH = p.OH;
    OW = p.OW;
    OHOW = p.OHOW;
    k = 0;
  }
  __device__ __forceinline__ void load() {
    const int kb = k + ks;
    int co = kb / KK;
    const int rem = kb - co * KK;
    int kh = rem / KW;
    int kw = rem - kh * KW;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const int th = ihp - kh * dh, tw = iwp - kw * dw;
      bool valid = ok && (kb + e) < K;
      int off = 0;
      if constexpr (UNIT) {
        valid = valid && unsigned(th) < unsigned(OH) && unsigned(tw) < unsigned(OW);
        off = co * OHOW + th * OW + tw;
      } else {
        valid = valid && th >= 0 && tw >= 0 && th % sh == 0 && tw % sw == 0;
        const int oh = th / sh, ow = tw / sw;
        valid = valid && oh < OH && ow < OW;
        off = co * OHOW + oh * OW + ow;
      }
      v[e] = valid ? dyg[off] : 0.f;
      if (++kw == KW) {
        kw = 0;
        if (++kh == KH) {
          kh = 0;
          ++co;
        }
      }
    }
    k += BK;
  }
  __device__ __forceinline__ void store(float* lds) const {
    constexpr int LDK = BK + 4;
    const int tid = threadIdx.x;
    float* dst = lds + (tid % ROWS) * LDK + ks;
    if constexpr (EPT % 4 == 0) {
#pragma unroll
      for (int e = 0; e < EPT; e += 4)
        *reinterpret_cast<f32x4*>(dst + e) = f32x4{v[e], v[e + 1], v[e + 2], v[e + 3]};
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e) dst[e] = v[e];
    }
  }
};

// dWeight A operand: rows = co, k = output position; element dy[img][co][q].
// Also keeps each thread's running row sums for dBias.
template <int ROWS, int BK>
struct DyRowsLoader {
  static constexpr int RPP = kThreads / BK;
  static constexpr int PASSES = ROWS / RPP;
  static_assert(PASSES >= 1 && ROWS % RPP == 0, "DyRowsLoader tiling");
  float v[PASSES];
  float bsum[PASSES];
  int coff[PASSES];
  bool ok[PASSES];
  const float* dyg;
  int k, kk, kmax, OHOW, COHOW;
  __device__ void init(const ConvArgs& p, int row0, int g, int k0, int kmax_) {
    const int tid = threadIdx.x;
    kk = tid % BK;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      const int co = row0 + tid / BK + q * RPP;
      ok[q] = co < p.Cout_g;
      coff[q] = ok[q] ? co * p.OHOW : 0;
      bsum[q] = 0.f;
    }
    dyg = p.dy + int64_t(g) * p.Cout_g * p.OHOW;
    OHOW = p.OHOW;
    COHOW = p.Cout * p.OHOW;
    k = k0;
    kmax = kmax_;
  }
  __device__ __forceinline__ void load() {
    const int kx = k + kk;
    const bool kin = kx < kmax;
    const int img = kx / OHOW;
    const int base = img * COHOW + (kx - img * OHOW);
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      v[q] = (ok[q] && kin) ? dyg[base + coff[q]] : 0.f;
      bsum[q] += v[q];
    }
    k += BK;
  }
  __device__ __forceinline__ void store(float* lds) const {
    constexpr int LDK = BK + 4;
    const int tid = threadIdx.x;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) lds[(tid / BK + q * RPP) * LDK + kk] = v[q];
  }
};

// dWeight B operand: rows = (ci, kh, kw), k = output position;
// element x[img][ci][oh*sh - ph + kh*dh][ow*sw - pw + kw*dw].
template <int ROWS, int BK>
struct XColsLoader {
  static constexpr int RPP = kThreads / BK;
  static constexpr int PASSES = ROWS / RPP;
  static_assert(PASSES >= 1 && ROWS % RPP == 0, "XColsLoader tiling");
  float v[PASSES];
  int coff[PASSES];
  int khd[PASSES];
  int kwd[PASSES];
  const float* xg;
  int k, kk, kmax, OHOW, OW, sh, sw, H, W, CHW;
  __device__ void init(const ConvArgs& p, int col0, int g, int k0, int kmax_) {
    const int tid = threadIdx.x;
    kk = tid % BK;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      const int n = col0 + tid / BK + q * RPP;
      const bool ok = n < p.Ncols;
      const int nn = ok ? n : 0;
      const int ci = nn / p.KK;
      const int r = nn - ci * p.KK;
      const int kh = r / p.KW;
      const int kw = r - kh * p.KW;
      coff[q] = ci * p.HW;
      // An invalid row gets an offset that always fails the bounds test.
      khd[q] = ok ? kh * p.dh - p.ph : INT_MIN / 2;
      kwd[q] = kw * p.dw - p.pw;
    }
    xg = p.x + int64_t(g) * p.Cin_g * p.HW;
    OHOW = p.OHOW;
    OW = p.OW;
    sh = p.sh;
    sw = p.sw;
    H = p.H;
    W = p.W;
    CHW = p.Cin * p.HW;
    k = k0;
    kmax = kmax_;
  }
  __device__ __forceinline__ void load() {
    const int kx = k + kk;
    const bool kin = kx < kmax;
    const int img = kx / OHOW;
    const int q0 = kx - img * OHOW;
    const int oh = q0 / OW;
    const int ow = q0 - oh * OW;
    const int ihb = oh * sh, iwb = ow * sw;
    const float* xi = xg + int64_t(img) * CHW;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      const int ih = ihb + khd[q], iw = iwb + kwd[q];
      const bool valid = kin && unsigned(ih) < unsigned(H) && unsigned(iw) < unsigned(W);
      v[q] = valid ? xi[coff[q] + ih * W + iw] : 0.f;
    }
    k += BK;
  }
  __device__ __forceinline__ void store(float* lds) const {
    constexpr int LDK = BK + 4;
    const int tid = threadIdx.x;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) lds[(tid / BK + q * RPP) * LDK + kk] = v[q];
  }
};

// ------------------------------------------------------------------ kernels
template <class C, Mode MA>
__global__ __launch_bounds__(256) void conv_fwd_kernel(ConvArgs p) {
  __shared__ __attribute__((aligned(16))) float smem[C::SMEM_FLOATS];
  const int g = blockIdx.z;
  int tm, tn;
  tile_coords(xcd_remap(blockIdx.x, p.tiles_m * p.tiles_n), p.tiles_m, p.tiles_n, tm, tn);
  const int row0 = tm * C::BM, col0 = tn * C::BN;
  StridedLoader<C::BM, C::BK, MA> la;
  la.init(p.w + int64_t(g) * p.Cout_g * p.K, p.K, 1, row0, p.M, 0, p.K);
  Im2colLoader<C::BN, C::BK> lb;
  lb.init(p, col0, g);
  Acc<C> acc;
  mainloop<C>(acc, la, lb, (p.K + C::BK - 1) / C::BK, smem);
  for_each_acc<C>(acc, [&](int r, int c, float v) {
    const int co = row0 + r, pos = col0 + c;
    if (co < p.M && pos < p.Ncols) {
      const int img = pos / p.OHOW;
      const int q = pos - img * p.OHOW;
      const int oc = g * p.Cout_g + co;
      p.out[(int64_t(img) * p.Cout + oc) * p.OHOW + q] = v + (p.bias ? p.bias[oc] : 0.f);
    }
  });
}

template <class C, bool UNIT>
__global__ __launch_bounds__(256) void conv_dx_kernel(ConvArgs p) {
  __shared__ __attribute__((aligned(16))) float smem[C::SMEM_FLOATS];
  const int g = blockIdx.z;
  int tm, tn;
  tile_coords(xcd_remap(blockIdx.x, p.tiles_m * p.tiles_n), p.tiles_m, p.tiles_n, tm, tn);
  const int row0 = tm * C::BM, col0 = tn * C::BN;
  WeightTLoader<C::BM, C::BK> la;
  la.init(p, row0, g);
  DyGatherLoader<C::BN, C::BK, UNIT> lb;
  lb.init(p, col0, g);
  Acc<C> acc;
  mainloop<C>(acc, la, lb, (p.K + C::BK - 1) / C::BK, smem);
  for_each_acc<C>(acc, [&](int r, int c, float v) {
    const int ci = row0 + r, pos = col0 + c;
    if (ci < p.M && pos < p.Ncols) {
      const int img = pos / p.HW;
      const int q = pos - img * p.HW;
      p.out[(int64_t(img) * p.Cin + g * p.Cin_g + ci) * p.HW + q] = v;
    }
  });
}

// Sum of `v` over the BK consecutive lanes that share a row (fixed butterfly).
template <int BK>
__device__ __forceinline__ float row_lane_sum(float v) {
#pragma unroll
  for (int m = BK / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, BK);
  return v;
}

template <class C>
__global__ __launch_bounds__(256) void conv_dw_kernel(ConvArgs p) {
  __shared__ __attribute__((aligned(16))) float smem[C::SMEM_FLOATS];
  __shared__ int s_last;
  const int g = blockIdx.z, split = blockIdx.y;
  const int ntiles = p.tiles_m * p.tiles_n;
  const int tile = xcd_remap(blockIdx.x, ntiles);
  int tm, tn;
  tile_coords(tile, p.tiles_m, p.tiles_n, tm, tn);
  const int row0 = tm * C::BM, col0 = tn * C::BN;
  const int k_begin = split * p.kps;
  const int k_end = min(p.K, k_begin + p.kps);
  DyRowsLoader<C::BM, C::BK> la;
  la.init(p, row0, g, k_begin, k_end);
  XColsLoader<C::BN, C::BK> lb;
  lb.init(p, col0, g, k_begin, k_end);
  Acc<C> acc;
  mainloop<C>(acc, la, lb, (k_end - k_begin + C::BK - 1) / C::BK, smem);

  const int tid = threadIdx.x;
  const bool do_db = p.db != nullptr && tn == 0;
  constexpr int RPP = kThreads / C::BK;
  constexpr int PASSES = C::BM / RPP;
  float* dwg = p.out + int64_t(g) * p.Cout_g * p.Ncols;

  if (p.splits == 1) {
    if (dwg != nullptr && p.out != nullptr)
      for_each_acc<C>(acc, [&](int r, int c, float v) {
        const int co = row0 + r, n = col0 + c;
        if (co < p.M && n < p.Ncols) dwg[int64_t(co) * p.Ncols + n] = v;
      });
    if (do_db) {
#pragma unroll
      for (int q = 0; q < PASSES; ++q) {
        const float s = row_lane_sum<C::BK>(la.bsum[q]);
        const int co = row0 + tid / C::BK + q * RPP;
        if (tid % C::BK == 0 && co < p.M) p.db[g * p.Cout_g + co] = s;
      }
    }
    return;
  }

  // Partial tile -> workspace in register order; dBias partial per row.
  constexpr int TILE = C::BM * C::BN;
  const int64_t tile_id = int64_t(g) * ntiles + tile;
  float* wsp = p.ws + (tile_id * p.splits + split) * TILE;
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) wsp[acc_slot<C>(i, j, v)] = acc.v[i][j][v];
  if (do_db) {
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      const float s = row_lane_sum<C::BK>(la.bsum[q]);
      const int rl = tid / C::BK + q * RPP;
      if (tid % C::BK == 0)
        p.ws_db[((int64_t(g) * p.tiles_m + tm) * p.splits + split) * C::BM + rl] = s;
    }
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = atomicAdd(&p.counters[tile_id], 1u);
    s_last = prev == unsigned(p.splits - 1);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  // Last arrival: fixed-order sum over splits, then the epilogue.
  const float* wst = p.ws + tile_id * p.splits * TILE;
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int slot = acc_slot<C>(i, j, v);
        float s = 0.f;
        for (int sp = 0; sp < p.splits; ++sp) s += wst[int64_t(sp) * TILE + slot];
        acc.v[i][j][v] = s;
      }
  if (p.out != nullptr)
    for_each_acc<C>(acc, [&](int r, int c, float v) {
      const int co = row0 + r, n = col0 + c;
      if (co < p.M && n < p.Ncols) dwg[int64_t(co) * p.Ncols + n] = v;
    });
  if (do_db && tid < C::BM && row0 + tid < p.M) {
    const float* wdb = p.ws_db + (int64_t(g) * p.tiles_m + tm) * p.splits * C::BM;
    float s = 0.f;
    for (int sp = 0; sp < p.splits; ++sp) s += wdb[sp * C::BM + tid];
    p.db[g * p.Cout_g + row0 + tid] = s;
  }
  if (tid == 0) p.counters[tile_id] = 0u;
}

// ----------------------------------------------------------- direct kernels
__global__ void conv_fwd_direct_kernel(ConvArgs p) {
  const int64_t total = int64_t(p.N) * p.Cout * p.OHOW;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += int64_t(gridDim.x) * blockDim.x) {
    const int ow = int(idx % p.OW);
    const int oh = int((idx / p.OW) % p.OH);
    const int oc = int((idx / p.OHOW) % p.Cout);
    const int img = int(idx / (int64_t(p.Cout) * p.OHOW));
    const int g = oc / p.Cout_g;
    float sum = p.bias ? p.bias[oc] : 0.f;
    for (int c = 0; c < p.Cin_g; ++c) {
      const int ic = g * p.Cin_g + c;
      for (int kh = 0; kh < p.KH; ++kh) {
        const int ih = oh * p.sh - p.ph + kh * p.dh;
        if (ih < 0 || ih >= p.H) continue;
        for (int kw = 0; kw < p.KW; ++kw) {
          const int iw = ow * p.sw - p.pw + kw * p.dw;
          if (iw < 0 || iw >= p.W) continue;
          sum += p.x[(int64_t(img) * p.Cin + ic) * p.HW + ih * p.W + iw] *
                 p.w[((int64_t(oc) * p.Cin_g + c) * p.KH + kh) * p.KW + kw];
        }
      }
    }
    p.out[idx] = sum;
  }
}

__global__ void conv_dx_direct_kernel(ConvArgs p) {
  const int64_t total = int64_t(p.N) * p.Cin * p.HW;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += int64_t(gridDim.x) * blockDim.x) {
    const int iw = int(idx % p.W);
    const int ih = int((idx / p.W) % p.H);
    const int ic = int((idx / p.HW) % p.Cin);
    const int img = int(idx / (int64_t(p.Cin) * p.HW));
    const int g = ic / p.Cin_g, c = ic % p.Cin_g;
    float sum = 0.f;
    for (int co = 0; co < p.Cout_g; ++co) {
      const int oc = g * p.Cout_g + co;
      for (int kh = 0; kh < p.KH; ++kh) {
        const int th = ih + p.ph - kh * p.dh;
        if (th < 0 || th % p.sh != 0) continue;
        const int oh = th / p.sh;
        if (oh >= p.OH) continue;
        for (int kw = 0; kw < p.KW; ++kw) {
          const int tw = iw + p.pw - kw * p.dw;
          if (tw < 0 || tw % p.sw != 0) continue;
          const int ow = tw / p.sw;
          if (ow >= p.OW) continue;
          sum += p.dy[(int64_t(img) * p.Cout + oc) * p.OHOW + oh * p.OW + ow] *
                 p.w[((int64_t(oc) * p.Cin_g + c) * p.KH + kh) * p.KW + kw];
        }
      }
    }
    p.out[idx] = sum;
  }
}

__global__ void conv_dw_direct_kernel(ConvArgs p) {
  const int64_t total = int64_t(p.Cout) * p.Cin_g * p.KK;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += int64_t(gridDim.x) * blockDim.x) {
    const int kw = int(idx % p.KW);
    const int kh = int((idx / p.KW) % p.KH);
    const int c = int((idx / p.KK) % p.Cin_g);
    const int oc = int(idx / (int64_t(p.KK) * p.Cin_g));
    const int ic = (oc / p.Cout_g) * p.Cin_g + c;
    float sum = 0.f;
    for (int img = 0; img < p.N; ++img)
      for (int oh = 0; oh < p.OH; ++oh) {
        const int ih = oh * p.sh - p.ph + kh * p.dh;
        if (ih < 0 || ih >= p.H) continue;
        for (int ow = 0; ow < p.OW; ++ow) {
          const int iw = ow * p.sw - p.pw + kw * p.dw;
          if (iw < 0 || iw >= p.W) continue;
          sum += p.x[(int64_t(img) * p.Cin + ic) * p.HW + ih * p.W + iw] *
                 p.dy[(int64_t(img) * p.Cout + oc) * p.OHOW + oh * p.OW + ow];
        }
      }
    p.out[idx] = sum;
  }
}

// No-scratch dWeight: one workgroup per weight, strided partial sums and a
// fixed LDS tree (conv2d_backward_weight_reduce.comp:13-38).
__global__ __launch_bounds__(256) void conv_dw_reduce_kernel(ConvArgs p) {
  __shared__ float part[256];
  const int64_t total = int64_t(p.Cout) * p.Cin_g * p.KK;
  const int64_t positions = int64_t(p.N) * p.OHOW;
  for (int64_t idx = blockIdx.x; idx < total; idx += gridDim.x) {
    const int kw = int(idx % p.KW);
    const int kh = int((idx / p.KW) % p.KH);
    const int c = int((idx / p.KK) % p.Cin_g);
    const int oc = int(idx / (int64_t(p.KK) * p.Cin_g));
    const int ic = (oc / p.Cout_g) * p.Cin_g + c;
    float sum = 0.f;
    for (int64_t r = threadIdx.x; r < positions; r += 256) {
      const int img = int(r / p.OHOW);
      const int q = int(r - int64_t(img) * p.OHOW);
      const int oh = q / p.OW, ow = q - oh * p.OW;
      const int ih = oh * p.sh - p.ph + kh * p.dh, iw = ow * p.sw - p.pw + kw * p.dw;
      if (unsigned(ih) < unsigned(p.H) && unsigned(iw) < unsigned(p.W))
        sum += p.x[(int64_t(img) * p.Cin + ic) * p.HW + ih * p.W + iw] *
               p.dy[(int64_t(img) * p.Cout + oc) * p.OHOW + q];
    }
    part[threadIdx.x] = sum;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
      if (int(threadIdx.x) < s) part[threadIdx.x] += part[threadIdx.x + s];
      __syncthreads();
    }
    if (threadIdx.x == 0) p.out[idx] = part[0];
    __syncthreads();
  }
}

// dBias: one workgroup per output channel, strided partial sums + LDS tree.
__global__ __launch_bounds__(256) void conv_db_reduce_kernel(ConvArgs p) {
  __shared__ float part[256];
  const int64_t positions = int64_t(p.N) * p.OHOW;
  for (int oc = blockIdx.x; oc < p.Cout; oc += gridDim.x) {
    float sum = 0.f;
    for (int64_t r = threadIdx.x; r < positions; r += 256) {
      const int img = int(r / p.OHOW);
      const int q = int(r - int64_t(img) * p.OHOW);
      sum += p.dy[(int64_t(img) * p.Cout + oc) * p.OHOW + q];
    }
    part[threadIdx.x] = sum;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
      if (int(threadIdx.x) < s) part[threadIdx.x] += part[threadIdx.x + s];
      __syncthreads();
    }
    if (threadIdx.x == 0) p.db[oc] = part[0];
    __syncthreads();
  }
}

// Serial per-channel dBias (conv2d_backward_bias.comp:9-27).
__global__ void conv_db_direct_kernel(ConvArgs p) {
  for (int oc = blockIdx.x * blockDim.x + threadIdx.x; oc < p.Cout; oc += gridDim.x * blockDim.x) {
    float sum = 0.f;
    for (int img = 0; img < p.N; ++img)
      for (int q = 0; q < p.OHOW; ++q) sum += p.dy[(int64_t(img) * p.Cout + oc) * p.OHOW + q];
    p.db[oc] = sum;
  }
}

// ------------------------------------------------------------------ host
using TileL = Cfg<128, 128, 16, 2>;  // 128 x 128, waves 2 x 2 (64 x 64 each)
using TileM = Cfg<64, 128, 16, 2>;   // 64 x 128, waves 2 x 2 (32 x 64 each)
using TileS = Cfg<64, 64, 16, 2>;    // 64 x 64, waves 2 x 2 (32 x 32 each)

int checked_desc(mx_conv2d_desc* d) {
  MX_REQUIRE(d, MX_ERR_INVALID, "conv2d: null descriptor");
  MX_REQUIRE(d->n > 0 && d->cin > 0 && d->cout > 0 && d->h > 0 && d->w > 0 && d->kh > 0 && d->kw > 0 &&
                 d->sh > 0 && d->sw > 0 && d->dh > 0 && d->dw > 0 && d->ph >= 0 && d->pw >= 0 &&
                 d->groups > 0 && d->cin % d->groups == 0 && d->cout % d->groups == 0,
             MX_ERR_INVALID, "Vulkan convolution: invalid shapes or parameters");
  for (int64_t v : {d->h, d->w, d->kh, d->kw, d->sh, d->sw, d->ph, d->pw, d->dh, d->dw})
    MX_REQUIRE(v <= INT32_MAX, MX_ERR_INVALID, "Vulkan convolution: spatial parameters exceed int32 coordinates");
  MX_REQUIRE(d->dh * (d->kh - 1) <= INT32_MAX && d->dw * (d->kw - 1) <= INT32_MAX, MX_ERR_INVALID,
             "Vulkan convolution: effective filter exceeds int32 coordinates");
  MX_REQUIRE(d->h + 2 * d->ph >= d->dh * (d->kh - 1) + 1 && d->w + 2 * d->pw >= d->dw * (d->kw - 1) + 1,
             MX_ERR_INVALID, "Vulkan convolution: effective kernel exceeds padded input");
  d->oh = (d->h + 2 * d->ph - d->dh * (d->kh - 1) - 1) / d->sh + 1;
  d->ow = (d->w + 2 * d->pw - d->dw * (d->kw - 1) - 1) / d->sw + 1;
  MX_REQUIRE(d->oh > 0 && d->ow > 0, MX_ERR_INVALID, "Vulkan convolution: empty output");
  MX_REQUIRE((d->oh - 1) * d->sh + d->dh * (d->kh - 1) <= INT32_MAX &&
                 (d->ow - 1) * d->sw + d->dw * (d->kw - 1) <= INT32_MAX && d->h - 1 + d->ph <= INT32_MAX &&
                 d->w - 1 + d->pw <= INT32_MAX,
             MX_ERR_INVALID, "Vulkan convolution: spatial indexing exceeds int32 coordinates");
  // Kernels index elements with 32-bit offsets inside each tensor.
  const int64_t kk = d->kh * d->kw;
  MX_REQUIRE(d->n * d->cin * d->h * d->w <= INT32_MAX && d->n * d->cout * d->oh * d->ow <= INT32_MAX &&
                 d->cout * (d->cin / d->groups) * kk <= INT32_MAX,
             MX_ERR_INVALID, "Vulkan convolution: input/weight/output indexing overflow");
  return MX_OK;
}

ConvArgs make_args(const mx_conv2d_desc& d) {
  ConvArgs p{};
  p.N = int(d.n);
  p.Cin = int(d.cin);
  p.H = int(d.h);
  p.W = int(d.w);
  p.Cout = int(d.cout);
  p.KH = int(d.kh);
  p.KW = int(d.kw);
  p.OH = int(d.oh);
  p.OW = int(d.ow);
  p.sh = int(d.sh);
  p.sw = int(d.sw);
  p.ph = int(d.ph);
  p.pw = int(d.pw);
  p.dh = int(d.dh);
  p.dw = int(d.dw);
  p.G = int(d.groups);
  p.Cin_g = p.Cin / p.G;
  p.Cout_g = p.Cout / p.G;
  p.KK = p.KH * p.KW;
  p.HW = p.H * p.W;
  p.OHOW = p.OH * p.OW;
  return p;
}

int linear_blocks(int64_t total) { return int(std::min<int64_t>((total + 255) / 256, 1 << 20)); }

bool winograd_applicable(const mx_conv2d_desc& d) {
  return d.kh == 3 && d.kw == 3 && d.sh == 1 && d.sw == 1 && d.dh == 1 && d.dw == 1;
}

// Reference heuristic (csrc/ops/convolution.cpp:423-482) restated for the
// MFMA candidates: implicit GEMM whenever the GEMM is not degenerate, Winograd
// only for the grouped 3x3 case the reference routes there by default.
int select_algo(const mx_conv2d_desc& d, int phase, int requested, int* algo) {
  const int64_t cin_g = d.cin / d.groups, cout_g = d.cout / d.groups;
  const int64_t rows = d.n * d.oh * d.ow, cols = cin_g * d.kh * d.kw;
  switch (phase) {
    case MX_CONV_FORWARD:
      if (requested == MX_CONV_ALGO_WINOGRAD) {
        MX_REQUIRE(winograd_applicable(d), MX_ERR_UNSUPPORTED,
                   "Forced Vulkan convolution forward candidate winograd_f2 exceeds device limits, workspace "
                   "budget, or operator applicability");
        *algo = MX_CONV_ALGO_WINOGRAD;
        return MX_OK;
      }
      MX_REQUIRE(requested != MX_CONV_ALGO_REDUCE, MX_ERR_UNSUPPORTED,
                 "reduce is not a forward convolution algorithm");
      if (requested != MX_CONV_ALGO_AUTO) {
        *algo = requested;
        return MX_OK;
      }
      if (winograd_applicable(d) && d.groups >= 4 && cin_g >= 16 && cout_g >= 16 && rows >= 2048)
        *algo = MX_CONV_ALGO_WINOGRAD;
      else if (cout_g >= 8 && cols >= 16 && rows >= 32)
        *algo = MX_CONV_ALGO_IMPLICIT_GEMM;
      else
        *algo = MX_CONV_ALGO_DIRECT;
      return MX_OK;
    case MX_CONV_DINPUT:
      MX_REQUIRE(requested != MX_CONV_ALGO_WINOGRAD && requested != MX_CONV_ALGO_REDUCE, MX_ERR_UNSUPPORTED,
                 "dinput supports direct and implicit_gemm only");
      if (requested != MX_CONV_ALGO_AUTO) {
        *algo = requested;
        return MX_OK;
      }
      *algo = (cin_g >= 2 && cout_g >= 8 && d.n * d.h * d.w >= 32) ? MX_CONV_ALGO_IMPLICIT_GEMM
                                                                   : MX_CONV_ALGO_DIRECT;
      return MX_OK;
    case MX_CONV_DWEIGHT:
      MX_REQUIRE(requested != MX_CONV_ALGO_WINOGRAD, MX_ERR_UNSUPPORTED, "winograd is forward only");
      if (requested != MX_CONV_ALGO_AUTO) {
        *algo = requested;
        return MX_OK;
      }
      if (cout_g >= 8 && cols >= 16 && cols * d.cout > 4096)
        *algo = MX_CONV_ALGO_IMPLICIT_GEMM;
      else if (rows >= 128)
        *algo = MX_CONV_ALGO_REDUCE;
      else
        *algo = MX_CONV_ALGO_DIRECT;
      return MX_OK;
    case MX_CONV_DBIAS:
      MX_REQUIRE(requested == MX_CONV_ALGO_AUTO || requested == MX_CONV_ALGO_DIRECT ||
                     requested == MX_CONV_ALGO_REDUCE,
                 MX_ERR_UNSUPPORTED, "dbias supports direct and reduce only");
      *algo = requested == MX_CONV_ALGO_AUTO ? (rows >= 128 ? MX_CONV_ALGO_REDUCE : MX_CONV_ALGO_DIRECT)
                                             : requested;
      return MX_OK;
    default:
      return set_error(MX_ERR_INVALID, cat("conv2d: bad phase ", phase));
  }
}

template <class C>
void set_tiles(ConvArgs& p) {
  p.tiles_m = (p.M + C::BM - 1) / C::BM;
  p.tiles_n = (p.Ncols + C::BN - 1) / C::BN;
}

// Tile shape from the GEMM view (per group M x Ncols, times groups).
int pick_tile(int M, int Ncols, int G) {
  const int64_t big = int64_t((M + 127) / 128) * ((Ncols + 127) / 128) * G;
  if (M > 64 && big >= cu_count()) return 0;
  const int64_t mid = int64_t((M + 63) / 64) * ((Ncols + 127) / 128) * G;
  if (mid >= cu_count()) return 1;
  return 2;
}

template <class C>
int launch_fwd(ConvArgs p, bool kvec, hipStream_t s) {
  set_tiles<C>(p);
  dim3 grid(p.tiles_m * p.tiles_n, 1, p.G);
  if (kvec)
    hipLaunchKernelGGL((conv_fwd_kernel<C, Mode::KVEC>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((conv_fwd_kernel<C, Mode::KSCALAR>), grid, dim3(256), 0, s, p);
  MX_HIP(hipGetLastError());
  return MX_OK;
}

template <class C>
int launch_dx(ConvArgs p, bool unit, hipStream_t s) {
  set_tiles<C>(p);
  dim3 grid(p.tiles_m * p.tiles_n, 1, p.G);
  if (unit)
    hipLaunchKernelGGL((conv_dx_kernel<C, true>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((conv_dx_kernel<C, false>), grid, dim3(256), 0, s, p);
  MX_HIP(hipGetLastError());
  return MX_OK;
}

struct DwPlan {
  int tile = 2;
  int splits = 1;
  int kps = 0;
  int64_t ws_bytes = 0;
  int64_t db_bytes = 0;
  int64_t counters = 0;
};

template <class C>
DwPlan plan_dw_cfg(const ConvArgs& p, int tile) {
  DwPlan pl;
  pl.tile = tile;
  const int64_t tiles = int64_t((p.M + C::BM - 1) / C::BM) * ((p.Ncols + C::BN - 1) / C::BN);
  const int64_t blocks = tiles * p.G;
  const int64_t target = 2LL * cu_count();
  const int64_t max_splits = std::max<int64_t>(1, (p.K + 4 * C::BK - 1) / (4 * C::BK));  // >= 4 slabs each
  int64_t splits = std::max<int64_t>(1, std::min<int64_t>(max_splits, (target + blocks - 1) / blocks));
  splits = std::min<int64_t>(splits, 65535);
  int64_t kps = (p.K + splits - 1) / splits;
  kps = (kps + C::BK - 1) / C::BK * C::BK;
  splits = (p.K + kps - 1) / kps;
  pl.splits = int(splits);
  pl.kps = int(kps);
  if (splits > 1) {
    pl.ws_bytes = blocks * splits * int64_t(C::BM) * C::BN * 4;
    pl.db_bytes = int64_t(p.G) * ((p.M + C::BM - 1) / C::BM) * splits * C::BM * 4;
    pl.counters = blocks;
  }
  return pl;
}

DwPlan plan_dw(const ConvArgs& p) {
  const int t = pick_tile(p.M, p.Ncols, p.G);
  if (t == 0) return plan_dw_cfg<TileL>(p, 0);
  if (t == 1) return plan_dw_cfg<TileM>(p, 1);
  return plan_dw_cfg<TileS>(p, 2);
}

template <class C>
int launch_dw(ConvArgs p, const DwPlan& pl, hipStream_t s) {
  set_tiles<C>(p);
  p.splits = pl.splits;
  p.kps = pl.kps;
  Scratch ws, wsdb;
  if (pl.splits > 1) {
    MX_TRY(ws.alloc(size_t(pl.ws_bytes), s));
    p.ws = ws.as<float>();
    if (p.db) {
      MX_TRY(wsdb.alloc(size_t(pl.db_bytes), s));
      p.ws_db = wsdb.as<float>();
    }
    MX_TRY(tile_counters(s, size_t(pl.counters), &p.counters));
  }
  dim3 grid(p.tiles_m * p.tiles_n, pl.splits, p.G);
  hipLaunchKernelGGL((conv_dw_kernel<C>), grid, dim3(256), 0, s, p);
  MX_HIP(hipGetLastError());
  return MX_OK;
}

}  // namespace

// Winograd forward lives in mx_winograd.hip.
int winograd_forward(const mx_conv2d_desc& d, const float* x, const float* w, const float* bias, float* y,
                     hipStream_t s);

}  // namespace mx

using namespace mx;

extern "C" {

int mx_conv2d_check(mx_conv2d_desc* desc) {
  MX_ABI_BEGIN
  return checked_desc(desc);
  MX_ABI_END
}

int mx_conv2d_select(const mx_conv2d_desc* desc, int phase, int requested, int* algo) {
  MX_ABI_BEGIN
  mx_conv2d_desc d = *desc;
  MX_TRY(checked_desc(&d));
  return select_algo(d, phase, requested, algo);
  MX_ABI_END
}

int mx_conv2d_forward(const mx_conv2d_desc* desc, const float* x, const float* w, const float* bias, float* y,
                      int algo, void* stream) {
  MX_ABI_BEGIN
  mx_conv2d_desc d = *desc;
  MX_TRY(checked_desc(&d));
  MX_REQUIRE(x && w && y, MX_ERR_INVALID, "conv2d forward: null tensor");
  int chosen = 0;
  MX_TRY(select_algo(d, MX_CONV_FORWARD, algo, &chosen));
  hipStream_t s = resolve_stream(stream);
  if (chosen == MX_CONV_ALGO_WINOGRAD) return winograd_forward(d, x, w, bias, y, s);
  ConvArgs p = make_args(d);
  p.x = x;
  p.w = w;
  p.bias = bias;
  p.out = y;
  if (chosen == MX_CONV_ALGO_DIRECT) {
    hipLaunchKernelGGL(conv_fwd_direct_kernel, dim3(linear_blocks(d.n * d.cout * d.oh * d.ow)), dim3(256), 0, s, p);
    MX_HIP(hipGetLastError());
    return MX_OK;
  }
  p.M = p.Cout_g;
  p.Ncols = p.N * p.OHOW;
  p.K = p.Cin_g * p.KK;
  const bool kvec = (p.K % 4 == 0) && ((reinterpret_cast<uintptr_t>(w) & 15u) == 0);
  switch (pick_tile(p.M, p.Ncols, p.G)) {
    case 0: return launch_fwd<TileL>(p, kvec, s);
    case 1: return launch_fwd<TileM>(p, kvec, s);
    default: return launch_fwd<TileS>(p, kvec, s);
  }
  MX_ABI_END
}

int mx_conv2d_backward_input(const mx_conv2d_desc* desc, const float* dy, const float* w, float* dx, int algo,
                             void* stream) {
  MX_ABI_BEGIN
  mx_conv2d_desc d = *desc;
  MX_TRY(checked_desc(&d));
  MX_REQUIRE(dy && w && dx, MX_ERR_INVALID, "conv2d dinput: null tensor");
  int chosen = 0;
  MX_TRY(select_algo(d, MX_CONV_DINPUT, algo, &chosen));
  hipStream_t s = resolve_stream(stream);
  ConvArgs p = make_args(d);
  p.dy = dy;
  p.w = w;
  p.out = dx;
  if (chosen == MX_CONV_ALGO_DIRECT) {
    hipLaunchKernelGGL(conv_dx_direct_kernel, dim3(linear_blocks(d.n * d.cin * d.h * d.w)), dim3(256), 0, s, p);
    MX_HIP(hipGetLastError());
    return MX_OK;
  }
  p.M = p.Cin_g;
  p.Ncols = p.N * p.HW;
  p.K = p.Cout_g * p.KK;
  const bool unit = p.sh == 1 && p.sw == 1;
  switch (pick_tile(p.M, p.Ncols, p.G)) {
    case 0: return launch_dx<TileL>(p, unit, s);
    case 1: return launch_dx<TileM>(p, unit, s);
    default: return launch_dx<TileS>(p, unit, s);
  }
  MX_ABI_END
}

int mx_conv2d_backward_bias(const mx_conv2d_desc* desc, const float* dy, float* db, void* stream) {
  MX_ABI_BEGIN
  mx_conv2d_desc d = *desc;
  MX_TRY(checked_desc(&d));
  MX_REQUIRE(dy && db, MX_ERR_INVALID, "conv2d dbias: null tensor");
  hipStream_t s = resolve_stream(stream);
  ConvArgs p = make_args(d);
  p.dy = dy;
  p.db = db;
  int chosen = 0;
  MX_TRY(select_algo(d, MX_CONV_DBIAS, MX_CONV_ALGO_AUTO, &chosen));
  if (chosen == MX_CONV_ALGO_DIRECT)
    hipLaunchKernelGGL(conv_db_direct_kernel, dim3(linear_blocks(d.cout)), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(conv_db_reduce_kernel, dim3(unsigned(std::min<int64_t>(d.cout, 65535))), dim3(256), 0, s, p);
  MX_HIP(hipGetLastError());
  return MX_OK;
  MX_ABI_END
}

int mx_conv2d_backward_weight(const mx_conv2d_desc* desc, const float* x, const float* dy, float* dw, float* db,
                              int algo, void* stream) {
  MX_ABI_BEGIN
  mx_conv2d_desc d = *desc;
  MX_TRY(checked_desc(&d));
  MX_REQUIRE(x && dy, MX_ERR_INVALID, "conv2d dweight: null tensor");
  if (!dw && !db) return MX_OK;
  if (!dw) return mx_conv2d_backward_bias(desc, dy, db, stream);
  int chosen = 0;
  MX_TRY(select_algo(d, MX_CONV_DWEIGHT, algo, &chosen));
  hipStream_t s = resolve_stream(stream);
  ConvArgs p = make_args(d);
  p.x = x;
  p.dy = dy;
  p.out = dw;
  if (chosen != MX_CONV_ALGO_IMPLICIT_GEMM) {
    if (chosen == MX_CONV_ALGO_DIRECT)
      hipLaunchKernelGGL(conv_dw_direct_kernel, dim3(linear_blocks(d.cout * (d.cin / d.groups) * d.kh * d.kw)),
                         dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL(conv_dw_reduce_kernel,
                         dim3(unsigned(std::min<int64_t>(d.cout * (d.cin / d.groups) * d.kh * d.kw, 1 << 20))),
                         dim3(256), 0, s, p);
    MX_HIP(hipGetLastError());
    if (db) return mx_conv2d_backward_bias(desc, dy, db, stream);
    return MX_OK;
  }
  p.db = db;
  p.M = p.Cout_g;
  p.Ncols = p.Cin_g * p.KK;
  p.K = p.N * p.OHOW;
  const DwPlan pl = plan_dw(p);
  switch (pl.tile) {
    case 0: return launch_dw<TileL>(p, pl, s);
    case 1: return launch_dw<TileM>(p, pl, s);
    default: return launch_dw<TileS>(p, pl, s);
  }
  MX_ABI_END
}

int mx_conv2d_kernel_name(const mx_conv2d_desc* desc, int phase, int algo, char* buf, size_t len) {
  MX_ABI_BEGIN
  mx_conv2d_desc d = *desc;
  MX_TRY(checked_desc(&d));
  int chosen = 0;
  MX_TRY(select_algo(d, phase, algo, &chosen));
  ConvArgs p = make_args(d);
  static const char* tiles[] = {"128x128x16", "64x128x16", "64x64x16"};
  std::string name;
  if (phase == MX_CONV_DBIAS) {
    name = chosen == MX_CONV_ALGO_DIRECT ? "conv_db_direct_kernel" : "conv_db_reduce_kernel";
  } else if (chosen == MX_CONV_ALGO_WINOGRAD) {
    name = "wino_filter_kernel";
  } else if (chosen == MX_CONV_ALGO_DIRECT) {
    name = phase == MX_CONV_FORWARD ? "conv_fwd_direct_kernel"
           : phase == MX_CONV_DINPUT ? "conv_dx_direct_kernel" : "conv_dw_direct_kernel";
  } else if (chosen == MX_CONV_ALGO_REDUCE) {
    name = "conv_dw_reduce_kernel";
  } else if (phase == MX_CONV_FORWARD) {
    name = cat("conv_fwd_kernel<", tiles[pick_tile(p.Cout_g, p.N * p.OHOW, p.G)], ">");
  } else if (phase == MX_CONV_DINPUT) {
    name = cat("conv_dx_kernel<", tiles[pick_tile(p.Cin_g, p.N * p.HW, p.G)], ">");
  } else {
    p.M = p.Cout_g;
    p.Ncols = p.Cin_g * p.KK;
    p.K = p.N * p.OHOW;
    name = cat("conv_dw_kernel<", tiles[plan_dw(p).tile], ">");
  }
  if (len) {
    std::strncpy(buf, name.c_str(), len - 1);
    buf[len - 1] = 0;
  }
  return MX_OK;
  MX_ABI_END
}

int mx_conv2d_dweight_plan(const mx_conv2d_desc* desc, int64_t* splits, int64_t* span, int64_t* workspace_bytes) {
  MX_ABI_BEGIN
  mx_conv2d_desc d = *desc;
  MX_TRY(checked_desc(&d));
  ConvArgs p = make_args(d);
  p.M = p.Cout_g;
  p.Ncols = p.Cin_g * p.KK;
  p.K = p.N * p.OHOW;
  const DwPlan pl = plan_dw(p);
  if (splits) *splits = pl.splits;
  if (span) *span = pl.kps;
  if (workspace_bytes) *workspace_bytes = pl.ws_bytes + pl.db_bytes;
  return MX_OK;
  MX_ABI_END
}

}  // extern "C"
