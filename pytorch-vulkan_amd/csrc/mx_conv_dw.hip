// Conv2D dWeight (+ fused dBias) as a split-K implicit GEMM on FP32 MFMA (gfx950).
//
// Reference behaviour followed: conv2d_backward_weight_tiled_body.glsl:1-71
// (dW[co, (ci,kh,kw)] = sum over positions of dy[co, pos] * im2col(x)[pos, (ci,kh,kw)]),
// conv2d_backward_weight_finalize.comp:9-18 (partials over position splits
// summed in split order) and csrc/ops/convolution.cpp:204-238 (split plan).
//
// K = N*OH*OW is split over blockIdx.y.  With one split the tile is stored
// directly; otherwise every split writes a full-size partial dW (and the
// column-0 tiles a partial dBias, from row sums of the dy operand they already
// stream) and conv_dw_finalize_kernel sums the partials in fixed split order,
// so the result is deterministic for a given plan.
#include <type_traits>

#include "mx_conv_common.hpp"

namespace mx {
namespace conv {
namespace {

// Sum of `v` over the W consecutive lanes that share a row (fixed butterfly).
template <int W>
__device__ __forceinline__ float row_lane_sum(float v) {
#pragma unroll
  for (int m = W / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, W);
  return v;
}

template <class C, class LA, class LB>
MX_TILE_KERNEL(C) void conv_dw_kernel(ConvArgs p) {
  __shared__ __attribute__((aligned(16))) float smem[C::SMEM_FLOATS];
  const int g = blockIdx.z, split = blockIdx.y;
  int tm, tn;
  tile_coords(xcd_remap(blockIdx.x, p.tiles_m * p.tiles_n), p.tiles_m, p.tiles_n, tm, tn);
  const int row0 = tm * C::BM, col0 = tn * C::BN;
  const int k_begin = split * p.kps;
  const int k_end = min(p.K, k_begin + p.kps);
  LA la;
  la.init(p, row0, g, k_begin, k_end);
  LB lb;
  lb.init(p, col0, g, k_begin, k_end);
  Acc<C> acc;
  mainloop<C>(acc, la, lb, (k_end - k_begin + C::BK - 1) / C::BK, smem);

  const int64_t dw_elems = int64_t(p.G) * p.Cout_g * p.Ncols;
  float* dst = (p.splits == 1 ? p.out : p.ws + split * dw_elems) + int64_t(g) * p.Cout_g * p.Ncols;
  // Column n of the GEMM is weight column n, or with channel-blocked columns
  // (channel block cb, tap t, channel in block c) weight column (16cb + c)*KK + t.
  int ccol[C::FN];
  bool cok[C::FN];
  const int kblk = p.KK * kChanBlock;
#pragma unroll
  for (int j = 0; j < C::FN; ++j) {
    const int n = col0 + acc_col<C>(j);
    cok[j] = n < p.Ncols;
    if (p.cols_blocked) {
      const int cb = n / kblk, rem = n - cb * kblk;
      const int t = rem / kChanBlock;
      ccol[j] = cb * kblk + (rem - t * kChanBlock) * p.KK + t;
    } else {
      ccol[j] = n;
    }
  }
  for_each_acc_row<C>([&](int r, int i, int v) {
    const int co = row0 + r;
    if (co >= p.M) return;
    float* d = dst + int64_t(co) * p.Ncols;
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
      if (cok[j]) d[ccol[j]] = acc.v[i][j][v];
  });
  if (p.db != nullptr && tn == 0) {
    float* dbd = (p.splits == 1 ? p.db : p.ws_db + int64_t(split) * p.Cout) + g * p.Cout_g;
    const int tid = threadIdx.x;
#pragma unroll
    for (int q = 0; q < LA::PASSES; ++q) {
      const float s = row_lane_sum<LA::LPR>(la.bsum[q]);
      const int co = row0 + tid / LA::LPR + q * LA::RPP;
      if (tid % LA::LPR == 0 && co < p.M) dbd[co] = s;
    }
  }
}

// dw[i] = sum over splits (in order) of ws[split][i]; same for db.
__global__ void conv_dw_finalize_kernel(const float* __restrict__ ws, const float* __restrict__ ws_db,
                                        float* __restrict__ dw, float* __restrict__ db, int64_t n_dw, int n_db,
                                        int splits) {
  const int64_t total = n_dw + n_db;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += int64_t(gridDim.x) * blockDim.x) {
    float s = 0.f;
    if (idx < n_dw) {
#pragma unroll 8
      for (int sp = 0; sp < splits; ++sp) s += ws[sp * n_dw + idx];
      dw[idx] = s;
    } else {
      const int64_t j = idx - n_dw;
#pragma unroll 8
      for (int sp = 0; sp < splits; ++sp) s += ws_db[sp * int64_t(n_db) + j];
      db[j] = s;
    }
  }
}

__global__ void conv_sum_splits_kernel(const float* __restrict__ ws, int splits, int64_t n, float* __restrict__ out,
                                       const float* __restrict__ bias, int hw, int cout) {
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < n;
       idx += int64_t(gridDim.x) * blockDim.x) {
    float s = 0.f;
#pragma unroll 8
    for (int sp = 0; sp < splits; ++sp) s += ws[sp * n + idx];
    if (bias) s += bias[(idx / hw) % cout];
    out[idx] = s;
  }
}

template <class C, class LA>
int launch_b(ConvArgs p, int bmode, hipStream_t s) {
  p.tiles_m = (p.M + C::BM - 1) / C::BM;
  p.tiles_n = (p.Ncols + C::BN - 1) / C::BN;
  const dim3 grid(p.tiles_m * p.tiles_n, p.splits, p.G);
  if (bmode == B_VEC) {
    hipLaunchKernelGGL((conv_dw_kernel<C, LA, PosKLoader<C::BN, C::BK, false>>), grid, dim3(kThreads), 0, s, p);
  } else {
    // The x-column gather over 256 columns, or paired with the scalar dy rows
    // on a 256-wide tile, does not fit the register budget; the planner never
    // picks those.
    constexpr bool dy_rows = std::is_same_v<LA, DyRowsLoader<C::BM, C::BK>>;
    constexpr bool fits = C::BN <= 128 && (C::BM * C::BN <= 128 * 128 || !dy_rows);
    if constexpr (fits) {
      if (p.cols_blocked)
        hipLaunchKernelGGL((conv_dw_kernel<C, LA, XColsLoader<C::BN, C::BK, true>>), grid, dim3(kThreads), 0, s, p);
      else
        hipLaunchKernelGGL((conv_dw_kernel<C, LA, XColsLoader<C::BN, C::BK, false>>), grid, dim3(kThreads), 0, s, p);
    } else {
      return set_error(MX_ERR_INVALID, "conv2d dweight: tile too large for two gathered operands");
    }
  }
  MX_HIP(hipGetLastError());
  return MX_OK;
}

template <class C>
int launch_a(const ConvArgs& p, int amode, int bmode, hipStream_t s) {
  if (amode == B_VEC) return launch_b<C, PosKLoader<C::BM, C::BK, true>>(p, bmode, s);
  return launch_b<C, DyRowsLoader<C::BM, C::BK>>(p, bmode, s);
}

}  // namespace

int conv_dw_launch(const ConvArgs& p, int tile, int amode, int bmode, hipStream_t s) {
  switch (tile) {
    case TALL: return launch_a<TileTall>(p, amode, bmode, s);
    case WIDE: return launch_a<TileWide>(p, amode, bmode, s);
    case SQ: return launch_a<TileSq>(p, amode, bmode, s);
    case FLAT: return launch_a<TileFlat>(p, amode, bmode, s);
    case NARROW: return launch_a<TileNarrow>(p, amode, bmode, s);
    default: return launch_a<TileSmall>(p, amode, bmode, s);
  }
}

int conv_sum_splits(const float* ws, int splits, int64_t n, float* out, const float* bias, int hw, int cout,
                    hipStream_t s) {
  const int blocks = int(std::min<int64_t>((n + 255) / 256, 1 << 20));
  hipLaunchKernelGGL(conv_sum_splits_kernel, dim3(blocks), dim3(256), 0, s, ws, splits, n, out, bias, hw, cout);
  MX_HIP(hipGetLastError());
  return MX_OK;
}

int conv_dw_finalize(const ConvArgs& p, float* dw, float* db, hipStream_t s) {
  const int64_t n_dw = int64_t(p.G) * p.Cout_g * p.Ncols;
  const int n_db = db ? p.Cout : 0;
  const int64_t total = n_dw + n_db;
  const int blocks = int(std::min<int64_t>((total + 255) / 256, 1 << 20));
  hipLaunchKernelGGL(conv_dw_finalize_kernel, dim3(blocks), dim3(256), 0, s, p.ws, p.ws_db, dw, db, n_dw, n_db,
                     p.splits);
  MX_HIP(hipGetLastError());
  return MX_OK;
}

}  // namespace conv
}  // namespace mx
