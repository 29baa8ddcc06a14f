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
  // The (tile, split) grid is remapped as one sequence, tiles fastest, so
  // the tiles of a split -- which read the same dy and x range -- share an
  // XCD's L2 even when a split has fewer tiles than there are XCDs (the
  // 7x7 stem: 3 tiles over 147 columns).
  const int g = blockIdx.z;
  const int ntiles = p.tiles_m * p.tiles_n;
  const int lin = xcd_remap(int(blockIdx.y) * int(gridDim.x) + int(blockIdx.x), int(gridDim.x * gridDim.y));
  const int split = lin / ntiles;
  int tm, tn;
  tile_coords(lin - split * ntiles, p.tiles_m, p.tiles_n, tm, tn);
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
  // This group's dW (or partial; weights are below 2^31 bytes) as a buffer
  // resource: stores outside the valid rows / columns go to kOffNone and are
  // dropped, so they run straight through without branches.  Column n of the
  // GEMM is weight column n, or with channel-blocked columns (channel block
  // cb, tap t, channel in block c) weight column (16cb + c)*KK + t.
  const i32x4 ro = buffer_rsrc(dst, int64_t(p.Cout_g) * p.Ncols * 4);
  uint32_t ccol[C::FN];
  const int kblk = p.KK * kChanBlock;
#pragma unroll
  for (int j = 0; j < C::FN; ++j) {
    const int n = col0 + acc_col<C>(j);
    int c = n;
    if (p.cols_blocked) {
      const int cb = n / kblk, rem = n - cb * kblk;
      const int t = rem / kChanBlock;
      c = cb * kblk + (rem - t * kChanBlock) * p.KK + t;
    }
    ccol[j] = n < p.Ncols ? uint32_t(c) * 4u : kOffNone;
  }
  for_each_acc_row<C>([&](int r, int i, int v) {
    const int co = row0 + r;
    const bool rok = co < p.M;
    const uint32_t roff = uint32_t(co * p.Ncols) * 4u;
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
      bstore(acc.v[i][j][v], ro, (rok && ccol[j] != kOffNone) ? roff + ccol[j] : kOffNone, 0);
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

// dw[i] = sum over the K splits of ws[split][i]; same for db (elements past
// n_dw).  A workgroup takes 64 lanes' worth of elements; wave q sums splits
// q, q + 4, q + 8, ... in order, and the four partials are added in wave
// order, so the result is the same on every run and many splits of a small
// dW keep four times more loads in flight than one thread per element would.
// The first n4 = n_dw / 4 groups of four (n4 = 0 unless the host found ws
// and dw 16-byte aligned) are summed as 16-byte vectors, E = 256 / Q groups
// per workgroup; workgroups past them take the rest (dw's tail, then db) one
// element per lane.  Each output is summed by Q lanes (chain q takes splits
// q, q + Q, ...), whose sums are added in chain order: a fixed order for a
// given split count.  Q = 16 when there are many splits keeps every split's
// load in flight at once (C1's Winograd weight gradient: 98 ranges, 6 loads
// per lane instead of 25).
template <int Q>
__global__ __launch_bounds__(256) void conv_dw_finalize_kernel(const float* __restrict__ ws,
                                                               const float* __restrict__ ws_db, float* __restrict__ dw,
                                                               float* __restrict__ db, int64_t n_dw, int n_db,
                                                               int splits, int64_t n4) {
  constexpr int E = 256 / Q;
  __shared__ f32x4 part[Q][E];
  const int e = threadIdx.x % E, q = threadIdx.x / E;
  const int64_t vblocks = (n4 + E - 1) / E;
  if (int64_t(blockIdx.x) < vblocks) {
    const int64_t g4 = int64_t(blockIdx.x) * E + e;
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    if (g4 < n4) {
      const f32x4* src = reinterpret_cast<const f32x4*>(ws) + g4;
      const int64_t stride4 = n_dw / 4;
#pragma unroll 4
      for (int sp = q; sp < splits; sp += Q) s += src[sp * stride4];
    }
    part[q][e] = s;
    __syncthreads();
    if (q == 0 && g4 < n4) {
      f32x4 t = part[0][e];
#pragma unroll
      for (int i = 1; i < Q; ++i) t += part[i][e];
      reinterpret_cast<f32x4*>(dw)[g4] = t;
    }
    return;
  }
  const int64_t idx = 4 * n4 + (int64_t(blockIdx.x) - vblocks) * E + e;
  float s = 0.f;
  if (idx < n_dw) {
    const float* src = ws + idx;
#pragma unroll 4
    for (int sp = q; sp < splits; sp += Q) s += src[sp * n_dw];
  } else if (idx < n_dw + n_db) {
    const float* src = ws_db + (idx - n_dw);
#pragma unroll 4
    for (int sp = q; sp < splits; sp += Q) s += src[sp * int64_t(n_db)];
  }
  part[q][e][0] = s;
  __syncthreads();
  if (q == 0) {
    float v = part[0][e][0];
#pragma unroll
    for (int i = 1; i < Q; ++i) v += part[i][e][0];
    if (idx < n_dw) dw[idx] = v;
    else if (idx < n_dw + n_db) db[idx - n_dw] = v;
  }
}

// out[i] = sum over splits (in order) of ws[split][i] (+ bias of i's channel).
// VEC: 16-byte vectors; the host guarantees n % 4 == 0, hw % 4 == 0 (one
// channel per vector) and aligned buffers.  Indices are 32-bit: a launch's
// output is one buffer-addressable tensor (< 2^31 bytes).
template <bool VEC>
__global__ void conv_sum_splits_kernel(const float* __restrict__ ws, int splits, int64_t n, float* __restrict__ out,
                                       const float* __restrict__ bias, int hw, int cout) {
  const uint32_t n_vec = uint32_t(VEC ? n / 4 : n);
  for (uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x; idx < n_vec; idx += gridDim.x * blockDim.x) {
    if constexpr (VEC) {
      const float4* src = reinterpret_cast<const float4*>(ws) + idx;
      float4 s = *src;
#pragma unroll 4
      for (int sp = 1; sp < splits; ++sp) {
        src += n_vec;
        const float4 v = *src;
        s.x += v.x;
        s.y += v.y;
        s.z += v.z;
        s.w += v.w;
      }
      if (bias) {
        const float b = bias[(4 * idx / uint32_t(hw)) % uint32_t(cout)];
        s.x += b;
        s.y += b;
        s.z += b;
        s.w += b;
      }
      reinterpret_cast<float4*>(out)[idx] = s;
    } else {
      float s = 0.f;
#pragma unroll 8
      for (int sp = 0; sp < splits; ++sp) s += ws[sp * n + idx];
      if (bias) s += bias[(idx / uint32_t(hw)) % uint32_t(cout)];
      out[idx] = s;
    }
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

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int conv_sum_splits(const float* ws, int splits, int64_t n, float* out, const float* bias, int hw, int cout,
                    hipStream_t s) {
  const bool vec = n % 4 == 0 && (!bias || hw % 4 == 0) && aligned16(ws) && aligned16(out);
  const int64_t items = vec ? n / 4 : n;
  const int blocks = int(std::min<int64_t>((items + 255) / 256, 1 << 20));
  if (vec)
    hipLaunchKernelGGL(conv_sum_splits_kernel<true>, dim3(blocks), dim3(256), 0, s, ws, splits, n, out, bias, hw,
                       cout);
  else
    hipLaunchKernelGGL(conv_sum_splits_kernel<false>, dim3(blocks), dim3(256), 0, s, ws, splits, n, out, bias, hw,
                       cout);
  MX_HIP(hipGetLastError());
  return MX_OK;
}

namespace {
// Finalize launch: vector groups when ws and out are 16-byte aligned and the
// partial planes stay so (n % 4 == 0), scalar elements for the rest.
int launch_finalize(const float* ws, const float* ws_db, float* out, float* db, int64_t n, int n_db, int splits,
                    hipStream_t s) {
  const bool vec = n % 4 == 0 && (reinterpret_cast<uintptr_t>(ws) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  const int64_t n4 = vec ? n / 4 : 0;
  const bool wide = splits >= 32;
  const int64_t E = wide ? 16 : 64;
  const int64_t blocks = (n4 + E - 1) / E + (n - 4 * n4 + n_db + E - 1) / E;
  MX_REQUIRE(blocks <= INT32_MAX, MX_ERR_UNSUPPORTED, "conv2d dweight: finalize grid too large");
  if (wide)
    hipLaunchKernelGGL(conv_dw_finalize_kernel<16>, dim3(unsigned(blocks)), dim3(256), 0, s, ws, ws_db, out, db, n,
                       n_db, splits, n4);
  else
    hipLaunchKernelGGL(conv_dw_finalize_kernel<4>, dim3(unsigned(blocks)), dim3(256), 0, s, ws, ws_db, out, db, n,
                       n_db, splits, n4);
  MX_HIP(hipGetLastError());
  return MX_OK;
}
}  // namespace

int conv_dw_finalize(const ConvArgs& p, float* dw, float* db, hipStream_t s) {
  return launch_finalize(p.ws, p.ws_db, dw, db, int64_t(p.G) * p.Cout_g * p.Ncols, db ? p.Cout : 0, p.splits, s);
}

int sum_partials(const float* ws, int splits, int64_t n, float* out, hipStream_t s) {
  return launch_finalize(ws, nullptr, out, nullptr, n, 0, splits, s);
}

int sum_partials(const float* ws, const float* ws_db, int splits, int64_t n, int n_db, float* out, float* out_db,
                 hipStream_t s) {
  return launch_finalize(ws, ws_db, out, out_db, n, out_db ? n_db : 0, splits, s);
}

}  // namespace conv
}  // namespace mx
