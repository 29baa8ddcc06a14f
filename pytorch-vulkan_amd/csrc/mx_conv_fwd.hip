// Conv2D forward as an implicit GEMM on FP32 MFMA (gfx950).
//
// Reference behaviour followed: csrc/shaders/conv2d_tiled_body.glsl:1-87
// (implicit-GEMM forward, bias in the store) and
// csrc/ops/convolution.cpp:641-665 (dispatch(Forward)).
//   C[co, pos] = Wp[co, k] x im2col(x)[k, pos] + bias[co]
// with k the gathered K order over (ci, kh, kw) (mx_conv_common.hpp); the
// weights are packed to it when it differs from their own [co][ci][kh][kw].
// A is read 16 bytes per lane (rows padded to a multiple of four floats by
// the host when K is not); B is the im2col gather, or for an unpadded 1x1
// stride-1 convolution the input itself read as rows of four positions.
#include "mx_conv_common.hpp"

namespace mx {
namespace conv {
namespace {

template <class C, Mode MA, class LB>
MX_TILE_KERNEL(C) void conv_fwd_kernel(ConvArgs p) {
  __shared__ __attribute__((aligned(16))) float smem[C::SMEM_FLOATS];
  const int g = blockIdx.z;
  int tm, tn;
  tile_coords(xcd_remap(blockIdx.x, p.tiles_m * p.tiles_n), p.tiles_m, p.tiles_n, tm, tn);
  const int row0 = tm * C::BM, col0 = tn * C::BN;
  const int split = blockIdx.y;
  const int k0 = split * p.kps, k1 = min(p.K, k0 + p.kps);
  BufStridedLoader<C::BM, C::BK, MA> la;
  la.init(p.wt + int64_t(g) * p.Cout_g * p.ldw, int64_t(p.Cout_g) * p.ldw * 4, p.ldw, 1, row0, p.M, k0, k1);
  LB lb;
  lb.init(p, col0, g, k0, k1);
  Acc<C> acc;
  mainloop<C>(acc, la, lb, (k1 - k0 + C::BK - 1) / C::BK, smem);
  // With split-K the tile goes to this split's partial output (bias added by
  // the finalize).
  float* const out = p.splits == 1 ? p.out : p.ws + split * p.out_elems;
  const float* const bias = p.splits == 1 ? p.bias : nullptr;
  // The output (one launch's, below 2^31 bytes) as a buffer resource: a
  // store outside the tile's valid rows / columns goes to kOffNone and is
  // dropped, so the epilogue has no branches.  Stores count in the same
  // vector-memory counter as loads, so the bias values of a fragment row
  // block are all loaded before its first store: a load between stores would
  // make every later store wait for the earlier ones to complete.
  const i32x4 ro = buffer_rsrc(out, p.out_elems * 4);
  // Output byte offset of each fragment column (img * Cout * OHOW + q), once.
  uint32_t cbase[C::FN];
#pragma unroll
  for (int j = 0; j < C::FN; ++j) {
    const int pos = col0 + acc_col<C>(j);
    const int img = (pos < p.Ncols ? pos : 0) / p.OHOW;
    cbase[j] = pos < p.Ncols ? uint32_t(img * p.Cout * p.OHOW + (pos - img * p.OHOW)) * 4u : kOffNone;
  }
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
    float b[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int co = row0 + acc_row<C>(i, v);
      b[v] = (bias && co < p.M) ? bias[g * p.Cout_g + co] : 0.f;
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int co = row0 + acc_row<C>(i, v);
      const bool rok = co < p.M;
      const uint32_t roff = uint32_t((g * p.Cout_g + co) * p.OHOW) * 4u;
#pragma unroll
      for (int j = 0; j < C::FN; ++j)
        bstore(acc.v[i][j][v] + b[v], ro, (rok && cbase[j] != kOffNone) ? roff + cbase[j] : kOffNone, 0);
    }
  }
}

// Wp[g][co][k] = w[g*Cout_g + co][ci][kh][kw] with k the blocked gathered
// order (channel block, kh, kw, channel in block).  32-bit indices: the
// weights are below 2^31 bytes.
__global__ void conv_fwd_pack_kernel(ConvArgs p, float* wp) {
  const uint32_t total = uint32_t(p.Cout) * p.Cin_g * p.KK;
  const uint32_t kblk = p.KK * kChanBlock;
  for (uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += gridDim.x * blockDim.x) {
    const uint32_t oc = idx / uint32_t(p.K);
    const uint32_t k = idx - oc * uint32_t(p.K);
    const uint32_t cb = k / kblk, rem = k - cb * kblk;
    const uint32_t t = rem / kChanBlock;  // kh * KW + kw
    const uint32_t ci = cb * kChanBlock + rem - t * kChanBlock;
    wp[idx] = p.w[(uint32_t(oc) * p.Cin_g + ci) * p.KK + t];
  }
}

// wp[row][k] = w[row][k] for k < K, zero for K <= k < ldw: rows of a
// multiple of four floats, so the weight operand is read 16 bytes per lane
// whatever K is (the 7x7 stem has K = 147).
__global__ void conv_fwd_pad_kernel(const float* __restrict__ w, float* __restrict__ wp, uint32_t rows, uint32_t K,
                                    uint32_t ldw) {
  const uint32_t total = rows * ldw;
  for (uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += gridDim.x * blockDim.x) {
    const uint32_t r = idx / ldw, k = idx - r * ldw;
    wp[idx] = k < K ? w[r * K + k] : 0.f;
  }
}

template <class C, Mode MA>
int launch_b(ConvArgs p, int bmode, hipStream_t s) {
  p.tiles_m = (p.M + C::BM - 1) / C::BM;
  p.tiles_n = (p.Ncols + C::BN - 1) / C::BN;
  const dim3 grid(p.tiles_m * p.tiles_n, p.splits, p.G);
  if (bmode == B_VEC) {
    hipLaunchKernelGGL((conv_fwd_kernel<C, MA, PosQuadLoader<C::BN, C::BK, false>>), grid, dim3(kThreads), 0, s, p);
  } else if constexpr (MA == Mode::KVEC) {
    if (blocked_channels(p.Cin_g))
      hipLaunchKernelGGL((conv_fwd_kernel<C, MA, Im2colLoader<C::BN, C::BK, true>>), grid, dim3(kThreads), 0, s, p);
    else
      hipLaunchKernelGGL((conv_fwd_kernel<C, MA, Im2colLoader<C::BN, C::BK, false>>), grid, dim3(kThreads), 0, s, p);
  } else {
    // Scalar weight rows mean unpacked weights: channels not blocked, or a
    // 1x1 kernel, whose blocked and plain K orders are the same.
    hipLaunchKernelGGL((conv_fwd_kernel<C, MA, Im2colLoader<C::BN, C::BK, false>>), grid, dim3(kThreads), 0, s, p);
  }
  MX_HIP(hipGetLastError());
  return MX_OK;
}

// The weight operand is always read 16 bytes per lane: the host pads rows
// whose length is not a multiple of four (conv_fwd_pad_kernel).
template <class C>
int launch_a(const ConvArgs& p, Mode ma, int bmode, hipStream_t s) {
  if (ma != Mode::KVEC || p.ldw % 4 != 0) return set_error(MX_ERR_INVALID, "conv2d forward: weight rows not padded");
  return launch_b<C, Mode::KVEC>(p, bmode, s);
}

}  // namespace

int conv_fwd_pack_weights(const ConvArgs& p, float* wp, hipStream_t s) {
  const int64_t total = int64_t(p.Cout) * p.Cin_g * p.KK;
  hipLaunchKernelGGL(conv_fwd_pack_kernel, dim3(int(std::min<int64_t>((total + 255) / 256, 1 << 20))), dim3(256), 0,
                     s, p, wp);
  MX_HIP(hipGetLastError());
  return MX_OK;
}

int conv_fwd_pad_weights(const ConvArgs& p, float* wp, hipStream_t s) {
  const int64_t total = int64_t(p.Cout) * p.ldw;
  hipLaunchKernelGGL(conv_fwd_pad_kernel, dim3(int(std::min<int64_t>((total + 255) / 256, 1 << 20))), dim3(256), 0, s,
                     p.w, wp, uint32_t(p.Cout), uint32_t(p.K), uint32_t(p.ldw));
  MX_HIP(hipGetLastError());
  return MX_OK;
}

int conv_fwd_launch(const ConvArgs& p, int tile, Mode ma, int bmode, hipStream_t s) {
  switch (tile) {
    case TALL: return launch_a<TileTall>(p, ma, bmode, s);
    case WIDE: return launch_a<TileWide>(p, ma, bmode, s);
    case SQ: return launch_a<TileSq>(p, ma, bmode, s);
    case FLAT: return launch_a<TileFlat>(p, ma, bmode, s);
    default: return launch_a<TileSmallShallow>(p, ma, bmode, s);
  }
}

}  // namespace conv
}  // namespace mx
