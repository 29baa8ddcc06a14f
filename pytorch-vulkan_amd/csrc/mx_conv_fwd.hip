// Conv2D forward as an implicit GEMM on FP32 MFMA (gfx950).
//
// Reference behaviour followed: csrc/shaders/conv2d_tiled_body.glsl:1-87
// (implicit-GEMM forward, bias in the store) and
// csrc/ops/convolution.cpp:641-665 (dispatch(Forward)).
//   C[co, pos] = W[co, (ci,kh,kw)] x im2col(x)[(ci,kh,kw), pos] + bias[co]
// A (weights, k contiguous) is read 16 bytes per lane when K % 4 == 0; B is
// the im2col gather, or for an unpadded 1x1 stride-1 convolution the input
// itself read as rows of four positions.
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
  StridedLoader<C::BM, C::BK, MA> la;
  la.init(p.w + int64_t(g) * p.Cout_g * p.K, p.K, 1, row0, p.M, 0, p.K);
  LB lb;
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

template <class C, Mode MA>
int launch_b(ConvArgs p, int bmode, hipStream_t s) {
  p.tiles_m = (p.M + C::BM - 1) / C::BM;
  p.tiles_n = (p.Ncols + C::BN - 1) / C::BN;
  const dim3 grid(p.tiles_m * p.tiles_n, 1, p.G);
  if (bmode == B_VEC)
    hipLaunchKernelGGL((conv_fwd_kernel<C, MA, PosQuadLoader<C::BN, C::BK, false>>), grid, dim3(kThreads), 0, s, p);
  else
    hipLaunchKernelGGL((conv_fwd_kernel<C, MA, Im2colLoader<C::BN, C::BK>>), grid, dim3(kThreads), 0, s, p);
  MX_HIP(hipGetLastError());
  return MX_OK;
}

template <class C>
int launch_a(const ConvArgs& p, Mode ma, int bmode, hipStream_t s) {
  if (ma == Mode::KVEC) return launch_b<C, Mode::KVEC>(p, bmode, s);
  return launch_b<C, Mode::KSCALAR>(p, bmode, s);
}

}  // namespace

int conv_fwd_launch(const ConvArgs& p, int tile, Mode ma, int bmode, hipStream_t s) {
  switch (tile) {
    case TALL: return launch_a<TileTall>(p, ma, bmode, s);
    case WIDE: return launch_a<TileWide>(p, ma, bmode, s);
    case SQ: return launch_a<TileSq>(p, ma, bmode, s);
    case FLAT: return launch_a<TileFlat>(p, ma, bmode, s);
    default: return launch_a<TileSmall>(p, ma, bmode, s);
  }
}

}  // namespace conv
}  // namespace mx
