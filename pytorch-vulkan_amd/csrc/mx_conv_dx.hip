// Conv2D dInput as one implicit GEMM per stride phase on FP32 MFMA (gfx950).
//
// Reference behaviour followed: csrc/shaders/conv2d_backward_input_tiled_body.glsl:1-95
// (dInput implicit GEMM: dx[ci, ipos] = sum over (co, kh, kw) of
// w[co][ci][kh][kw] * dy[co][(ih + ph - kh*dh)/sh][(iw + pw - kw*dw)/sw] where
// the division is exact) and csrc/ops/convolution.cpp:684-687.
//
// For stride s > 1 only the taps with (ih + ph - kh*dh) % sh == 0 contribute,
// and which taps those are depends only on ih % sh.  The input positions are
// therefore split into sh*sw phases (ih % sh, iw % sw); each phase is a dense
// GEMM over exactly its taps (th, tw), so no zero-inserted term is ever
// multiplied.  Phases no tap reaches are zero-filled.  Weights are first
// packed per phase as Wt_p[g][k][ci] (k the gathered K order over (co, th,
// tw), mx_conv_common.hpp) so the A operand has ci contiguous (16 bytes per
// lane); a 1x1 kernel needs no packing, w itself is [g][co][ci].
#include "mx_conv_common.hpp"

namespace mx {
namespace conv {
namespace {

// Wt_p[g][k][ci] = w[g*Cout_g + co][ci][kh0 + th*stph][kw0 + tw*stpw] with k
// the gathered K order over (co, th, tw): the A operand of phase p's GEMM,
// ci contiguous, at wt + set.ph[p].off.  One launch packs up to
// kMaxPackPhases phases (blockIdx.y = phase).  32-bit indices: the packed
// weights are below 2^31 bytes.
__global__ void conv_dx_pack_kernel(ConvArgs p, DxPackSet set, float* wt) {
  const DxPackPhase ph = set.ph[blockIdx.y];
  const uint32_t nt = ph.nth * ph.ntw;
  const uint32_t total = uint32_t(p.G) * ph.K * p.Cin_g;
  const bool blocked = blocked_channels(p.Cout_g);
  const uint32_t kblk = nt * kChanBlock;
  float* const dst = wt + ph.off;
  for (uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += gridDim.x * blockDim.x) {
    const uint32_t rest = idx / uint32_t(p.Cin_g);
    const uint32_t ci = idx - rest * uint32_t(p.Cin_g);
    const uint32_t g = rest / uint32_t(ph.K);
    const uint32_t k = rest - g * uint32_t(ph.K);
    uint32_t co, t;
    if (blocked) {
      const uint32_t cb = k / kblk, rem = k - cb * kblk;
      t = rem / kChanBlock;
      co = cb * kChanBlock + rem - t * kChanBlock;
    } else {
      co = k / nt;
      t = k - co * nt;
    }
    const uint32_t th = t / uint32_t(ph.ntw), tw = t - th * uint32_t(ph.ntw);
    const int kh = ph.kh0 + int(th) * ph.stph, kw = ph.kw0 + int(tw) * ph.stpw;
    dst[idx] = p.w[((int64_t(g * p.Cout_g + co) * p.Cin_g + ci) * p.KH + kh) * p.KW + kw];
  }
}

// dx = 0 everywhere (16-byte stores where the tensor allows): run before the
// phase GEMMs of a convolution whose stride leaves some input positions
// untouched by every tap; the GEMMs then overwrite the reached positions.
__global__ void conv_dx_zero_kernel(float* __restrict__ dx, int64_t n) {
  const int64_t n4 = n / 4;
  const bool vec = (reinterpret_cast<uintptr_t>(dx) & 15) == 0;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (vec) {
    for (; i < n4; i += stride) reinterpret_cast<float4*>(dx)[i] = float4{0.f, 0.f, 0.f, 0.f};
    i = 4 * n4 + (int64_t(blockIdx.x) * blockDim.x + threadIdx.x);
  }
  for (; i < n; i += stride) dx[i] = 0.f;
}

// One output tile (linear index `lin`, K split `split`, group g) of one
// stride phase.
template <class C, Mode MA, class LB>
__device__ __forceinline__ void dx_tile(const ConvArgs& p, int g, int lin, int split, float* smem) {
  int tm, tn;
  tile_coords(lin, p.tiles_m, p.tiles_n, tm, tn);
  const int row0 = tm * C::BM, col0 = tn * C::BN;
  const int k0 = split * p.kps, k1 = min(p.K, k0 + p.kps);
  BufStridedLoader<C::BM, C::BK, MA> la;  // element (ci, k) = wt[g][k][ci]
  la.init(p.wt + int64_t(g) * p.K * p.Cin_g, int64_t(p.K) * p.Cin_g * 4, 1, p.Cin_g, row0, p.M, k0, k1);
  LB lb;
  lb.init(p, col0, g, k0, k1);
  Acc<C> acc;
  mainloop<C>(acc, la, lb, (k1 - k0 + C::BK - 1) / C::BK, smem);
  float* const out = p.splits == 1 ? p.out : p.ws + split * p.out_elems;
  // (Not built for the 256-wide tiles, whose registers it would spill; the
  // host does not request it for them.)
  if constexpr (C::BM * C::BN <= 128 * 128) if (p.zfill) {
    // Phase (0, 0) of stride 2 x 2, W even: position (i, j) owns input rows
    // 2i, 2i + 1 (if < H) and columns 2j, 2j + 1; one 8-byte store per row.
    int cb[C::FN];
    bool ok[C::FN], row2[C::FN];
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
      const int pos = col0 + acc_col<C>(j);
      ok[j] = pos < p.Ncols;
      const int pp = ok[j] ? pos : 0;
      const int img = pp / p.HpWp;
      const int q = pp - img * p.HpWp;
      const int i = q / p.Wp;
      cb[j] = img * p.Cin * p.HW + 2 * i * p.W + 2 * (q - i * p.Wp);
      row2[j] = 2 * i + 1 < p.H;
    }
    for_each_acc_row<C>([&](int r, int i, int v) {
      const int ci = row0 + r;
      if (ci >= p.M) return;
      float* dst = out + int64_t(g * p.Cin_g + ci) * p.HW;
#pragma unroll
      for (int j = 0; j < C::FN; ++j) {
        if (!ok[j]) continue;
        *reinterpret_cast<float2*>(dst + cb[j]) = float2{acc.v[i][j][v], 0.f};
        if (row2[j]) *reinterpret_cast<float2*>(dst + cb[j] + p.W) = float2{0.f, 0.f};
      }
    });
    return;
  }
  // The output (one launch's dx, or one split's partial, below 2^31 bytes)
  // as a buffer resource: stores outside the tile's valid rows / columns go
  // to kOffNone and are dropped, so the stores run straight through without
  // a branch or a 64-bit address per element.  Byte offset of each fragment
  // column (img * Cin * HW + phase position), once.
  const i32x4 ro = buffer_rsrc(out, p.out_elems * 4);
  uint32_t cbase[C::FN];
#pragma unroll
  for (int j = 0; j < C::FN; ++j) {
    const int pos = col0 + acc_col<C>(j);
    const bool cok = pos < p.Ncols;
    const int pp = cok ? pos : 0;
    const int img = pp / p.HpWp;
    const int q = pp - img * p.HpWp;
    const int i = q / p.Wp;
    cbase[j] = cok ? uint32_t(img * p.Cin * p.HW + (p.pa + p.sh * i) * p.W + p.pb + p.sw * (q - i * p.Wp)) * 4u
                   : kOffNone;
  }
  for_each_acc_row<C>([&](int r, int i, int v) {
    const int ci = row0 + r;
    const bool rok = ci < p.M;
    const uint32_t roff = uint32_t((g * p.Cin_g + ci) * p.HW) * 4u;
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
      bstore(acc.v[i][j][v], ro, (rok && cbase[j] != kOffNone) ? roff + cbase[j] : kOffNone, 0);
  });
}

template <class C, Mode MA, class LB>
MX_TILE_KERNEL(C) void conv_dx_kernel(ConvArgs p) {
  __shared__ __attribute__((aligned(16))) float smem[C::SMEM_FLOATS];
  dx_tile<C, MA, LB>(p, blockIdx.z, xcd_remap(blockIdx.x, p.tiles_m * p.tiles_n), blockIdx.y, smem);
}

// Several stride phases in one launch (blockIdx.z = phase * G + group): the
// phases of a strided layer are each a fraction of its positions, and run one
// after another their launches leave most of the GPU idle.  The grid covers
// the phase with the most tiles; the others' surplus workgroups exit.
template <class C, Mode MA, class LB>
MX_TILE_KERNEL(C) void conv_dx_phases_kernel(DxPhaseSet set) {
  __shared__ __attribute__((aligned(16))) float smem[C::SMEM_FLOATS];
  const int ph = int(blockIdx.z) / set.G, g = int(blockIdx.z) - ph * set.G;
  const ConvArgs& p = set.q[ph];
  const int lin = xcd_remap(blockIdx.x, gridDim.x);
  if (lin >= p.tiles_m * p.tiles_n) return;
  dx_tile<C, MA, LB>(p, g, lin, blockIdx.y, smem);
}

template <class C, Mode MA>
int launch_b(ConvArgs p, int bmode, hipStream_t s) {
  p.tiles_m = (p.M + C::BM - 1) / C::BM;
  p.tiles_n = (p.Ncols + C::BN - 1) / C::BN;
  const dim3 grid(p.tiles_m * p.tiles_n, p.splits, p.G);
  if (bmode == B_VEC)
    hipLaunchKernelGGL((conv_dx_kernel<C, MA, PosQuadLoader<C::BN, C::BK, true>>), grid, dim3(kThreads), 0, s, p);
  else if (blocked_channels(p.Cout_g))
    hipLaunchKernelGGL((conv_dx_kernel<C, MA, PhaseGatherLoader<C::BN, C::BK, true>>), grid, dim3(kThreads), 0, s, p);
  else
    hipLaunchKernelGGL((conv_dx_kernel<C, MA, PhaseGatherLoader<C::BN, C::BK, false>>), grid, dim3(kThreads), 0, s, p);
  MX_HIP(hipGetLastError());
  return MX_OK;
}

template <class C>
int launch_a(const ConvArgs& p, Mode ma, int bmode, hipStream_t s) {
  if (ma == Mode::RVEC) return launch_b<C, Mode::RVEC>(p, bmode, s);
  return launch_b<C, Mode::RSCALAR>(p, bmode, s);
}

template <class C, Mode MA>
int launch_set_b(DxPhaseSet set, int bmode, hipStream_t s) {
  int most = 0;
  for (int i = 0; i < set.n; ++i) {
    ConvArgs& q = set.q[i];
    q.tiles_m = (q.M + C::BM - 1) / C::BM;
    q.tiles_n = (q.Ncols + C::BN - 1) / C::BN;
    most = std::max(most, q.tiles_m * q.tiles_n);
  }
  const dim3 grid(unsigned(most), unsigned(set.q[0].splits), unsigned(set.G * set.n));
  if (bmode == B_VEC)
    hipLaunchKernelGGL((conv_dx_phases_kernel<C, MA, PosQuadLoader<C::BN, C::BK, true>>), grid, dim3(kThreads), 0, s,
                       set);
  else if (blocked_channels(set.q[0].Cout_g))
    hipLaunchKernelGGL((conv_dx_phases_kernel<C, MA, PhaseGatherLoader<C::BN, C::BK, true>>), grid, dim3(kThreads), 0,
                       s, set);
  else
    hipLaunchKernelGGL((conv_dx_phases_kernel<C, MA, PhaseGatherLoader<C::BN, C::BK, false>>), grid, dim3(kThreads),
                       0, s, set);
  MX_HIP(hipGetLastError());
  return MX_OK;
}

template <class C>
int launch_set_a(const DxPhaseSet& set, Mode ma, int bmode, hipStream_t s) {
  if (ma == Mode::RVEC) return launch_set_b<C, Mode::RVEC>(set, bmode, s);
  return launch_set_b<C, Mode::RSCALAR>(set, bmode, s);
}

int grid_for(int64_t total) { return int(std::min<int64_t>((total + 255) / 256, 1 << 20)); }

}  // namespace

int conv_dx_pack_weights(const ConvArgs& p, const DxPackSet& set, float* wt, hipStream_t s) {
  int64_t most = 0;
  for (int i = 0; i < set.n; ++i) most = std::max<int64_t>(most, int64_t(p.G) * set.ph[i].K * p.Cin_g);
  hipLaunchKernelGGL(conv_dx_pack_kernel, dim3(grid_for(most), set.n), dim3(256), 0, s, p, set, wt);
  MX_HIP(hipGetLastError());
  return MX_OK;
}

int conv_dx_zero(float* dx, int64_t n, hipStream_t s) {
  hipLaunchKernelGGL(conv_dx_zero_kernel, dim3(grid_for((n + 3) / 4)), dim3(256), 0, s, dx, n);
  MX_HIP(hipGetLastError());
  return MX_OK;
}

int conv_dx_launch_set(const DxPhaseSet& set, int tile, Mode ma, int bmode, hipStream_t s) {
  if (set.n == 1) return conv_dx_launch(set.q[0], tile, ma, bmode, s);
  switch (tile) {
    case TALL: return launch_set_a<TileTall>(set, ma, bmode, s);
    case WIDE: return launch_set_a<TileWide>(set, ma, bmode, s);
    case SQ: return launch_set_a<TileSq>(set, ma, bmode, s);
    case FLAT: return launch_set_a<TileFlat>(set, ma, bmode, s);
    default: return launch_set_a<TileSmallShallow>(set, ma, bmode, s);
  }
}

int conv_dx_launch(const ConvArgs& p, int tile, Mode ma, int bmode, hipStream_t s) {
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
