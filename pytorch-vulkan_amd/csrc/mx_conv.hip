// FP32 NCHW Conv2D on gfx950: validation, algorithm selection, planning of
// the implicit-GEMM launches (mx_conv_fwd.hip, mx_conv_dx.hip,
// mx_conv_dw.hip), the direct kernels and the dBias reduction.
//
// Reference behaviour followed (mistrjirka/Pytorch-vulkan):
//   validation + output shape  csrc/ops/convolution.cpp:101-156
//   candidate menu / heuristic csrc/ops/convolution.cpp:357-482
//   dWeight split-K plan       csrc/ops/convolution.cpp:204-238
//   direct kernels             conv2d_forward.comp:11-43, conv2d_backward_input.comp:10-47,
//                              conv2d_backward_weight.comp:10-41
//   dBias                      conv2d_backward_bias_reduce.comp:10-24
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <numeric>
#include <string>
#include <vector>

#include "mx_conv_common.hpp"

namespace mx {
namespace {

using conv::ConvArgs;
using mfma::Mode;

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

// Depthwise forward (groups == Cin, Cout = m * Cin; conv2d_depthwise.comp:15-41).
// One workgroup per (image, input channel, 16 x 64 output tile): the input
// patch the tile reads (halo and zero padding included) is staged once in LDS
// and all m output channels that read this input channel are computed from
// it, so x is read from HBM once per tile and y written once.  Wave w owns
// output rows 4w .. 4w+3 of the tile, lane l output column l.  Each output
// starts from its bias and adds the taps in (kh, kw) order, as the shader
// does; a padded tap adds 0 * w.  A patch larger than the LDS budget (very
// large dilation) reads x directly (kStaged = false).
constexpr int kDwTileW = 64, kDwTileH = 16, kDwRowsPerWave = 4;
constexpr int kDwLdsFloats = 12288;  // 48 KiB

struct DepthwiseArgs {
  ConvArgs p;
  int tiles_w, tiles_h;
  int64_t tiles;
  int patch_h, patch_w;  // staged input rows / columns of one tile
};

template <bool kStaged>
__global__ __launch_bounds__(256) void conv_depthwise_kernel(DepthwiseArgs a) {
  __shared__ float patch[kStaged ? kDwLdsFloats : 1];
  const ConvArgs& p = a.p;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m = p.Cout_g;
  for (int64_t t = blockIdx.x; t < a.tiles; t += gridDim.x) {
    const int tw = int(t % a.tiles_w);
    const int th = int((t / a.tiles_w) % a.tiles_h);
    const int64_t plane = t / (int64_t(a.tiles_w) * a.tiles_h);  // img * Cin + ic
    const int ic = int(plane % p.Cin);
    const int img = int(plane / p.Cin);
    const float* xp = p.x + plane * p.HW;
    const int oh0 = th * kDwTileH, ow0 = tw * kDwTileW;
    const int ih0 = oh0 * p.sh - p.ph, iw0 = ow0 * p.sw - p.pw;
    if constexpr (kStaged) {
      const int n = a.patch_h * a.patch_w;
      for (int e = threadIdx.x; e < n; e += 256) {
        const int r = e / a.patch_w, c = e - r * a.patch_w;
        const int ih = ih0 + r, iw = iw0 + c;
        patch[e] = (ih >= 0 && ih < p.H && iw >= 0 && iw < p.W) ? xp[ih * p.W + iw] : 0.f;
      }
      __syncthreads();
    }
    const int ow = ow0 + lane;
    const int orow = wave * kDwRowsPerWave;
    for (int j = 0; j < m; ++j) {
      const int oc = ic * m + j;
      const float* wk = p.w + int64_t(oc) * p.KK;
      const float b = p.bias ? p.bias[oc] : 0.f;
      float acc[kDwRowsPerWave];
#pragma unroll
      for (int r = 0; r < kDwRowsPerWave; ++r) acc[r] = b;
      for (int kh = 0; kh < p.KH; ++kh)
        for (int kw = 0; kw < p.KW; ++kw) {
          const float wv = wk[kh * p.KW + kw];
          const int c = lane * p.sw + kw * p.dw;
#pragma unroll
          for (int r = 0; r < kDwRowsPerWave; ++r) {
            const int rr = (orow + r) * p.sh + kh * p.dh;
            float xv;
            if constexpr (kStaged) {
              // rr <= 15 sh + (KH-1) dh < patch_h and c <= 63 sw + (KW-1) dw < patch_w.
              xv = patch[rr * a.patch_w + c];
            } else {
              const int ih = ih0 + rr, iw = iw0 + c;
              xv = (ih >= 0 && ih < p.H && iw >= 0 && iw < p.W) ? xp[ih * p.W + iw] : 0.f;
            }
            acc[r] += xv * wv;
          }
        }
      float* yp = p.out + (int64_t(img) * p.Cout + oc) * p.OHOW;
#pragma unroll
      for (int r = 0; r < kDwRowsPerWave; ++r) {
        const int oh = oh0 + orow + r;
        if (oh < p.OH && ow < p.OW) yp[oh * p.OW + ow] = acc[r];
      }
    }
    if constexpr (kStaged) __syncthreads();  // the next tile restages the patch
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
  p.f_ohow = conv::fast_div(uint32_t(p.OHOW));
  p.f_ow = conv::fast_div(uint32_t(p.OW));
  p.f_hw = conv::fast_div(uint32_t(p.HW));
  p.f_kblk = conv::fast_div(uint32_t(p.KK * conv::kChanBlock));
  p.f_tapw = conv::fast_div(uint32_t(p.KW));
  p.f_kk = conv::fast_div(uint32_t(p.KK));
  return p;
}

bool depthwise_staged(const mx_conv2d_desc& d) {
  const int64_t ph = (kDwTileH - 1) * d.sh + (d.kh - 1) * d.dh + 1;
  const int64_t pw = (kDwTileW - 1) * d.sw + (d.kw - 1) * d.dw + 1;
  return ph * pw <= kDwLdsFloats;
}

int conv_depthwise_forward(const mx_conv2d_desc& d, const float* x, const float* w, const float* bias, float* y,
                           hipStream_t s) {
  DepthwiseArgs a{};
  a.p = make_args(d);
  a.p.x = x;
  a.p.w = w;
  a.p.bias = bias;
  a.p.out = y;
  a.tiles_w = int((d.ow + kDwTileW - 1) / kDwTileW);
  a.tiles_h = int((d.oh + kDwTileH - 1) / kDwTileH);
  a.tiles = d.n * d.cin * a.tiles_w * a.tiles_h;
  if (a.tiles == 0) return MX_OK;
  const dim3 grid(unsigned(std::min<int64_t>(a.tiles, 1 << 20)));
  if (depthwise_staged(d)) {
    a.patch_h = int((kDwTileH - 1) * d.sh + (d.kh - 1) * d.dh + 1);
    a.patch_w = int((kDwTileW - 1) * d.sw + (d.kw - 1) * d.dw + 1);
    hipLaunchKernelGGL(conv_depthwise_kernel<true>, grid, dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL(conv_depthwise_kernel<false>, grid, dim3(256), 0, s, a);
  }
  MX_HIP(hipGetLastError());
  return MX_OK;
}

int linear_blocks(int64_t total) { return int(std::min<int64_t>((total + 255) / 256, 1 << 20)); }

// Images per launch of the implicit-GEMM kernels: their loaders address each
// activation tensor with 32-bit byte offsets below kBufMaxBytes, so a larger
// batch runs as several launches over image chunks.  MX_CONV_BUFFER_LIMIT
// (bytes) lowers the bound, which lets the tests run the chunked path on small
// tensors.  Returns 0 when a single image does not fit.
int64_t images_per_launch(const mx_conv2d_desc& d) {
  // The weights are one buffer too (they cannot be split).
  if (d.cout * (d.cin / d.groups) * d.kh * d.kw * 4 >= conv::kBufMaxBytes) return 0;
  int64_t limit = conv::kBufMaxBytes;
  if (const char* e = std::getenv("MX_CONV_BUFFER_LIMIT")) {
    const long long v = std::atoll(e);
    if (v > 0 && v < limit) limit = v;
  }
  const int64_t per_img = std::max(d.cin * d.h * d.w, d.cout * d.oh * d.ow) * 4;
  return std::min<int64_t>(d.n, limit / per_img);
}

mx_conv2d_desc batch_slice(const mx_conv2d_desc& d, int64_t n) {
  mx_conv2d_desc c = d;
  c.n = n;
  return c;
}

// TORCH_VULKAN_CONV_TILE (csrc/ops/convolution.cpp:411-414): the reference's
// tile menu by name (:163-169) and the implicit-GEMM tile of this build each
// name forces.  Names keep their shape relations on this menu: base the
// smallest tile, wide the tile widest in positions, tall the one tallest in
// channels, the register tiles the square register-blocked ones; register3 and
// register3_hoist only for 3x3 filters, as the reference's fixed-3x3 tiles
// (:168-169, :369).  Unset or "auto" lets the planner choose (-1).
struct NamedTile {
  const char* name;
  int tile;
  bool fixed3x3;
};
constexpr NamedTile kNamedTiles[] = {{"base", conv::SMALL, false},   {"wide", conv::FLAT, false},
                                     {"tall", conv::TALL, false},    {"register", conv::SQ, false},
                                     {"register3", conv::WIDE, true}, {"register3_hoist", conv::SQ, true}};
constexpr int kNamedTileCount = int(sizeof(kNamedTiles) / sizeof(kNamedTiles[0]));

int tile_knob(int* idx) {
  *idx = -1;
  const char* v = std::getenv("TORCH_VULKAN_CONV_TILE");
  if (!v || !*v || std::strcmp(v, "auto") == 0) return MX_OK;
  for (int i = 0; i < kNamedTileCount; ++i)
    if (std::strcmp(v, kNamedTiles[i].name) == 0) *idx = i;
  MX_REQUIRE(*idx >= 0, MX_ERR_INVALID,
             "TORCH_VULKAN_CONV_TILE must be auto/base/wide/tall/register/register3/register3_hoist");
  return MX_OK;
}

// The tiles the planner may use for d's implicit GEMM under the knob: the
// named tile when this phase's loaders allow it, otherwise the base tile (the
// reference's fallback to tiled_base, :474-478).
unsigned knob_tiles(const mx_conv2d_desc& d, unsigned allowed) {
  int k = -1;
  if (tile_knob(&k) != MX_OK || k < 0) return allowed;
  const NamedTile& t = kNamedTiles[k];
  const unsigned base = allowed & (1u << conv::SMALL);
  if (t.fixed3x3 && !(d.kh == 3 && d.kw == 3)) return base ? base : allowed;
  const unsigned m = allowed & (1u << t.tile);
  return m ? m : (base ? base : allowed);
}

bool winograd_applicable(const mx_conv2d_desc& d) {
  return d.kh == 3 && d.kw == 3 && d.sh == 1 && d.sw == 1 && d.dh == 1 && d.dw == 1;
}

// AUTO's Winograd rule for 3x3 stride-1 layers with at least 32 channels per
// group on both sides, measured on MI355X per phase against the implicit GEMM
// (kernel time of each algorithm forced).  On typical layers the fused
// F(2x2,3x3) forward and input gradient take 0.50-0.89 of the implicit GEMM's
// time (8x64 channels at 56^2: 17.8 vs 35.6 us; 16x128 at 64^2: 98 vs 184;
// 16x512 at 8^2: 45.5 vs 60.0).  They lose where their channel walk (input
// channels for the forward, output channels for the input gradient) is long
// against the channels they produce, which sets their workgroup count, unless
// the layer has many positions: 16x1024 at 16^2 to 32 takes 98.5 vs 54.1 us,
// at 56^2 (8 images) 155 vs 254.  Over 401 layers per phase (batch 1-32,
// 7^2-56^2, 32-1024 x 32-512 channels) the rule below (Winograd from 16384
// positions, or from 512 when the walk is at most 4x the channels produced)
// sums to 2.0% (forward) and 2.4% (input gradient) above the faster algorithm
// per layer, a cut at 1024 positions to 6.7% and 4.6%.  The weight gradient's
// break-even follows the layer's work, not its positions: in two sweeps (342
// and 401 layers: batch 1-32, 7^2-56^2, 32-1024 input x 32-512 output
// channels, kernel time of each algorithm forced) it wins from
// 2^25 multiply-adds per filter tap (positions x input channels per group x
// output channels; 16x512 at 8^2 to 512: 46 vs 73 us) and loses below
// (8x32 at 16^2 to 64: 11.8 vs 10.5 us); summed over each sweep it costs
// 0.7-0.8% more than the faster algorithm per layer, a 2048-position cut
// 8-15% more.  This replaces the reference heuristic for these layers (its
// Winograd is a grouped-layer forward rule, csrc/ops/convolution.cpp:454-460,
// kept below); every other layer, and padding beyond 2, keeps the
// reference's choices.
bool winograd_auto(const mx_conv2d_desc& d, int phase) {
  if (!winograd_applicable(d) || d.ph > 2 || d.pw > 2 || d.cin / d.groups < 32 || d.cout / d.groups < 32)
    return false;
  const int64_t positions = d.n * d.oh * d.ow;
  if (phase == MX_CONV_DWEIGHT) return positions * (d.cin / d.groups) * d.cout >= (int64_t(1) << 25);
  const int64_t walk = (phase == MX_CONV_FORWARD ? d.cin : d.cout) / d.groups;
  const int64_t made = (phase == MX_CONV_FORWARD ? d.cout : d.cin) / d.groups;
  return positions >= 16384 || (positions >= 512 && walk <= 4 * made);
}

// Reference heuristic (csrc/ops/convolution.cpp:423-482) restated for the
// MFMA candidates: implicit GEMM whenever the GEMM is not degenerate, Winograd
// for the grouped 3x3 case the reference routes there by default and, in all
// three phases, for the 3x3 stride-1 layers where it measures faster on
// MI355X (winograd_auto).
int select_algo_heuristic(const mx_conv2d_desc& d, int phase, int requested, int* algo);

// The implicit GEMM runs one grid-z slice per group: past 65535 groups AUTO
// takes the direct kernels and a forced implicit GEMM is refused.
int select_algo(const mx_conv2d_desc& d, int phase, int requested, int* algo) {
  MX_TRY(select_algo_heuristic(d, phase, requested, algo));
  if (*algo == MX_CONV_ALGO_IMPLICIT_GEMM && d.groups > 65535) {
    MX_REQUIRE(requested != MX_CONV_ALGO_IMPLICIT_GEMM, MX_ERR_UNSUPPORTED,
               "conv2d implicit GEMM: at most 65535 groups (one launch slice per group)");
    *algo = MX_CONV_ALGO_DIRECT;
  }
  return MX_OK;
}

int select_algo_heuristic(const mx_conv2d_desc& d, int phase, int requested, int* algo) {
  const int64_t cin_g = d.cin / d.groups, cout_g = d.cout / d.groups;
  const int64_t rows = d.n * d.oh * d.ow, cols = cin_g * d.kh * d.kw;
  MX_REQUIRE(requested >= MX_CONV_ALGO_AUTO && requested <= MX_CONV_ALGO_DEPTHWISE, MX_ERR_INVALID,
             "conv2d: unknown algorithm ", requested);
  int knob = -1;
  MX_TRY(tile_knob(&knob));
  if (requested == MX_CONV_ALGO_IMPLICIT_GEMM && phase != MX_CONV_DBIAS && knob >= 0 &&
      kNamedTiles[knob].fixed3x3 && !(d.kh == 3 && d.kw == 3)) {
    static const char* names[] = {"forward", "dinput", "dweight"};
    return set_error(MX_ERR_UNSUPPORTED, cat("Forced Vulkan convolution ", names[phase], " candidate tiled_",
                                             kNamedTiles[knob].name,
                                             " exceeds device limits, workspace budget, or operator applicability"));
  }
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
      if (requested == MX_CONV_ALGO_DEPTHWISE)
        MX_REQUIRE(d.groups == d.cin, MX_ERR_UNSUPPORTED,
                   "Forced Vulkan convolution forward candidate depthwise exceeds device limits, workspace "
                   "budget, or operator applicability");
      if (requested != MX_CONV_ALGO_AUTO) {
        *algo = requested;
        return MX_OK;
      }
      // Small-channel layers (a 3-channel stem or output head) still go to
      // the MFMA implicit GEMM: a mostly-empty tile row is cheaper than the
      // direct kernel's per-output loop once the GEMM has real depth.
      if ((winograd_applicable(d) && d.groups >= 4 && cin_g >= 16 && cout_g >= 16 && rows >= 2048) ||
          winograd_auto(d, MX_CONV_FORWARD))
        *algo = MX_CONV_ALGO_WINOGRAD;
      else if (d.groups == d.cin && d.cin >= 8)
        *algo = MX_CONV_ALGO_DEPTHWISE;
      else if (cols >= 8 && rows >= 32 && cout_g * cols >= 64)
        *algo = MX_CONV_ALGO_IMPLICIT_GEMM;
      else
        *algo = MX_CONV_ALGO_DIRECT;
      return MX_OK;
    case MX_CONV_DINPUT:
      // Winograd input gradients are a choice of this build (the reference's
      // Winograd is forward only); AUTO keeps the reference's candidates.
      if (requested == MX_CONV_ALGO_WINOGRAD) {
        MX_REQUIRE(winograd_applicable(d) && d.ph <= 2 && d.pw <= 2, MX_ERR_UNSUPPORTED,
                   "Forced convolution dinput candidate winograd_f2 needs a 3x3 stride-1 dilation-1 layer with "
                   "padding <= 2");
        *algo = MX_CONV_ALGO_WINOGRAD;
        return MX_OK;
      }
      MX_REQUIRE(requested != MX_CONV_ALGO_REDUCE && requested != MX_CONV_ALGO_DEPTHWISE, MX_ERR_UNSUPPORTED,
                 "dinput supports direct, implicit_gemm and winograd only");
      if (requested != MX_CONV_ALGO_AUTO) {
        *algo = requested;
        return MX_OK;
      }
      if (winograd_auto(d, MX_CONV_DINPUT)) {
        *algo = MX_CONV_ALGO_WINOGRAD;
        return MX_OK;
      }
      *algo = (cin_g >= 2 && cout_g * d.kh * d.kw >= 8 && cin_g * cout_g * d.kh * d.kw >= 64 &&
               d.n * d.h * d.w >= 32)
                  ? MX_CONV_ALGO_IMPLICIT_GEMM
                  : MX_CONV_ALGO_DIRECT;
      return MX_OK;
    case MX_CONV_DWEIGHT:
      // Winograd weight gradients (the adjoint of the forward transform) are,
      // like Winograd input gradients, a choice of this build made on request.
      if (requested == MX_CONV_ALGO_WINOGRAD) {
        MX_REQUIRE(winograd_applicable(d), MX_ERR_UNSUPPORTED,
                   "Forced convolution dweight candidate winograd_f2 needs a 3x3 stride-1 dilation-1 layer");
        *algo = MX_CONV_ALGO_WINOGRAD;
        return MX_OK;
      }
      MX_REQUIRE(requested != MX_CONV_ALGO_DEPTHWISE, MX_ERR_UNSUPPORTED,
                 "depthwise is a forward convolution algorithm");
      if (requested != MX_CONV_ALGO_AUTO) {
        *algo = requested;
        return MX_OK;
      }
      if (winograd_auto(d, MX_CONV_DWEIGHT))
        *algo = MX_CONV_ALGO_WINOGRAD;
      else if (rows >= 64 && cout_g * cols >= 64)
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

// Per-tile figures for the planners: rows, columns, workgroups resident per
// CU, and the CU's MFMA throughput with a full set of such tiles, relative to
// 85% of its FP32 peak.  The rates (and the constants of plan_cost) were
// fitted to measured times of every (tile, split) plan on the 53 ResNet-50
// layers (forward, dInput, dWeight) on MI355X: the fitted planner's choices
// cost 1.5% more in total than the best measured plan per layer.
struct TileInfo {
  int bm, bn, per_cu;
  double rate;
  const char* name;
};
constexpr TileInfo kTileInfo[conv::NTILES] = {
    {256, 128, 2, 1.20, "256x128x16"}, {128, 256, 2, 1.22, "128x256x16"}, {128, 128, 2, 1.15, "128x128x16"},
    {64, 256, 2, 0.68, "64x256x16"},   {256, 64, 2, 0.76, "256x64x16"},   {64, 64, 4, 1.10, "64x64x32"}};

// Kernel tag of a tile for a phase: forward and dInput compile the small tile
// with 16-deep slabs (conv::TileSmallShallow).
const char* tile_name(int tile, int phase) {
  return (tile == conv::SMALL && phase != MX_CONV_DWEIGHT) ? "64x64x16" : kTileInfo[tile].name;
}

// Estimated time of one implicit GEMM (per group M x Ncols x K, G groups)
// with tile `ti` and K split `splits` ways of kps each, plus the finalize pass
// that sums the partial outputs.  A CU holding n tiles runs at
// rate * occ(n) of its share of 85% of the FP32 MFMA peak, occ rising from
// 0.75 with one resident tile to 1 with per_cu; tiles beyond that queue.  The
// finalize moves (splits + 1) outputs' bytes at an effective 3.1 TB/s.  The
// two constants were fitted on MI355X to every (tile, split) plan of 83
// layer phases (C3's implicit-GEMM layers and the small C1 / C4 layers, each
// plan forced and timed): the planner's picks sum to 0.1-0.4% above the
// best plan per layer on C3 and 1.5-1.6% on the small layers, against 0.5%
// and 8.9% with the earlier 0.56 and 8 TB/s.
double plan_cost(const TileInfo& ti, int64_t M, int64_t Ncols, int64_t G, int64_t splits, int64_t kps,
                 int64_t out_elems) {
  const double cu = cu_count();
  const double cu_flops = 0.85 * 157.3e12 / 256.0;
  const int64_t tiles = ((M + ti.bm - 1) / ti.bm) * ((Ncols + ti.bn - 1) / ti.bn) * G;
  const int64_t per_cu = (tiles * splits + int64_t(cu) - 1) / int64_t(cu);
  const double occ = std::min(1.0, 0.75 + 0.25 * double(per_cu - 1) / double(ti.per_cu - 1));
  double t = double(per_cu) * 2.0 * ti.bm * ti.bn * double(kps) / (cu_flops * ti.rate * occ) + 2e-6;
  if (splits > 1) t += double(splits + 1) * double(out_elems) * 4.0 / 3.1e12 + 3e-6;
  return t;
}

constexpr int kSplitBK = 32;         // K granularity of a split (a multiple of every loader run)
constexpr int kMinSplitSpan = 128;   // shortest K range worth a split

struct GemmPlan {
  int tile = conv::SQ;
  int splits = 1;
  int kps = 0;
};

// Cheapest (tile, K split) over the allowed tiles (bit mask over conv::Tile)
// and split counts up to max_splits.  A split plan needs `ws_per_split` bytes
// of partial outputs per split, all within the workspace budget `ws_limit`.
// MX_CONV_PLAN="tile,splits" (tile index in conv::Tile order) forces the tile
// when this phase and shape can use it, with the largest split count up to
// `splits` that the shape and the budget allow (for tests, tuning and
// diagnosis); a forced split for which the budget holds no split at all is an
// error, as a forced algorithm beyond the budget is in
// csrc/ops/convolution.cpp:472-473.
int plan_gemm(int64_t M, int64_t Ncols, int64_t K, int64_t G, unsigned tiles, int64_t max_splits,
              int64_t out_elems, int64_t ws_per_split, int64_t ws_limit, GemmPlan* out) {
  int force_tile = -1, force_splits = 0;
  if (const char* e = std::getenv("MX_CONV_PLAN")) {
    if (std::sscanf(e, "%d,%d", &force_tile, &force_splits) != 2 || force_tile < 0 || force_tile >= conv::NTILES ||
        !(tiles & (1u << force_tile)) || force_splits < 1)
      force_tile = -1;
  }
  GemmPlan best;
  double best_t = -1;
  bool budget_stop = false;
  static const int kSplits[] = {1, 2, 3, 4, 6, 8, 12, 16, 24, 32, 48, 64, 96, 128, 192, 256, 384, 512};
  for (int t = 0; t < conv::NTILES; ++t) {
    if (!(tiles & (1u << t)) || (force_tile >= 0 && t != force_tile)) continue;
    for (int want : kSplits) {
      if (want > max_splits || (force_tile >= 0 && want > force_splits)) break;
      int64_t kps = (K + want - 1) / want;
      kps = (kps + kSplitBK - 1) / kSplitBK * kSplitBK;
      const int64_t splits = (K + kps - 1) / kps;
      if (splits > 1 && kps < kMinSplitSpan) break;
      if (splits > 1 && splits * ws_per_split > ws_limit) {
        budget_stop = true;
        break;
      }
      const double cost = plan_cost(kTileInfo[t], M, Ncols, G, splits, kps, out_elems);
      if (force_tile >= 0 || best_t < 0 || cost < best_t) {  // forced: the largest split that fits
        best_t = cost;
        best.tile = t;
        best.splits = int(splits);
        best.kps = int(kps);
      }
    }
  }
  if (force_tile >= 0 && budget_stop && best.splits == 1)
    return set_error(MX_ERR_WORKSPACE, cat("Forced convolution plan ", force_tile, ",", force_splits,
                                           " exceeds the workspace budget (TORCH_VULKAN_CONV_WORKSPACE_MB)"));
  *out = best;
  return MX_OK;
}

constexpr unsigned kAllTiles = (1u << conv::NTILES) - 1;
constexpr unsigned kSinglePassTiles = kAllTiles & ~(1u << conv::NARROW);  // forward / dInput

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

// Stand-in operand address for plans made without data (the variant and
// plan queries): device allocations are at least 256-byte aligned.
const float* kAlignedNull = reinterpret_cast<const float*>(uintptr_t(256));
float* const kAlignedOut = reinterpret_cast<float*>(uintptr_t(256));

bool unpadded_1x1(const ConvArgs& p) {
  return p.KH == 1 && p.KW == 1 && p.sh == 1 && p.sw == 1 && p.ph == 0 && p.pw == 0;
}

// ----------------------------------------------------------------- forward
struct FwdPlan {
  ConvArgs p{};
  GemmPlan gp;
  bool packed = false;  // weights copied to the channel-blocked K order
  bool padded = false;  // weights copied to rows padded to a multiple of four floats
  int bmode = conv::B_GATHER;
  int64_t w_bytes = 0, ws_bytes = 0;
};

int plan_forward(const mx_conv2d_desc& d, const float* x, const float* w, const float* bias, float* y,
                 int64_t ws_limit, FwdPlan* f) {
  ConvArgs& p = f->p;
  p = make_args(d);
  p.x = x;
  p.w = w;
  p.wt = w;
  p.bias = bias;
  p.out = y;
  p.M = p.Cout_g;
  p.Ncols = p.N * p.OHOW;
  p.K = p.Cin_g * p.KK;
  f->packed = p.KK > 1 && conv::blocked_channels(p.Cin_g);
  // Weight rows are read 16 bytes per lane: a K that is not a multiple of
  // four, or unaligned weights, get a copy with rows padded to a multiple of
  // four floats.
  f->padded = !f->packed && (p.K % 4 != 0 || !aligned16(w));
  f->bmode = (unpadded_1x1(p) && p.HW % 4 == 0 && aligned16(x)) ? conv::B_VEC : conv::B_GATHER;
  p.out_elems = int64_t(p.N) * p.Cout * p.OHOW;
  MX_TRY(plan_gemm(p.Cout_g, int64_t(p.N) * p.OHOW, int64_t(p.Cin_g) * p.KK, p.G, knob_tiles(d, kSinglePassTiles), 512,
                   p.out_elems, p.out_elems * 4, ws_limit, &f->gp));
  p.splits = f->gp.splits;
  p.kps = f->gp.kps;
  p.ldw = f->padded ? (p.K + 3) / 4 * 4 : p.K;
  f->w_bytes = f->packed ? int64_t(p.Cout) * p.Cin_g * p.KK * 4 : f->padded ? int64_t(p.Cout) * p.ldw * 4 : 0;
  f->ws_bytes = f->gp.splits > 1 ? int64_t(f->gp.splits) * p.out_elems * 4 : 0;
  return MX_OK;
}

std::string fwd_variant(const FwdPlan& f) {
  const char* b = f.bmode == conv::B_VEC ? "PosQuad"
                  : conv::blocked_channels(f.p.Cin_g) ? "Im2col<blocked>" : "Im2col";
  return cat("conv_fwd_kernel<", tile_name(f.gp.tile, MX_CONV_FORWARD), ",KVEC,", b, ">",
             f.gp.splits > 1 ? "+split" : "");
}

// ----------------------------------------------------------------- dInput
// dInput stride phases.  Along one axis, phase a (input index = a mod s) is
// reached by the taps k with (a + pad - k*dil) % s == 0: k = k0 + t*step with
// step = s / gcd(s, dil); tap t reads output index i + off0 - t*(dil / gcd).
struct AxisPhase {
  int len = 0;   // input positions in the phase
  int taps = 0;
  int k0 = 0, step = 1, off0 = 0, dstep = 0;
};

AxisPhase axis_phase(int a, int in, int k, int s, int pad, int dil) {
  AxisPhase ph;
  ph.len = a < in ? (in - a + s - 1) / s : 0;
  const int gcd = std::gcd(s, dil);
  ph.step = s / gcd;
  ph.dstep = dil / gcd;
  int k0 = -1;
  for (int kk = 0; kk < std::min(k, ph.step); ++kk)
    if (((a + pad - kk * dil) % s + s) % s == 0) {
      k0 = kk;
      break;
    }
  if (k0 < 0) return ph;
  ph.k0 = k0;
  ph.taps = (k - 1 - k0) / ph.step + 1;
  ph.off0 = (a + pad - k0 * dil) / s;  // exact division
  return ph;
}

struct DxPlan {
  ConvArgs p{};
  std::vector<ConvArgs> phases;  // every phase with input positions (K == 0: no tap reaches it)
  std::vector<int> bmodes;       // per phase: B_VEC for a one-to-one phase read 16 bytes per lane
  GemmPlan gp;
  bool packed = false, vec_a = false, any_zero = false, zfill = false;
  int64_t out_elems = 0, w_bytes = 0, ws_bytes = 0;
};

// One GEMM per stride phase over exactly the taps that reach it, one
// (tile, split) plan for all of them made on the phase with the most work.
// Split-K only when every phase has taps, so every partial output element is
// written by some phase.
int plan_dinput(const mx_conv2d_desc& d, const float* dy, const float* w, float* dx, int64_t ws_limit, DxPlan* f) {
  ConvArgs& p = f->p;
  p = make_args(d);
  p.dy = dy;
  p.w = w;
  p.wt = w;
  p.out = dx;
  int64_t best_work = -1, bm = 0, bn = 0, bk = 0;
  for (int a = 0; a < p.sh; ++a) {
    const AxisPhase ah = axis_phase(a, p.H, p.KH, p.sh, p.ph, p.dh);
    for (int b = 0; b < p.sw; ++b) {
      const AxisPhase aw = axis_phase(b, p.W, p.KW, p.sw, p.pw, p.dw);
      if (ah.len == 0 || aw.len == 0) continue;
      ConvArgs q = p;
      q.pa = a;
      q.pb = b;
      q.Hp = ah.len;
      q.Wp = aw.len;
      q.HpWp = ah.len * aw.len;
      q.nth = ah.taps;
      q.ntw = aw.taps;
      q.offh0 = ah.off0;
      q.offw0 = aw.off0;
      q.dsh = ah.dstep;
      q.dsw = aw.dstep;
      q.kh0 = ah.k0;
      q.kw0 = aw.k0;
      q.stph = ah.step;
      q.stpw = aw.step;
      q.M = p.Cin_g;
      q.Ncols = p.N * q.HpWp;
      q.K = p.Cout_g * q.nth * q.ntw;
      if (q.K == 0) f->any_zero = true;
      const int64_t work = int64_t(q.K) * q.Ncols;
      if (work > best_work) {
        best_work = work;
        bm = q.M;
        bn = q.Ncols;
        bk = q.K;
      }
      f->phases.push_back(q);
    }
  }
  f->out_elems = int64_t(p.N) * p.Cin * p.HW;
  MX_TRY(plan_gemm(bm, bn, std::max<int64_t>(bk, 1), p.G, knob_tiles(d, kSinglePassTiles), f->any_zero ? 1 : 512,
                   f->out_elems, f->out_elems * 4, ws_limit, &f->gp));
  // A 1x1 kernel is already [g][co][ci]; larger kernels are packed per phase.
  f->packed = p.KK > 1;
  f->vec_a = p.Cin_g % 4 == 0 && (f->packed || aligned16(w));
  bool only_00 = true;
  for (const ConvArgs& q : f->phases)
    if (q.K != 0 && (q.pa != 0 || q.pb != 0)) only_00 = false;
  // Stride 2 x 2 with phase (0, 0) the only one reached and W even: the
  // GEMM writes the zeros of each 2x2 block itself (8-byte aligned stores).
  f->zfill = f->any_zero && only_00 && p.sh == 2 && p.sw == 2 && p.W % 2 == 0 &&
             (reinterpret_cast<uintptr_t>(dx) & 7) == 0 && f->gp.splits == 1 && f->gp.tile != conv::TALL &&
             f->gp.tile != conv::WIDE;
  for (ConvArgs& q : f->phases) {
    const bool one_to_one = q.nth == 1 && q.ntw == 1 && q.offh0 == 0 && q.offw0 == 0 && q.Hp == p.OH &&
                            q.Wp == p.OW && p.OHOW % 4 == 0 && aligned16(dy);
    f->bmodes.push_back(one_to_one ? conv::B_VEC : conv::B_GATHER);
    if (q.K == 0) continue;
    q.zfill = f->zfill ? 1 : 0;
    q.f_kblk = conv::fast_div(uint32_t(q.nth * q.ntw * conv::kChanBlock));
    q.f_tapw = conv::fast_div(uint32_t(q.ntw));
    q.f_kk = conv::fast_div(uint32_t(q.nth * q.ntw));
    q.splits = f->gp.splits;
    q.kps = int((q.K + f->gp.splits - 1) / f->gp.splits + kSplitBK - 1) / kSplitBK * kSplitBK;
    q.out_elems = f->out_elems;
  }
  f->w_bytes = f->packed ? int64_t(p.Cout) * p.Cin_g * p.KK * 4 : 0;
  f->ws_bytes = f->gp.splits > 1 ? int64_t(f->gp.splits) * f->out_elems * 4 : 0;
  return MX_OK;
}

std::string dx_variant(const DxPlan& f) {
  std::vector<std::string> names;
  for (size_t i = 0; i < f.phases.size(); ++i) {
    const ConvArgs& q = f.phases[i];
    if (q.K == 0) continue;
    // Phases sharing a loader run as one conv_dx_phases_kernel launch.
    int same = 0;
    for (size_t j = 0; j < f.phases.size(); ++j) same += f.phases[j].K != 0 && f.bmodes[j] == f.bmodes[i];
    const char* b = f.bmodes[i] == conv::B_VEC ? "PosQuad"
                    : conv::blocked_channels(q.Cout_g) ? "PhaseGather<blocked>" : "PhaseGather";
    std::string n = cat(same > 1 ? "conv_dx_phases_kernel<" : "conv_dx_kernel<", tile_name(f.gp.tile, MX_CONV_DINPUT),
                        ",", f.vec_a ? "RVEC" : "RSCALAR", ",", b, ">", f.gp.splits > 1 ? "+split" : "",
                        f.zfill ? "+zfill" : "");
    if (std::find(names.begin(), names.end(), n) == names.end()) names.push_back(n);
  }
  std::string out;
  for (const std::string& n : names) out += (out.empty() ? "" : " ") + n;
  return out.empty() ? "conv_dx_zero_kernel" : out;
}

// ----------------------------------------------------------------- dWeight
struct DwPlan {
  ConvArgs p{};
  GemmPlan gp;
  int amode = conv::B_GATHER, bmode = conv::B_GATHER;
  bool with_db = false;
  int64_t ws_bytes = 0, db_bytes = 0;
};

// dWeight: K = N*OH*OW positions, split so every CU gets work; each split
// writes one full-size partial dW (and a dBias partial) that the finalize
// re-reads.  The x operand is the column gather unless the kernel is an
// unpadded 1x1 stride-1 one with 4-aligned planes; dy is read as scalar rows
// when OH*OW % 4 != 0.  Gathers over 256 columns (and a 256-wide tile with
// both gathers) are not built.
int plan_dweight(const mx_conv2d_desc& d, const float* x, const float* dy, float* dw, float* db, int64_t ws_limit,
                 DwPlan* f) {
  ConvArgs& p = f->p;
  p = make_args(d);
  p.x = x;
  p.dy = dy;
  p.out = dw;
  p.db = db;
  const bool with_db = db != nullptr;
  p.M = p.Cout_g;
  p.Ncols = p.Cin_g * p.KK;
  p.K = p.N * p.OHOW;
  f->with_db = with_db;
  f->amode = (p.OHOW % 4 == 0 && aligned16(dy)) ? conv::B_VEC : conv::B_GATHER;
  f->bmode = (unpadded_1x1(p) && p.HW % 4 == 0 && aligned16(x)) ? conv::B_VEC : conv::B_GATHER;
  p.cols_blocked = f->bmode == conv::B_GATHER && conv::blocked_channels(p.Cin_g) ? 1 : 0;
  const int64_t out = int64_t(p.G) * p.Cout_g * p.Ncols;
  unsigned tiles = kAllTiles;
  if (f->bmode == conv::B_GATHER) tiles &= ~((1u << conv::WIDE) | (1u << conv::FLAT));
  if (f->bmode == conv::B_GATHER && f->amode == conv::B_GATHER) tiles &= ~(1u << conv::TALL);
  const int64_t per_split = out * 4 + (with_db ? int64_t(p.Cout) * 4 : 0);
  MX_TRY(plan_gemm(p.M, p.Ncols, p.K, p.G, knob_tiles(d, tiles), 65535, out, per_split, ws_limit, &f->gp));
  p.splits = f->gp.splits;
  p.kps = f->gp.kps;
  if (f->gp.splits > 1) {
    f->ws_bytes = int64_t(f->gp.splits) * out * 4;
    f->db_bytes = with_db ? int64_t(f->gp.splits) * p.Cout * 4 : 0;
  }
  return MX_OK;
}

std::string dw_variant(const DwPlan& f) {
  const char* a = f.amode == conv::B_VEC ? "PosK" : "DyRows";
  const char* b = f.bmode == conv::B_VEC ? "PosK" : f.p.cols_blocked ? "XCols<blocked>" : "XCols";
  return cat("conv_dw_kernel<", kTileInfo[f.gp.tile].name, ",", a, ",", b, ">", f.gp.splits > 1 ? "+split" : "",
             f.with_db ? "+db" : "");
}

}  // namespace

// Winograd lives in mx_winograd.hip.
int winograd_forward(const mx_conv2d_desc& d, const float* x, const float* w, const float* bias, float* y,
                     int64_t ws_limit, hipStream_t s);
int winograd_backward_input(const mx_conv2d_desc& d, const float* dy, const float* w, float* dx, int64_t ws_limit,
                            hipStream_t s);
int winograd_backward_weight(const mx_conv2d_desc& d, const float* x, const float* dy, float* dw, float* db,
                             int64_t ws_limit, float* ext, hipStream_t s);
int winograd_describe(const mx_conv2d_desc& d, int phase, bool with_bias, int64_t ws_limit, std::string* variant,
                      int64_t* ws_bytes);
int winograd_backward(const mx_conv2d_desc& d, const float* x, const float* w, const float* dy, float* dx, float* dw,
                      float* db, int64_t ws_limit, hipStream_t s, bool* done);
int winograd_backward_one_launch(const mx_conv2d_desc& d, int64_t ws_limit, bool with_db, bool* one);

namespace conv {
// Scratch budget of one convolution call (split-K partials, the Winograd
// weight gradient's range partials, the unfused Winograd transforms):
// TORCH_VULKAN_CONV_WORKSPACE_MB, an integer number of MiB in [0, 4096],
// 64 when unset (csrc/ops/convolution.cpp:239-247).  Weight-sized copies
// (packed or transformed filters) are not counted.
int workspace_limit(int64_t* bytes) {
  const char* v = std::getenv("TORCH_VULKAN_CONV_WORKSPACE_MB");
  if (!v || !*v) {
    *bytes = int64_t(64) << 20;
    return MX_OK;
  }
  char* end = nullptr;
  const unsigned long long mb = std::strtoull(v, &end, 10);
  MX_REQUIRE(*v != '-' && end != v && *end == '\0' && mb <= 4096, MX_ERR_INVALID,
             "TORCH_VULKAN_CONV_WORKSPACE_MB must be an integer in [0,4096]");
  *bytes = int64_t(mb) << 20;
  return MX_OK;
}
}  // namespace conv

}  // namespace mx

using namespace mx;

namespace {

// Entry points work on a copy of the caller's descriptor (checked_desc fills
// in its output size).
int copy_desc(const mx_conv2d_desc* desc, mx_conv2d_desc* d) {
  MX_REQUIRE(desc, MX_ERR_INVALID, "conv2d: null descriptor");
  *d = *desc;
  return MX_OK;
}

// Plan of one call of `phase` (no data touched): the algorithm that runs, the
// implicit GEMM's tile and K split, the scratch counted against the workspace
// budget and the kernel instantiations launched.
int describe(const mx_conv2d_desc* desc, int phase, int algo, int with_bias, mx_conv2d_plan_info* info) {
  mx_conv2d_desc d{};
  MX_TRY(copy_desc(desc, &d));
  MX_TRY(checked_desc(&d));
  int chosen = 0;
  MX_TRY(select_algo(d, phase, algo, &chosen));
  int64_t limit = 0;
  MX_TRY(conv::workspace_limit(&limit));
  mx_conv2d_plan_info r{};
  r.algo = chosen;
  r.tile = -1;
  r.splits = 1;
  std::string name;
  if (phase == MX_CONV_DBIAS) {
    name = chosen == MX_CONV_ALGO_DIRECT ? "conv_db_direct_kernel" : "conv_db_reduce_kernel";
  } else if (chosen == MX_CONV_ALGO_WINOGRAD) {
    MX_TRY(winograd_describe(d, phase, with_bias != 0, limit, &name, &r.workspace_bytes));
  } else if (chosen == MX_CONV_ALGO_DEPTHWISE) {
    name = depthwise_staged(d) ? "conv_depthwise_kernel<staged>" : "conv_depthwise_kernel<global>";
  } else if (chosen == MX_CONV_ALGO_DIRECT) {
    name = phase == MX_CONV_FORWARD  ? "conv_fwd_direct_kernel"
           : phase == MX_CONV_DINPUT ? "conv_dx_direct_kernel"
                                     : "conv_dw_direct_kernel";
    if (phase == MX_CONV_DWEIGHT && with_bias) name += " conv_db_reduce_kernel";
  } else if (chosen == MX_CONV_ALGO_REDUCE) {
    name = "conv_dw_reduce_kernel";
    if (with_bias) name += " conv_db_reduce_kernel";
  } else if (phase == MX_CONV_FORWARD) {
    FwdPlan f;
    MX_TRY(plan_forward(d, kAlignedNull, kAlignedNull, nullptr, kAlignedOut, limit, &f));
    name = fwd_variant(f);
    r.tile = f.gp.tile;
    r.splits = f.gp.splits;
    r.span = f.gp.kps;
    r.workspace_bytes = f.ws_bytes;
  } else if (phase == MX_CONV_DINPUT) {
    DxPlan f;
    MX_TRY(plan_dinput(d, kAlignedNull, kAlignedNull, kAlignedOut, limit, &f));
    name = dx_variant(f);
    r.tile = f.gp.tile;
    r.splits = f.gp.splits;
    r.span = f.gp.kps;
    r.workspace_bytes = f.ws_bytes;
  } else {
    DwPlan f;
    MX_TRY(plan_dweight(d, kAlignedNull, kAlignedNull, kAlignedOut, with_bias ? kAlignedOut : nullptr, limit, &f));
    name = dw_variant(f);
    r.tile = f.gp.tile;
    r.splits = f.gp.splits;
    r.span = f.gp.kps;
    r.workspace_bytes = f.ws_bytes + f.db_bytes;
  }
  if (images_per_launch(d) < d.n && (chosen == MX_CONV_ALGO_IMPLICIT_GEMM || chosen == MX_CONV_ALGO_WINOGRAD))
    name += "+batch_chunks";
  std::strncpy(r.variant, name.c_str(), sizeof r.variant - 1);
  *info = r;
  return MX_OK;
}

}  // namespace

extern "C" {

int mx_conv2d_check(mx_conv2d_desc* desc) {
  MX_ABI_BEGIN
  return checked_desc(desc);
  MX_ABI_END
}

int mx_conv2d_select(const mx_conv2d_desc* desc, int phase, int requested, int* algo) {
  MX_ABI_BEGIN
  mx_conv2d_desc d{};
  MX_TRY(copy_desc(desc, &d));
  MX_TRY(checked_desc(&d));
  return select_algo(d, phase, requested, algo);
  MX_ABI_END
}

int mx_conv2d_forward(const mx_conv2d_desc* desc, const float* x, const float* w, const float* bias, float* y,
                      int algo, void* stream) {
  MX_ABI_BEGIN
  mx_conv2d_desc d{};
  MX_TRY(copy_desc(desc, &d));
  MX_TRY(checked_desc(&d));
  MX_REQUIRE(x && w && y, MX_ERR_INVALID, "conv2d forward: null tensor");
  int chosen = 0;
  MX_TRY(select_algo(d, MX_CONV_FORWARD, algo, &chosen));
  int64_t limit = 0;
  MX_TRY(conv::workspace_limit(&limit));
  hipStream_t s = resolve_stream(stream);
  if (chosen == MX_CONV_ALGO_IMPLICIT_GEMM || chosen == MX_CONV_ALGO_WINOGRAD) {
    const int64_t nc = images_per_launch(d);
    MX_REQUIRE(nc > 0, MX_ERR_UNSUPPORTED, "conv2d forward: one image or the weights exceed the 2 GiB operand bound");
    if (nc < d.n) {
      for (int64_t n0 = 0; n0 < d.n; n0 += nc) {
        const mx_conv2d_desc c = batch_slice(d, std::min(nc, d.n - n0));
        MX_TRY(mx_conv2d_forward(&c, x + n0 * d.cin * d.h * d.w, w, bias, y + n0 * d.cout * d.oh * d.ow, chosen,
                                 stream));
      }
      return MX_OK;
    }
  }
  if (chosen == MX_CONV_ALGO_WINOGRAD) return winograd_forward(d, x, w, bias, y, limit, s);
  if (chosen == MX_CONV_ALGO_DEPTHWISE) return conv_depthwise_forward(d, x, w, bias, y, s);
  if (chosen == MX_CONV_ALGO_DIRECT) {
    ConvArgs p = make_args(d);
    p.x = x;
    p.w = w;
    p.bias = bias;
    p.out = y;
    hipLaunchKernelGGL(conv_fwd_direct_kernel, dim3(linear_blocks(d.n * d.cout * d.oh * d.ow)), dim3(256), 0, s, p);
    MX_HIP(hipGetLastError());
    return MX_OK;
  }
  FwdPlan f;
  MX_TRY(plan_forward(d, x, w, bias, y, limit, &f));
  ConvArgs& p = f.p;
  Scratch wp, ws;
  if (f.packed) {  // pack to the blocked K order
    MX_TRY(wp.alloc(size_t(f.w_bytes), s));
    MX_TRY(conv::conv_fwd_pack_weights(p, wp.as<float>(), s));
    p.wt = wp.as<float>();
  } else if (f.padded) {
    MX_TRY(wp.alloc(size_t(f.w_bytes), s));
    MX_TRY(conv::conv_fwd_pad_weights(p, wp.as<float>(), s));
    p.wt = wp.as<float>();
  }
  if (f.gp.splits == 1) return conv::conv_fwd_launch(p, f.gp.tile, Mode::KVEC, f.bmode, s);
  MX_TRY(ws.alloc(size_t(f.ws_bytes), s));
  p.ws = ws.as<float>();
  MX_TRY(conv::conv_fwd_launch(p, f.gp.tile, Mode::KVEC, f.bmode, s));
  return conv::conv_sum_splits(p.ws, f.gp.splits, p.out_elems, y, bias, p.OHOW, p.Cout, s);
  MX_ABI_END
}

int mx_conv2d_backward_input(const mx_conv2d_desc* desc, const float* dy, const float* w, float* dx, int algo,
                             void* stream) {
  MX_ABI_BEGIN
  mx_conv2d_desc d{};
  MX_TRY(copy_desc(desc, &d));
  MX_TRY(checked_desc(&d));
  MX_REQUIRE(dy && w && dx, MX_ERR_INVALID, "conv2d dinput: null tensor");
  int chosen = 0;
  MX_TRY(select_algo(d, MX_CONV_DINPUT, algo, &chosen));
  int64_t limit = 0;
  MX_TRY(conv::workspace_limit(&limit));
  hipStream_t s = resolve_stream(stream);
  if (chosen == MX_CONV_ALGO_IMPLICIT_GEMM || chosen == MX_CONV_ALGO_WINOGRAD) {
    const int64_t nc = images_per_launch(d);
    MX_REQUIRE(nc > 0, MX_ERR_UNSUPPORTED, "conv2d dinput: one image or the weights exceed the 2 GiB operand bound");
    if (nc < d.n) {
      for (int64_t n0 = 0; n0 < d.n; n0 += nc) {
        const mx_conv2d_desc c = batch_slice(d, std::min(nc, d.n - n0));
        MX_TRY(mx_conv2d_backward_input(&c, dy + n0 * d.cout * d.oh * d.ow, w, dx + n0 * d.cin * d.h * d.w,
                                        chosen, stream));
      }
      return MX_OK;
    }
  }
  if (chosen == MX_CONV_ALGO_WINOGRAD) return winograd_backward_input(d, dy, w, dx, limit, s);
  if (chosen == MX_CONV_ALGO_DIRECT) {
    ConvArgs p = make_args(d);
    p.dy = dy;
    p.w = w;
    p.out = dx;
    hipLaunchKernelGGL(conv_dx_direct_kernel, dim3(linear_blocks(d.n * d.cin * d.h * d.w)), dim3(256), 0, s, p);
    MX_HIP(hipGetLastError());
    return MX_OK;
  }
  DxPlan f;
  MX_TRY(plan_dinput(d, dy, w, dx, limit, &f));
  const ConvArgs& p = f.p;  // data pointers set; every phase is a copy of it
  Scratch wt, ws;
  if (f.packed) MX_TRY(wt.alloc(size_t(f.w_bytes), s));
  if (f.ws_bytes) MX_TRY(ws.alloc(size_t(f.ws_bytes), s));
  // Positions no tap reaches (a phase with K = 0) are zero: one contiguous
  // fill of dx, then the phase GEMMs overwrite the reached positions (such
  // plans never split K, so the GEMMs write dx directly) -- unless the GEMM
  // writes those zeros itself (zfill).
  if (f.any_zero && !f.zfill) MX_TRY(conv::conv_dx_zero(dx, f.out_elems, s));
  // Pack every reached phase's weights up front, each at its own offset
  // (the phases partition the taps, so they fit the weights' size), in
  // launches of up to kMaxPackPhases phases.
  if (f.packed) {
    conv::DxPackSet set{};
    uint32_t off = 0;
    for (ConvArgs& q : f.phases) {
      if (q.K == 0) continue;
      set.ph[set.n++] = conv::DxPackPhase{q.K, q.nth, q.ntw, q.kh0, q.kw0, q.stph, q.stpw, off};
      q.wt = wt.as<float>() + off;
      off += uint32_t(p.G) * uint32_t(q.K) * uint32_t(p.Cin_g);
      if (set.n == conv::kMaxPackPhases) {
        MX_TRY(conv::conv_dx_pack_weights(p, set, wt.as<float>(), s));
        set.n = 0;
      }
    }
    if (set.n > 0) MX_TRY(conv::conv_dx_pack_weights(p, set, wt.as<float>(), s));
  }
  // The reached phases in one launch per operand loader (up to four each,
  // fewer when phases x groups would pass the 65535 limit of grid z).
  const int max_set = int(std::max<int64_t>(1, std::min<int64_t>(conv::kMaxFusedPhases, 65535 / p.G)));
  for (int bmode : {int(conv::B_GATHER), int(conv::B_VEC)}) {
    conv::DxPhaseSet set{};
    set.G = p.G;
    for (size_t i = 0; i < f.phases.size(); ++i) {
      ConvArgs& q = f.phases[i];
      if (q.K == 0 || f.bmodes[i] != bmode) continue;
      q.ws = ws.as<float>();
      set.q[set.n++] = q;
      if (set.n == max_set) {
        MX_TRY(conv::conv_dx_launch_set(set, f.gp.tile, f.vec_a ? Mode::RVEC : Mode::RSCALAR, bmode, s));
        set.n = 0;
      }
    }
    if (set.n > 0) MX_TRY(conv::conv_dx_launch_set(set, f.gp.tile, f.vec_a ? Mode::RVEC : Mode::RSCALAR, bmode, s));
  }
  if (f.gp.splits > 1) return conv::conv_sum_splits(ws.as<float>(), f.gp.splits, f.out_elems, dx, nullptr, 1, 1, s);
  return MX_OK;
  MX_ABI_END
}

int mx_conv2d_backward_bias(const mx_conv2d_desc* desc, const float* dy, float* db, void* stream) {
  MX_ABI_BEGIN
  mx_conv2d_desc d{};
  MX_TRY(copy_desc(desc, &d));
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

}  // extern "C"

// Scratch of mx_conv2d_backward_weight_noalloc: one array per GPU, in the
// library's code object, so calls allocate nothing.  Host code uses the device
// address hipGetSymbolAddress returns for the current GPU (noalloc_scratch),
// never the array's name.
namespace mx {
namespace noalloc {
__device__ __align__(256) float scratch[MX_NOALLOC_SCRATCH_BYTES / 4];
}  // namespace noalloc
}  // namespace mx

namespace {

// dW (+ dB) of one call.  Scratch (split-K partials, the Winograd range
// partials, the partial gradients of a batch split into chunks) comes from
// `ext` when the caller provides `ext_bytes` of it, else from the
// stream-ordered allocator; with `ext` every plan is sized to fit and nothing
// is allocated.
int dweight_impl(const mx_conv2d_desc* desc, const float* x, const float* dy, float* dw, float* db, int algo,
                 float* ext, int64_t ext_bytes, void* stream) {
  mx_conv2d_desc d{};
  MX_TRY(copy_desc(desc, &d));
  MX_TRY(checked_desc(&d));
  MX_REQUIRE(x && dy, MX_ERR_INVALID, "conv2d dweight: null tensor");
  if (!dw && !db) return MX_OK;
  if (!dw) return mx_conv2d_backward_bias(desc, dy, db, stream);
  int chosen = 0;
  MX_TRY(select_algo(d, MX_CONV_DWEIGHT, algo, &chosen));
  int64_t limit = 0;
  MX_TRY(conv::workspace_limit(&limit));
  if (ext) limit = std::min(limit, ext_bytes);
  hipStream_t s = resolve_stream(stream);
  if (chosen == MX_CONV_ALGO_DIRECT || chosen == MX_CONV_ALGO_REDUCE) {
    ConvArgs p = make_args(d);
    p.x = x;
    p.dy = dy;
    p.out = dw;
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
  {
    const int64_t nc = images_per_launch(d);
    MX_REQUIRE(nc > 0, MX_ERR_UNSUPPORTED, "conv2d dweight: one image or the weights exceed the 2 GiB operand bound");
    if (nc < d.n) {
      // Sum of the chunks' gradients: the first chunk writes dw / db, the
      // others go through a scratch copy added in chunk order.  With a caller
      // workspace that copy takes its tail and the chunks plan within the rest.
      const int64_t nw = d.cout * (d.cin / d.groups) * d.kh * d.kw;
      const int64_t tmp_bytes = (nw + (db ? d.cout : 0)) * 4;
      Scratch tmp;
      float* tw = nullptr;
      int64_t sub_bytes = 0;
      if (ext) {
        MX_REQUIRE(tmp_bytes <= limit, MX_ERR_WORKSPACE, "conv2d dweight: the partial gradient of a chunked batch (",
                   tmp_bytes, " bytes) exceeds the ", limit, "-byte workspace");
        sub_bytes = (limit - tmp_bytes) / 256 * 256;
        tw = ext + sub_bytes / 4;
      } else {
        MX_TRY(tmp.alloc(size_t(tmp_bytes), s));
        tw = tmp.as<float>();
      }
      float* tb = db ? tw + nw : nullptr;
      for (int64_t n0 = 0; n0 < d.n; n0 += nc) {
        const mx_conv2d_desc c = batch_slice(d, std::min(nc, d.n - n0));
        const float* xc = x + n0 * d.cin * d.h * d.w;
        const float* dyc = dy + n0 * d.cout * d.oh * d.ow;
        float* sub_ext = ext ? ext : nullptr;
        if (n0 == 0) {
          MX_TRY(dweight_impl(&c, xc, dyc, dw, db, chosen, sub_ext, sub_bytes, stream));
        } else {
          MX_TRY(dweight_impl(&c, xc, dyc, tw, tb, chosen, sub_ext, sub_bytes, stream));
          MX_TRY(mx_add_f32(dw, dw, tw, 1.f, nw, stream));
          if (db) MX_TRY(mx_add_f32(db, db, tb, 1.f, d.cout, stream));
        }
      }
      return MX_OK;
    }
  }
  if (chosen == MX_CONV_ALGO_WINOGRAD) {
    return winograd_backward_weight(d, x, dy, dw, db, limit, ext, s);
  }
  DwPlan f;
  MX_TRY(plan_dweight(d, x, dy, dw, db, limit, &f));
  ConvArgs& p = f.p;
  if (f.gp.splits == 1) return conv::conv_dw_launch(p, f.gp.tile, f.amode, f.bmode, s);
  Scratch ws, wsdb;
  if (ext) {
    // The plan fits: ws_bytes + db_bytes <= limit <= ext_bytes.
    p.ws = ext;
    p.ws_db = db ? ext + f.ws_bytes / 4 : nullptr;
  } else {
    MX_TRY(ws.alloc(size_t(f.ws_bytes), s));
    p.ws = ws.as<float>();
    if (db) {
      MX_TRY(wsdb.alloc(size_t(f.db_bytes), s));
      p.ws_db = wsdb.as<float>();
    }
  }
  MX_TRY(conv::conv_dw_launch(p, f.gp.tile, f.amode, f.bmode, s));
  return conv::conv_dw_finalize(p, dw, db, s);
}

constexpr int64_t kNoAllocBytes = MX_NOALLOC_SCRATCH_BYTES;
constexpr int kNoAllocDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kNoAllocDevices] = {};

// The current GPU's copy of `scratch`, looked up on the first call there.
int noalloc_scratch(float** out) {
  const int dev = current_device();
  MX_REQUIRE(dev >= 0 && dev < kNoAllocDevices, MX_ERR_INVALID, "device ", dev, " out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    MX_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(mx::noalloc::scratch)));
    MX_REQUIRE(ptr, MX_ERR_HIP, "hipGetSymbolAddress returned no address for the scratch array");
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return MX_OK;
}

}  // namespace

extern "C" {

int mx_conv2d_backward_weight(const mx_conv2d_desc* desc, const float* x, const float* dy, float* dw, float* db,
                              int algo, void* stream) {
  MX_ABI_BEGIN
  return dweight_impl(desc, x, dy, dw, db, algo, nullptr, 0, stream);
  MX_ABI_END
}

int mx_conv2d_backward(const mx_conv2d_desc* desc, const float* x, const float* w, const float* dy, float* dx,
                       float* dw, float* db, int algo_dx, int algo_dw, void* stream) {
  MX_ABI_BEGIN
  mx_conv2d_desc d{};
  MX_TRY(copy_desc(desc, &d));
  MX_TRY(checked_desc(&d));
  if (dx && (dw || db)) {
    int ax = 0, aw = 0;
    MX_TRY(select_algo(d, MX_CONV_DINPUT, algo_dx, &ax));
    if (dw) MX_TRY(select_algo(d, MX_CONV_DWEIGHT, algo_dw, &aw));
    if (dw && ax == MX_CONV_ALGO_WINOGRAD && aw == MX_CONV_ALGO_WINOGRAD && images_per_launch(d) >= d.n) {
      MX_REQUIRE(x && w && dy, MX_ERR_INVALID, "conv2d backward: null tensor");
      int64_t limit = 0;
      MX_TRY(conv::workspace_limit(&limit));
      bool done = false;
      MX_TRY(winograd_backward(d, x, w, dy, dx, dw, db, limit, resolve_stream(stream), &done));
      if (done) return MX_OK;
    }
  }
  if (dx) MX_TRY(mx_conv2d_backward_input(desc, dy, w, dx, algo_dx, stream));
  if (dw || db) MX_TRY(mx_conv2d_backward_weight(desc, x, dy, dw, db, algo_dw, stream));
  return MX_OK;
  MX_ABI_END
}

int mx_conv2d_backward_one_launch(const mx_conv2d_desc* desc, int algo_dx, int algo_dw, int with_bias,
                                  int* one_launch) {
  MX_ABI_BEGIN
  mx_conv2d_desc d{};
  MX_TRY(copy_desc(desc, &d));
  MX_REQUIRE(one_launch, MX_ERR_INVALID, "mx_conv2d_backward_one_launch: null argument");
  MX_TRY(checked_desc(&d));
  *one_launch = 0;
  int ax = 0, aw = 0;
  MX_TRY(select_algo(d, MX_CONV_DINPUT, algo_dx, &ax));
  MX_TRY(select_algo(d, MX_CONV_DWEIGHT, algo_dw, &aw));
  if (ax == MX_CONV_ALGO_WINOGRAD && aw == MX_CONV_ALGO_WINOGRAD && images_per_launch(d) >= d.n) {
    int64_t limit = 0;
    MX_TRY(conv::workspace_limit(&limit));
    bool one = false;
    MX_TRY(winograd_backward_one_launch(d, limit, with_bias != 0, &one));
    *one_launch = one ? 1 : 0;
  }
  return MX_OK;
  MX_ABI_END
}

int mx_conv2d_backward_weight_noalloc(const mx_conv2d_desc* desc, const float* x, const float* dy, float* dw,
                                      float* db, int algo, void* stream) {
  MX_ABI_BEGIN
  MX_REQUIRE(desc, MX_ERR_INVALID, "conv2d dweight: null descriptor");
  float* ws = nullptr;
  MX_TRY(noalloc_scratch(&ws));
  return dweight_impl(desc, x, dy, dw, db, algo, ws, kNoAllocBytes, stream);
  MX_ABI_END
}

int mx_conv2d_kernel_name(const mx_conv2d_desc* desc, int phase, int algo, char* buf, size_t len) {
  MX_ABI_BEGIN
  MX_REQUIRE(buf || !len, MX_ERR_INVALID, "mx_conv2d_kernel_name: null buffer");
  mx_conv2d_plan_info info{};
  MX_TRY(describe(desc, phase, algo, 1, &info));
  std::string name;
  if (phase == MX_CONV_DBIAS) {
    name = info.variant;
  } else if (info.algo == MX_CONV_ALGO_WINOGRAD) {
    // The variant names the kernel that carries the call: "wino_ws16_kernel<
    // even,filter>+flip", "wino_dw_ws_kernel+ranges", or the unfused passes'
    // batched GEMM "wino_unfused(gemm_kernel<..>)".
    const std::string v = info.variant;
    const size_t open = v.find('(');
    if (open != std::string::npos) {
      name = v.substr(open + 1, v.rfind(')') - open - 1);
    } else {
      name = v.substr(0, v.find_first_of("<+"));
    }
  } else if (info.algo == MX_CONV_ALGO_DEPTHWISE) {
    name = "conv_depthwise_kernel";
  } else if (info.algo == MX_CONV_ALGO_DIRECT) {
    name = phase == MX_CONV_FORWARD  ? "conv_fwd_direct_kernel"
           : phase == MX_CONV_DINPUT ? "conv_dx_direct_kernel"
                                     : "conv_dw_direct_kernel";
  } else if (info.algo == MX_CONV_ALGO_REDUCE) {
    name = "conv_dw_reduce_kernel";
  } else {
    const char* kind = phase == MX_CONV_FORWARD ? "conv_fwd_kernel" : phase == MX_CONV_DINPUT ? "conv_dx_kernel"
                                                                                                : "conv_dw_kernel";
    name = cat(kind, "<", tile_name(info.tile, phase), ">");
  }
  if (len) {
    std::strncpy(buf, name.c_str(), len - 1);
    buf[len - 1] = 0;
  }
  return MX_OK;
  MX_ABI_END
}

int mx_conv2d_plan(const mx_conv2d_desc* desc, int phase, int algo, int with_bias, mx_conv2d_plan_info* info) {
  MX_ABI_BEGIN
  MX_REQUIRE(desc && info, MX_ERR_INVALID, "mx_conv2d_plan: null argument");
  return describe(desc, phase, algo, with_bias, info);
  MX_ABI_END
}

int mx_conv2d_dweight_plan(const mx_conv2d_desc* desc, int64_t* splits, int64_t* span, int64_t* workspace_bytes) {
  MX_ABI_BEGIN
  mx_conv2d_desc d{};
  MX_TRY(copy_desc(desc, &d));
  MX_TRY(checked_desc(&d));
  int64_t limit = 0;
  MX_TRY(conv::workspace_limit(&limit));
  DwPlan f;
  MX_TRY(plan_dweight(d, kAlignedNull, kAlignedNull, kAlignedOut, kAlignedOut, limit, &f));
  if (splits) *splits = f.gp.splits;
  if (span) *span = f.gp.kps;
  if (workspace_bytes) *workspace_bytes = f.ws_bytes + f.db_bytes;
  return MX_OK;
  MX_ABI_END
}

}  // extern "C"
