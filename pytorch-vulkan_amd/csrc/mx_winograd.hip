// Winograd F(2x2, 3x3) forward convolution (3x3, stride 1, dilation 1).
//
// Transform matrices follow the reference shaders
// (conv2d_winograd_weights.comp:17-28, conv2d_winograd_input.comp:24-37,
// conv2d_winograd_gemm_output.comp:46-63):
//   U = G g G^T,  G = [[1,0,0],[1/2,1/2,1/2],[1/2,-1/2,1/2],[0,0,1]]
//   V = B^T d B,  B^T = [[1,0,-1,0],[0,1,1,0],[0,-1,1,0],[0,1,0,-1]]
//   Y = A^T M A + bias,  A^T = [[1,1,1,0],[0,1,-1,-1]]
// on 4x4 input tiles at stride 2.  The 16 products M_t = U_t V_t (one per
// transform coordinate t, every group) run as a single batched FP32 MFMA GEMM
// of batch 16*groups.  Layouts: U [16*G][Cout_g][Cin_g], V [16*G][Cin_g][T],
// M [16*G][Cout_g][T] with T = N * ceil(OH/2) * ceil(OW/2).
#include <hip/hip_runtime.h>

#include <algorithm>

#include "mx_internal.hpp"

namespace mx {
namespace {

struct WinoArgs {
  const float* x;
  const float* w;
  const float* bias;
  float* y;
  float* U;
  float* V;
  float* M;
  int N, Cin, H, W, Cout, OH, OW, ph, pw, G, Cin_g, Cout_g, TH, TW, T;
};

__global__ void wino_filter_kernel(WinoArgs p) {
  const int64_t total = int64_t(p.Cout) * p.Cin_g;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += int64_t(gridDim.x) * blockDim.x) {
    const int oc = int(idx / p.Cin_g), ci = int(idx % p.Cin_g);
    const int g = oc / p.Cout_g, co = oc % p.Cout_g;
    float k[3][3];
    for (int r = 0; r < 3; ++r)
      for (int c = 0; c < 3; ++c) k[r][c] = p.w[idx * 9 + r * 3 + c];
    float z[4][3];
    for (int c = 0; c < 3; ++c) {
      z[0][c] = k[0][c];
      z[1][c] = 0.5f * (k[0][c] + k[1][c] + k[2][c]);
      z[2][c] = 0.5f * (k[0][c] - k[1][c] + k[2][c]);
      z[3][c] = k[2][c];
    }
    const int64_t plane = int64_t(p.Cout_g) * p.Cin_g;
    const int64_t off = int64_t(co) * p.Cin_g + ci;
    for (int r = 0; r < 4; ++r) {
      const float u[4] = {z[r][0], 0.5f * (z[r][0] + z[r][1] + z[r][2]), 0.5f * (z[r][0] - z[r][1] + z[r][2]),
                          z[r][2]};
      for (int c = 0; c < 4; ++c) p.U[(int64_t(r * 4 + c) * p.G + g) * plane + off] = u[c];
    }
  }
}

__global__ void wino_input_kernel(WinoArgs p) {
  const int64_t total = int64_t(p.Cin) * p.T;
  const int per_image = p.TH * p.TW;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += int64_t(gridDim.x) * blockDim.x) {
    const int ch = int(idx / p.T), tile = int(idx % p.T);
    const int img = tile / per_image, pos = tile % per_image;
    const int y0 = (pos / p.TW) * 2 - p.ph, x0 = (pos % p.TW) * 2 - p.pw;
    const float* xc = p.x + (int64_t(img) * p.Cin + ch) * p.H * p.W;
    float d[4][4];
    for (int r = 0; r < 4; ++r)
      for (int c = 0; c < 4; ++c) {
        const int iy = y0 + r, ix = x0 + c;
        d[r][c] = (unsigned(iy) < unsigned(p.H) && unsigned(ix) < unsigned(p.W)) ? xc[iy * p.W + ix] : 0.f;
      }
    float z[4][4];
    for (int c = 0; c < 4; ++c) {
      z[0][c] = d[0][c] - d[2][c];
      z[1][c] = d[1][c] + d[2][c];
      z[2][c] = d[2][c] - d[1][c];
      z[3][c] = d[1][c] - d[3][c];
    }
    const int g = ch / p.Cin_g, ci = ch % p.Cin_g;
    const int64_t plane = int64_t(p.Cin_g) * p.T;
    const int64_t off = int64_t(ci) * p.T + tile;
    for (int r = 0; r < 4; ++r) {
      const float v[4] = {z[r][0] - z[r][2], z[r][1] + z[r][2], z[r][2] - z[r][1], z[r][1] - z[r][3]};
      for (int c = 0; c < 4; ++c) p.V[(int64_t(r * 4 + c) * p.G + g) * plane + off] = v[c];
    }
  }
}

__global__ void wino_output_kernel(WinoArgs p) {
  const int64_t total = int64_t(p.Cout) * p.T;
  const int per_image = p.TH * p.TW;
  const int64_t plane = int64_t(p.Cout_g) * p.T;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += int64_t(gridDim.x) * blockDim.x) {
    const int oc = int(idx / p.T), tile = int(idx % p.T);
    const int g = oc / p.Cout_g, co = oc % p.Cout_g;
    float m[16];
    for (int t = 0; t < 16; ++t) m[t] = p.M[(int64_t(t) * p.G + g) * plane + int64_t(co) * p.T + tile];
    float r0[4], r1[4];
    for (int c = 0; c < 4; ++c) {
      r0[c] = m[c] + m[4 + c] + m[8 + c];
      r1[c] = m[4 + c] - m[8 + c] - m[12 + c];
    }
    const float b = p.bias ? p.bias[oc] : 0.f;
    const float v00 = r0[0] + r0[1] + r0[2] + b;
    const float v01 = r0[1] - r0[2] - r0[3] + b;
    const float v10 = r1[0] + r1[1] + r1[2] + b;
    const float v11 = r1[1] - r1[2] - r1[3] + b;
    const int img = tile / per_image, pos = tile % per_image;
    const int oy = (pos / p.TW) * 2, ox = (pos % p.TW) * 2;
    float* yo = p.y + (int64_t(img) * p.Cout + oc) * p.OH * p.OW;
    if (oy < p.OH && ox < p.OW) yo[oy * p.OW + ox] = v00;
    if (oy < p.OH && ox + 1 < p.OW) yo[oy * p.OW + ox + 1] = v01;
    if (oy + 1 < p.OH && ox < p.OW) yo[(oy + 1) * p.OW + ox] = v10;
    if (oy + 1 < p.OH && ox + 1 < p.OW) yo[(oy + 1) * p.OW + ox + 1] = v11;
  }
}

int blocks_for(int64_t total) { return int(std::min<int64_t>((total + 255) / 256, 1 << 20)); }

}  // namespace

int winograd_forward(const mx_conv2d_desc& d, const float* x, const float* w, const float* bias, float* y,
                     hipStream_t s) {
  WinoArgs p{};
  p.x = x;
  p.w = w;
  p.bias = bias;
  p.y = y;
  p.N = int(d.n);
  p.Cin = int(d.cin);
  p.H = int(d.h);
  p.W = int(d.w);
  p.Cout = int(d.cout);
  p.OH = int(d.oh);
  p.OW = int(d.ow);
  p.ph = int(d.ph);
  p.pw = int(d.pw);
  p.G = int(d.groups);
  p.Cin_g = p.Cin / p.G;
  p.Cout_g = p.Cout / p.G;
  p.TH = (p.OH + 1) / 2;
  p.TW = (p.OW + 1) / 2;
  const int64_t T = int64_t(p.N) * p.TH * p.TW;
  MX_REQUIRE(T <= INT32_MAX && 16 * int64_t(p.Cin) * T <= INT32_MAX && 16 * int64_t(p.Cout) * T <= INT32_MAX,
             MX_ERR_UNSUPPORTED, "winograd: transformed tensors exceed int32 indexing");
  p.T = int(T);
  Scratch U, V, M;
  MX_TRY(U.alloc(size_t(16) * p.Cout * p.Cin_g * 4, s));
  MX_TRY(V.alloc(size_t(16) * p.Cin * T * 4, s));
  MX_TRY(M.alloc(size_t(16) * p.Cout * T * 4, s));
  p.U = U.as<float>();
  p.V = V.as<float>();
  p.M = M.as<float>();
  hipLaunchKernelGGL(wino_filter_kernel, dim3(blocks_for(int64_t(p.Cout) * p.Cin_g)), dim3(256), 0, s, p);
  MX_HIP(hipGetLastError());
  hipLaunchKernelGGL(wino_input_kernel, dim3(blocks_for(int64_t(p.Cin) * T)), dim3(256), 0, s, p);
  MX_HIP(hipGetLastError());
  mx_gemm_desc gd{};
  gd.batch = 16 * int64_t(p.G);
  gd.m = p.Cout_g;
  gd.n = T;
  gd.k = p.Cin_g;
  gd.a_stride_b = int64_t(p.Cout_g) * p.Cin_g;
  gd.a_stride_m = p.Cin_g;
  gd.a_stride_k = 1;
  gd.b_stride_b = int64_t(p.Cin_g) * T;
  gd.b_stride_k = T;
  gd.b_stride_n = 1;
  gd.c_stride_b = int64_t(p.Cout_g) * T;
  gd.ldc = T;
  gd.alpha = 1.f;
  gd.beta = 0.f;
  gd.bias_kind = MX_BIAS_NONE;
  MX_TRY(mx_gemm_f32(&gd, p.U, p.V, nullptr, p.M, s));
  hipLaunchKernelGGL(wino_output_kernel, dim3(blocks_for(int64_t(p.Cout) * T)), dim3(256), 0, s, p);
  MX_HIP(hipGetLastError());
  return MX_OK;
}

}  // namespace mx
