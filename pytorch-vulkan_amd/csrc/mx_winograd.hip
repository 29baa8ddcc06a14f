// Winograd F(2x2, 3x3) convolution (3x3, stride 1, dilation 1): the forward
// pass, and the input gradient of such a layer, which is itself a 3x3 stride-1
// convolution of dy with the filter flipped in both spatial axes and its
// channel axes swapped per group, at padding 2 - p:
//   dx[n, g*C + c, i, j] = sum_{o, r, s} dy[n, g*O + o, i + r - (2 - p), ...]
//                                        * w[g*O + o, c, 2 - r, 2 - s]
// (C, O the layer's input and output channels per group).  The filter
// transforms read w in that order (`flip`); everything after them is the
// forward kernel unchanged.
//
// Transform matrices follow the reference shaders
// (conv2d_winograd_weights.comp:17-28, conv2d_winograd_input.comp:24-37,
// conv2d_winograd_gemm_output.comp:46-63):
//   U = G g G^T,  G = [[1,0,0],[1/2,1/2,1/2],[1/2,-1/2,1/2],[0,0,1]]
//   V = B^T d B,  B^T = [[1,0,-1,0],[0,1,1,0],[0,-1,1,0],[0,1,0,-1]]
//   Y = A^T M A + bias,  A^T = [[1,1,1,0],[0,1,-1,-1]]
// on 4x4 input tiles at stride 2, M_t = U_t V_t for each of the 16 transform
// coordinates t.
//
// Fused kernel (the default): one workgroup computes 64 output channels x 32
// tiles for all 16 coordinates.  Per slab of 8 input channels it stages the
// transformed filter U (precomputed once per call by the filter launch,
// [G][16][Cpad][Opad], output channels contiguous, zero padded, or for
// short channel walks transformed from w in the kernel) and transforms the
// 4x4 input patches it loads straight into LDS, so V never goes to HBM; the
// 16 products run as
// v_mfma_f32_16x16x4f32 with each wave holding all 16 coordinates of a 32
// channel x 16 tile block, so the output transform A^T M A and the bias are
// applied in registers and M never goes to HBM either.
//
// Unfused kernels (launches with few tiles, or MX_WINOGRAD_FUSED=0): the
// filter, input and output
// transforms run as separate passes around one batched MFMA GEMM of batch
// 16*groups over U [16*G][Cout_g][Cin_g], V [16*G][Cin_g][T],
// M [16*G][Cout_g][T] with T = N * ceil(OH/2) * ceil(OW/2).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <string>

#include "mfma_core.hpp"
#include "mx_internal.hpp"

namespace mx {
namespace conv {
int sum_partials(const float* ws, const float* ws_db, int splits, int64_t n, int n_db, float* out, float* out_db,
                 hipStream_t s);
}
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
  int flip;  // filter is the flipped, channel-swapped layer filter (input gradient)
};

__global__ void wino_filter_kernel(WinoArgs p) {
  const int64_t total = int64_t(p.Cout) * p.Cin_g;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += int64_t(gridDim.x) * blockDim.x) {
    const int oc = int(idx / p.Cin_g), ci = int(idx % p.Cin_g);
    const int g = oc / p.Cout_g, co = oc % p.Cout_g;
    float k[3][3];
    if (p.flip) {
      // Layer filter [G*Cin_g][Cout_g][3][3]: element (oc, ci) is layer
      // output channel g*Cin_g + ci, layer input channel co, flipped taps.
      const float* src = p.w + ((int64_t(g) * p.Cin_g + ci) * p.Cout_g + co) * 9;
      for (int r = 0; r < 3; ++r)
        for (int c = 0; c < 3; ++c) k[r][c] = src[8 - (r * 3 + c)];
    } else {
      for (int r = 0; r < 3; ++r)
        for (int c = 0; c < 3; ++c) k[r][c] = p.w[idx * 9 + r * 3 + c];
    }
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

// ------------------------------------------------------------ fused kernel
namespace fused {
using mfma::f32x4;
using mfma::i32x4;
using mfma::kOffNone;
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int BO = 64;  // output channels per workgroup
constexpr int BT = 32;  // tiles per workgroup
constexpr int BK = 8;   // input channels per slab
// A 16x16x4 MFMA step takes k index kq = lane / 16 of its four; a lane runs
// two steps per slab, so it needs slab channels 2 kq and 2 kq + 1.  Both
// stages keep those two adjacent: A [coord][kq][o][2], B [coord][kq][t][2],
// and a lane's fragments for one coordinate are one 8-byte read each at a
// constant offset from its base.
constexpr int ROW_A = 2 * BO;  // floats per (coord, kq) row
constexpr int ROW_B = 2 * BT;
constexpr int A_FLOATS = 16 * 4 * ROW_A;
constexpr int B_FLOATS = 16 * 4 * ROW_B;
constexpr int A_PASSES = A_FLOATS / 4 / mfma::kThreads;  // float4 loads per thread per slab
static_assert(A_PASSES == 8, "filter slab tiling");
static_assert(BK * BT == mfma::kThreads, "one input patch per thread per slab");

struct Args {
  const float* x;    // [N][Cin][H][W]
  const float* U;    // [G][16][nslab][4][Opad][2]
  const float* w;    // the layer filter, for kernels that transform it themselves
  const float* bias;
  float* y;          // [N][Cout][OH][OW]
  int64_t x_bytes, u_bytes, y_bytes, w_bytes;
  int Cin, H, W, Cout, OH, OW, ph, pw, C, O, Cpad, Opad, TH, TW, T, n_ob, nslab;
  mfma::FastDiv f_thw, f_tw;
};

// A thread's 4x4 input patch for one slab: each row is one 16-byte load at
// the row's first column, the slab's channel offset added in 32-bit
// arithmetic.  Rows outside the image keep the kOffNone offset and read
// zeros; columns outside it read the neighbouring row's values and are
// zeroed in patch().  A patch whose rows would start before the tensor or end
// past it (only at the tensor's first and last rows) is read again element by
// element in fix(), after which no value kept comes from a load that was
// partly out of range.
struct PatchRows {
  uint32_t row_off[4];  // byte offset of row r's first column, kOffNone off the image
  uint32_t col_ok;      // bit cc: column cc inside the image
  uint32_t f_off, l_off;  // offsets of the first and last rows inside the image (0 when none)
  f32x4 xr[4];
  uint32_t sx;          // slab offset of the rows held
  bool whole;           // the row loads were inside the tensor

  __device__ __forceinline__ void init(int64_t plane, int y0, int x0, bool tok, int H, int W) {
    f_off = l_off = 0;
    bool seen = false;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int iy = y0 + r;
      const bool ok = tok && unsigned(iy) < unsigned(H);
      // x0 may be negative (left padding): the offset is then taken modulo
      // 2^32, and fix() re-reads the one patch whose row starts before the
      // tensor.
      row_off[r] = ok ? uint32_t(((plane + iy) * W + x0) * 4) : kOffNone;
      if (ok && !seen) f_off = row_off[r];
      if (ok) l_off = row_off[r];
      seen = seen || ok;
    }
    col_ok = 0;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) col_ok |= (unsigned(x0 + cc) < unsigned(W) ? 1u : 0u) << cc;
  }
  // Rows of the slab at byte offset s; a channel past the group's (padding)
  // reads zeros.
  __device__ __forceinline__ void load(const i32x4& rx, uint32_t s, uint32_t x_bytes, bool chan_ok) {
    sx = s;
    whole = !chan_ok | ((int(f_off + s) >= 0) & (l_off + s + 16u <= x_bytes));  // no short-circuit branch
#pragma unroll
    for (int r = 0; r < 4; ++r) xr[r] = mfma::bload4(rx, chan_ok ? row_off[r] + s : kOffNone, 0);
  }
  __device__ __forceinline__ void fix(const i32x4& rx) {
    if (!whole) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        // Offsets formed here, not hoisted out of the slab loop into 16
        // registers held for the whole kernel.
        uint32_t ro = row_off[r];
        asm volatile("" : "+v"(ro));
#pragma unroll
        for (int cc = 0; cc < 4; ++cc)
          xr[r][cc] = mfma::bload(rx, ((col_ok >> cc) & 1u) ? ro + 4u * cc : kOffNone, sx);
      }
    }
  }
  // The same patch element by element (one load per element inside the
  // image, the slab in the scalar offset), for the two-workgroup fused
  // kernel, where the row loads' column selects and the rare re-read cost
  // more than the twelve loads they save.
  __device__ __forceinline__ void load_elements(const i32x4& rx, uint32_t s, bool chan_ok, float (&d)[16]) const {
    const uint32_t cmask = chan_ok ? col_ok : 0u;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int cc = 0; cc < 4; ++cc)
        d[r * 4 + cc] = mfma::bload(rx, ((cmask >> cc) & 1u) ? row_off[r] + 4u * cc : kOffNone, s);
  }
  __device__ __forceinline__ void patch(float (&d)[16]) const {
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) d[r * 4 + cc] = ((col_ok >> cc) & 1u) ? xr[r][cc] : 0.f;
  }
};

// U' for the padded (c, o) range, zero outside the real one: channel c of
// coordinate t at [g][t][c / 8][(c % 8) / 2][o][c % 2].
// With `flip`, w is the layer filter [G*C][O][3][3] of an input gradient:
// element (o, c) reads layer output channel g*C + c, input channel o, taps
// reversed.
// One thread per (g, channel pair c, c + 1, o), o fastest: the two channels
// of a pair are adjacent in U', so each coordinate is one 8-byte store and a
// wave writes 512 contiguous bytes.
// u = G k G^T for one 3x3 filter k (row-major), G = [[1,0,0],[1/2,1/2,1/2],
// [1/2,-1/2,1/2],[0,0,1]].  The filter launch and the kernels that transform
// the filter themselves share this arithmetic, so their U' are bit-identical.
__device__ __forceinline__ void filter_math(const float (&k)[9], float (&u)[16]) {
  float z[4][3];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    z[0][j] = k[j];
    z[1][j] = 0.5f * (k[j] + k[3 + j] + k[6 + j]);
    z[2][j] = 0.5f * (k[j] - k[3 + j] + k[6 + j]);
    z[3][j] = k[6 + j];
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    u[r * 4 + 0] = z[r][0];
    u[r * 4 + 1] = 0.5f * (z[r][0] + z[r][1] + z[r][2]);
    u[r * 4 + 2] = 0.5f * (z[r][0] - z[r][1] + z[r][2]);
    u[r * 4 + 3] = z[r][2];
  }
}

__device__ __forceinline__ void filter_transform(const float* __restrict__ w, int C, int O, int g, int o, int c,
                                                 bool flip, float (&u)[16]) {
  if (o >= O || c >= C) {
#pragma unroll
    for (int t = 0; t < 16; ++t) u[t] = 0.f;
    return;
  }
  float k[9];
  if (flip) {
    const float* src = w + ((int64_t(g) * C + c) * O + o) * 9;
#pragma unroll
    for (int j = 0; j < 9; ++j) k[j] = src[8 - j];
  } else {
    const float* src = w + ((int64_t(g) * O + o) * C + c) * 9;
#pragma unroll
    for (int j = 0; j < 9; ++j) k[j] = src[j];
  }
  filter_math(k, u);
}

__global__ void filter_kernel(const float* __restrict__ w, float* __restrict__ U, int C, int O, int Cpad, int Opad,
                              int G, bool flip) {
  const int pairs = Cpad / 2;
  const int64_t total = int64_t(G) * pairs * Opad;
  const int nslab = Cpad / BK;
  for (int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += int64_t(gridDim.x) * blockDim.x) {
    const int o = int(idx % Opad);
    const int64_t rest = idx / Opad;
    const int c = 2 * int(rest % pairs), g = int(rest / pairs);
    float u0[16], u1[16];
    filter_transform(w, C, O, g, o, c, flip, u0);
    filter_transform(w, C, O, g, o, c + 1, flip, u1);
    const int slab = c / BK, kq = (c % BK) >> 1;
#pragma unroll
    for (int t = 0; t < 16; ++t)
      *reinterpret_cast<f32x2*>(U + (((int64_t(g) * 16 + t) * nslab + slab) * 4 + kq) * int64_t(Opad) * 2 + 2 * o) =
          f32x2{u0[t], u1[t]};
  }
}

// Fused (warp-specialized kernel) or unfused passes.  The fused kernel holds
// one workgroup per CU, so a launch with long channel walks and fewer
// workgroups than half the CUs leaves the chip idle where the unfused passes'
// batched GEMM spreads the same work: measured on MI355X, 512 channels at
// 8x8, batch 16 (64 workgroups of 64 slabs) run 89.5 us fused and 47.6
// unfused.  From half the CUs up, or with short walks (<= 16 slabs, where
// the unfused passes' V and M round trips dominate), the fused kernel wins:
// 16 x 256 x 16^2 (128 workgroups of 32 slabs) 49.8 vs 58.0 us, C1's layer
// 18.2 vs 21.2, every 3x3 layer of the C3 and C4 stacks 8-20% faster.
bool prefer_fused(int64_t workgroups, int nslab) {
  return 2 * workgroups >= int64_t(cu_count()) || nslab <= 16;
}

}  // namespace fused

// ------------------------------------------------------------ warp-specialized fused kernel
// A workgroup of eight waves in two roles.  Waves 0-3 (consumers) run only
// the fragment reads and MFMAs of slab s, then the output transform; waves
// 4-7 (producers) load slab s + 2 and transform slab s + 1 (the input patches
// by B^T d B, the filter copied from U' or transformed from w) into the
// other of two LDS stages.  Each SIMD holds one wave of each role, so its
// matrix core runs one wave's products while the other wave's staging
// instructions issue; had every wave done both, as in a single-role kernel,
// the staging would issue between the products (measured on MI355X: C1's
// layer 21.2 -> 18.2 us, the C3 / C4 3x3 layers 8-20% faster than the
// single-role kernels this one replaced).  One barrier per slab, reached by
// both roles the same number of times (1 + nslab).  The products run by
// quads of coordinates (the first k step of four coordinates, then the
// second), so a product and the next one on the same accumulator are eight
// MFMAs apart.  96 KB of LDS: one workgroup per CU.
namespace ws {
using fused::A_FLOATS;
using fused::A_PASSES;
using fused::B_FLOATS;
using fused::BK;
using fused::BO;
using fused::BT;
using fused::f32x2;
using fused::PatchRows;
using fused::ROW_A;
using fused::ROW_B;
using mfma::f32x4;
using mfma::i32x4;
using mfma::kOffNone;

// FILT: 0 reads U' (written by the filter launch); 1 / 2 have the producers
// transform the layer filter w themselves (2: flipped and channel-swapped,
// for an input gradient), so no filter launch runs.  Producer thread (kq, o)
// then loads the 3x3 filters of output channel o0 + o, slab channels 2 kq and
// 2 kq + 1, and stores their 16 coordinates as 8-byte pairs (a wave writes
// 512 contiguous bytes per coordinate).
// The kernel body for logical block b of group g, on LDS stages the caller
// provides (the backward kernel runs it beside the weight gradient's body).
template <bool RAGGED, int FILT>
__device__ __forceinline__ void ws_body(const fused::Args& p, int b, int g, float* __restrict__ As0,
                                        float* __restrict__ Bs0, float* __restrict__ As1, float* __restrict__ Bs1) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ob = b % p.n_ob, tb = b / p.n_ob;
  const int o0 = ob * BO, t0 = tb * BT;
  const int nslab = p.nslab;  // even: the host pads the channels to 16

  if (wave >= 4) {
    // ---- producers: the pipelined kernel's loads and stores, thread ptid.
    const int ptid = tid - 256;
    const i32x4 ru = mfma::buffer_rsrc(p.U, p.u_bytes);
    const int a_row = ptid >> 5, a_f4 = ptid & 31;
    const uint32_t a_off = uint32_t(
        ((((int64_t(g) * 16 + (a_row >> 2)) * p.nslab) * 4 + (a_row & 3)) * int64_t(p.Opad) * 2 + 2 * o0 +
         4 * a_f4) *
        4);
    const uint32_t a_sstep = uint32_t(4) * p.Opad * 2 * 4;
    const uint32_t a_qstep = uint32_t(2) * p.nslab * a_sstep;
    const i32x4 rx = mfma::buffer_rsrc(p.x, p.x_bytes);
    const int b_t = (ptid & 15) | ((ptid >> 1) & 16);
    const int b_c = ((ptid >> 4) & 1) | ((ptid >> 5) & 6);
    // A slab's loaded registers.  (Two sets, loading two slabs ahead,
    // measured no faster: the producers are not waiting on load latency.)
    struct Set {
      f32x4 av[FILT ? 1 : A_PASSES];
      f32x4 wv[2][2];
      float wl[2];
      PatchRows px;
    };
    Set sa_;
    PatchRows& px = sa_.px;
    {
      const int t = t0 + b_t;
      const bool tok = t < p.T;
      const uint32_t tt = tok ? uint32_t(t) : 0u;
      const uint32_t img = mfma::fdiv(tt, p.f_thw);
      const uint32_t pos = tt - img * uint32_t(p.TH * p.TW);
      const uint32_t ty = mfma::fdiv(pos, p.f_tw), tx = pos - ty * uint32_t(p.TW);
      const int y0 = int(2 * ty) - p.ph, x0 = int(2 * tx) - p.pw;
      const int64_t plane = (int64_t(img) * p.Cin + int64_t(g) * p.C + b_c) * p.H;
      px.init(plane, y0, x0, tok, p.H, p.W);
    }
    const uint32_t x_sstep = uint32_t(BK) * p.H * p.W * 4;
    const i32x4 rw = mfma::buffer_rsrc(p.w, FILT ? p.w_bytes : 0);
    const int f_o = ptid & 63, f_kq = ptid >> 6;
    const bool f_ook = o0 + f_o < p.O;
    // Byte offset of filter (o0 + f_o, channel c): forward w[g*O + o][c],
    // flipped w[g*C + c][o].
    auto f_off = [&](int c) {
      const int64_t e = FILT == 2 ? (int64_t(g) * p.C + c) * p.O + o0 + f_o : (int64_t(g) * p.O + o0 + f_o) * p.C + c;
      return (f_ook && c < p.C) ? uint32_t(e * 36) : kOffNone;
    };
    auto load = [&](Set& r, int slab) {
      const uint32_t sa = uint32_t(slab) * a_sstep, sx = uint32_t(slab) * x_sstep;
      if constexpr (FILT) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const uint32_t off = f_off(slab * BK + 2 * f_kq + j);
          r.wv[j][0] = mfma::bload4(rw, off, 0);
          r.wv[j][1] = mfma::bload4(rw, off, 16);
          r.wl[j] = mfma::bload(rw, off, 32);
        }
      } else {
#pragma unroll
        for (int q = 0; q < A_PASSES; ++q) r.av[q] = mfma::bload4(ru, a_off, sa + uint32_t(q) * a_qstep);
      }
      r.px.load(rx, sx, uint32_t(p.x_bytes), !RAGGED || slab * BK + b_c < p.C);
    };
    auto store = [&](Set& r, float* As, float* Bs) {
      r.px.fix(rx);
      const f32x4(&av)[FILT ? 1 : A_PASSES] = r.av;
      const f32x4(&wv)[2][2] = r.wv;
      const float(&wl)[2] = r.wl;
      float* const b_st = Bs + (b_c >> 1) * ROW_B + 2 * b_t + (b_c & 1);
      if constexpr (FILT) {
        float u[2][16];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float v[9] = {wv[j][0][0], wv[j][0][1], wv[j][0][2], wv[j][0][3], wv[j][1][0],
                              wv[j][1][1], wv[j][1][2], wv[j][1][3], wl[j]};
          float k[9];
#pragma unroll
          for (int e = 0; e < 9; ++e) k[e] = FILT == 2 ? v[8 - e] : v[e];
          fused::filter_math(k, u[j]);
        }
        float* const a_st = As + f_kq * ROW_A + 2 * f_o;
#pragma unroll
        for (int t = 0; t < 16; ++t) *reinterpret_cast<f32x2*>(a_st + t * 4 * ROW_A) = f32x2{u[0][t], u[1][t]};
      } else {
        float* const a_st = As + a_row * ROW_A + 4 * a_f4;
#pragma unroll
        for (int q = 0; q < A_PASSES; ++q) *reinterpret_cast<f32x4*>(a_st + q * 8 * ROW_A) = av[q];
      }
      float d[16];
      r.px.patch(d);
      float z[16];
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        z[0 * 4 + cc] = d[0 * 4 + cc] - d[2 * 4 + cc];
        z[1 * 4 + cc] = d[1 * 4 + cc] + d[2 * 4 + cc];
        z[2 * 4 + cc] = d[2 * 4 + cc] - d[1 * 4 + cc];
        z[3 * 4 + cc] = d[1 * 4 + cc] - d[3 * 4 + cc];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        b_st[(i * 4 + 0) * 4 * ROW_B] = z[i * 4 + 0] - z[i * 4 + 2];
        b_st[(i * 4 + 1) * 4 * ROW_B] = z[i * 4 + 1] + z[i * 4 + 2];
        b_st[(i * 4 + 2) * 4 * ROW_B] = z[i * 4 + 2] - z[i * 4 + 1];
        b_st[(i * 4 + 3) * 4 * ROW_B] = z[i * 4 + 1] - z[i * 4 + 3];
      }
    };
    load(sa_, 0);
    store(sa_, As0, Bs0);
    load(sa_, 1);
    __syncthreads();  // stage 0 holds slab 0
    // Trip s stores slab s + 1 into the stage slab s - 1 used (the consumers
    // finished reading it before the previous barrier) and loads slab s + 2;
    // past the last slab nothing is stored.
    for (int s = 0; s < nslab; s += 2) {
      store(sa_, As1, Bs1);  // slab s + 1 (s + 1 < nslab: nslab is even)
      load(sa_, min(s + 2, nslab - 1));
      __syncthreads();
      if (s + 2 < nslab) {
        store(sa_, As0, Bs0);  // slab s + 2
        load(sa_, min(s + 3, nslab - 1));
      }
      __syncthreads();
    }
    return;
  }

  // ---- consumers: wave (wo, wt) owns output channels wo*32 .. +31 and tiles
  // wt*16 .. +15 of the block, for all 16 coordinates.
  const int wo = wave >> 1, wt = wave & 1;
  const int kq = lane >> 4, li = lane & 15;
  f32x4 acc[16][2];
#pragma unroll
  for (int t = 0; t < 16; ++t) acc[t][0] = acc[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto slab = [&](const float* Ac, const float* Bc) {
    const f32x2* const a_frag = reinterpret_cast<const f32x2*>(Ac + kq * ROW_A + 2 * (wo * 32 + li));
    const f32x2* const b_frag = reinterpret_cast<const f32x2*>(Bc + kq * ROW_B + 2 * (wt * 16 + li));
    f32x2 fa0[4], fa1[4], fb[4];
    auto frags = [&](int q) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 4 * q + j;
        fb[j] = b_frag[t * 2 * ROW_B];
        fa0[j] = a_frag[t * 2 * ROW_A];
        fa1[j] = a_frag[t * 2 * ROW_A + 16];
      }
    };
    // Coordinates in quads, as in the pipelined kernel.
    auto quad = [&](int q) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int t = 4 * q + j;
          acc[t][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa0[j][h], fb[j][h], acc[t][0], 0, 0, 0);
          acc[t][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa1[j][h], fb[j][h], acc[t][1], 0, 0, 0);
        }
    };
    frags(0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      quad(q);
      if (q < 3) {
        frags(q + 1);
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 14, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  __syncthreads();  // stage 0 holds slab 0
  for (int s = 0; s < nslab; s += 2) {
    slab(As0, Bs0);
    __syncthreads();
    slab(As1, Bs1);
    __syncthreads();
  }

  // Output transform (the fused kernel's epilogue).
  const int t = t0 + wt * 16 + li;
  if (t >= p.T) return;
  const uint32_t img = mfma::fdiv(uint32_t(t), p.f_thw);
  const uint32_t pos = uint32_t(t) - img * uint32_t(p.TH * p.TW);
  const uint32_t ty = mfma::fdiv(pos, p.f_tw), tx = pos - ty * uint32_t(p.TW);
  const int oy = int(2 * ty), ox = int(2 * tx);
  const bool right = ox + 1 < p.OW, below = oy + 1 < p.OH;
  float bias_v[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int o = o0 + wo * 32 + i * 16 + 4 * kq + v;
      bias_v[i][v] = (p.bias && o < p.O) ? p.bias[g * p.O + o] : 0.f;
    }
  const i32x4 ry = mfma::buffer_rsrc(p.y, p.y_bytes);
  const uint32_t row_step = uint32_t(p.OW) * 4u;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int o = o0 + wo * 32 + i * 16 + 4 * kq + v;
      float m[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) m[q] = acc[q][i][v];
      float r0[4], r1[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        r0[c] = m[c] + m[4 + c] + m[8 + c];
        r1[c] = m[4 + c] - m[8 + c] - m[12 + c];
      }
      const float bb = bias_v[i][v];
      const bool ok = o < p.O;
      const uint32_t off =
          uint32_t(((img * uint32_t(p.Cout) + uint32_t(g * p.O + o)) * uint32_t(p.OH) + uint32_t(oy)) *
                       uint32_t(p.OW) +
                   uint32_t(ox)) *
          4u;
      mfma::bstore(r0[0] + r0[1] + r0[2] + bb, ry, ok ? off : kOffNone, 0);
      mfma::bstore(r0[1] - r0[2] - r0[3] + bb, ry, (ok && right) ? off + 4u : kOffNone, 0);
      mfma::bstore(r1[0] + r1[1] + r1[2] + bb, ry, (ok && below) ? off + row_step : kOffNone, 0);
      mfma::bstore(r1[1] - r1[2] - r1[3] + bb, ry, (ok && below && right) ? off + row_step + 4u : kOffNone, 0);
    }
}

template <bool RAGGED, int FILT>
__global__ __launch_bounds__(512) void wino_ws_kernel(fused::Args p) {
  __shared__ __attribute__((aligned(16))) float As0[A_FLOATS];
  __shared__ __attribute__((aligned(16))) float Bs0[B_FLOATS];
  __shared__ __attribute__((aligned(16))) float As1[A_FLOATS];
  __shared__ __attribute__((aligned(16))) float Bs1[B_FLOATS];
  ws_body<RAGGED, FILT>(p, mfma::xcd_remap(blockIdx.x, gridDim.x), blockIdx.y, As0, Bs0, As1, Bs1);
}

// The same roles with 16 tiles per workgroup: 80 KB of LDS and at most 128
// VGPRs, so two workgroups share a CU and one's prologue and epilogue (the
// first slabs' loads, the output transform and its stores) overlap the
// other's products.  Consumer wave w owns output channels w*16 .. +15 and all
// 16 tiles; producer waves 4-5 transform the 128 input patches of a slab,
// waves 6-7 copy the slab's filter (64 floats per thread).  Same U' layout,
// accumulation order and epilogue as the 32-tile kernel: bit-identical.
constexpr int BT16 = 16;
constexpr int ROW_B16 = 2 * BT16;
constexpr int B16_FLOATS = 16 * 4 * ROW_B16;

// FILT 1 / 2: waves 6-7 transform the layer filter w (2: flipped and
// channel-swapped) instead of copying U': thread (half, o) the four filters
// of output channel o0 + o and slab channels 4 half .. 4 half + 3.
template <bool RAGGED, int FILT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 4))) void wino_ws16_kernel(fused::Args p) {
  __shared__ __attribute__((aligned(16))) float As0[A_FLOATS];
  __shared__ __attribute__((aligned(16))) float Bs0[B16_FLOATS];
  __shared__ __attribute__((aligned(16))) float As1[A_FLOATS];
  __shared__ __attribute__((aligned(16))) float Bs1[B16_FLOATS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.y;
  const int b = mfma::xcd_remap(blockIdx.x, gridDim.x);
  const int ob = b % p.n_ob, tb = b / p.n_ob;
  const int o0 = ob * BO, t0 = tb * BT16;
  const int nslab = p.nslab;  // even: the host pads the channels to 16

  if (wave >= 6) {
    // ---- filter producers: rows a_row .. of the slab's U' block, 16 floats
    // (four 16-byte chunks) per (coordinate, k pair) row and thread.
    const int ptid = tid - 384;  // 0 .. 127
    const i32x4 ru = mfma::buffer_rsrc(p.U, p.u_bytes);
    const int a_row = ptid >> 5, a_f4 = ptid & 31;  // 4 rows per pass, 16 passes
    const uint32_t a_off = uint32_t(
        ((((int64_t(g) * 16 + (a_row >> 2)) * p.nslab) * 4 + (a_row & 3)) * int64_t(p.Opad) * 2 + 2 * o0 +
         4 * a_f4) *
        4);
    const uint32_t a_sstep = uint32_t(4) * p.Opad * 2 * 4;
    const uint32_t a_cstep = uint32_t(p.nslab) * a_sstep;  // one coordinate
    f32x4 av[FILT ? 1 : 16];
    // In-kernel filter: the 4 x 9 taps of this thread's filters.
    const i32x4 rw = mfma::buffer_rsrc(p.w, FILT ? p.w_bytes : 0);
    const int f_o = ptid & 63, f_h = ptid >> 6;
    const bool f_ook = o0 + f_o < p.O;
    float wk[FILT ? 36 : 1];
    auto load = [&](int slab) {
      if constexpr (FILT == 0) {
        const uint32_t sa = uint32_t(slab) * a_sstep;
#pragma unroll
        for (int q = 0; q < 16; ++q) av[q] = mfma::bload4(ru, a_off, sa + uint32_t(q) * a_cstep);
      } else {
        const int c = slab * BK + 4 * f_h;
        if constexpr (FILT == 1) {
          // w[g*O + o][c .. c + 3]: 36 contiguous floats (channels past C read
          // the next row's or nothing and are zeroed in store()).
          const uint32_t off = f_ook ? uint32_t(((int64_t(g) * p.O + o0 + f_o) * p.C + c) * 36) : kOffNone;
#pragma unroll
          for (int i = 0; i < 9; ++i) {
            const f32x4 v = mfma::bload4(rw, off, uint32_t(i) * 16);
            wk[4 * i] = v[0], wk[4 * i + 1] = v[1], wk[4 * i + 2] = v[2], wk[4 * i + 3] = v[3];
          }
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t off =
                (f_ook && c + j < p.C) ? uint32_t(((int64_t(g) * p.C + c + j) * p.O + o0 + f_o) * 36) : kOffNone;
            const f32x4 v0 = mfma::bload4(rw, off, 0), v1 = mfma::bload4(rw, off, 16);
            wk[9 * j] = v0[0], wk[9 * j + 1] = v0[1], wk[9 * j + 2] = v0[2], wk[9 * j + 3] = v0[3];
            wk[9 * j + 4] = v1[0], wk[9 * j + 5] = v1[1], wk[9 * j + 6] = v1[2], wk[9 * j + 7] = v1[3];
            wk[9 * j + 8] = mfma::bload(rw, off, 32);
          }
        }
      }
    };
    int f_slab = 0;  // slab whose taps wk holds (for the channel bound)
    auto store = [&](float* As) {
      if constexpr (FILT == 0) {
        float* const a_st = As + a_row * ROW_A + 4 * a_f4;
#pragma unroll
        for (int q = 0; q < 16; ++q) *reinterpret_cast<f32x4*>(a_st + q * 4 * ROW_A) = av[q];
      } else {
        const int c = f_slab * BK + 4 * f_h;
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
          float u[2][16];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int j = 2 * pr + h;
            float k[9];
#pragma unroll
            for (int e = 0; e < 9; ++e) k[e] = (c + j < p.C) ? wk[9 * j + (FILT == 2 ? 8 - e : e)] : 0.f;
            fused::filter_math(k, u[h]);
          }
          float* const a_st = As + (2 * f_h + pr) * ROW_A + 2 * f_o;
#pragma unroll
          for (int t = 0; t < 16; ++t) *reinterpret_cast<f32x2*>(a_st + t * 4 * ROW_A) = f32x2{u[0][t], u[1][t]};
        }
      }
    };
    load(0);
    f_slab = 0;
    store(As0);
    load(1);
    __syncthreads();
    for (int s = 0; s < nslab; s += 2) {
      f_slab = s + 1;
      store(As1);
      load(min(s + 2, nslab - 1));
      __syncthreads();
      if (s + 2 < nslab) {
        f_slab = s + 2;
        store(As0);
        load(min(s + 3, nslab - 1));
      }
      __syncthreads();
    }
    return;
  }
  if (wave >= 4) {
    // ---- patch producers: thread ptid owns slab tile b_t and channel b_c;
    // a half-wave's V stores are 32 consecutive floats.
    const int ptid = tid - 256;  // 0 .. 127
    const i32x4 rx = mfma::buffer_rsrc(p.x, p.x_bytes);
    const int b_t = ptid & 15;
    const int b_c = ((ptid >> 4) & 1) | ((ptid >> 5) << 1);
    PatchRows px;
    {
      const int t = t0 + b_t;
      const bool tok = t < p.T;
      const uint32_t tt = tok ? uint32_t(t) : 0u;
      const uint32_t img = mfma::fdiv(tt, p.f_thw);
      const uint32_t pos = tt - img * uint32_t(p.TH * p.TW);
      const uint32_t ty = mfma::fdiv(pos, p.f_tw), tx = pos - ty * uint32_t(p.TW);
      const int y0 = int(2 * ty) - p.ph, x0 = int(2 * tx) - p.pw;
      const int64_t plane = (int64_t(img) * p.Cin + int64_t(g) * p.C + b_c) * p.H;
      px.init(plane, y0, x0, tok, p.H, p.W);
    }
    const uint32_t x_sstep = uint32_t(BK) * p.H * p.W * 4;
    auto load = [&](int slab) {
      px.load(rx, uint32_t(slab) * x_sstep, uint32_t(p.x_bytes), !RAGGED || slab * BK + b_c < p.C);
    };
    auto store = [&](float* Bs) {
      px.fix(rx);
      float* const b_st = Bs + (b_c >> 1) * ROW_B16 + 2 * b_t + (b_c & 1);
      float d[16];
      px.patch(d);
      float z[16];
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        z[0 * 4 + cc] = d[0 * 4 + cc] - d[2 * 4 + cc];
        z[1 * 4 + cc] = d[1 * 4 + cc] + d[2 * 4 + cc];
        z[2 * 4 + cc] = d[2 * 4 + cc] - d[1 * 4 + cc];
        z[3 * 4 + cc] = d[1 * 4 + cc] - d[3 * 4 + cc];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        b_st[(i * 4 + 0) * 4 * ROW_B16] = z[i * 4 + 0] - z[i * 4 + 2];
        b_st[(i * 4 + 1) * 4 * ROW_B16] = z[i * 4 + 1] + z[i * 4 + 2];
        b_st[(i * 4 + 2) * 4 * ROW_B16] = z[i * 4 + 2] - z[i * 4 + 1];
        b_st[(i * 4 + 3) * 4 * ROW_B16] = z[i * 4 + 1] - z[i * 4 + 3];
      }
    };
    load(0);
    store(Bs0);
    load(1);
    __syncthreads();
    for (int s = 0; s < nslab; s += 2) {
      store(Bs1);
      load(min(s + 2, nslab - 1));
      __syncthreads();
      if (s + 2 < nslab) {
        store(Bs0);
        load(min(s + 3, nslab - 1));
      }
      __syncthreads();
    }
    return;
  }

  // ---- consumers: wave w owns output channels w*16 .. +15 and the 16 tiles.
  const int kq = lane >> 4, li = lane & 15;
  f32x4 acc[16];
#pragma unroll
  for (int t = 0; t < 16; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto slab = [&](const float* Ac, const float* Bc) {
    const f32x2* const a_frag = reinterpret_cast<const f32x2*>(Ac + kq * ROW_A + 2 * (wave * 16 + li));
    const f32x2* const b_frag = reinterpret_cast<const f32x2*>(Bc + kq * ROW_B16 + 2 * li);
    f32x2 fa[4], fb[4];
    auto frags = [&](int q) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 4 * q + j;
        fb[j] = b_frag[t * 2 * ROW_B16];
        fa[j] = a_frag[t * 2 * ROW_A];
      }
    };
    auto quad = [&](int q) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[4 * q + j] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[j][h], fb[j][h], acc[4 * q + j], 0, 0, 0);
    };
    frags(0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      quad(q);
      if (q < 3) {
        frags(q + 1);
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  __syncthreads();  // stage 0 holds slab 0
  for (int s = 0; s < nslab; s += 2) {
    slab(As0, Bs0);
    __syncthreads();
    slab(As1, Bs1);
    __syncthreads();
  }

  // Output transform (the 32-tile kernel's epilogue).
  const int t = t0 + li;
  if (t >= p.T) return;
  const uint32_t img = mfma::fdiv(uint32_t(t), p.f_thw);
  const uint32_t pos = uint32_t(t) - img * uint32_t(p.TH * p.TW);
  const uint32_t ty = mfma::fdiv(pos, p.f_tw), tx = pos - ty * uint32_t(p.TW);
  const int oy = int(2 * ty), ox = int(2 * tx);
  const bool right = ox + 1 < p.OW, below = oy + 1 < p.OH;
  float bias_v[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int o = o0 + wave * 16 + 4 * kq + v;
    bias_v[v] = (p.bias && o < p.O) ? p.bias[g * p.O + o] : 0.f;
  }
  const i32x4 ry = mfma::buffer_rsrc(p.y, p.y_bytes);
  const uint32_t row_step = uint32_t(p.OW) * 4u;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int o = o0 + wave * 16 + 4 * kq + v;
    float m[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) m[q] = acc[q][v];
    float r0[4], r1[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      r0[c] = m[c] + m[4 + c] + m[8 + c];
      r1[c] = m[4 + c] - m[8 + c] - m[12 + c];
    }
    const float bb = bias_v[v];
    const bool ok = o < p.O;
    const uint32_t off =
        uint32_t(((img * uint32_t(p.Cout) + uint32_t(g * p.O + o)) * uint32_t(p.OH) + uint32_t(oy)) * uint32_t(p.OW) +
                 uint32_t(ox)) *
        4u;
    mfma::bstore(r0[0] + r0[1] + r0[2] + bb, ry, ok ? off : kOffNone, 0);
    mfma::bstore(r0[1] - r0[2] - r0[3] + bb, ry, (ok && right) ? off + 4u : kOffNone, 0);
    mfma::bstore(r1[0] + r1[1] + r1[2] + bb, ry, (ok && below) ? off + row_step : kOffNone, 0);
    mfma::bstore(r1[1] - r1[2] - r1[3] + bb, ry, (ok && below && right) ? off + row_step + 4u : kOffNone, 0);
  }
}
}  // namespace ws

// ------------------------------------------------------------ fused dWeight
// Weight gradient of a 3x3 stride-1 layer as the adjoint of the forward
// transform: with M_t = U_t V_t and Y = A^T M A, U = G w G^T,
//   dM = A dY A^T   (4x4 per 2x2 output tile of dy),
//   dU_t[o][c] = sum over tiles k of dM_t[o][k] V_t[c][k],
//   dw = G^T dU G   (3x3 from 4x4).
// V is the forward's input transform of the same 4x4 patches.  One workgroup
// computes 64 output x 32 input channels of dU for all 16 coordinates over
// one range of tiles (the GEMM's K); slabs of 8 tiles are transformed on the
// way into LDS (dM from two 2x2 dy tiles per thread, V from one x patch per
// thread) in the layout of the forward kernel, so the products are the same
// v_mfma_f32_16x16x4f32 schedule.  The epilogue applies G^T dU G in
// registers and writes the tile range's 3x3 partial, summed over ranges in a
// fixed order by a second launch.
namespace fused_dw {
using fused::BK;  // tiles per slab
using fused::BO;  // output channels per workgroup
using fused::f32x2;
// The forward kernel's stage layout with each (coord, k pair) row padded by
// 8 floats, so consecutive rows start 8 banks apart: the dM stores (four k
// pairs per 16 lanes) and the V stores (four pairs x two halves per 32
// lanes) then hit distinct banks (unpadded they were 4-way conflicts).
constexpr int ROW_A = fused::ROW_A + 8;
constexpr int ROW_B = fused::ROW_B + 8;
constexpr int A_FLOATS = 16 * 4 * ROW_A;
constexpr int B_FLOATS = 16 * 4 * ROW_B;
using mfma::f32x4;
using mfma::i32x4;
using mfma::kOffNone;
constexpr int BC = fused::BT;  // input channels per workgroup (the forward's tile columns)
static_assert(BK * BC == mfma::kThreads, "one x patch per thread per slab");
static_assert(BK * BO == 2 * mfma::kThreads, "two dy tiles per thread per slab");

struct Args {
  const float* x;   // [N][Cin][H][W]
  const float* dy;  // [N][Cout][OH][OW]
  float* out;       // [range][G][O][C][3][3]
  float* out_db;    // [range][G][O] dBias partials, or null
  int64_t x_bytes, dy_bytes;
  int Cin, H, W, Cout, OH, OW, ph, pw, C, O, TH, TW, T, n_ob, n_cb, kps;
  mfma::FastDiv f_thw, f_tw;
};

// A workgroup decodes the tiles of its range once, in chunks of up to
// kChunk tiles, into a table in LDS.  Row offsets are in bytes and leave out
// the channel term, which each lane adds (saturating, so a sentinel stays out
// of range); kRowNone marks a row outside the image or a tile past the range.
constexpr int kChunk = 512;
constexpr uint32_t kRowNone = 0x80000000u;
constexpr uint32_t kXRare = 1u << 5, kYRare = 1u << 6;
struct alignas(16) TileEntry {
  uint32_t xrow[4];  // x patch rows (columns x0 .. x0 + 3)
  uint32_t yrow[2];  // dy tile rows (columns ox, ox + 1)
  int xfirst;        // element offset of the patch's top-left corner (may be negative)
  // bits 0-3: x column cc inside the image; 4: dy column ox + 1 inside;
  // kXRare / kYRare: a row segment may leave the tensor for some channel;
  // 8-11: x row r inside; 12-13: dy row r inside.
  uint32_t bits;
};

// Tile t -> image and the top-left output coordinate (2 ty, 2 tx).
__device__ __forceinline__ void tile_origin(uint32_t t, const Args& p, uint32_t& img, int& oy, int& ox) {
  img = mfma::fdiv(t, p.f_thw);
  const uint32_t pos = t - img * uint32_t(p.TH * p.TW);
  const uint32_t ty = mfma::fdiv(pos, p.f_tw);
  oy = int(2 * ty);
  ox = int(2 * (pos - ty * uint32_t(p.TW)));
}

// Tiles k0 .. k0 + n - 1 of a range ending at k1 into the LDS table, by
// `nthreads` threads; entries at or past k1 read nothing.
__device__ __forceinline__ void decode_tiles(const Args& p, TileEntry* tiles, int k0, int k1, int n, int tid,
                                             int nthreads) {
  const int HW = p.H * p.W, OHW = p.OH * p.OW;  // the tensors hold fewer than 2^29 floats
  const int x_elems = int(p.x_bytes >> 2), dy_elems = int(p.dy_bytes >> 2);
  for (int i = tid; i < n; i += nthreads) {
    const int t = k0 + i;
    const bool tok = t < k1;
    uint32_t img;
    int oy, ox;
    tile_origin(tok ? uint32_t(t) : 0u, p, img, oy, ox);
    const int y0 = oy - p.ph, x0 = ox - p.pw;
    TileEntry e;
    e.xfirst = int(img) * p.Cin * HW + y0 * p.W + x0;
    const int yfirst = int(img) * p.Cout * OHW + oy * p.OW + ox;
    uint32_t bits = uint32_t(ox + 1 < p.OW) << 4;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) bits |= uint32_t(unsigned(x0 + cc) < unsigned(p.W)) << cc;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool ok = tok && unsigned(y0 + r) < unsigned(p.H);
      bits |= uint32_t(ok) << (8 + r);
      e.xrow[r] = ok ? uint32_t(e.xfirst + r * p.W) * 4u : kRowNone;
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const bool ok = tok && oy + r < p.OH;
      bits |= uint32_t(ok) << (12 + r);
      e.yrow[r] = ok ? uint32_t(yfirst + r * p.OW) * 4u : kRowNone;
    }
    // Checked for the largest channel, so every channel's lanes agree; a
    // tile past the range reads nothing and is never rare.
    if (tok && (e.xfirst < 0 || e.xfirst + 3 * p.W + 4 + (p.Cin - 1) * HW > x_elems)) bits |= kXRare;
    if (tok && yfirst + p.OW + 2 + (p.Cout - 1) * OHW > dy_elems) bits |= kYRare;
    e.bits = bits;
    tiles[i] = e;
  }
}

// One thread's part of a slab: the x patch of input channel b_c for slab
// tile b_t (one patch per thread), and the dy tiles of output channel a_o
// for slab tiles 2 a_kq and 2 a_kq + 1 (the k pair one MFMA lane
// multiplies), with their transforms into an LDS stage.
//
// Each row of the x patch and of a dy tile is one 16- or 8-byte load at the
// row's first column; a row outside the image reads zeros.  Columns outside
// the image read the neighbouring row's values and are zeroed in store()
// from the column bits.  A tile whose rows may start before the tensor or end
// past it (only at the tensor's first and last rows) is read again element
// by element in store(), after the slab's loads have landed, so the rare path
// adds no wait to the common one and no load it keeps is ever partly out of
// range.
struct SlabIO {
  i32x4 rdy, rx;
  int a_o, a_kq, b_c, b_t, HW, OHW, W, OW;
  bool o_ok, c_ok;
  uint32_t dy_chan, x_chan, xc_bytes, yc_bytes;
  f32x4 xr[4];     // the x patch's rows
  uint32_t xbits;  // the patch's TileEntry::bits
  f32x2 yr[2][2];  // the dy tiles' rows
  uint32_t ybits[2];
  float dsum;      // this thread's dy values, for dBias

  __device__ __forceinline__ void init(const Args& p, int tid, int g, int o0, int c0) {
    rdy = mfma::buffer_rsrc(p.dy, p.dy_bytes);
    rx = mfma::buffer_rsrc(p.x, p.x_bytes);
    a_o = tid >> 2;
    a_kq = tid & 3;
    b_c = tid >> 3;
    b_t = tid & 7;
    o_ok = o0 + a_o < p.O;
    c_ok = c0 + b_c < p.C;
    dy_chan = uint32_t(g * p.O + o0 + a_o);
    x_chan = uint32_t(g * p.C + c0 + b_c);
    HW = p.H * p.W;
    OHW = p.OH * p.OW;
    W = p.W;
    OW = p.OW;
    xc_bytes = c_ok ? x_chan * uint32_t(HW) * 4u : kRowNone;
    yc_bytes = o_ok ? dy_chan * uint32_t(OHW) * 4u : kRowNone;
    dsum = 0.f;
  }
  __device__ __forceinline__ void load(const TileEntry* tiles, int slab) {
    const TileEntry* ex = &tiles[slab * BK + b_t];
    const uint4 xo = *reinterpret_cast<const uint4*>(ex->xrow);
    xbits = ex->bits;
    xr[0] = mfma::bload4(rx, __builtin_elementwise_add_sat(xo.x, xc_bytes), 0);
    xr[1] = mfma::bload4(rx, __builtin_elementwise_add_sat(xo.y, xc_bytes), 0);
    xr[2] = mfma::bload4(rx, __builtin_elementwise_add_sat(xo.z, xc_bytes), 0);
    xr[3] = mfma::bload4(rx, __builtin_elementwise_add_sat(xo.w, xc_bytes), 0);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const TileEntry* ey = &tiles[slab * BK + 2 * a_kq + j];
      const uint2 yo = *reinterpret_cast<const uint2*>(ey->yrow);
      ybits[j] = ey->bits;
      yr[j][0] = mfma::bload2(rdy, __builtin_elementwise_add_sat(yo.x, yc_bytes), 0);
      yr[j][1] = mfma::bload2(rdy, __builtin_elementwise_add_sat(yo.y, yc_bytes), 0);
    }
  }
  __device__ __forceinline__ void store(const TileEntry* tiles, int slab, float* As, float* Bs) {
    float* const a_st = As + a_kq * ROW_A + 2 * a_o;                       // [coord][kq][o][2]
    float* const b_st = Bs + (b_t >> 1) * ROW_B + 2 * b_c + (b_t & 1);    // [coord][kq][c][2]
    if (xbits & kXRare) {
      const int first = tiles[slab * BK + b_t].xfirst + int(x_chan) * HW;
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
          const bool ok = c_ok && ((xbits >> (8 + r)) & 1u) && ((xbits >> cc) & 1u);
          xr[r][cc] = mfma::bload(rx, ok ? uint32_t(first + r * W + cc) * 4u : kOffNone, 0);
        }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
      if (ybits[j] & kYRare) {
        // Row 0 of a tile inside the range is always inside the image.
        const int first = int(tiles[slab * BK + 2 * a_kq + j].yrow[0] >> 2) + int(dy_chan) * OHW;
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
          for (int cc = 0; cc < 2; ++cc) {
            const bool ok = o_ok && ((ybits[j] >> (12 + r)) & 1u) && (cc == 0 || ((ybits[j] >> 4) & 1u));
            yr[j][r][cc] = mfma::bload(rdy, ok ? uint32_t(first + r * OW + cc) * 4u : kOffNone, 0);
          }
      }
    float gy[2][4];  // two 2x2 dy tiles
    float d[16];     // one 4x4 x patch
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        gy[j][r * 2] = yr[j][r][0];
        gy[j][r * 2 + 1] = ((ybits[j] >> 4) & 1u) ? yr[j][r][1] : 0.f;
      }
    dsum += ((gy[0][0] + gy[0][1]) + (gy[0][2] + gy[0][3])) + ((gy[1][0] + gy[1][1]) + (gy[1][2] + gy[1][3]));
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) d[r * 4 + cc] = ((xbits >> cc) & 1u) ? xr[r][cc] : 0.f;
    // dM = A g A^T, A = [[1,0],[1,1],[1,-1],[0,-1]], for both tiles.
    float m[2][16];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float z[4][2];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        z[0][c] = gy[j][c];
        z[1][c] = gy[j][c] + gy[j][2 + c];
        z[2][c] = gy[j][c] - gy[j][2 + c];
        z[3][c] = -gy[j][2 + c];
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        m[j][r * 4 + 0] = z[r][0];
        m[j][r * 4 + 1] = z[r][0] + z[r][1];
        m[j][r * 4 + 2] = z[r][0] - z[r][1];
        m[j][r * 4 + 3] = -z[r][1];
      }
    }
#pragma unroll
    for (int q = 0; q < 16; ++q) *reinterpret_cast<f32x2*>(a_st + q * 4 * ROW_A) = f32x2{m[0][q], m[1][q]};
    // V = B^T d B
    float z[16];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      z[0 * 4 + cc] = d[0 * 4 + cc] - d[2 * 4 + cc];
      z[1 * 4 + cc] = d[1 * 4 + cc] + d[2 * 4 + cc];
      z[2 * 4 + cc] = d[2 * 4 + cc] - d[1 * 4 + cc];
      z[3 * 4 + cc] = d[1 * 4 + cc] - d[3 * 4 + cc];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      b_st[(r * 4 + 0) * 4 * ROW_B] = z[r * 4 + 0] - z[r * 4 + 2];
      b_st[(r * 4 + 1) * 4 * ROW_B] = z[r * 4 + 1] + z[r * 4 + 2];
      b_st[(r * 4 + 2) * 4 * ROW_B] = z[r * 4 + 2] - z[r * 4 + 1];
      b_st[(r * 4 + 3) * 4 * ROW_B] = z[r * 4 + 1] - z[r * 4 + 3];
    }
  }
  // dBias of the range: every dy element lies in exactly one tile, and the
  // workgroups of the first input-channel block read each one once; the four
  // lanes of an output channel (a_kq = 0..3, adjacent) hold its slab tiles.
  __device__ __forceinline__ void write_db(const Args& p, int range, int g, int ngroups, int o0) const {
    float t = dsum;
    t += __shfl_xor(t, 1);
    t += __shfl_xor(t, 2);
    if (a_kq == 0 && o_ok) p.out_db[(int64_t(range) * ngroups + g) * p.O + o0 + a_o] = t;
  }
};

// dw = G^T dU G, G = [[1,0,0],[1/2,1/2,1/2],[1/2,-1/2,1/2],[0,0,1]], of a
// wave's 32 output x 16 input channels, written as the range's 3x3 partial.
// 16x16x4 layout: lane l, register v holds row 4 (l / 16) + v (output
// channel) and column l % 16 (input channel).
__device__ __forceinline__ void write_dw(const Args& p, const f32x4 (&acc)[16][2], int range, int g, int ngroups,
                                         int o0, int c0, int wo, int wc, int kq, int li) {
  const int c = c0 + wc * 16 + li;
  if (c >= p.C) return;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int o = o0 + wo * 32 + i * 16 + 4 * kq + v;
      if (o >= p.O) continue;
      float u[16];
#pragma unroll
      for (int q = 0; q < 16; ++q) u[q] = acc[q][i][v];
      float z[3][4];
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        const float s12 = 0.5f * (u[4 + cc] + u[8 + cc]);
        z[0][cc] = u[cc] + s12;
        z[1][cc] = 0.5f * (u[4 + cc] - u[8 + cc]);
        z[2][cc] = s12 + u[12 + cc];
      }
      float* dst = p.out + ((int64_t(range) * ngroups + g) * p.O + o) * int64_t(p.C) * 9 + int64_t(c) * 9;
#pragma unroll
      for (int r = 0; r < 3; ++r) {
        const float s12 = 0.5f * (z[r][1] + z[r][2]);
        dst[r * 3 + 0] = z[r][0] + s12;
        dst[r * 3 + 1] = 0.5f * (z[r][1] - z[r][2]);
        dst[r * 3 + 2] = s12 + z[r][3];
      }
    }
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void wino_dw_kernel(Args p) {
  __shared__ __attribute__((aligned(16))) float smem[A_FLOATS + B_FLOATS];
  __shared__ TileEntry tiles[kChunk];
  float* As = smem;
  float* Bs = smem + A_FLOATS;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = blockIdx.y;
  // Blocks of one tile range are consecutive, so they share an XCD and read
  // the same x and dy tiles through its L2.
  const int b = mfma::xcd_remap(blockIdx.x, gridDim.x);
  const int nblk = p.n_ob * p.n_cb;
  const int range = b / nblk, ob = (b % nblk) % p.n_ob, cb = (b % nblk) / p.n_ob;
  const int o0 = ob * BO, c0 = cb * BC;
  const int k_begin = range * p.kps;
  const int k_end = min(p.T, k_begin + p.kps);
  SlabIO io;
  io.init(p, tid, g, o0, c0);

  // Wave (wo, wc) owns output channels wo*32 .. +31 (two 16-row blocks) and
  // input channels wc*16 .. +15 of the block, for all 16 coordinates.
  const int wo = wave >> 1, wc = wave & 1;
  const int kq = lane >> 4, li = lane & 15;
  f32x4 acc[16][2];
#pragma unroll
  for (int t = 0; t < 16; ++t) acc[t][0] = acc[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  const f32x2* const a_frag = reinterpret_cast<const f32x2*>(As + kq * ROW_A + 2 * (wo * 32 + li));
  const f32x2* const b_frag = reinterpret_cast<const f32x2*>(Bs + kq * ROW_B + 2 * (wc * 16 + li));
  auto mma = [&]() {
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const f32x2 fb = b_frag[t * 2 * ROW_B];
      const f32x2 fa0 = a_frag[t * 2 * ROW_A];
      const f32x2 fa1 = a_frag[t * 2 * ROW_A + 16];  // output channels + 16
      acc[t][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa0[0], fb[0], acc[t][0], 0, 0, 0);
      acc[t][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa1[0], fb[0], acc[t][1], 0, 0, 0);
      acc[t][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa0[1], fb[1], acc[t][0], 0, 0, 0);
      acc[t][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa1[1], fb[1], acc[t][1], 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
    for (int t = 0; t < 6; ++t) {
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
  };

  for (int k0 = k_begin; k0 < k_end; k0 += kChunk) {
    const int k1 = min(k_end, k0 + kChunk);
    const int nslab = (k1 - k0 + BK - 1) / BK;
    decode_tiles(p, tiles, k0, k1, nslab * BK, tid, mfma::kThreads);
    __syncthreads();
    io.load(tiles, 0);
    for (int sl = 0; sl < nslab; ++sl) {
      io.store(tiles, sl, As, Bs);
      __syncthreads();
      io.load(tiles, min(sl + 1, nslab - 1));  // the last slab re-reads itself: no branch around the loads
      __builtin_amdgcn_sched_barrier(0);
      mma();
      __syncthreads();
    }
  }
  if (p.out_db && cb == 0) io.write_db(p, range, g, gridDim.y, o0);
  write_dw(p, acc, range, g, gridDim.y, o0, c0, wo, wc, kq, li);
}

// The weight gradient with the warp-specialized split of the forward kernel:
// waves 4-7 (producers) load and transform slab s + 1 (dM and V) into the
// other of two LDS stages while waves 0-3 (consumers) multiply slab s; one
// barrier per slab.  A range holds at most kChunk tiles, decoded once; an odd
// slab count runs one more slab of tiles past the range (they read nothing).
// Producers own the dBias sums, consumers the accumulators and the
// G^T dU G epilogue.  Same products per coordinate in the same order as the
// single-role kernel.  106 KB of LDS stages + 16 KB tile table: one
// workgroup of eight waves per CU.
// VEC_OUT (output channels a multiple of 64, input channels of 32): the
// consumers write the block's 3x3 partial (64 x 32 x 9 floats) to LDS and
// all eight waves copy it out as 16-byte stores of whole rows, instead of
// each lane storing its 72 values one float at a time (C1: 14.4 MB of
// partials, 7 us of scattered stores).
constexpr int kResRow = BC * 9;  // floats of one output channel's row in the result tile

// The kernel body for logical block b of group g on caller-provided LDS
// (the backward kernel runs it beside the input gradient's body).
template <bool VEC_OUT>
__device__ __forceinline__ void dw_ws_body(const Args& p, int b, int g, float* __restrict__ As0,
                                           float* __restrict__ Bs0, float* __restrict__ As1, float* __restrict__ Bs1,
                                           TileEntry* __restrict__ tiles) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nblk = p.n_ob * p.n_cb;
  const int range = b / nblk, ob = (b % nblk) % p.n_ob, cb = (b % nblk) / p.n_ob;
  const int o0 = ob * BO, c0 = cb * BC;
  const int k_begin = range * p.kps;
  const int k_end = min(p.T, k_begin + p.kps);  // the host keeps p.kps <= kChunk
  const int nslab = ((k_end - k_begin + BK - 1) / BK + 1) & ~1;  // even, >= 2
  decode_tiles(p, tiles, k_begin, k_end, nslab * BK, tid, 2 * mfma::kThreads);
  __syncthreads();

  if (wave >= 4) {
    SlabIO io;
    io.init(p, tid - mfma::kThreads, g, o0, c0);
    io.load(tiles, 0);
    io.store(tiles, 0, As0, Bs0);
    io.load(tiles, 1);
    __syncthreads();  // stage 0 holds slab 0
    for (int s = 0; s < nslab; s += 2) {
      io.store(tiles, s + 1, As1, Bs1);
      io.load(tiles, min(s + 2, nslab - 1));
      __syncthreads();
      if (s + 2 < nslab) {
        io.store(tiles, s + 2, As0, Bs0);
        io.load(tiles, min(s + 3, nslab - 1));
      }
      __syncthreads();
    }
    if (p.out_db && cb == 0) io.write_db(p, range, g, gridDim.y, o0);
    if constexpr (!VEC_OUT) return;
  }
  if (wave >= 4) {
    __syncthreads();  // the consumers' result tile is in LDS
  } else {
  const int wo = wave >> 1, wc = wave & 1;
  const int kq = lane >> 4, li = lane & 15;
  f32x4 acc[16][2];
#pragma unroll
  for (int t = 0; t < 16; ++t) acc[t][0] = acc[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto slab = [&](const float* Ac, const float* Bc) {
    const f32x2* const a_frag = reinterpret_cast<const f32x2*>(Ac + kq * ROW_A + 2 * (wo * 32 + li));
    const f32x2* const b_frag = reinterpret_cast<const f32x2*>(Bc + kq * ROW_B + 2 * (wc * 16 + li));
    f32x2 fa0[4], fa1[4], fb[4];
    auto frags = [&](int q) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 4 * q + j;
        fb[j] = b_frag[t * 2 * ROW_B];
        fa0[j] = a_frag[t * 2 * ROW_A];
        fa1[j] = a_frag[t * 2 * ROW_A + 16];
      }
    };
    auto quad = [&](int q) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int t = 4 * q + j;
          acc[t][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa0[j][h], fb[j][h], acc[t][0], 0, 0, 0);
          acc[t][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(fa1[j][h], fb[j][h], acc[t][1], 0, 0, 0);
        }
    };
    frags(0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      quad(q);
      if (q < 3) {
        frags(q + 1);
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 14, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  __syncthreads();  // stage 0 holds slab 0
  for (int s = 0; s < nslab; s += 2) {
    slab(As0, Bs0);
    __syncthreads();
    slab(As1, Bs1);
    __syncthreads();
  }
  if constexpr (!VEC_OUT) {
    write_dw(p, acc, range, g, gridDim.y, o0, c0, wo, wc, kq, li);
    return;
  } else {
    // G^T dU G as in write_dw, into the result tile: rows 0-29 in As0, 30-59
    // in As1, 60-63 in Bs0 (the stages are free after the last barrier).
    const int c = wc * 16 + li;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int o = wo * 32 + i * 16 + 4 * kq + v;
        float u[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) u[q] = acc[q][i][v];
        float z[3][4];
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
          const float s12 = 0.5f * (u[4 + cc] + u[8 + cc]);
          z[0][cc] = u[cc] + s12;
          z[1][cc] = 0.5f * (u[4 + cc] - u[8 + cc]);
          z[2][cc] = s12 + u[12 + cc];
        }
        float* dst = (o < 30 ? As0 + o * kResRow : o < 60 ? As1 + (o - 30) * kResRow : Bs0 + (o - 60) * kResRow) +
                     c * 9;
#pragma unroll
        for (int r = 0; r < 3; ++r) {
          const float s12 = 0.5f * (z[r][1] + z[r][2]);
          dst[r * 3 + 0] = z[r][0] + s12;
          dst[r * 3 + 1] = 0.5f * (z[r][1] - z[r][2]);
          dst[r * 3 + 2] = s12 + z[r][3];
        }
      }
    __syncthreads();
  }
  }
  if constexpr (VEC_OUT) {
    // 64 rows of 288 floats (72 16-byte chunks) to [range][g][o][c][3][3].
    float* const out = p.out + ((int64_t(range) * gridDim.y + g) * p.O + o0) * int64_t(p.C) * 9 + int64_t(c0) * 9;
    for (int f4 = tid; f4 < BO * (kResRow / 4); f4 += 2 * mfma::kThreads) {
      const int o = f4 / (kResRow / 4), q = f4 - o * (kResRow / 4);
      const float* src =
          (o < 30 ? As0 + o * kResRow : o < 60 ? As1 + (o - 30) * kResRow : Bs0 + (o - 60) * kResRow) + 4 * q;
      *reinterpret_cast<f32x4*>(out + int64_t(o) * p.C * 9 + 4 * q) = *reinterpret_cast<const f32x4*>(src);
    }
  }
}

template <bool VEC_OUT>
__global__ __launch_bounds__(512) void wino_dw_ws_kernel(Args p) {
  __shared__ __attribute__((aligned(16))) float As0[A_FLOATS];
  __shared__ __attribute__((aligned(16))) float Bs0[B_FLOATS];
  __shared__ __attribute__((aligned(16))) float As1[A_FLOATS];
  __shared__ __attribute__((aligned(16))) float Bs1[B_FLOATS];
  __shared__ TileEntry tiles[kChunk];
  dw_ws_body<VEC_OUT>(p, mfma::xcd_remap(blockIdx.x, gridDim.x), blockIdx.y, As0, Bs0, As1, Bs1, tiles);
}

}  // namespace fused_dw

// ------------------------------------------------------------ backward kernel
// The input and weight gradients of one 3x3 stride-1 layer in one launch:
// workgroups 0 .. n_dw - 1 run the weight gradient's warp-specialized body,
// the rest the fused kernel's body on dy with the flipped filter (dx).  A
// dependent launch costs about 3 us on MI355X even when empty, and each of
// the two launches alone leaves CUs idle at the end (C1: 196 workgroups of
// each on 256 CUs); together the longer weight-gradient workgroups start
// first and the input-gradient ones fill the CUs as they free up.  Each body
// is the one its own kernel runs, so the results are bit-identical to the
// two separate calls.  LDS: the larger body's stages and tile table (120 KB).
namespace bwd {
constexpr int kFwdFloats = 2 * (fused::A_FLOATS + fused::B_FLOATS);
constexpr int kDwStage = fused_dw::A_FLOATS + fused_dw::B_FLOATS;
constexpr int kLdsFloats = 2 * kDwStage + fused_dw::kChunk * int(sizeof(fused_dw::TileEntry) / 4);
static_assert(kFwdFloats <= kLdsFloats, "the input gradient's stages fit the weight gradient's");

template <bool RAGGED, bool VEC_OUT, int FILT>
__global__ __launch_bounds__(512) void wino_bwd_kernel(fused::Args pf, fused_dw::Args pw, int n_dw) {
  __shared__ __attribute__((aligned(16))) float lds[kLdsFloats];
  const int bx = blockIdx.x;
  if (bx < n_dw) {
    fused_dw::dw_ws_body<VEC_OUT>(pw, mfma::xcd_remap(bx, n_dw), blockIdx.y, lds, lds + fused_dw::A_FLOATS,
                                  lds + kDwStage, lds + kDwStage + fused_dw::A_FLOATS,
                                  reinterpret_cast<fused_dw::TileEntry*>(lds + 2 * kDwStage));
  } else {
    const int n_dx = int(gridDim.x) - n_dw;
    ws::ws_body<RAGGED, FILT>(pf, mfma::xcd_remap(bx - n_dw, n_dx), blockIdx.y, lds, lds + fused::A_FLOATS,
                           lds + fused::A_FLOATS + fused::B_FLOATS, lds + 2 * fused::A_FLOATS + fused::B_FLOATS);
  }
}
}  // namespace bwd

int winograd_unfused(const mx_conv2d_desc& d, const float* x, const float* w, const float* bias, float* y,
                     bool flip, int64_t chunk, hipStream_t s);

}  // namespace

namespace {
// The batched GEMM of the unfused passes: M_t = U_t V_t for the 16*G
// coordinates, U [16*G][Cout_g][Cin_g], V [16*G][Cin_g][T], M [16*G][Cout_g][T].
mx_gemm_desc unfused_gemm_desc(int G, int Cout_g, int Cin_g, int64_t T) {
  mx_gemm_desc gd{};
  gd.batch = 16 * int64_t(G);
  gd.m = Cout_g;
  gd.n = T;
  gd.k = Cin_g;
  gd.a_stride_b = int64_t(Cout_g) * Cin_g;
  gd.a_stride_m = Cin_g;
  gd.a_stride_k = 1;
  gd.b_stride_b = int64_t(Cin_g) * T;
  gd.b_stride_k = T;
  gd.b_stride_n = 1;
  gd.c_stride_b = int64_t(Cout_g) * T;
  gd.ldc = T;
  gd.alpha = 1.f;
  gd.beta = 0.f;
  gd.bias_kind = MX_BIAS_NONE;
  return gd;
}

int winograd_unfused(const mx_conv2d_desc& d, const float* x, const float* w, const float* bias, float* y,
                     bool flip, int64_t chunk, hipStream_t s) {
  WinoArgs p{};
  p.flip = flip ? 1 : 0;
  p.w = w;
  p.bias = bias;
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
  const int64_t T = chunk * p.TH * p.TW;  // tiles of one chunk of images
  MX_REQUIRE(T <= INT32_MAX && 16 * int64_t(p.Cin) * T <= INT32_MAX && 16 * int64_t(p.Cout) * T <= INT32_MAX,
             MX_ERR_UNSUPPORTED, "winograd: transformed tensors exceed int32 indexing");
  Scratch U, V, M;
  MX_TRY(U.alloc(size_t(16) * p.Cout * p.Cin_g * 4, s));
  MX_TRY(V.alloc(size_t(16) * p.Cin * T * 4, s));
  MX_TRY(M.alloc(size_t(16) * p.Cout * T * 4, s));
  p.U = U.as<float>();
  p.V = V.as<float>();
  p.M = M.as<float>();
  hipLaunchKernelGGL(wino_filter_kernel, dim3(blocks_for(int64_t(p.Cout) * p.Cin_g)), dim3(256), 0, s, p);
  MX_HIP(hipGetLastError());
  // Images in chunks that reuse V and M (the workspace budget sets the chunk).
  for (int64_t n0 = 0; n0 < d.n; n0 += chunk) {
    p.N = int(std::min(chunk, d.n - n0));
    p.T = p.N * p.TH * p.TW;
    p.x = x + n0 * p.Cin * p.H * p.W;
    p.y = y + n0 * p.Cout * p.OH * p.OW;
    hipLaunchKernelGGL(wino_input_kernel, dim3(blocks_for(int64_t(p.Cin) * p.T)), dim3(256), 0, s, p);
    MX_HIP(hipGetLastError());
    const mx_gemm_desc gd = unfused_gemm_desc(p.G, p.Cout_g, p.Cin_g, p.T);
    MX_TRY(mx_gemm_f32(&gd, p.U, p.V, nullptr, p.M, s));
    hipLaunchKernelGGL(wino_output_kernel, dim3(blocks_for(int64_t(p.Cout) * p.T)), dim3(256), 0, s, p);
    MX_HIP(hipGetLastError());
  }
  return MX_OK;
}
}  // namespace

namespace {
// Launch plan of a Winograd convolution: the fused kernel's arguments (all
// but the data pointers), its grid, and whether the fused or the unfused
// passes run.  The unfused passes need U, V and M in scratch; V and M cover
// as many images at a time as the workspace budget holds (`chunk`), and when
// not even one image fits the fused kernel runs instead (it needs only the
// transformed filter, which like a packed weight copy is not counted).
struct RunPlan {
  fused::Args p{};
  int G = 1;
  int64_t blocks = 0;
  bool fused = true;
  bool filt = false;          // the fused kernel transforms the filter itself (no filter launch)
  bool t16 = false;           // the 16-tile fused kernel (two workgroups per CU)
  int64_t chunk = 0;          // images per unfused pass
  int64_t unfused_bytes = 0;  // U, V and M of one pass
};

int plan_run(const mx_conv2d_desc& d, int64_t ws_limit, RunPlan* r) {
  fused::Args& p = r->p;
  p.Cin = int(d.cin);
  p.H = int(d.h);
  p.W = int(d.w);
  p.Cout = int(d.cout);
  p.OH = int(d.oh);
  p.OW = int(d.ow);
  p.ph = int(d.ph);
  p.pw = int(d.pw);
  r->G = int(d.groups);
  p.C = p.Cin / r->G;
  p.O = p.Cout / r->G;
  // The fused kernel runs two slabs per loop trip: channels padded to 16
  // (zero filter rows).
  p.Cpad = (p.C + 2 * fused::BK - 1) / (2 * fused::BK) * (2 * fused::BK);
  p.Opad = (p.O + fused::BO - 1) / fused::BO * fused::BO;
  p.TH = (p.OH + 1) / 2;
  p.TW = (p.OW + 1) / 2;
  p.n_ob = p.Opad / fused::BO;
  p.nslab = p.Cpad / fused::BK;
  p.f_tw = mfma::fast_div(uint32_t(p.TW));
  p.f_thw = mfma::fast_div(uint32_t(p.TH * p.TW));
  const int64_t u_bytes = int64_t(r->G) * 16 * p.Cpad * p.Opad * 4;
  MX_REQUIRE(u_bytes < mfma::kBufMaxBytes, MX_ERR_UNSUPPORTED, "winograd: the transformed filter exceeds 2 GiB");
  p.u_bytes = u_bytes;
  // The caller splits batches so the input stays one buffer resource with
  // 32-bit offsets (images_per_launch).
  p.x_bytes = d.n * int64_t(p.Cin) * p.H * p.W * 4;
  p.y_bytes = d.n * int64_t(p.Cout) * p.OH * p.OW * 4;
  const int64_t T = d.n * int64_t(p.TH) * p.TW;
  MX_REQUIRE(p.x_bytes < mfma::kBufMaxBytes && p.y_bytes < mfma::kBufMaxBytes && T <= INT32_MAX, MX_ERR_UNSUPPORTED,
             "winograd: an operand exceeds the 2 GiB bound");
  p.T = int(T);
  r->blocks = (T + fused::BT - 1) / fused::BT * p.n_ob;
  MX_REQUIRE(r->blocks <= INT32_MAX, MX_ERR_UNSUPPORTED, "winograd: grid too large");
  const int64_t wgs = r->blocks * r->G;
  // MX_WINOGRAD_FUSED=1 / 0 forces the fused / unfused kernels (tests, tuning).
  r->fused = fused::prefer_fused(wgs, p.nslab);
  if (const char* e = std::getenv("MX_WINOGRAD_FUSED"))
    if (e[0] == '0' || e[0] == '1') r->fused = e[0] == '1';
  const int64_t u_plain = 16 * int64_t(p.Cout) * p.C * 4;
  const int64_t per_image = 16 * (int64_t(p.Cin) + p.Cout) * p.TH * p.TW * 4;
  const int64_t fit = ws_limit > u_plain ? (ws_limit - u_plain) / per_image : 0;
  if (!r->fused && fit < 1) r->fused = true;
  if (!r->fused) {
    const int64_t passes = (d.n + fit - 1) / fit;
    r->chunk = (d.n + passes - 1) / passes;
    r->unfused_bytes = u_plain + per_image * r->chunk;
  }
  // With at most 4 slabs the producers transform the filter themselves: a
  // dependent launch costs about 3 us on MI355X even when empty, more than
  // the filter's work (20 -> 24 channels at 9x11, batch 4: 8.8 -> 6.8 us); on
  // longer walks every workgroup redoing the transform costs more than the
  // launch (C1's layer 18.3 -> 19.3 us, 64 x 56^2 80.6 -> 105.4).
  // MX_WINOGRAD_FILTER=0 / 1 forces the filter launch / the in-kernel
  // transform (tests, tuning).
  r->filt = p.nslab <= 4;
  if (const char* e = std::getenv("MX_WINOGRAD_FILTER"))
    if (e[0] == '0' || e[0] == '1') r->filt = e[0] == '1';
  r->filt = r->filt && r->fused;
  // The 16-tile kernel (two workgroups per CU, one's prologue and epilogue
  // under the other's products) wins while the transformed filter is small
  // enough to stay in L2 for the twice as many workgroups that read it: 64 x
  // 64 channels at 56^2, batch 64, 96.3 -> 84.4 us, 128 x 128 at 28^2 93.9 ->
  // 79.5, 256 x 256 at 16^2, batch 16, 49.0 -> 34.7; at 512 x 512 (a 16.8 MB
  // U') it loses (91.2 -> 94.9).  MX_WINOGRAD_T16=0 / 1 forces it off / on.
  r->t16 = int64_t(p.Cpad) * p.Opad <= 256 * 256;
  if (const char* e = std::getenv("MX_WINOGRAD_T16"))
    if (e[0] == '0' || e[0] == '1') r->t16 = e[0] == '1';
  r->t16 = r->t16 && r->fused;
  if (r->filt) {
    p.w_bytes = int64_t(d.cout) * p.C * 9 * 4;
    MX_REQUIRE(p.w_bytes < mfma::kBufMaxBytes, MX_ERR_UNSUPPORTED, "winograd: the filter exceeds 2 GiB");
  }
  return MX_OK;
}

// The convolution d of x with filter w (read flipped and channel-swapped when
// `flip`), Winograd F(2x2,3x3), plus bias.
int winograd_run(const mx_conv2d_desc& d, const float* x, const float* w, const float* bias, float* y, bool flip,
                 int64_t ws_limit, hipStream_t s) {
  RunPlan r;
  MX_TRY(plan_run(d, ws_limit, &r));
  fused::Args& p = r.p;
  if (p.T == 0) return MX_OK;
  if (!r.fused) return winograd_unfused(d, x, w, bias, y, flip, r.chunk, s);
  p.bias = bias;
  p.x = x;
  p.y = y;
  const dim3 grid{unsigned(r.blocks), unsigned(r.G), 1u};
  const bool ragged = p.C % (2 * fused::BK) != 0;
  if (r.filt && r.t16) {
    p.w = w;
    const dim3 grid16{unsigned((int64_t(p.T) + ws::BT16 - 1) / ws::BT16 * p.n_ob), unsigned(r.G), 1u};
    void (*k16)(fused::Args) = flip ? (ragged ? ws::wino_ws16_kernel<true, 2> : ws::wino_ws16_kernel<false, 2>)
                                    : (ragged ? ws::wino_ws16_kernel<true, 1> : ws::wino_ws16_kernel<false, 1>);
    hipLaunchKernelGGL(k16, grid16, dim3(512), 0, s, p);
    MX_HIP(hipGetLastError());
    return MX_OK;
  }
  if (r.filt) {
    p.w = w;
    void (*kern)(fused::Args) = flip ? (ragged ? ws::wino_ws_kernel<true, 2> : ws::wino_ws_kernel<false, 2>)
                                     : (ragged ? ws::wino_ws_kernel<true, 1> : ws::wino_ws_kernel<false, 1>);
    hipLaunchKernelGGL(kern, grid, dim3(512), 0, s, p);
    MX_HIP(hipGetLastError());
    return MX_OK;
  }
  Scratch U;
  MX_TRY(U.alloc(size_t(p.u_bytes), s));
  p.U = U.as<float>();
  // 64-thread blocks: a small filter (64 x 64 is 2,048 threads) then spreads
  // over 32 CUs instead of 8, and its scattered reads queue on more of them.
  const int64_t filter_threads = int64_t(r.G) * (p.Cpad / 2) * p.Opad;
  hipLaunchKernelGGL(fused::filter_kernel, dim3(unsigned(std::min<int64_t>((filter_threads + 63) / 64, 1 << 20))),
                     dim3(64), 0, s, w, U.as<float>(), p.C, p.O, p.Cpad, p.Opad, r.G, flip);
  MX_HIP(hipGetLastError());
  if (r.t16) {
    const dim3 grid16{unsigned((int64_t(p.T) + ws::BT16 - 1) / ws::BT16 * p.n_ob), unsigned(r.G), 1u};
    void (*k16)(fused::Args) = ragged ? ws::wino_ws16_kernel<true, 0> : ws::wino_ws16_kernel<false, 0>;
    hipLaunchKernelGGL(k16, grid16, dim3(512), 0, s, p);
    MX_HIP(hipGetLastError());
    return MX_OK;
  }
  void (*kern)(fused::Args) = ragged ? ws::wino_ws_kernel<true, 0> : ws::wino_ws_kernel<false, 0>;
  hipLaunchKernelGGL(kern, grid, dim3(512), 0, s, p);
  MX_HIP(hipGetLastError());
  return MX_OK;
}

// Launch plan of the Winograd weight gradient: K ranges of output tiles sized
// so the launch fills every CU twice (at least four slabs each), as few as
// the workspace budget requires for their partials (one range writes dw
// directly, with no scratch).
struct DwRunPlan {
  fused_dw::Args p{};
  int G = 1;
  int64_t blocks = 0, ranges = 1, n_dw = 0, n_db = 0;
  bool ws = false;  // the warp-specialized kernel (ranges of at most fused_dw::kChunk tiles)
};

// with_db: the kernel also writes the dBias partials (Cout per range).
int plan_dw_run(const mx_conv2d_desc& d, int64_t ws_limit, bool with_db, DwRunPlan* r) {
  fused_dw::Args& p = r->p;
  p.Cin = int(d.cin);
  p.H = int(d.h);
  p.W = int(d.w);
  p.Cout = int(d.cout);
  p.OH = int(d.oh);
  p.OW = int(d.ow);
  p.ph = int(d.ph);
  p.pw = int(d.pw);
  r->G = int(d.groups);
  p.C = p.Cin / r->G;
  p.O = p.Cout / r->G;
  p.TH = (p.OH + 1) / 2;
  p.TW = (p.OW + 1) / 2;
  p.n_ob = (p.O + fused_dw::BO - 1) / fused_dw::BO;
  p.n_cb = (p.C + fused_dw::BC - 1) / fused_dw::BC;
  p.f_tw = mfma::fast_div(uint32_t(p.TW));
  p.f_thw = mfma::fast_div(uint32_t(p.TH * p.TW));
  // The caller splits batches so both operands stay buffer-addressable.
  p.x_bytes = d.n * int64_t(p.Cin) * p.H * p.W * 4;
  p.dy_bytes = d.n * int64_t(p.Cout) * p.OH * p.OW * 4;
  const int64_t T = d.n * int64_t(p.TH) * p.TW;
  MX_REQUIRE(p.x_bytes < mfma::kBufMaxBytes && p.dy_bytes < mfma::kBufMaxBytes && T <= INT32_MAX, MX_ERR_UNSUPPORTED,
             "winograd dweight: an operand exceeds the 2 GiB bound");
  r->n_dw = int64_t(p.Cout) * p.C * 9;
  r->n_db = with_db ? p.Cout : 0;
  r->blocks = int64_t(p.n_ob) * p.n_cb * r->G;
  const int64_t fit = ws_limit / ((r->n_dw + r->n_db) * 4);
  // Warp-specialized kernel: one workgroup per CU, so ranges fill the CUs
  // once (whole slab pairs, at most kChunk tiles each, as many as the
  // workspace holds; one range writes dw directly).  MX_WINO_DW_WS=0 / 1
  // forces the single-role / warp-specialized kernel (tests, tuning).
  {
    const int64_t want = fit >= 2 ? std::max<int64_t>(1, std::min<int64_t>(cu_count() / r->blocks, fit)) : 1;
    int64_t kps = (T + want - 1) / want;
    kps = (kps + 2 * fused_dw::BK - 1) / (2 * fused_dw::BK) * (2 * fused_dw::BK);
    r->ws = kps <= fused_dw::kChunk;
    if (const char* e = std::getenv("MX_WINO_DW_WS"))
      if (e[0] == '0' || e[0] == '1') r->ws = e[0] == '1' && kps <= fused_dw::kChunk;
    if (r->ws) {
      r->ranges = std::max<int64_t>(1, (T + kps - 1) / kps);
      MX_REQUIRE(r->blocks * r->ranges <= INT32_MAX && r->G <= 65535, MX_ERR_UNSUPPORTED,
                 "winograd dweight: grid too large");
      p.kps = int(kps);
      p.T = int(T);
      return MX_OK;
    }
  }
  int64_t per_cu = 2;
  if (const char* e = std::getenv("MX_WINO_DW_PER_CU")) per_cu = std::max(1, std::atoi(e));
  int64_t want = std::max<int64_t>(1, (per_cu * int64_t(cu_count()) + r->blocks - 1) / r->blocks);
  want = fit >= 2 ? std::min(want, fit) : 1;
  int64_t kps = (T + want - 1) / want;
  kps = std::max<int64_t>(kps, 4 * fused_dw::BK);
  kps = (kps + fused_dw::BK - 1) / fused_dw::BK * fused_dw::BK;
  r->ranges = std::max<int64_t>(1, (T + kps - 1) / kps);
  MX_REQUIRE(r->blocks * r->ranges <= INT32_MAX && r->G <= 65535, MX_ERR_UNSUPPORTED,
             "winograd dweight: grid too large");
  p.kps = int(kps);
  p.T = int(T);
  return MX_OK;
}
}  // namespace

int winograd_forward(const mx_conv2d_desc& d, const float* x, const float* w, const float* bias, float* y,
                     int64_t ws_limit, hipStream_t s) {
  return winograd_run(d, x, w, bias, y, false, ws_limit, s);
}

// dw (and db when given) of the 3x3 stride-1 layer d (any padding): the
// fused adjoint kernel over K ranges of tiles, then a fixed-order sum of the
// ranges' partials.  The partials go to `ext` when the caller provides the
// workspace (at least ws_limit bytes), else to a stream-ordered allocation.
int winograd_backward_weight(const mx_conv2d_desc& d, const float* x, const float* dy, float* dw, float* db,
                             int64_t ws_limit, float* ext, hipStream_t s) {
  DwRunPlan r;
  MX_TRY(plan_dw_run(d, ws_limit, db != nullptr, &r));
  fused_dw::Args& p = r.p;
  p.x = x;
  p.dy = dy;
  Scratch ws;
  float* partials = ext;
  if (r.ranges > 1 && !ext) {
    MX_TRY(ws.alloc(size_t(r.ranges) * size_t(r.n_dw + r.n_db) * 4, s));
    partials = ws.as<float>();
  }
  float* const partials_db = r.ranges > 1 ? partials + r.ranges * r.n_dw : nullptr;
  p.out = r.ranges > 1 ? partials : dw;
  p.out_db = db ? (r.ranges > 1 ? partials_db : db) : nullptr;
  if (r.ws) {
    const bool vec_out = p.O % fused_dw::BO == 0 && p.C % fused_dw::BC == 0 && (reinterpret_cast<uintptr_t>(p.out) & 15) == 0;
    void (*kern)(fused_dw::Args) = vec_out ? fused_dw::wino_dw_ws_kernel<true> : fused_dw::wino_dw_ws_kernel<false>;
    hipLaunchKernelGGL(kern, dim3(unsigned(r.blocks / r.G * r.ranges), unsigned(r.G)), dim3(512), 0, s, p);
  }
  else
    hipLaunchKernelGGL(fused_dw::wino_dw_kernel, dim3(unsigned(r.blocks / r.G * r.ranges), unsigned(r.G)),
                       dim3(256), 0, s, p);
  MX_HIP(hipGetLastError());
  if (r.ranges > 1)
    return conv::sum_partials(partials, partials_db, int(r.ranges), r.n_dw, int(r.n_db), dw, db, s);
  return MX_OK;
}

namespace {
// The transposed description of a Winograd input gradient (see below).
mx_conv2d_desc dinput_as_forward(const mx_conv2d_desc& d) {
  mx_conv2d_desc t = d;
  t.cin = d.cout;
  t.h = d.oh;
  t.w = d.ow;
  t.cout = d.cin;
  t.ph = 2 - d.ph;
  t.pw = 2 - d.pw;
  t.oh = d.h;
  t.ow = d.w;
  return t;
}
}  // namespace

// Kernels a Winograd call of `phase` launches and the scratch it counts
// against the workspace budget.
int winograd_describe(const mx_conv2d_desc& d, int phase, bool with_bias, int64_t ws_limit, std::string* variant,
                      int64_t* ws_bytes) {
  if (phase == MX_CONV_DWEIGHT) {
    DwRunPlan r;
    MX_TRY(plan_dw_run(d, ws_limit, with_bias, &r));
    *variant = cat(r.ws ? "wino_dw_ws_kernel" : "wino_dw_kernel", r.ranges > 1 ? "+ranges" : "");
    *ws_bytes = r.ranges > 1 ? r.ranges * (r.n_dw + r.n_db) * 4 : 0;
    return MX_OK;
  }
  RunPlan r;
  MX_TRY(plan_run(phase == MX_CONV_DINPUT ? dinput_as_forward(d) : d, ws_limit, &r));
  if (r.fused) {
    *variant = cat(r.t16 ? "wino_ws16_kernel<" : "wino_ws_kernel<", r.p.C % (2 * fused::BK) ? "ragged" : "even",
                   r.filt ? ",filter>" : ">");
    *ws_bytes = 0;
  } else {
    // U, V and M are fresh mx_malloc blocks (256-byte aligned).
    const mx_gemm_desc gd = unfused_gemm_desc(r.G, r.p.O, r.p.C, r.chunk * r.p.TH * r.p.TW);
    const float* aligned = reinterpret_cast<const float*>(uintptr_t(256));
    char gname[96];
    MX_TRY(mx_gemm_variant(&gd, aligned, aligned, gname, sizeof gname));
    *variant = cat("wino_unfused(", gname, ")", r.chunk < d.n ? "+chunks" : "");
    *ws_bytes = r.unfused_bytes;
  }
  if (phase == MX_CONV_DINPUT) *variant += "+flip";
  return MX_OK;
}

// dx of the 3x3 stride-1 layer d: the forward convolution of dy
// [N][Cout][OH][OW] with the flipped filter at padding 2 - p, whose output is
// [N][Cin][H][W] since H = OH + 2 (2 - p) - 2.  Needs p <= 2.
int winograd_backward_input(const mx_conv2d_desc& d, const float* dy, const float* w, float* dx, int64_t ws_limit,
                            hipStream_t s) {
  return winograd_run(dinput_as_forward(d), dy, w, nullptr, dx, true, ws_limit, s);
}

// Whether both Winograd gradients of the 3x3 stride-1 layer d run as one
// backward launch (*one), with the plans that launch uses.  One launch pays
// for tiny layers, where launch overhead dominates (33 -> 40 channels at
// 17x15: 20.2 -> 15.4 us), and where two launches of short walks (<= 8 slabs)
// would each leave CUs idle but together fill them at least one and a half
// times over, with the input gradient alone fitting the CUs once (C1's layer:
// 196 + 196 workgroups, 45.1 -> 39.6 us).  Otherwise the 16-tile
// input-gradient kernel's two workgroups per CU win (64 x 28^2, batch 16: 33.3
// vs 34.1; 128 x 28^2, batch 8: 46.3 vs 48.7; 256 x 16^2, batch 16: 68.9 vs
// 82.0).  MX_WINOGRAD_BWD=0 / 1 forces the two launches / the one launch.
static int winograd_backward_plan(const mx_conv2d_desc& d, int64_t ws_limit, bool with_db, RunPlan* rf,
                                  DwRunPlan* rw, bool* one) {
  *one = false;
  if (d.ph > 2 || d.pw > 2) return MX_OK;
  MX_TRY(plan_run(dinput_as_forward(d), ws_limit, rf));
  MX_TRY(plan_dw_run(d, ws_limit, with_db, rw));
  if (!rf->fused || !rw->ws || rf->p.T == 0 || rw->p.T == 0) return MX_OK;
  const int64_t cus = cu_count(), n_dx32 = rf->blocks * rf->G, n_dw_all = rw->blocks * rw->ranges;
  bool o = 4 * (n_dx32 + n_dw_all) <= cus ||
           (rf->p.nslab <= 8 && n_dx32 <= cus && 2 * (n_dx32 + n_dw_all) >= 3 * cus);
  if (const char* e = std::getenv("MX_WINOGRAD_BWD"))
    if (e[0] == '0' || e[0] == '1') o = e[0] == '1';
  *one = o;
  return MX_OK;
}

int winograd_backward_one_launch(const mx_conv2d_desc& d, int64_t ws_limit, bool with_db, bool* one) {
  RunPlan rf;
  DwRunPlan rw;
  return winograd_backward_plan(d, ws_limit, with_db, &rf, &rw, one);
}

// dx, dw and db of the 3x3 stride-1 layer d in one backward launch (after
// the flipped filter transform, before the weight gradient's range sum) when
// both gradients take the fused Winograd paths: the input gradient the fused
// kernel with U' from the filter launch, the weight gradient the
// warp-specialized kernel.  *done = false (nothing launched) otherwise; the
// caller then runs the two gradients one after the other.
int winograd_backward(const mx_conv2d_desc& d, const float* x, const float* w, const float* dy, float* dx, float* dw,
                      float* db, int64_t ws_limit, hipStream_t s, bool* done) {
  *done = false;
  RunPlan rf;
  DwRunPlan rw;
  bool one = false;
  MX_TRY(winograd_backward_plan(d, ws_limit, db != nullptr, &rf, &rw, &one));
  if (!one) return MX_OK;
  // Input gradient: the fused kernel's arguments as winograd_run sets them.
  fused::Args& pf = rf.p;
  pf.bias = nullptr;
  pf.x = dy;
  pf.y = dx;
  // With walks of <= 8 slabs the input-gradient workgroups transform the
  // flipped filter themselves, saving the filter launch (C1 40.1 -> 39.6 us;
  // 512 channels 201 -> 218, so not on long walks).  MX_WINOGRAD_FILTER=0 /
  // 1 forces the filter launch / the in-kernel transform.
  bool in_filt = rf.p.nslab <= 8;
  if (const char* e = std::getenv("MX_WINOGRAD_FILTER"))
    if (e[0] == '0' || e[0] == '1') in_filt = e[0] == '1';
  Scratch U;
  if (in_filt) {
    pf.w = w;
    pf.w_bytes = int64_t(d.cout) * (d.cin / d.groups) * 9 * 4;
  } else {
    MX_TRY(U.alloc(size_t(pf.u_bytes), s));
    pf.U = U.as<float>();
    const int64_t filter_threads = int64_t(rf.G) * (pf.Cpad / 2) * pf.Opad;
    hipLaunchKernelGGL(fused::filter_kernel, dim3(unsigned(std::min<int64_t>((filter_threads + 63) / 64, 1 << 20))),
                       dim3(64), 0, s, w, U.as<float>(), pf.C, pf.O, pf.Cpad, pf.Opad, rf.G, true);
    MX_HIP(hipGetLastError());
  }
  // Weight gradient: as winograd_backward_weight sets it.
  fused_dw::Args& pw = rw.p;
  pw.x = x;
  pw.dy = dy;
  Scratch ws;
  float* partials = nullptr;
  if (rw.ranges > 1) {
    MX_TRY(ws.alloc(size_t(rw.ranges) * size_t(rw.n_dw + rw.n_db) * 4, s));
    partials = ws.as<float>();
  }
  float* const partials_db = rw.ranges > 1 ? partials + rw.ranges * rw.n_dw : nullptr;
  pw.out = rw.ranges > 1 ? partials : dw;
  pw.out_db = db ? (rw.ranges > 1 ? partials_db : db) : nullptr;
  const bool vec_out =
      pw.O % fused_dw::BO == 0 && pw.C % fused_dw::BC == 0 && (reinterpret_cast<uintptr_t>(pw.out) & 15) == 0;
  const bool ragged = pf.C % (2 * fused::BK) != 0;
  const int64_t n_dw = rw.blocks / rw.G * rw.ranges, n_dx = rf.blocks;
  MX_REQUIRE(n_dw + n_dx <= INT32_MAX && rf.G == rw.G, MX_ERR_UNSUPPORTED, "winograd backward: grid too large");
  void (*kern)(fused::Args, fused_dw::Args, int) =
      in_filt ? (ragged ? (vec_out ? bwd::wino_bwd_kernel<true, true, 2> : bwd::wino_bwd_kernel<true, false, 2>)
                        : (vec_out ? bwd::wino_bwd_kernel<false, true, 2> : bwd::wino_bwd_kernel<false, false, 2>))
              : (ragged ? (vec_out ? bwd::wino_bwd_kernel<true, true, 0> : bwd::wino_bwd_kernel<true, false, 0>)
                        : (vec_out ? bwd::wino_bwd_kernel<false, true, 0> : bwd::wino_bwd_kernel<false, false, 0>));
  hipLaunchKernelGGL(kern, dim3(unsigned(n_dw + n_dx), unsigned(rw.G)), dim3(512), 0, s, pf, pw, int(n_dw));
  MX_HIP(hipGetLastError());
  *done = true;
  if (rw.ranges > 1)
    return conv::sum_partials(partials, partials_db, int(rw.ranges), rw.n_dw, int(rw.n_db), dw, db, s);
  return MX_OK;
}

}  // namespace mx
