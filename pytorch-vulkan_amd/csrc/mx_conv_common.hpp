// Shared pieces of the implicit-GEMM Conv2D kernels (forward, dInput,
// dWeight): the argument block, the operand loaders and the tile menu.
//
// GEMM views (per group g):
//   forward : C[co, pos]        = Wp[co, k(ci,kh,kw)]   x im2col(x)[k(ci,kh,kw), pos]
//   dInput  : C[ci, ppos]       = Wt_p[ci, k(co,th,tw)] x gather_p(dy)[k(co,th,tw), ppos]
//             k(.) is the gathered K order (kChanBlock below).
//             one GEMM per stride phase p = (ih % sh, iw % sw); ppos runs over
//             the input positions of that phase and (th, tw) over the taps
//             that reach it, so no zero-inserted term is ever multiplied.
//   dWeight : C[co, (ci,kh,kw)] = dy[co, pos]           x im2col(x)^T[pos, (ci,kh,kw)]
//             K = N*OH*OW split across workgroups; per-split partials are
//             summed in fixed split order by a finalize kernel.
//
// Loaders feed the double-buffered MFMA main loop (mfma_core.hpp).  Where the
// operand is a plain strided matrix (1x1 stride-1 unpadded convolutions, the
// dy operand of dWeight, the packed weights of dInput) the loaders read 16
// bytes per lane; gathers with halo checks read 4 bytes per lane, consecutive
// lanes on consecutive positions.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>

#include "mfma_core.hpp"
#include "mx_internal.hpp"

namespace mx {
namespace conv {

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
  // dInput stride phase: input positions ih = pa + sh*i (i < Hp),
  // iw = pb + sw*j (j < Wp); tap th reaches dy row i + offh0 - th*dsh, tap tw
  // dy column j + offw0 - tw*dsw.
  // Tap th is kernel row kh0 + th*stph (tw: kernel column kw0 + tw*stpw).
  int pa, pb, Hp, Wp, HpWp, nth, ntw, offh0, offw0, dsh, dsw, kh0, kw0, stph, stpw;
  const float* wt;  // weights packed to the gathered K order: forward [g][co][k], dInput [g][k][ci]
  // Split-K partials (splits > 1): forward / dInput write their tile to
  // ws + split * out_elems at the output's own offsets; dWeight writes
  // [split][G*Cout_g][Cin_g*KK] and the dBias partials to ws_db [split][Cout].
  float* ws;
  float* ws_db;
  int64_t out_elems;
};

// Gathered K order.  With a channel count that is a multiple of kChanBlock
// the K index of the forward / dInput GEMMs runs over (channel block, kh, kw,
// channel in block): a loader's run of consecutive k (at most kChanBlock) then
// shares one tap, so one bounds test covers it and its addresses are one
// channel plane apart, while the taps of one channel block stay within a few
// slabs (the input lines they share stay in L1).  Other channel counts keep
// the plain (channel, kh, kw) order.  The weights are packed to match.
constexpr int kChanBlock = 16;
__host__ __device__ constexpr bool blocked_channels(int c) { return c % kChanBlock == 0; }

// ------------------------------------------------------------------ loaders
// Forward B operand (gather): rows = output positions (img, oh, ow), k in
// the gathered K order over (ci, kh, kw); element
// x[img][g*Cin_g + ci][oh*sh - ph + kh*dh][ow*sw - pw + kw*dw].  Each thread
// holds EPT consecutive k of one position.
template <int ROWS, int BK>
struct Im2colLoader {
  static constexpr bool KMAJOR = false;
  static constexpr bool DEEP = false;  // its per-thread state leaves no room for a second set at 64x64
  int kstep = BK;  // k advance per load(); the main loop may set 2 * BK
  static constexpr int EPT = ROWS * BK / kThreads;
  static_assert(ROWS <= kThreads && EPT >= 1 && BK % EPT == 0 && kChanBlock % EPT == 0, "Im2colLoader tiling");
  float v[EPT];
  const float* xg;
  int ih0, iw0, ks, k, kmax;
  bool ok, blocked;
  int KK, KBLK, KH, KW, dh, dw, H, W, HW;
  __device__ __forceinline__ void init(const ConvArgs& p, int col0, int g, int k0, int kmax_) {
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
    blocked = blocked_channels(p.Cin_g);
    KK = p.KK;
    KBLK = p.KK * kChanBlock;
    KH = p.KH;
    KW = p.KW;
    dh = p.dh;
    dw = p.dw;
    H = p.H;
    W = p.W;
    HW = p.HW;
    k = k0;
    kmax = kmax_;
  }
  __device__ __forceinline__ void load() {
    const int kb = k + ks;
    if (blocked) {
      // (channel block, kh, kw, channel in block): the run shares one tap.
      const int cb = kb / KBLK;
      const int rem = kb - cb * KBLK;
      const int t = rem / kChanBlock;
      const int kh = t / KW, kw = t - (t / KW) * KW;
      const int c = cb * kChanBlock + (rem - t * kChanBlock);
      const int ih = ih0 + kh * dh, iw = iw0 + kw * dw;
      const bool valid = ok && kb < kmax && unsigned(ih) < unsigned(H) && unsigned(iw) < unsigned(W);
      const float* src = xg + (c * HW + ih * W + iw);
#pragma unroll
      for (int e = 0; e < EPT; ++e) v[e] = load_or_zero(src + e * HW, valid);
    } else {
      // (ci, kh, kw) with kw fastest.
      int ci = kb / KK;
      const int rem = kb - ci * KK;
      int kh = rem / KW;
      int kw = rem - kh * KW;
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const int ih = ih0 + kh * dh, iw = iw0 + kw * dw;
        const bool valid = ok && (kb + e) < kmax && unsigned(ih) < unsigned(H) && unsigned(iw) < unsigned(W);
        v[e] = load_or_zero(xg + ci * HW + ih * W + iw, valid);
        if (++kw == KW) {
          kw = 0;
          if (++kh == KH) {
            kh = 0;
            ++ci;
          }
        }
      }
    }
    k += kstep;
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

// rows = positions taken four at a time, k = channel: element
// base[img * cs + k * hw + q] for position (img, q).  Needs hw % 4 == 0 and a
// 16-byte aligned base so a quad of positions is one aligned 16-byte read.
// Forward B operand of an unpadded 1x1 stride-1 convolution (x, k = ci) and
// dInput B operand of an unpadded 1x1 convolution (dy, k = co).
template <int ROWS, int BK, bool DY>
struct PosQuadLoader {
  static constexpr bool KMAJOR = true;
  int kstep = BK;  // k advance per load(); the main loop may set 2 * BK
  static constexpr int TPK = ROWS / 4;        // threads per k
  static constexpr int KPP = kThreads / TPK;  // k per pass
  static constexpr int PASSES = BK / KPP;
  static_assert(PASSES >= 1 && BK % KPP == 0, "PosQuadLoader tiling");
  f32x4 v[PASSES];
  const float* ptr;
  int hw, k, kmax, kk;
  bool ok;
  __device__ __forceinline__ void init(const ConvArgs& p, int col0, int g, int k0, int kmax_) {
    const int tid = threadIdx.x;
    kk = tid / TPK;
    const float* base = DY ? p.dy + int64_t(g) * p.Cout_g * p.OHOW : p.x + int64_t(g) * p.Cin_g * p.HW;
    const int cs = DY ? p.Cout * p.OHOW : p.Cin * p.HW;
    hw = DY ? p.OHOW : p.HW;
    const int pos = col0 + 4 * (tid % TPK);
    ok = pos < p.Ncols;
    const int pp = ok ? pos : 0;
    const int img = pp / hw;
    ptr = base + int64_t(img) * cs + (pp - img * hw);
    k = k0;
    kmax = kmax_;
  }
  __device__ __forceinline__ void load() {
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      const int kx = k + kk + q * KPP;
      v[q] = load4_or_zero(ptr + int64_t(kx) * hw, ok && kx < kmax);
    }
    k += kstep;
  }
  __device__ __forceinline__ void store(float* lds) const {
    constexpr int LDR = ROWS + 4;
    const int tid = threadIdx.x;
#pragma unroll
    for (int q = 0; q < PASSES; ++q)
      *reinterpret_cast<f32x4*>(lds + (kk + q * KPP) * LDR + 4 * (tid % TPK)) = v[q];
  }
};

// dInput B operand (gather) for one stride phase: rows = phase positions
// (img, i, j), k in the gathered K order over (co, th, tw); element
// dy[img][g*Cout_g + co][i + offh0 - th*dsh][j + offw0 - tw*dsw].
template <int ROWS, int BK>
struct PhaseGatherLoader {
  static constexpr bool KMAJOR = false;
  int kstep = BK;  // k advance per load(); the main loop may set 2 * BK
  static constexpr int EPT = ROWS * BK / kThreads;
  static_assert(ROWS <= kThreads && EPT >= 1 && BK % EPT == 0 && kChanBlock % EPT == 0, "PhaseGatherLoader tiling");
  float v[EPT];
  const float* dyg;
  int ib, jb, ks, k, kmax;
  bool ok, blocked;
  int NT, KBLK, nth, ntw, dsh, dsw, OH, OW, OHOW;
  __device__ __forceinline__ void init(const ConvArgs& p, int col0, int g, int k0, int kmax_) {
    const int tid = threadIdx.x;
    const int r = tid % ROWS;
    ks = (tid / ROWS) * EPT;
    const int pos = col0 + r;
    ok = pos < p.Ncols;
    const int pp = ok ? pos : 0;
    const int img = pp / p.HpWp;
    const int q = pp - img * p.HpWp;
    const int i = q / p.Wp;
    const int j = q - i * p.Wp;
    ib = i + p.offh0;
    jb = j + p.offw0;
    dyg = p.dy + (int64_t(img) * p.Cout + int64_t(g) * p.Cout_g) * p.OHOW;
    blocked = blocked_channels(p.Cout_g);
    NT = p.nth * p.ntw;
    KBLK = NT * kChanBlock;
    nth = p.nth;
    ntw = p.ntw;
    dsh = p.dsh;
    dsw = p.dsw;
    OH = p.OH;
    OW = p.OW;
    OHOW = p.OHOW;
    k = k0;
    kmax = kmax_;
  }
  __device__ __forceinline__ void load() {
    const int kb = k + ks;
    if (blocked) {
      // (channel block, th, tw, channel in block): the run shares one tap.
      const int cb = kb / KBLK;
      const int rem = kb - cb * KBLK;
      const int t = rem / kChanBlock;
      const int th = t / ntw, tw = t - (t / ntw) * ntw;
      const int co = cb * kChanBlock + (rem - t * kChanBlock);
      const int oh = ib - th * dsh, ow = jb - tw * dsw;
      const bool valid = ok && kb < kmax && unsigned(oh) < unsigned(OH) && unsigned(ow) < unsigned(OW);
      const float* src = dyg + (co * OHOW + oh * OW + ow);
#pragma unroll
      for (int e = 0; e < EPT; ++e) v[e] = load_or_zero(src + e * OHOW, valid);
    } else {
      // (co, th, tw) with tw fastest.
      int co = kb / NT;
      const int rem = kb - co * NT;
      int th = rem / ntw;
      int tw = rem - th * ntw;
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const int oh = ib - th * dsh, ow = jb - tw * dsw;
        const bool valid = ok && (kb + e) < kmax && unsigned(oh) < unsigned(OH) && unsigned(ow) < unsigned(OW);
        v[e] = load_or_zero(dyg + co * OHOW + oh * OW + ow, valid);
        if (++tw == ntw) {
          tw = 0;
          if (++th == nth) {
            th = 0;
            ++co;
          }
        }
      }
    }
    k += kstep;
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

// dWeight operands with k = output position.  Every loader exposes the
// thread -> row map (rows tid / LPR + q * RPP) used by the dBias row sums.
//
// dy rows (A, rows = co), scalar: element dy[img][co][q]; lanes along k.
template <int ROWS, int BK>
struct DyRowsLoader {
  static constexpr bool KMAJOR = false;
  static constexpr bool DEEP = false;  // a pointer offset, flag and row sum per pass: one register set
  int kstep = BK;  // k advance per load(); the main loop may set 2 * BK
  static constexpr int LPR = BK;  // lanes per row
  static constexpr int RPP = kThreads / BK;
  static constexpr int PASSES = ROWS / RPP;
  static_assert(PASSES >= 1 && ROWS % RPP == 0, "DyRowsLoader tiling");
  float v[PASSES];
  float bsum[PASSES];
  int coff[PASSES];
  bool ok[PASSES];
  const float* dyg;
  int k, kk, kmax, OHOW, COHOW;
  __device__ __forceinline__ void init(const ConvArgs& p, int row0, int g, int k0, int kmax_) {
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
    // One register set (DEEP = false): clamped 32-bit offsets and a select.
    const int kx = k + kk;
    const bool kin = kx < kmax;
    const int kc = kin ? kx : 0;
    const int img = kc / OHOW;
    const int base = img * COHOW + (kc - img * OHOW);
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      const bool use = ok[q] && kin;
      const float t = dyg[use ? base + coff[q] : 0];
      v[q] = use ? t : 0.f;
      bsum[q] += v[q];
    }
    k += kstep;
  }
  __device__ __forceinline__ void store(float* lds) const {
    constexpr int LDK = BK + 4;
    const int tid = threadIdx.x;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) lds[(tid / BK + q * RPP) * LDK + kk] = v[q];
  }
};

// rows = channel, k = position, 16 bytes along k: element base[img*cs + row*hw + q].
// Needs hw % 4 == 0, a 16-byte aligned base and k0 % 4 == 0.  dWeight A
// operand (DY: dy, rows = co, keeps dBias row sums) and the dWeight B operand
// of an unpadded 1x1 stride-1 convolution (x, rows = ci).
template <int ROWS, int BK, bool DY>
struct PosKLoader {
  static constexpr bool KMAJOR = false;
  int kstep = BK;  // k advance per load(); the main loop may set 2 * BK
  static constexpr int LPR = BK / 4;  // lanes per row
  static constexpr int RPP = kThreads / LPR;
  static constexpr int PASSES = ROWS / RPP;
  static_assert(PASSES >= 1 && ROWS % RPP == 0, "PosKLoader tiling");
  f32x4 v[PASSES];
  float bsum[PASSES];
  int roff[PASSES];
  bool ok[PASSES];
  const float* base;
  int k, kq, kmax, hw, cs;
  __device__ __forceinline__ void init(const ConvArgs& p, int row0, int g, int k0, int kmax_) {
    const int tid = threadIdx.x;
    kq = tid % LPR;
    base = DY ? p.dy + int64_t(g) * p.Cout_g * p.OHOW : p.x + int64_t(g) * p.Cin_g * p.HW;
    cs = DY ? p.Cout * p.OHOW : p.Cin * p.HW;
    hw = DY ? p.OHOW : p.HW;
    const int R = DY ? p.Cout_g : p.Ncols;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      const int row = row0 + tid / LPR + q * RPP;
      ok[q] = row < R;
      roff[q] = ok[q] ? row * hw : 0;
      bsum[q] = 0.f;
    }
    k = k0;
    kmax = kmax_;
  }
  __device__ __forceinline__ void load() {
    const int kx = k + 4 * kq;
    const bool kin = kx < kmax;
    const int img = kx / hw;
    const float* src = base + int64_t(img) * cs + (kx - img * hw);
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      v[q] = load4_or_zero(src + roff[q], ok[q] && kin);
      if constexpr (DY) bsum[q] += (v[q][0] + v[q][1]) + (v[q][2] + v[q][3]);
    }
    k += kstep;
  }
  __device__ __forceinline__ void store(float* lds) const {
    constexpr int LDK = BK + 4;
    const int tid = threadIdx.x;
#pragma unroll
    for (int q = 0; q < PASSES; ++q)
      *reinterpret_cast<f32x4*>(lds + (tid / LPR + q * RPP) * LDK + 4 * kq) = v[q];
  }
};

// dWeight B operand (gather): rows = (ci, kh, kw), k = output position;
// element x[img][ci][oh*sh - ph + kh*dh][ow*sw - pw + kw*dw].
template <int ROWS, int BK>
struct XColsLoader {
  static constexpr bool KMAJOR = false;
  static constexpr bool DEEP = false;  // three per-pass offsets: one register set
  int kstep = BK;  // k advance per load(); the main loop may set 2 * BK
  static constexpr int RPP = kThreads / BK;
  static constexpr int PASSES = ROWS / RPP;
  static_assert(PASSES >= 1 && ROWS % RPP == 0, "XColsLoader tiling");
  float v[PASSES];
  int coff[PASSES];
  int khd[PASSES];
  int kwd[PASSES];
  const float* xg;
  int k, kk, kmax, OHOW, OW, sh, sw, H, W, CHW;
  __device__ __forceinline__ void init(const ConvArgs& p, int col0, int g, int k0, int kmax_) {
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
    // One register set (DEEP = false): clamped 32-bit offsets and a select.
    const int kx = k + kk;
    const bool kin = kx < kmax;
    const int kc = kin ? kx : 0;
    const int img = kc / OHOW;
    const int q0 = kc - img * OHOW;
    const int oh = q0 / OW;
    const int ow = q0 - oh * OW;
    const int ihb = oh * sh, iwb = ow * sw;
    const float* xi = xg + int64_t(img) * CHW;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      const int ih = ihb + khd[q], iw = iwb + kwd[q];
      const bool valid = kin && unsigned(ih) < unsigned(H) && unsigned(iw) < unsigned(W);
      const float t = xi[valid ? coff[q] + ih * W + iw : 0];
      v[q] = valid ? t : 0.f;
    }
    k += kstep;
  }
  __device__ __forceinline__ void store(float* lds) const {
    constexpr int LDK = BK + 4;
    const int tid = threadIdx.x;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) lds[(tid / BK + q * RPP) * LDK + kk] = v[q];
  }
};

// ------------------------------------------------------------------ tiles
// Tile menu (BM x BN x BK, wave grid rows, waves per SIMD).
using TileTall = Cfg<256, 128, 16, 2, 2>;   // 4 waves of 128 x 64
using TileWide = Cfg<128, 256, 16, 2, 2>;   // 4 waves of 64 x 128
using TileSq = Cfg<128, 128, 16, 2, 2>;     // 4 waves of 64 x 64
using TileFlat = Cfg<64, 256, 16, 1, 2>;    // 4 waves of 64 x 64 in a row
using TileNarrow = Cfg<256, 64, 16, 4, 2>;  // 4 waves of 64 x 64 in a column
using TileSmall = Cfg<64, 64, 32, 2, 4>;    // 4 waves of 32 x 32, 32-deep slabs
enum Tile : int { TALL = 0, WIDE, SQ, FLAT, NARROW, SMALL, NTILES };

// Operand modes the launchers dispatch on.
enum BMode : int { B_GATHER = 0, B_VEC = 1 };

int conv_fwd_launch(const ConvArgs& p, int tile, Mode ma, int bmode, hipStream_t s);
int conv_dx_launch(const ConvArgs& p, int tile, Mode ma, int bmode, hipStream_t s);
int conv_dw_launch(const ConvArgs& p, int tile, int amode, int bmode, hipStream_t s);
int conv_dx_pack_weights(const ConvArgs& p, float* wt, hipStream_t s);
int conv_fwd_pack_weights(const ConvArgs& p, float* wt, hipStream_t s);
int conv_dx_zero_phase(const ConvArgs& p, hipStream_t s);
int conv_dw_finalize(const ConvArgs& p, float* dw, float* db, hipStream_t s);
// out[i] = sum over splits of ws[split][i] (+ bias[(i / hw) % cout] when bias).
int conv_sum_splits(const float* ws, int splits, int64_t n, float* out, const float* bias, int hw, int cout,
                    hipStream_t s);

}  // namespace conv
}  // namespace mx
