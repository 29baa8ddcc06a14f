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
  int ldw;          // forward: row pitch of wt in floats (K, or K rounded up to 4 in a padded copy)
  // dInput, stride 2 x 2 with only phase (0, 0) reached (a 1x1 stride-2
  // layer): each phase output also writes the three unreached positions of
  // its 2x2 input block as zeros (8-byte stores), in place of a separate fill.
  int zfill;
  // Split-K partials (splits > 1): forward / dInput write their tile to
  // ws + split * out_elems at the output's own offsets; dWeight writes
  // [split][G*Cout_g][Cin_g*KK] and the dBias partials to ws_db [split][Cout].
  float* ws;
  float* ws_db;
  int64_t out_elems;
  // Per-lane divisions of the loaders' inner loops: position -> image
  // (OH*OW), row (OW) and, for the 16-byte k loaders, image of a k index (hw
  // of the operand read along k).
  FastDiv f_ohow, f_ow, f_hw;
  // Blocked K walk of the forward / dInput gathers: k -> (channel block,
  // tap) by taps * kChanBlock, tap -> (row, column) by the tap-grid width
  // (forward: KK * 16 and KW; dInput phase: nth * ntw * 16 and ntw).
  FastDiv f_kblk, f_tapw;
  FastDiv f_kk;  // non-blocked gathers: taps per channel (forward KK, dInput phase nth * ntw)
  // dWeight: the B gather runs its columns in the channel-blocked order
  // (channel block, kh, kw, channel in block); the epilogue maps them back.
  int cols_blocked;
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
// All activation operands are read through buffer resources (mfma_core.hpp):
// a lane computes one 32-bit byte offset per run of elements (kOffNone when
// masked, which reads zeros), the run's stride is a scalar offset, and no
// instruction touches a loaded value before store() writes it to LDS, so the
// loads of the next slabs stay in flight behind the MFMAs.  K decompositions
// that are the same for a whole wave are made wave-uniform
// (readfirstlane) and run on the scalar unit.

__device__ __forceinline__ int wave_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Forward B operand (gather): rows = output positions (img, oh, ow), k in
// the gathered K order over (ci, kh, kw); element
// x[img][g*Cin_g + ci][oh*sh - ph + kh*dh][ow*sw - pw + kw*dw].  Each thread
// holds EPT consecutive k of one position; a wave's 64 threads share their
// k run (ROWS is a multiple of 64), so the (ci, kh, kw) walk is scalar.
template <int ROWS, int BK, bool BLOCKED>
struct Im2colLoader {
  static constexpr bool KMAJOR = false;
  int kstep = BK;  // k advance per load(); the main loop may set 2 * BK
  static constexpr int EPT = ROWS * BK / kThreads;
  static_assert(ROWS % 64 == 0 && ROWS <= kThreads && EPT >= 1 && BK % EPT == 0 && kChanBlock % EPT == 0,
                "Im2colLoader tiling");
  float v[EPT];
  i32x4 rs;
  uint32_t xoff;  // bytes to (img, first channel of the group, 0, 0)
  int ih0, iw0, ks, k, kmax;
  bool ok;
  FastDiv f_kblk, f_kw, f_kk;
  int KK, KBLK, KH, KW, dh, dw, H, W, HW;
  __device__ __forceinline__ void init(const ConvArgs& p, int col0, int g, int k0, int kmax_) {
    const int tid = threadIdx.x;
    const int r = tid % ROWS;
    ks = wave_uniform((tid / ROWS) * EPT);
    const int pos = col0 + r;
    ok = pos < p.Ncols;
    const int pp = ok ? pos : 0;
    const int img = pp / p.OHOW;
    const int q = pp - img * p.OHOW;
    const int oh = q / p.OW;
    const int ow = q - oh * p.OW;
    ih0 = ok ? oh * p.sh - p.ph : INT_MIN / 2;  // fails every bounds test
    iw0 = ow * p.sw - p.pw;
    xoff = uint32_t((int64_t(img) * p.Cin + int64_t(g) * p.Cin_g) * p.HW * 4);
    rs = buffer_rsrc(p.x, int64_t(p.N) * p.Cin * p.HW * 4);
    f_kblk = p.f_kblk;
    f_kw = p.f_tapw;
    f_kk = p.f_kk;
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
    const int kb = k + ks;  // wave-uniform
    if constexpr (BLOCKED) {
      // (channel block, kh, kw, channel in block): the run shares one tap.
      const int cb = int(fdiv(uint32_t(kb), f_kblk));
      const int rem = kb - cb * KBLK;
      const int t = rem / kChanBlock;
      const int kh = int(fdiv(uint32_t(t), f_kw));
      const int kw = t - kh * KW;
      const int c = cb * kChanBlock + (rem - t * kChanBlock);
      const int ih = ih0 + kh * dh, iw = iw0 + kw * dw;
      const bool valid = (kb < kmax) & (unsigned(ih) < unsigned(H)) & (unsigned(iw) < unsigned(W));
      const uint32_t voff = valid ? xoff + uint32_t(ih * W + iw) * 4u : kOffNone;
      const uint32_t s0 = uint32_t(c) * uint32_t(HW) * 4u;
#pragma unroll
      for (int e = 0; e < EPT; ++e) v[e] = bload(rs, voff, s0 + uint32_t(e * HW) * 4u);
    } else {
      // (ci, kh, kw) with kw fastest, decomposed per element by multiply-high
      // divisions of the wave-uniform k on the scalar unit (readfirstlane
      // keeps it there: a channel offset the compiler thinks divergent turns
      // each load into a loop over distinct values).  Out-of-range positions
      // carry ih0 far below zero, so one bounds test covers them and nothing
      // branches.
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const int ke = wave_uniform(kb + e);
        const int ci = int(fdiv(uint32_t(ke), f_kk));
        const int rem = ke - ci * KK;
        const int kh = int(fdiv(uint32_t(rem), f_kw));
        const int kw = rem - kh * KW;
        const int ih = ih0 + kh * dh, iw = iw0 + kw * dw;
        const bool valid = (ke < kmax) & (unsigned(ih) < unsigned(H)) & (unsigned(iw) < unsigned(W));
        v[e] = bload(rs, valid ? xoff + uint32_t(ih * W + iw) * 4u : kOffNone, uint32_t(ci) * uint32_t(HW) * 4u);
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
  i32x4 rs;
  uint32_t voff, hw4;
  int k, kmax, kk;
  __device__ __forceinline__ void init(const ConvArgs& p, int col0, int g, int k0, int kmax_) {
    const int tid = threadIdx.x;
    kk = tid / TPK;
    const int cs = DY ? p.Cout * p.OHOW : p.Cin * p.HW;
    const int hw = DY ? p.OHOW : p.HW;
    const int64_t gbase = DY ? int64_t(g) * p.Cout_g * p.OHOW : int64_t(g) * p.Cin_g * p.HW;
    rs = buffer_rsrc(DY ? p.dy : p.x, int64_t(p.N) * cs * 4);
    const int pos = col0 + 4 * (tid % TPK);
    const bool ok = pos < p.Ncols;
    const int pp = ok ? pos : 0;
    const int img = pp / hw;
    voff = ok ? uint32_t((gbase + int64_t(img) * cs + (pp - img * hw) + int64_t(kk) * hw) * 4) : kOffNone;
    hw4 = uint32_t(hw) * 4u;
    k = k0;
    kmax = kmax_;
  }
  __device__ __forceinline__ void load() {
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      const int kx = k + kk + q * KPP;
      v[q] = bload4(rs, kx < kmax ? voff : kOffNone, uint32_t(k + q * KPP) * hw4);
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
// dy[img][g*Cout_g + co][i + offh0 - th*dsh][j + offw0 - tw*dsw].  The k run
// of a wave is shared, as in Im2colLoader.
template <int ROWS, int BK, bool BLOCKED>
struct PhaseGatherLoader {
  static constexpr bool KMAJOR = false;
  int kstep = BK;  // k advance per load(); the main loop may set 2 * BK
  static constexpr int EPT = ROWS * BK / kThreads;
  static_assert(ROWS % 64 == 0 && ROWS <= kThreads && EPT >= 1 && BK % EPT == 0 && kChanBlock % EPT == 0,
                "PhaseGatherLoader tiling");
  float v[EPT];
  i32x4 rs;
  uint32_t doff;  // bytes to (img, first channel of the group, 0, 0)
  int ib, jb, ks, k, kmax;
  bool ok;
  FastDiv f_kblk, f_tw, f_nt;
  int NT, KBLK, nth, ntw, dsh, dsw, OH, OW, OHOW;
  __device__ __forceinline__ void init(const ConvArgs& p, int col0, int g, int k0, int kmax_) {
    const int tid = threadIdx.x;
    const int r = tid % ROWS;
    ks = wave_uniform((tid / ROWS) * EPT);
    const int pos = col0 + r;
    ok = pos < p.Ncols;
    const int pp = ok ? pos : 0;
    const int img = pp / p.HpWp;
    const int q = pp - img * p.HpWp;
    const int i = q / p.Wp;
    const int j = q - i * p.Wp;
    ib = ok ? i + p.offh0 : INT_MIN / 2;  // fails every bounds test
    jb = j + p.offw0;
    doff = uint32_t((int64_t(img) * p.Cout + int64_t(g) * p.Cout_g) * p.OHOW * 4);
    rs = buffer_rsrc(p.dy, int64_t(p.N) * p.Cout * p.OHOW * 4);
    f_kblk = p.f_kblk;
    f_tw = p.f_tapw;
    f_nt = p.f_kk;
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
    const int kb = k + ks;  // wave-uniform
    if constexpr (BLOCKED) {
      // (channel block, th, tw, channel in block): the run shares one tap.
      const int cb = int(fdiv(uint32_t(kb), f_kblk));
      const int rem = kb - cb * KBLK;
      const int t = rem / kChanBlock;
      const int th = int(fdiv(uint32_t(t), f_tw));
      const int tw = t - th * ntw;
      const int co = cb * kChanBlock + (rem - t * kChanBlock);
      const int oh = ib - th * dsh, ow = jb - tw * dsw;
      const bool valid = (kb < kmax) & (unsigned(oh) < unsigned(OH)) & (unsigned(ow) < unsigned(OW));
      const uint32_t voff = valid ? doff + uint32_t(oh * OW + ow) * 4u : kOffNone;
      const uint32_t s0 = uint32_t(co) * uint32_t(OHOW) * 4u;
#pragma unroll
      for (int e = 0; e < EPT; ++e) v[e] = bload(rs, voff, s0 + uint32_t(e * OHOW) * 4u);
    } else {
      // (co, th, tw) with tw fastest, decomposed per element from the
      // wave-uniform k on the scalar unit; out-of-range positions carry ib far
      // below zero, so nothing branches.
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const int ke = wave_uniform(kb + e);
        const int co = int(fdiv(uint32_t(ke), f_nt));
        const int rem = ke - co * NT;
        const int th = int(fdiv(uint32_t(rem), f_tw));
        const int tw = rem - th * ntw;
        const int oh = ib - th * dsh, ow = jb - tw * dsw;
        const bool valid = (ke < kmax) & (unsigned(oh) < unsigned(OH)) & (unsigned(ow) < unsigned(OW));
        v[e] = bload(rs, valid ? doff + uint32_t(oh * OW + ow) * 4u : kOffNone, uint32_t(co) * uint32_t(OHOW) * 4u);
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
// thread -> row map (rows tid / LPR + q * RPP) used by the dBias row sums,
// which store() accumulates (after the loads have landed).
//
// dy rows (A, rows = co), scalar: element dy[img][co][q]; lanes along k.
template <int ROWS, int BK>
struct DyRowsLoader {
  static constexpr bool KMAJOR = false;
  int kstep = BK;  // k advance per load(); the main loop may set 2 * BK
  static constexpr int LPR = BK;  // lanes per row
  static constexpr int RPP = kThreads / BK;
  static constexpr int PASSES = ROWS / RPP;
  static_assert(PASSES >= 1 && ROWS % RPP == 0, "DyRowsLoader tiling");
  float v[PASSES];
  mutable float bsum[PASSES];
  bool rok[PASSES];
  i32x4 rs;
  uint32_t roff, pass4, cohow4;
  FastDiv f_ohow;
  int k, kk, kmax, OHOW;
  __device__ __forceinline__ void init(const ConvArgs& p, int row0, int g, int k0, int kmax_) {
    const int tid = threadIdx.x;
    kk = tid % BK;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      rok[q] = row0 + tid / BK + q * RPP < p.Cout_g;
      bsum[q] = 0.f;
    }
    rs = buffer_rsrc(p.dy, int64_t(p.N) * p.Cout * p.OHOW * 4);
    roff = uint32_t((int64_t(g) * p.Cout_g + row0 + tid / BK) * p.OHOW * 4);
    pass4 = uint32_t(RPP) * uint32_t(p.OHOW) * 4u;
    cohow4 = uint32_t(p.Cout) * uint32_t(p.OHOW) * 4u;
    f_ohow = p.f_ohow;
    OHOW = p.OHOW;
    k = k0;
    kmax = kmax_;
  }
  __device__ __forceinline__ void load() {
    const int kx = k + kk;
    const bool kin = kx < kmax;
    const uint32_t img = fdiv(uint32_t(kx), f_ohow);
    const uint32_t base = kin ? img * cohow4 + roff + (uint32_t(kx) - img * uint32_t(OHOW)) * 4u : kOffNone;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) v[q] = bload(rs, rok[q] ? base : kOffNone, uint32_t(q) * pass4);
    k += kstep;
  }
  __device__ __forceinline__ void store(float* lds) const {
    constexpr int LDK = BK + 4;
    const int tid = threadIdx.x;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      lds[(tid / BK + q * RPP) * LDK + kk] = v[q];
      bsum[q] += v[q];
    }
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
  mutable float bsum[PASSES];
  bool rok[PASSES];
  i32x4 rs;
  uint32_t roff, pass4, cs4;
  FastDiv f_hw;
  int k, kq, kmax, hw;
  __device__ __forceinline__ void init(const ConvArgs& p, int row0, int g, int k0, int kmax_) {
    const int tid = threadIdx.x;
    kq = tid % LPR;
    const int cs = DY ? p.Cout * p.OHOW : p.Cin * p.HW;
    hw = DY ? p.OHOW : p.HW;
    const int64_t gbase = DY ? int64_t(g) * p.Cout_g : int64_t(g) * p.Cin_g;
    f_hw = DY ? p.f_ohow : p.f_hw;
    const int R = DY ? p.Cout_g : p.Ncols;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      rok[q] = row0 + tid / LPR + q * RPP < R;
      bsum[q] = 0.f;
    }
    rs = buffer_rsrc(DY ? p.dy : p.x, int64_t(p.N) * cs * 4);
    roff = uint32_t((gbase + row0 + tid / LPR) * hw * 4);
    pass4 = uint32_t(RPP) * uint32_t(hw) * 4u;
    cs4 = uint32_t(cs) * 4u;
    k = k0;
    kmax = kmax_;
  }
  __device__ __forceinline__ void load() {
    const int kx = k + 4 * kq;
    const bool kin = kx < kmax;
    const uint32_t img = fdiv(uint32_t(kx), f_hw);
    const uint32_t base = kin ? img * cs4 + roff + (uint32_t(kx) - img * uint32_t(hw)) * 4u : kOffNone;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) v[q] = bload4(rs, rok[q] ? base : kOffNone, uint32_t(q) * pass4);
    k += kstep;
  }
  __device__ __forceinline__ void store(float* lds) const {
    constexpr int LDK = BK + 4;
    const int tid = threadIdx.x;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) {
      *reinterpret_cast<f32x4*>(lds + (tid / LPR + q * RPP) * LDK + 4 * kq) = v[q];
      if constexpr (DY) bsum[q] += (v[q][0] + v[q][1]) + (v[q][2] + v[q][3]);
    }
  }
};

// dWeight B operand (gather): rows = (ci, kh, kw), k = output position;
// element x[img][ci][oh*sh - ph + kh*dh][ow*sw - pw + kw*dw].  Lanes run along
// k (one position each); a thread's PASSES rows are consecutive.  With a
// channel count that is a multiple of kChanBlock the rows are taken in the
// channel-blocked order (channel block, kh, kw, channel in block), so a
// thread's rows share one tap: one bounds test and one offset, the channels a
// plane apart in the scalar offset (ConvArgs::cols_blocked tells the epilogue
// to map the columns back).  Other channel counts test each row.
template <int ROWS, int BK, bool BLOCKED>
struct XColsLoader {
  static constexpr bool KMAJOR = false;
  // Per-row offsets of the plain order leave room for one register set only.
  static constexpr bool DEEP = BLOCKED;
  int kstep = BK;  // k advance per load(); the main loop may set 2 * BK
  static constexpr int RPP = kThreads / BK;
  static constexpr int PASSES = ROWS / RPP;
  static constexpr int NR = BLOCKED ? 1 : PASSES;  // rows with their own tap / channel
  static_assert(PASSES >= 1 && ROWS % RPP == 0 && kChanBlock % PASSES == 0, "XColsLoader tiling");
  float v[PASSES];
  i32x4 rs;
  uint32_t coff[NR];  // bytes to the row's channel plane (blocked: the run's first channel)
  int khd[NR], kwd[NR];
  FastDiv f_ohow, f_ow;
  uint32_t chw4, hw4;
  int k, kk, kmax, OHOW, OW, sh, sw, H, W;
  __device__ __forceinline__ void init(const ConvArgs& p, int col0, int g, int k0, int kmax_) {
    const int tid = threadIdx.x;
    kk = tid % BK;
    const int n0 = col0 + (tid / BK) * PASSES;
    if constexpr (BLOCKED) {
      // The PASSES rows n0.. lie in one 16-channel block and share tap t.
      const int kblk = p.KK * kChanBlock;
      const int cb = n0 / kblk, rem = n0 - cb * kblk;
      const int t = rem / kChanBlock;
      const int ci0 = cb * kChanBlock + (rem - t * kChanBlock);
      const int kh = t / p.KW, kw = t - (t / p.KW) * p.KW;
      coff[0] = uint32_t((int64_t(g) * p.Cin_g + ci0) * p.HW * 4);
      // A run past the last column gets a tap offset that always fails the bounds test.
      khd[0] = n0 < p.Ncols ? kh * p.dh - p.ph : INT_MIN / 2;
      kwd[0] = kw * p.dw - p.pw;
    } else {
#pragma unroll
      for (int q = 0; q < PASSES; ++q) {
        const int n = n0 + q;
        const bool ok = n < p.Ncols;
        const int nn = ok ? n : 0;
        const int ci = nn / p.KK;
        const int r = nn - ci * p.KK;
        const int kh = r / p.KW;
        const int kw = r - kh * p.KW;
        coff[q] = uint32_t((int64_t(g) * p.Cin_g + ci) * p.HW * 4);
        khd[q] = ok ? kh * p.dh - p.ph : INT_MIN / 2;
        kwd[q] = kw * p.dw - p.pw;
      }
    }
    rs = buffer_rsrc(p.x, int64_t(p.N) * p.Cin * p.HW * 4);
    f_ohow = p.f_ohow;
    f_ow = p.f_ow;
    chw4 = uint32_t(p.Cin) * uint32_t(p.HW) * 4u;
    hw4 = uint32_t(p.HW) * 4u;
    OHOW = p.OHOW;
    OW = p.OW;
    sh = p.sh;
    sw = p.sw;
    H = p.H;
    W = p.W;
    k = k0;
    kmax = kmax_;
  }
  __device__ __forceinline__ void load() {
    const int kx = k + kk;
    const bool kin = kx < kmax;
    const uint32_t img = fdiv(uint32_t(kx), f_ohow);
    const uint32_t q0 = uint32_t(kx) - img * uint32_t(OHOW);
    const uint32_t oh = fdiv(q0, f_ow);
    const int ihb = int(oh) * sh, iwb = int(q0 - oh * uint32_t(OW)) * sw;
    const uint32_t ibase = img * chw4;
    if constexpr (BLOCKED) {
      const int ih = ihb + khd[0], iw = iwb + kwd[0];
      const bool valid = kin && unsigned(ih) < unsigned(H) && unsigned(iw) < unsigned(W);
      const uint32_t voff = valid ? ibase + coff[0] + uint32_t(ih * W + iw) * 4u : kOffNone;
#pragma unroll
      for (int q = 0; q < PASSES; ++q) v[q] = bload(rs, voff, uint32_t(q) * hw4);
    } else {
#pragma unroll
      for (int q = 0; q < PASSES; ++q) {
        const int ih = ihb + khd[q], iw = iwb + kwd[q];
        const bool valid = kin && unsigned(ih) < unsigned(H) && unsigned(iw) < unsigned(W);
        v[q] = bload(rs, valid ? ibase + coff[q] + uint32_t(ih * W + iw) * 4u : kOffNone, 0u);
      }
    }
    k += kstep;
  }
  __device__ __forceinline__ void store(float* lds) const {
    constexpr int LDK = BK + 4;
    const int tid = threadIdx.x;
#pragma unroll
    for (int q = 0; q < PASSES; ++q) lds[((tid / BK) * PASSES + q) * LDK + kk] = v[q];
  }
};

// ------------------------------------------------------------------ tiles
// Tile menu (BM x BN x BK, wave grid rows, waves per SIMD).
using TileTall = Cfg<256, 128, 16, 2, 2>;   // 4 waves of 128 x 64
using TileWide = Cfg<128, 256, 16, 2, 2>;   // 4 waves of 64 x 128
using TileSq = Cfg<128, 128, 16, 2, 2>;     // 4 waves of 64 x 64
using TileFlat = Cfg<64, 256, 16, 1, 2>;    // 4 waves of 64 x 64 in a row
using TileNarrow = Cfg<256, 64, 16, 4, 2>;  // 4 waves of 64 x 64 in a column
using TileSmall = Cfg<64, 64, 32, 2, 4>;    // 4 waves of 32 x 32, 32-deep slabs (dWeight)
// Forward and dInput run the small tile with 16-deep slabs: half the LDS and
// load registers, so five workgroups fit a CU instead of four (measured on
// the ResNet-50 layers: 1x1 forwards and input gradients 2-15% faster; the
// weight gradients, whose K runs over positions, are faster with 32-deep
// slabs).
using TileSmallShallow = Cfg<64, 64, 16, 2, 5>;
enum Tile : int { TALL = 0, WIDE, SQ, FLAT, NARROW, SMALL, NTILES };

// Operand modes the launchers dispatch on.
enum BMode : int { B_GATHER = 0, B_VEC = 1 };

int conv_fwd_launch(const ConvArgs& p, int tile, Mode ma, int bmode, hipStream_t s);
int conv_dx_launch(const ConvArgs& p, int tile, Mode ma, int bmode, hipStream_t s);
// Up to kMaxFusedPhases stride phases of one dInput (same tile, loaders and
// split count) in one launch.
constexpr int kMaxFusedPhases = 4;
struct DxPhaseSet {
  ConvArgs q[kMaxFusedPhases];
  int n, G;
};
int conv_dx_launch_set(const DxPhaseSet& set, int tile, Mode ma, int bmode, hipStream_t s);
int conv_dw_launch(const ConvArgs& p, int tile, int amode, int bmode, hipStream_t s);
// Weight packing of several dInput stride phases in one launch.
constexpr int kMaxPackPhases = 16;
struct DxPackPhase {
  int K, nth, ntw, kh0, kw0, stph, stpw;
  uint32_t off;  // floats from the packed buffer's start
};
struct DxPackSet {
  int n;
  DxPackPhase ph[kMaxPackPhases];
};
int conv_dx_pack_weights(const ConvArgs& p, const DxPackSet& set, float* wt, hipStream_t s);
int conv_fwd_pack_weights(const ConvArgs& p, float* wt, hipStream_t s);
int conv_fwd_pad_weights(const ConvArgs& p, float* wt, hipStream_t s);
int conv_dx_zero(float* dx, int64_t n, hipStream_t s);
int conv_dw_finalize(const ConvArgs& p, float* dw, float* db, hipStream_t s);
// out[i] = sum over splits of ws[split][i] (+ bias[(i / hw) % cout] when bias).
int conv_sum_splits(const float* ws, int splits, int64_t n, float* out, const float* bias, int hw, int cout,
                    hipStream_t s);
// out[i] = sum of ws[split][i] over the splits in a fixed order (the dWeight
// finalize: 64 elements per workgroup, four interleaved phases of splits),
// for few elements over many splits.
int sum_partials(const float* ws, int splits, int64_t n, float* out, hipStream_t s);
// The same for two arrays of partials in one launch: ws [splits][n] into
// out and ws_db [splits][n_db] into out_db.
int sum_partials(const float* ws, const float* ws_db, int splits, int64_t n, int n_db, float* out, float* out_db,
                 hipStream_t s);

}  // namespace conv
}  // namespace mx
