// FP32 MFMA tile machinery for gfx950 (CDNA4), shared by the GEMM and the
// implicit-GEMM convolution kernels.
//
// A 256-thread workgroup (4 wave64) computes a BM x BN tile of C = A x B.
// Operands are staged through LDS in double-buffered BK slabs.  Each operand
// loader chooses its LDS layout: row-major with k contiguous ([row][BK + 4])
// or k-major with rows contiguous ([k][ROWS + 4]), whichever its global
// reads can fill with conflict-free 16-byte LDS stores (a row-contiguous
// operand written row-major would be a strided transpose).  Each wave owns a
// (BM/WAVES_M) x (BN/WAVES_N) sub-tile built from 32x32 blocks of
// v_mfma_f32_32x32x2f32.  Inside a slab the k index is permuted so that lane
// half h (lane / 32) handles k in [h*BK/2, (h+1)*BK/2): from a row-major
// stage a lane fetches its BK/2 operand values with ds_read_b128, from a
// k-major stage with one ds_read_b32 per k (32 consecutive rows per half
// wave), and the A/B fragments stay consistent because both use the same
// permutation.  Summation order within a 32x32 block is the MFMA's own (FP32
// accumulate).
//
// Cfg::OCC is the register budget in waves per SIMD the kernels are compiled
// for (amdgpu_waves_per_eu): 2 keeps a 128 x 128 tile in 256 registers so two
// workgroups share a CU and hide each other's slab-load latency.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mx {
namespace mfma {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;

template <int BM_, int BN_, int BK_, int WAVES_M_, int OCC_ = 2>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, OCC = OCC_;
  static constexpr int WAVES_M = WAVES_M_, WAVES_N = 4 / WAVES_M_;
  static constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
  static constexpr int FM = WTM / 32, FN = WTN / 32;
  static constexpr int PAD = 4;
  static constexpr int LDK = BK + PAD;
  static constexpr int KH = BK / 2;
  // A stage holds either layout: [rows][BK + PAD] or [BK][rows + PAD].
  static constexpr int A_STAGE = (BM * LDK > BK * (BM + PAD)) ? BM * LDK : BK * (BM + PAD);
  static constexpr int B_STAGE = (BN * LDK > BK * (BN + PAD)) ? BN * LDK : BK * (BN + PAD);
  static constexpr int SMEM_FLOATS = 2 * (A_STAGE + B_STAGE);
  static constexpr int ACC_REGS = FM * FN * 16;
  static_assert(WAVES_M * WAVES_N == 4, "4 waves per workgroup");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32");
  static_assert(BK % 8 == 0, "BK must be a multiple of 8");
};

// Qualifiers of a tile kernel compiled for configuration C.
#define MX_TILE_KERNEL(C) \
  __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(C::OCC, C::OCC)))

template <class C>
struct Acc {
  f32x16 v[C::FM][C::FN];
};

// Branch-free guarded loads: a masked element reads a zero from kZeroPage
// instead of its own address, so the loop has no control flow and no
// instruction touches a loaded value before it is stored to LDS one slab
// later.  (A branch or a select right after the load makes the compiler wait
// for every load in flight, prefetched slabs included.)
static __device__ __attribute__((aligned(16))) float kZeroPage[4];  // zero-initialised, never written

__device__ __forceinline__ float load_or_zero(const float* p, bool ok) { return *(ok ? p : kZeroPage); }
__device__ __forceinline__ f32x4 load4_or_zero(const float* p, bool ok) {
  return *reinterpret_cast<const f32x4*>(ok ? p : kZeroPage);
}

// Raw buffer loads.  An operand tensor becomes one buffer resource (base,
// byte extent) held in scalar registers; a lane supplies a 32-bit byte offset
// and the per-element stride goes in the scalar offset, so a run of loads
// costs no vector ALU work beyond its first offset.  The hardware range check
// returns zero for an offset at or past the extent: a masked lane uses
// kOffNone, which needs every operand to end below 2^31 bytes (kBufMaxBytes,
// enforced by the host, which splits larger batches).
typedef int i32x4 __attribute__((ext_vector_type(4)));
extern "C" __device__ float mx_raw_buffer_load_f32(i32x4 rsrc, int voffset, int soffset, int aux) __asm(
    "llvm.amdgcn.raw.buffer.load.f32");
extern "C" __device__ f32x4 mx_raw_buffer_load_v4f32(i32x4 rsrc, int voffset, int soffset, int aux) __asm(
    "llvm.amdgcn.raw.buffer.load.v4f32");
typedef float f32x2 __attribute__((ext_vector_type(2)));
extern "C" __device__ f32x2 mx_raw_buffer_load_v2f32(i32x4 rsrc, int voffset, int soffset, int aux) __asm(
    "llvm.amdgcn.raw.buffer.load.v2f32");
// Vector-memory store through the same resource: a store at an offset past
// the extent (kOffNone) is dropped by the range check.
extern "C" __device__ void mx_raw_buffer_store_f32(float v, i32x4 rsrc, int voffset, int soffset, int aux) __asm(
    "llvm.amdgcn.raw.buffer.store.f32");

constexpr uint32_t kOffNone = 0x80000000u;
constexpr int64_t kBufMaxBytes = 0x7FFF0000;

// Word 3 = 0x00020000: 32-bit data format, raw (stride 0) addressing.
__device__ __forceinline__ i32x4 buffer_rsrc(const void* base, int64_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r.x = __builtin_amdgcn_readfirstlane(int(uint32_t(a)));
  r.y = __builtin_amdgcn_readfirstlane(int(uint32_t(a >> 32) & 0xFFFFu));
  r.z = __builtin_amdgcn_readfirstlane(int(uint32_t(bytes)));
  r.w = 0x00020000;
  return r;
}
__device__ __forceinline__ float bload(const i32x4& r, uint32_t voff, uint32_t soff) {
  return mx_raw_buffer_load_f32(r, int(voff), int(soff), 0);
}
__device__ __forceinline__ f32x4 bload4(const i32x4& r, uint32_t voff, uint32_t soff) {
  return mx_raw_buffer_load_v4f32(r, int(voff), int(soff), 0);
}
__device__ __forceinline__ f32x2 bload2(const i32x4& r, uint32_t voff, uint32_t soff) {
  return mx_raw_buffer_load_v2f32(r, int(voff), int(soff), 0);
}
__device__ __forceinline__ void bstore(float v, const i32x4& r, uint32_t voff, uint32_t soff) {
  mx_raw_buffer_store_f32(v, r, int(voff), int(soff), 0);
}

// n / d for n < 2^31 by multiply-high (m, l from fast_div(d) on the host):
// (umulhi(n, m) + n) >> l with l = ceil(log2 d), m = 2^32 (2^l - d) / d + 1.
struct FastDiv {
  uint32_t m;
  uint32_t l;
};
inline FastDiv fast_div(uint32_t d) {
  uint32_t l = 0;
  while ((uint64_t(1) << l) < d) ++l;
  const uint64_t m = ((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1;
  return FastDiv{uint32_t(m), l};
}
__device__ __forceinline__ uint32_t fdiv(uint32_t n, FastDiv f) { return (__umulhi(n, f.m) + n) >> f.l; }

// Row (within one pass) of the 16-byte chunk thread `tid` moves for a
// row-major stage with TPR threads per row.  With four threads per row, LDS
// serves a 16-byte store eight lanes at a time over 32 banks: rows r and r + 1
// at a 20-float pitch overlap in four banks, rows r and r + 4 sit 16 banks
// apart.  Swapping bits 0 and 2 of the row index pairs rows r and r + 4 in
// each group of eight lanes; global coalescing is unchanged (four lanes still
// read 64 contiguous bytes of one row).
template <int TPR>
__device__ __forceinline__ int kvec_row(int tid) {
  const int j = tid / TPR;
  if constexpr (TPR == 4) return (j & ~5) | ((j & 1) << 2) | ((j >> 2) & 1);
  return j;
}

template <class C>
__device__ __forceinline__ void acc_zero(Acc<C>& acc) {
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc.v[i][j][r] = 0.f;
}

// Operand fragment for one 32-row block: the KH k values (this lane's half of
// the slab) of row `row` of a stage in either layout.
template <class C, int ROWS, bool KMAJOR>
__device__ __forceinline__ void load_frag(float (&f)[C::KH], const float* stage, int row, int h) {
  if constexpr (KMAJOR) {
    constexpr int LDR = ROWS + C::PAD;
    const float* src = stage + h * C::KH * LDR + row;
#pragma unroll
    for (int q = 0; q < C::KH; ++q) f[q] = src[q * LDR];
  } else {
    const float* src = stage + row * C::LDK + h * C::KH;
#pragma unroll
    for (int q = 0; q < C::KH; q += 4) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(src + q);
      f[q + 0] = t[0];
      f[q + 1] = t[1];
      f[q + 2] = t[2];
      f[q + 3] = t[3];
    }
  }
}

// One BK slab: fragments from LDS, BK/2 MFMA steps per 32x32 block.
template <class C, bool KMA, bool KMB>
__device__ __forceinline__ void mma_slab(Acc<C>& acc, const float* As, const float* Bs, int wm,
                                         int wn, int lane) {
  const int r = lane & 31, h = lane >> 5;
  float a[C::FM][C::KH];
  float b[C::FN][C::KH];
#pragma unroll
  for (int i = 0; i < C::FM; ++i) load_frag<C, C::BM, KMA>(a[i], As, wm * C::WTM + i * 32 + r, h);
#pragma unroll
  for (int j = 0; j < C::FN; ++j) load_frag<C, C::BN, KMB>(b[j], Bs, wn * C::WTN + j * 32 + r, h);
  // All fragment reads are in flight before the first MFMA; the MFMAs then
  // wait only on their own operands (LDS returns in order).
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < C::KH; ++s)
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN; ++j)
        acc.v[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s], b[j][s], acc.v[i][j], 0, 0, 0);
}

// Loaders that keep per-thread row sums (dBias) add those of a second copy.
template <class L>
__device__ __forceinline__ auto merge_row_sums(L& a, const L& b, int) -> decltype(a.bsum[0], void()) {
#pragma unroll
  for (int q = 0; q < int(sizeof(a.bsum) / sizeof(a.bsum[0])); ++q) a.bsum[q] += b.bsum[q];
}
template <class L>
__device__ __forceinline__ void merge_row_sums(L&, const L&, long) {}

// Main loop over nk slabs.  Loaders expose load() (global -> registers,
// advancing their k cursor by kstep), store(lds) and KMAJOR (the LDS layout
// store() writes).  Two LDS stages.
//
// Tiles up to 128 x 128 keep two register sets per operand: set 0 carries the
// even slabs and set 1 the odd ones (each cursor steps two slabs), so the
// global loads of slab t + 2 are in flight while slab t is multiplied and
// slab t + 1 is written to LDS -- two slabs of MFMA time cover the load
// latency.  Larger tiles (and scalar strided operands) have the registers for
// one set only; the 256-wide tiles' longer slabs (4096 MFMA cycles per wave)
// cover one slab of latency.
template <class C, class LA, class LB>
__device__ __forceinline__ void mainloop_1deep(Acc<C>& acc, LA& la, LB& lb, int nk, float* smem) {
  float* As = smem;
  float* Bs = smem + 2 * C::A_STAGE;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
  acc_zero<C>(acc);
  if (nk <= 0) return;
  la.load();
  lb.load();
  la.store(As);
  lb.store(Bs);
  __syncthreads();
  // Loads past the last slab read zeros (the loaders mask k >= kmax) into a
  // stage nobody reads; issuing them unconditionally keeps the loop free of
  // branches.
  for (int t = 0; t < nk; ++t) {
    const int cur = t & 1;
    la.load();
    lb.load();
    mma_slab<C, LA::KMAJOR, LB::KMAJOR>(acc, As + cur * C::A_STAGE, Bs + cur * C::B_STAGE, wm, wn, lane);
    la.store(As + (cur ^ 1) * C::A_STAGE);
    lb.store(Bs + (cur ^ 1) * C::B_STAGE);
    __syncthreads();
  }
}

// Loaders declare DEEP = false when a second register set would not fit
// (scalar strided modes hold a 64-bit pointer per row pass).
template <class L>
constexpr auto deep_ok(int) -> decltype(L::DEEP, bool()) { return L::DEEP; }
template <class L>
constexpr bool deep_ok(long) { return true; }

template <class C, class LA, class LB>
__device__ __forceinline__ void mainloop(Acc<C>& acc, LA& la0, LB& lb0, int nk, float* smem) {
  if constexpr (C::BM * C::BN > 128 * 128 || !deep_ok<LA>(0) || !deep_ok<LB>(0)) {
    mainloop_1deep<C>(acc, la0, lb0, nk, smem);
  } else {
  float* const As0 = smem;
  float* const As1 = smem + C::A_STAGE;
  float* const Bs0 = smem + 2 * C::A_STAGE;
  float* const Bs1 = Bs0 + C::B_STAGE;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
  acc_zero<C>(acc);
  if (nk <= 0) return;
  LA la1 = la0;
  LB lb1 = lb0;
  la0.kstep = lb0.kstep = la1.kstep = lb1.kstep = 2 * C::BK;
  la1.k += C::BK;
  lb1.k += C::BK;
  // Loads past the last slab read zeros (the loaders mask k >= kmax) into a
  // stage nobody reads; issuing loads and stores unconditionally keeps the
  // loop free of branches, so the waits before each store cover only the
  // older register set.
  la0.load();
  lb0.load();
  la1.load();
  lb1.load();
  la0.store(As0);
  lb0.store(Bs0);
  __syncthreads();
  // With 16-deep slabs an odd slab count runs one more slab, of zeros (the
  // loaders mask k >= kmax): a loop with one exit keeps the accumulators in
  // the same registers across iterations, where an exit between the two
  // halves made the compiler copy them every iteration.  (The 32-deep
  // weight-gradient tile keeps the exit: without it, it spills.)
  for (int t = 0; t < nk; t += 2) {
    // Slab t (stage 0); slab t + 1 waits in set 1.
    la0.load();
    lb0.load();
    mma_slab<C, LA::KMAJOR, LB::KMAJOR>(acc, As0, Bs0, wm, wn, lane);
    la1.store(As1);
    lb1.store(Bs1);
    __syncthreads();
    if constexpr (C::BK >= 32) {
      if (t + 1 >= nk) break;
    }
    // Slab t + 1 (stage 1); slab t + 2 waits in set 0.
    la1.load();
    lb1.load();
    mma_slab<C, LA::KMAJOR, LB::KMAJOR>(acc, As1, Bs1, wm, wn, lane);
    la0.store(As0);
    lb0.store(Bs0);
    __syncthreads();
  }
  merge_row_sums(la0, la1, 0);
  }
}

// Visits every accumulator with its (row, col) inside the BM x BN tile.
// 32x32x2 f32 output layout: lane l, register v -> row 8*(v/4) + 4*(l/32) + v%4,
// column l%32.
template <class C, class F>
__device__ __forceinline__ void for_each_acc(const Acc<C>& acc, F&& f) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
  const int r = lane & 31, h = lane >> 5;
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = wm * C::WTM + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        const int col = wn * C::WTN + j * 32 + r;
        f(row, col, acc.v[i][j][v]);
      }
}

// Same walk with the fragment column index j (0..FN) of each value: every
// value of one j shares this lane's column.
template <class C, class F>
__device__ __forceinline__ void for_each_acc_j(const Acc<C>& acc, F&& f) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / C::WAVES_N, wn = wave % C::WAVES_N;
  const int r = lane & 31, h = lane >> 5;
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int row = wm * C::WTM + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        const int col = wn * C::WTN + j * 32 + r;
        f(row, col, j, acc.v[i][j][v]);
      }
}

// This lane's column inside the tile for fragment column j.
template <class C>
__device__ __forceinline__ int acc_col(int j) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  return (wave % C::WAVES_N) * C::WTN + j * 32 + (lane & 31);
}

// This lane's row inside the tile for accumulator (i, v).
template <class C>
__device__ __forceinline__ int acc_row(int i, int v) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  return (wave / C::WAVES_N) * C::WTM + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
}

// Epilogue walk by rows: f(row, i, v) once per accumulator row of this lane;
// the callee loops over the FN fragment columns (acc.v[i][j][v]) with column
// data it computed once (acc_col), so per-element work is one add and a store.
template <class C, class F>
__device__ __forceinline__ void for_each_acc_row(F&& f) {
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) f(acc_row<C>(i, v), i, v);
}

// Register-order index of accumulator (i, j, v) of this thread: partial tiles
// are spilled and reloaded in this order, fully coalesced.
template <class C>
__device__ __forceinline__ int acc_slot(int i, int j, int v) {
  return ((i * C::FN + j) * 16 + v) * kThreads + threadIdx.x;
}

// ---------------------------------------------------------------- loaders
// Operand element (row, k) = base[row * s_row + k * s_k] for rows
// [row0, row0 + ROWS) clipped to R and k < kmax (zero outside).
enum class Mode : int {
  KVEC = 0,     // k contiguous, 16-byte aligned: float4 along k
  RVEC = 1,     // rows contiguous, 16-byte aligned: float4 along rows
  KSCALAR = 2,  // consecutive lanes -> consecutive k
  RSCALAR = 3   // consecutive lanes -> consecutive rows
};

template <int ROWS, int BK, Mode MODE>
struct StridedLoader;

template <int ROWS, int BK>
struct StridedLoader<ROWS, BK, Mode::KVEC> {
  static constexpr bool KMAJOR = false;
  int kstep = BK;  // k advance per load(); the main loop may set 2 * BK
  static constexpr int TPR = BK / 4;                 // threads per row
  static constexpr int RPP = kThreads / TPR;         // rows per pass
  static constexpr int PASSES = ROWS / RPP;
  static_assert(PASSES >= 1 && ROWS % RPP == 0, "KVEC tiling");
  f32x4 v[PASSES];
  const float* ptr[PASSES];
  bool ok[PASSES];
  int k, kmax, kq;
  __device__ __forceinline__ void init(const float* base, int64_t s_row, int64_t /*s_k*/, int row0, int R, int k0,
                       int kmax_) {
    const int tid = threadIdx.x;
    kq = tid % TPR;
    k = k0;
    kmax = kmax_;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int row = row0 + kvec_row<TPR>(tid) + p * RPP;
      ok[p] = row < R;
      ptr[p] = base + (ok[p] ? int64_t(row) * s_row : 0) + 4 * kq;
    }
  }
  __device__ __forceinline__ void load() {
    const int kk = k + 4 * kq;
    const bool kin = kk < kmax;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) v[p] = load4_or_zero(ptr[p] + k, ok[p] && kin);
    k += kstep;
  }
  __device__ __forceinline__ void store(float* lds) const {
    const int tid = threadIdx.x;
    constexpr int LDK = BK + 4;
#pragma unroll
    for (int p = 0; p < PASSES; ++p)
      *reinterpret_cast<f32x4*>(lds + (kvec_row<TPR>(tid) + p * RPP) * LDK + 4 * kq) = v[p];
  }
};

template <int ROWS, int BK>
struct StridedLoader<ROWS, BK, Mode::RVEC> {
  // Rows are contiguous in memory: each thread reads 4 rows at one k with a
  // 16-byte load and writes them unchanged into the k-major stage.
  static constexpr bool KMAJOR = true;
  int kstep = BK;  // k advance per load(); the main loop may set 2 * BK
  static constexpr int TPK = ROWS / 4;               // threads per k
  static constexpr int KPP = kThreads / TPK;         // k per pass
  static constexpr int PASSES = BK / KPP;
  static_assert(PASSES >= 1 && BK % KPP == 0, "RVEC tiling");
  f32x4 v[PASSES];
  const float* ptr;
  int64_t s_k;
  bool ok;
  int k, kmax, kk;
  __device__ __forceinline__ void init(const float* base, int64_t /*s_row*/, int64_t s_k_, int row0, int R, int k0,
                       int kmax_) {
    const int tid = threadIdx.x;
    const int rq = tid % TPK;
    kk = tid / TPK;
    const int row = row0 + 4 * rq;
    ok = row < R;
    ptr = base + (ok ? row : 0);
    s_k = s_k_;
    k = k0;
    kmax = kmax_;
  }
  __device__ __forceinline__ void load() {
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int kx = k + kk + p * KPP;
      v[p] = load4_or_zero(ptr + int64_t(kx) * s_k, ok && kx < kmax);
    }
    k += kstep;
  }
  __device__ __forceinline__ void store(float* lds) const {
    const int tid = threadIdx.x;
    constexpr int LDR = ROWS + 4;
#pragma unroll
    for (int p = 0; p < PASSES; ++p)
      *reinterpret_cast<f32x4*>(lds + (kk + p * KPP) * LDR + 4 * (tid % TPK)) = v[p];
  }
};

template <int ROWS, int BK>
struct StridedLoader<ROWS, BK, Mode::KSCALAR> {
  static constexpr bool KMAJOR = false;
  static constexpr bool DEEP = false;
  int kstep = BK;  // k advance per load(); the main loop may set 2 * BK
  static constexpr int RPP = kThreads / BK;
  static constexpr int PASSES = ROWS / RPP;
  static_assert(PASSES >= 1 && ROWS % RPP == 0, "KSCALAR tiling");
  float v[PASSES];
  const float* ptr[PASSES];
  bool ok[PASSES];
  int64_t s_k;
  int k, kmax, kk;
  __device__ __forceinline__ void init(const float* base, int64_t s_row, int64_t s_k_, int row0, int R, int k0, int kmax_) {
    const int tid = threadIdx.x;
    kk = tid % BK;
    s_k = s_k_;
    k = k0;
    kmax = kmax_;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int row = row0 + tid / BK + p * RPP;
      ok[p] = row < R;
      ptr[p] = base + (ok[p] ? int64_t(row) * s_row : 0);
    }
  }
  __device__ __forceinline__ void load() {
    const int kx = k + kk;
    const bool kin = kx < kmax;
    const int64_t off = int64_t(kx) * s_k;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) v[p] = load_or_zero(ptr[p] + off, ok[p] && kin);
    k += kstep;
  }
  __device__ __forceinline__ void store(float* lds) const {
    const int tid = threadIdx.x;
    constexpr int LDK = BK + 4;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) lds[(tid / BK + p * RPP) * LDK + kk] = v[p];
  }
};

template <int ROWS, int BK>
struct StridedLoader<ROWS, BK, Mode::RSCALAR> {
  static constexpr bool KMAJOR = false;
  static constexpr bool DEEP = false;
  int kstep = BK;  // k advance per load(); the main loop may set 2 * BK
  static_assert(kThreads % ROWS == 0 || ROWS % kThreads == 0, "RSCALAR tiling");
  static constexpr int EPT = ROWS * BK / kThreads;   // consecutive k per thread
  static_assert(ROWS <= kThreads, "RSCALAR expects ROWS <= 256");
  float v[EPT];
  const float* ptr;
  int64_t s_k;
  bool ok;
  int k, kmax, ks;
  __device__ __forceinline__ void init(const float* base, int64_t s_row, int64_t s_k_, int row0, int R, int k0, int kmax_) {
    const int tid = threadIdx.x;
    const int r = tid % ROWS;
    ks = (tid / ROWS) * EPT;
    const int row = row0 + r;
    ok = row < R;
    ptr = base + (ok ? int64_t(row) * s_row : 0);
    s_k = s_k_;
    k = k0;
    kmax = kmax_;
  }
  __device__ __forceinline__ void load() {
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const int kx = k + ks + e;
      v[e] = load_or_zero(ptr + int64_t(kx) * s_k, ok && kx < kmax);
    }
    k += kstep;
  }
  __device__ __forceinline__ void store(float* lds) const {
    const int tid = threadIdx.x;
    constexpr int LDK = BK + 4;
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

// The same operand views through a buffer resource over [base, base + bytes)
// (bytes < kBufMaxBytes, 32-bit element strides): per-lane byte offsets are
// fixed at init, the k cursor moves the scalar offset, and masked elements
// read zero through the range check.  Used for convolution weights; the
// general GEMM keeps StridedLoader (its operands may exceed the 2^31 range).
template <int ROWS, int BK, Mode MODE>
struct BufStridedLoader;

template <int ROWS, int BK>
struct BufStridedLoader<ROWS, BK, Mode::KVEC> {
  static constexpr bool KMAJOR = false;
  int kstep = BK;
  static constexpr int TPR = BK / 4;
  static constexpr int RPP = kThreads / TPR;
  static constexpr int PASSES = ROWS / RPP;
  static_assert(PASSES >= 1 && ROWS % RPP == 0, "KVEC tiling");
  f32x4 v[PASSES];
  i32x4 rs;
  uint32_t off[PASSES];
  int k, kmax, kq;
  __device__ __forceinline__ void init(const float* base, int64_t bytes, int s_row, int /*s_k*/, int row0, int R,
                                       int k0, int kmax_) {
    const int tid = threadIdx.x;
    kq = tid % TPR;
    rs = buffer_rsrc(base, bytes);
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
      const int row = row0 + kvec_row<TPR>(tid) + p * RPP;
      off[p] = row < R ? uint32_t(row * s_row + 4 * kq) * 4u : kOffNone;
    }
    k = k0;
    kmax = kmax_;
  }
  __device__ __forceinline__ void load() {
    const bool kin = k + 4 * kq < kmax;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) v[p] = bload4(rs, kin ? off[p] : kOffNone, uint32_t(k) * 4u);
    k += kstep;
  }
  __device__ __forceinline__ void store(float* lds) const {
    const int tid = threadIdx.x;
    constexpr int LDK = BK + 4;
#pragma unroll
    for (int p = 0; p < PASSES; ++p)
      *reinterpret_cast<f32x4*>(lds + (kvec_row<TPR>(tid) + p * RPP) * LDK + 4 * kq) = v[p];
  }
};

template <int ROWS, int BK>
struct BufStridedLoader<ROWS, BK, Mode::RVEC> {
  static constexpr bool KMAJOR = true;
  int kstep = BK;
  static constexpr int TPK = ROWS / 4;
  static constexpr int KPP = kThreads / TPK;
  static constexpr int PASSES = BK / KPP;
  static_assert(PASSES >= 1 && BK % KPP == 0, "RVEC tiling");
  f32x4 v[PASSES];
  i32x4 rs;
  uint32_t off, sk4;
  int k, kmax, kk;
  __device__ __forceinline__ void init(const float* base, int64_t bytes, int /*s_row*/, int s_k, int row0, int R,
                                       int k0, int kmax_) {
    const int tid = threadIdx.x;
    kk = tid / TPK;
    const int row = row0 + 4 * (tid % TPK);
    rs = buffer_rsrc(base, bytes);
    off = row < R ? uint32_t(row + kk * s_k) * 4u : kOffNone;
    sk4 = uint32_t(s_k) * 4u;
    k = k0;
    kmax = kmax_;
  }
  __device__ __forceinline__ void load() {
#pragma unroll
    for (int p = 0; p < PASSES; ++p)
      v[p] = bload4(rs, k + kk + p * KPP < kmax ? off : kOffNone, uint32_t(k + p * KPP) * sk4);
    k += kstep;
  }
  __device__ __forceinline__ void store(float* lds) const {
    const int tid = threadIdx.x;
    constexpr int LDR = ROWS + 4;
#pragma unroll
    for (int p = 0; p < PASSES; ++p)
      *reinterpret_cast<f32x4*>(lds + (kk + p * KPP) * LDR + 4 * (tid % TPK)) = v[p];
  }
};

template <int ROWS, int BK>
struct BufStridedLoader<ROWS, BK, Mode::RSCALAR> {
  static constexpr bool KMAJOR = false;
  int kstep = BK;
  static_assert(ROWS % 64 == 0 && ROWS <= kThreads, "RSCALAR tiling");
  static constexpr int EPT = ROWS * BK / kThreads;  // consecutive k per thread (wave-uniform run)
  float v[EPT];
  i32x4 rs;
  uint32_t off, sk4;
  int k, kmax, ks;
  __device__ __forceinline__ void init(const float* base, int64_t bytes, int s_row, int s_k, int row0, int R, int k0,
                                       int kmax_) {
    const int tid = threadIdx.x;
    ks = __builtin_amdgcn_readfirstlane((tid / ROWS) * EPT);
    const int row = row0 + tid % ROWS;
    rs = buffer_rsrc(base, bytes);
    off = row < R ? uint32_t(row * s_row) * 4u : kOffNone;
    sk4 = uint32_t(s_k) * 4u;
    k = k0;
    kmax = kmax_;
  }
  __device__ __forceinline__ void load() {
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const int kx = k + ks + e;  // wave-uniform
      v[e] = bload(rs, kx < kmax ? off : kOffNone, uint32_t(kx) * sk4);
    }
    k += kstep;
  }
  __device__ __forceinline__ void store(float* lds) const {
    const int tid = threadIdx.x;
    constexpr int LDK = BK + 4;
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

// Bijective block remap so that consecutive logical tiles land on the same
// XCD (hardware dispatches workgroup b to XCD b % 8): tiles that share an
// operand panel then share that XCD's L2.
__device__ __forceinline__ int xcd_remap(int b, int n) {
  constexpr int X = 8;
  if (n < 2 * X) return b;
  const int per = n / X, rem = n % X;
  const int xcd = b % X, idx = b / X;
  return xcd < rem ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
}

// Logical tile id -> (tile_m, tile_n) in GROUP_M-row bands (raster order
// within a band) so a wave of resident tiles reuses A and B panels.
__device__ __forceinline__ void tile_coords(int t, int tiles_m, int tiles_n, int& tm, int& tn) {
  constexpr int GROUP_M = 8;
  const int band = GROUP_M * tiles_n;
  const int g = t / band;
  const int first_m = g * GROUP_M;
  const int gm = min(tiles_m - first_m, GROUP_M);
  const int in = t % band;
  tm = first_m + in % gm;
  tn = in / gm;
}

}  // namespace mfma
}  // namespace mx
