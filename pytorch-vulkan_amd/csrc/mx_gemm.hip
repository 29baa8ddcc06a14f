// FP32 strided / batched GEMM with fused alpha, beta*bias epilogue on gfx950
// MFMA (v_mfma_f32_32x32x2f32).
//
// Covers the reference's matmul_strided{,_reg}{,_bias}.comp and
// bmm_strided.comp (mm_impl csrc/ops/mm.cpp:244-343, addmm_bias_vulkan
// csrc/ops/mm.cpp:835-879, bmm_impl csrc/ops/bmm.cpp:16-68): A and B are read
// straight from arbitrary strided views (a transposed weight costs no copy),
// and the bias add of nn.Linear happens in the store.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>

#include "mfma_core.hpp"
#include "mx_internal.hpp"

namespace mx {
namespace {

using namespace mfma;

struct GemmArgs {
  const float* a;
  const float* b;
  const float* bias;
  float* c;
  int64_t a_sb, a_sm, a_sk;
  int64_t b_sb, b_sk, b_sn;
  int64_t c_sb, ldc;
  int64_t bias_sb, bias_sm, bias_sn;
  int M, N, K, batch, batch0;
  int tiles_m, tiles_n;
  float alpha, beta;
  int bias_kind;
};

template <class C, Mode MA, Mode MB>
MX_TILE_KERNEL(C) void gemm_kernel(GemmArgs p) {
  __shared__ __attribute__((aligned(16))) float smem[C::SMEM_FLOATS];
  int tm, tn;
  tile_coords(xcd_remap(blockIdx.x, p.tiles_m * p.tiles_n), p.tiles_m, p.tiles_n, tm, tn);
  const int row0 = tm * C::BM, col0 = tn * C::BN;
  const int64_t bz = int64_t(p.batch0) + blockIdx.z;
  StridedLoader<C::BM, C::BK, MA> la;
  StridedLoader<C::BN, C::BK, MB> lb;
  la.init(p.a + bz * p.a_sb, p.a_sm, p.a_sk, row0, p.M, 0, p.K);
  lb.init(p.b + bz * p.b_sb, p.b_sn, p.b_sk, col0, p.N, 0, p.K);
  Acc<C> acc;
  mainloop<C>(acc, la, lb, (p.K + C::BK - 1) / C::BK, smem);
  float* __restrict__ cb = p.c + bz * p.c_sb;
  const float* __restrict__ bias = p.bias ? p.bias + bz * p.bias_sb : nullptr;
  const float alpha = p.alpha, beta = p.beta;
  const int kind = (p.bias_kind == MX_BIAS_NONE || beta == 0.f) ? MX_BIAS_NONE : p.bias_kind;
  int ccol[C::FN];
  float bcol[C::FN];
#pragma unroll
  for (int j = 0; j < C::FN; ++j) {
    ccol[j] = col0 + acc_col<C>(j);
    // Column bias (nn.Linear): one value per fragment column, loaded once.
    bcol[j] = (kind == MX_BIAS_COL && ccol[j] < p.N) ? beta * bias[int64_t(ccol[j]) * p.bias_sn] : 0.f;
  }
  // Two separate walks: stores and loads share the vector-memory counter, so
  // a bias load between stores makes every later store wait for the earlier
  // ones; only the matrix-bias walk (baddbmm) reads memory between stores.
  if (kind == MX_BIAS_MATRIX) {
    for_each_acc_row<C>([&](int r, int i, int v) {
      const int row = row0 + r;
      if (row >= p.M) return;
      float* __restrict__ crow = cb + int64_t(row) * p.ldc;
      const float* __restrict__ brow = bias + int64_t(row) * p.bias_sm;
#pragma unroll
      for (int j = 0; j < C::FN; ++j)
        if (ccol[j] < p.N) crow[ccol[j]] = alpha * acc.v[i][j][v] + beta * brow[int64_t(ccol[j]) * p.bias_sn];
    });
    return;
  }
  for_each_acc_row<C>([&](int r, int i, int v) {
    const int row = row0 + r;
    if (row >= p.M) return;
    float* __restrict__ crow = cb + int64_t(row) * p.ldc;
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
      if (ccol[j] < p.N) crow[ccol[j]] = alpha * acc.v[i][j][v] + bcol[j];
  });
}

// k == 0: C = beta * bias (or zeros when beta == 0 / no bias).
__global__ void gemm_k0_kernel(GemmArgs p) {
  const int64_t total = int64_t(p.batch) * p.M * p.N;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int col = int(i % p.N);
    const int64_t rest = i / p.N;
    const int row = int(rest % p.M);
    const int bz = int(rest / p.M);
    float out = 0.f;
    if (p.bias_kind != MX_BIAS_NONE && p.beta != 0.f) {
      const float* bias = p.bias + int64_t(bz) * p.bias_sb;
      const float bv = p.bias_kind == MX_BIAS_COL ? bias[int64_t(col) * p.bias_sn]
                                                  : bias[int64_t(row) * p.bias_sm + int64_t(col) * p.bias_sn];
      out = p.beta * bv;
    }
    p.c[int64_t(bz) * p.c_sb + int64_t(row) * p.ldc + col] = out;
  }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

// Operand layout -> loader mode.  rows = m for A, n for B.
Mode pick_mode(const float* base, int64_t s_row, int64_t s_k, int64_t s_batch, int64_t batch, int64_t R,
               int64_t K) {
  const bool batch_ok = batch <= 1 || s_batch % 4 == 0;
  if (s_k == 1 && aligned16(base) && s_row % 4 == 0 && batch_ok && K % 4 == 0) return Mode::KVEC;
  if (s_row == 1 && aligned16(base) && s_k % 4 == 0 && batch_ok && R % 4 == 0) return Mode::RVEC;
  if (s_k == 1) return Mode::KSCALAR;
  if (s_row == 1) return Mode::RSCALAR;
  return std::llabs(s_k) <= std::llabs(s_row) ? Mode::KSCALAR : Mode::RSCALAR;
}

template <class C, Mode MA, Mode MB>
int launch3(GemmArgs p, hipStream_t s) {
  const int ntiles = p.tiles_m * p.tiles_n;
  for (int b0 = 0; b0 < p.batch; b0 += 65535) {
    p.batch0 = b0;
    const dim3 grid(ntiles, 1, std::min(p.batch - b0, 65535));
    hipLaunchKernelGGL((gemm_kernel<C, MA, MB>), grid, dim3(kThreads), 0, s, p);
    MX_HIP(hipGetLastError());
  }
  return MX_OK;
}

template <class C, Mode MA>
int launch2(const GemmArgs& p, Mode mb, hipStream_t s) {
  switch (mb) {
    case Mode::KVEC: return launch3<C, MA, Mode::KVEC>(p, s);
    case Mode::RVEC: return launch3<C, MA, Mode::RVEC>(p, s);
    case Mode::KSCALAR: return launch3<C, MA, Mode::KSCALAR>(p, s);
    default: return launch3<C, MA, Mode::RSCALAR>(p, s);
  }
}

template <class C>
int launch1(GemmArgs p, Mode ma, Mode mb, hipStream_t s) {
  p.tiles_m = (p.M + C::BM - 1) / C::BM;
  p.tiles_n = (p.N + C::BN - 1) / C::BN;
  switch (ma) {
    case Mode::KVEC: return launch2<C, Mode::KVEC>(p, mb, s);
    case Mode::RVEC: return launch2<C, Mode::RVEC>(p, mb, s);
    case Mode::KSCALAR: return launch2<C, Mode::KSCALAR>(p, mb, s);
    default: return launch2<C, Mode::RSCALAR>(p, mb, s);
  }
}

// 256-row tiles are built for the 16-byte operand modes only (scalar modes
// would need a register per row pass).
template <class C>
int launch1_vec(GemmArgs p, Mode ma, Mode mb, hipStream_t s) {
  p.tiles_m = (p.M + C::BM - 1) / C::BM;
  p.tiles_n = (p.N + C::BN - 1) / C::BN;
  if (ma == Mode::KVEC)
    return mb == Mode::KVEC ? launch3<C, Mode::KVEC, Mode::KVEC>(p, s) : launch3<C, Mode::KVEC, Mode::RVEC>(p, s);
  return mb == Mode::KVEC ? launch3<C, Mode::RVEC, Mode::KVEC>(p, s) : launch3<C, Mode::RVEC, Mode::RVEC>(p, s);
}

bool is_vec(Mode m) { return m == Mode::KVEC || m == Mode::RVEC; }

// Tile menu (BM x BN x BK, wave grid, waves per SIMD).  All keep two or more
// workgroups resident per CU.
using TileTall = Cfg<256, 128, 16, 2, 2>;  // 4 waves of 128 x 64
using TileWide = Cfg<128, 256, 16, 2, 2>;  // 4 waves of 64 x 128
using TileSq = Cfg<128, 128, 16, 2, 2>;    // 4 waves of 64 x 64
using TileSmall = Cfg<64, 64, 16, 2, 4>;   // 4 waves of 32 x 32

struct TileChoice {
  int bm, bn, per_cu;
  double rate;  // throughput of a CU full of such tiles, relative to 256 x 128
};
constexpr TileChoice kTiles[] = {{256, 128, 2, 1.0}, {128, 256, 2, 1.0}, {128, 128, 2, 0.94}, {64, 64, 4, 0.6}};

// Cheapest tile by a wave-quantised cost model: rounds of resident tiles
// times the time of one round (per_cu tiles per CU at the relative rate).
// MX_GEMM_TILE=<index into kTiles> forces a tile (tuning and diagnosis; the
// 256-wide tiles only for 16-byte operand modes).  `kernel` (mx_gemm_kernel)
// forces the 64x64 tile or keeps the choice among the large ones.
int pick_gemm_tile(int64_t m, int64_t n, int64_t batch, bool vec, int kernel) {
  if (const char* e = std::getenv("MX_GEMM_TILE")) {
    const int t = std::atoi(e);
    if (t >= (vec ? 0 : 2) && t < 4) return t;
  }
  if (kernel == MX_GEMM_KERNEL_TILED) return 3;
  const int last = kernel == MX_GEMM_KERNEL_REGISTER ? 3 : 4;
  int best = 2;
  double best_cost = 0;
  for (int i = vec ? 0 : 2; i < last; ++i) {
    const TileChoice& t = kTiles[i];
    const int64_t tiles = ((m + t.bm - 1) / t.bm) * ((n + t.bn - 1) / t.bn) * batch;
    const int64_t slots = int64_t(cu_count()) * t.per_cu;
    const double cost = double((tiles + slots - 1) / slots) * t.per_cu * t.bm * t.bn / t.rate;
    if (i == (vec ? 0 : 2) || cost < best_cost) {
      best = i;
      best_cost = cost;
    }
  }
  return best;
}

}  // namespace
}  // namespace mx

using namespace mx;

namespace mx {
namespace {

const char* mode_name(Mode m) {
  switch (m) {
    case Mode::KVEC: return "KVEC";
    case Mode::RVEC: return "RVEC";
    case Mode::KSCALAR: return "KSCALAR";
    default: return "RSCALAR";
  }
}

// Validated arguments, operand modes and tile of one mx_gemm_f32 call (the
// pointers only decide alignment; nothing is read).  Returns MX_OK with
// *empty set when the call writes nothing.
struct GemmPlan {
  GemmArgs p{};
  Mode ma = Mode::KVEC, mb = Mode::KVEC;
  int tile = 2;
  bool empty = false;
};

int plan_gemm(const mx_gemm_desc* d, const float* a, const float* b, const float* bias, float* c, GemmPlan* g) {
  MX_REQUIRE(d, MX_ERR_INVALID, "mx_gemm_f32: null descriptor");
  MX_REQUIRE(d->batch >= 0 && d->m >= 0 && d->n >= 0 && d->k >= 0, MX_ERR_INVALID,
             "mx_gemm_f32: negative dimension");
  MX_REQUIRE(d->m <= INT32_MAX && d->n <= INT32_MAX && d->k <= INT32_MAX && d->batch <= INT32_MAX,
             MX_ERR_INVALID, "mx_gemm_f32: dimension exceeds int32");
  MX_REQUIRE(d->bias_kind >= MX_BIAS_NONE && d->bias_kind <= MX_BIAS_MATRIX, MX_ERR_INVALID,
             "mx_gemm_f32: bad bias kind");
  MX_REQUIRE(d->kernel >= MX_GEMM_KERNEL_AUTO && d->kernel <= MX_GEMM_KERNEL_REGISTER, MX_ERR_INVALID,
             "mx_gemm: unknown kernel class ", d->kernel);
  g->empty = d->batch == 0 || d->m == 0 || d->n == 0;
  if (g->empty) return MX_OK;
  GemmArgs& p = g->p;
  p.a = a ? a + d->a_offset : nullptr;
  p.b = b ? b + d->b_offset : nullptr;
  p.bias = bias ? bias + d->bias_offset : nullptr;
  p.c = c ? c + d->c_offset : nullptr;
  p.a_sb = d->a_stride_b;
  p.a_sm = d->a_stride_m;
  p.a_sk = d->a_stride_k;
  p.b_sb = d->b_stride_b;
  p.b_sk = d->b_stride_k;
  p.b_sn = d->b_stride_n;
  p.c_sb = d->c_stride_b;
  p.ldc = d->ldc;
  p.bias_sb = d->bias_stride_b;
  p.bias_sm = d->bias_stride_m;
  p.bias_sn = d->bias_stride_n;
  p.M = int(d->m);
  p.N = int(d->n);
  p.K = int(d->k);
  p.batch = int(d->batch);
  p.alpha = d->alpha;
  p.beta = d->beta;
  p.bias_kind = d->bias_kind;
  if (d->k == 0) return MX_OK;
  MX_REQUIRE(((d->m + 63) / 64) * ((d->n + 63) / 64) <= INT32_MAX, MX_ERR_INVALID, "mx_gemm_f32: too many tiles");
  g->ma = pick_mode(p.a, p.a_sm, p.a_sk, p.a_sb, p.batch, p.M, p.K);
  g->mb = pick_mode(p.b, p.b_sn, p.b_sk, p.b_sb, p.batch, p.N, p.K);
  g->tile = pick_gemm_tile(d->m, d->n, d->batch, is_vec(g->ma) && is_vec(g->mb), d->kernel);
  return MX_OK;
}

constexpr const char* kTileNames[] = {"256x128x16", "128x256x16", "128x128x16", "64x64x16"};

}  // namespace
}  // namespace mx

extern "C" int mx_gemm_f32(const mx_gemm_desc* d, const float* a, const float* b, const float* bias,
                           float* c, void* stream) {
  MX_ABI_BEGIN
  GemmPlan g;
  MX_TRY(plan_gemm(d, a, b, bias, c, &g));
  if (g.empty) return MX_OK;
  MX_REQUIRE(c, MX_ERR_INVALID, "mx_gemm_f32: null output");
  MX_REQUIRE(d->bias_kind == MX_BIAS_NONE || bias, MX_ERR_INVALID, "mx_gemm_f32: null bias");
  hipStream_t s = resolve_stream(stream);
  GemmArgs& p = g.p;
  if (d->k == 0) {
    const int64_t total = d->batch * d->m * d->n;
    const int blocks = int(std::min<int64_t>((total + 255) / 256, 65535));
    hipLaunchKernelGGL(gemm_k0_kernel, dim3(blocks), dim3(256), 0, s, p);
    MX_HIP(hipGetLastError());
    return MX_OK;
  }
  MX_REQUIRE(a && b, MX_ERR_INVALID, "mx_gemm_f32: null operand");
  switch (g.tile) {
    case 0: return launch1_vec<TileTall>(p, g.ma, g.mb, s);
    case 1: return launch1_vec<TileWide>(p, g.ma, g.mb, s);
    case 2: return launch1<TileSq>(p, g.ma, g.mb, s);
    default: return launch1<TileSmall>(p, g.ma, g.mb, s);
  }
  MX_ABI_END
}

extern "C" int mx_gemm_variant(const mx_gemm_desc* d, const float* a, const float* b, char* buf, size_t len) {
  MX_ABI_BEGIN
  MX_REQUIRE(buf || !len, MX_ERR_INVALID, "mx_gemm_variant: null buffer");
  GemmPlan g;
  MX_TRY(plan_gemm(d, a, b, nullptr, nullptr, &g));
  std::string name;
  if (g.empty) {
    name = "none";
  } else if (d->k == 0) {
    name = "gemm_k0_kernel";
  } else {
    const int kind = (d->bias_kind == MX_BIAS_NONE || d->beta == 0.f) ? MX_BIAS_NONE : d->bias_kind;
    name = cat("gemm_kernel<", kTileNames[g.tile], ",", mode_name(g.ma), ",", mode_name(g.mb), ">",
               kind == MX_BIAS_COL ? "+bias_col" : kind == MX_BIAS_MATRIX ? "+bias_matrix" : "",
               d->batch > 65535 ? "+batch_chunks" : "");
  }
  if (len) {
    std::strncpy(buf, name.c_str(), len - 1);
    buf[len - 1] = 0;
  }
  return MX_OK;
  MX_ABI_END
}
