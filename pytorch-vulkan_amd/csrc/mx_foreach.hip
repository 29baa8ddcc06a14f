// Multi-tensor pointwise kernels behind torch.optim's foreach path
// (_foreach_mul_ / add_ / div_ / lerp_ / addcmul_ / addcdiv_ / maximum_ /
// sqrt / add.List) and the per-tensor lerp / addcmul / addcdiv / maximum /
// minimum registrations (reference: csrc/ops/optimizer_primitives.cpp:12-202,
// optimizer_pointwise.comp).  A list of tensors is one launch: a device table
// of entries walked in 4096-element chunks dealt round-robin to the
// workgroups (the layout of the fused AdamW kernel), 16-byte loads where an
// entry's streams are aligned.  A new launch starts only where an entry writes
// memory an earlier entry of the same launch reads or writes, so a list that
// repeats a tensor updates it in list order, as torch's per-tensor loop does.
//
// Per-element arithmetic is torch's CPU kernel for each op (the parity target):
//   lerp     |w| < 0.5 ? fma(w, e - s, s) : fma(w - 1, e - s, e)   (vectorised Lerp)
//   addcmul  fma(v * t1, t2, s)         addcdiv  s + (v * t1) / t2
//   add(alpha) fma(other, alpha, self)  maximum / minimum: NaN wins, else the second operand unless
//            the first is greater / smaller (the vector max / min instructions: max(-0, +0) = +0)
//   mul / div: one IEEE operation; sqrt within one ulp (torch's CPU sqrt is not
//   correctly rounded either).  No other multiply-add contraction.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "mx_internal.hpp"

namespace mx {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kVec = 4;                // float4 per stream per thread per chunk
constexpr int kChunk = 256 * 4 * kVec;  // elements per chunk

struct FeEntry {
  float* out;
  const float* a;
  const float* b;
  const float* c;
  int64_t numel;
  int64_t chunk_begin;
  float s;
  int vec;
};

template <int OP>
__device__ __forceinline__ float fe_apply(float a, float b, float c, float s) {
#pragma clang fp contract(off)
  switch (OP) {
    case MX_FOREACH_MUL_SCALAR: return a * s;
    case MX_FOREACH_ADD_SCALAR: return a + s;
    case MX_FOREACH_DIV_SCALAR: return a / s;
    case MX_FOREACH_LERP_SCALAR: {
      const float d = b - a;
      return fabsf(s) < 0.5f ? fmaf(s, d, a) : fmaf(s - 1.f, d, b);
    }
    case MX_FOREACH_LERP_TENSOR: {
      const float d = b - a;
      return fabsf(c) < 0.5f ? fmaf(c, d, a) : fmaf(c - 1.f, d, b);
    }
    case MX_FOREACH_ADDCMUL: return fmaf(s * b, c, a);
    case MX_FOREACH_ADDCDIV: return a + (s * b) / c;
    case MX_FOREACH_MAXIMUM: return (a != a || b != b) ? __builtin_nanf("") : (a > b ? a : b);
    case MX_FOREACH_MINIMUM: return (a != a || b != b) ? __builtin_nanf("") : (a < b ? a : b);
    case MX_FOREACH_SQRT: return sqrtf(a);
    default: return fmaf(b, s, a);  // MX_FOREACH_ADD_LIST
  }
}

template <int OP>
constexpr bool reads_b() {
  return OP == MX_FOREACH_LERP_SCALAR || OP == MX_FOREACH_LERP_TENSOR || OP == MX_FOREACH_ADDCMUL ||
         OP == MX_FOREACH_ADDCDIV || OP == MX_FOREACH_MAXIMUM || OP == MX_FOREACH_MINIMUM ||
         OP == MX_FOREACH_ADD_LIST;
}
template <int OP>
constexpr bool reads_c() {
  return OP == MX_FOREACH_LERP_TENSOR || OP == MX_FOREACH_ADDCMUL || OP == MX_FOREACH_ADDCDIV;
}

template <int OP>
__global__ __launch_bounds__(256) void foreach_kernel(const FeEntry* __restrict__ tab, int ntens,
                                                      int64_t total_chunks) {
  FeEntry e = tab[0];
  int64_t e_end = (e.numel + kChunk - 1) / kChunk;
  for (int64_t ch = blockIdx.x; ch < total_chunks; ch += gridDim.x) {
    if (ch >= e_end || ch < e.chunk_begin) {
      int lo = 0, hi = ntens - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (tab[mid].chunk_begin <= ch)
          lo = mid;
        else
          hi = mid - 1;
      }
      e = tab[lo];
      e_end = e.chunk_begin + (e.numel + kChunk - 1) / kChunk;
    }
    const int64_t base = (ch - e.chunk_begin) * kChunk + int64_t(threadIdx.x) * 4;
    if (e.vec && base + (kVec - 1) * 1024 + 3 < e.numel) {
      f32x4 a4[kVec], b4[kVec], c4[kVec];
#pragma unroll
      for (int u = 0; u < kVec; ++u) {
        const int64_t i = base + u * 1024;
        a4[u] = *reinterpret_cast<const f32x4*>(e.a + i);
        if constexpr (reads_b<OP>()) b4[u] = *reinterpret_cast<const f32x4*>(e.b + i);
        if constexpr (reads_c<OP>()) c4[u] = *reinterpret_cast<const f32x4*>(e.c + i);
      }
#pragma unroll
      for (int u = 0; u < kVec; ++u) {
        f32x4 r;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          r[j] = fe_apply<OP>(a4[u][j], reads_b<OP>() ? b4[u][j] : 0.f, reads_c<OP>() ? c4[u][j] : 0.f, e.s);
        *reinterpret_cast<f32x4*>(e.out + base + u * 1024) = r;
      }
    } else {
      for (int u = 0; u < kVec; ++u)
        for (int64_t i = base + u * 1024; i < min(base + u * 1024 + 4, e.numel); ++i)
          e.out[i] = fe_apply<OP>(e.a[i], reads_b<OP>() ? e.b[i] : 0.f, reads_c<OP>() ? e.c[i] : 0.f, e.s);
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct Interval {
  uintptr_t lo, hi;
  int64_t entry;
  bool written;
};

// For each entry j, the latest earlier entry whose memory conflicts with j's
// (one of the two writes bytes the other touches), or -1.
std::vector<int64_t> latest_conflict(const mx_foreach_tensor* t, int64_t n) {
  std::vector<Interval> iv;
  iv.reserve(size_t(n) * 4);
  for (int64_t i = 0; i < n; ++i) {
    if (t[i].numel <= 0) continue;
    const uintptr_t bytes = uintptr_t(t[i].numel) * 4;
    auto add = [&](const void* p, bool w) {
      if (p) iv.push_back({reinterpret_cast<uintptr_t>(p), reinterpret_cast<uintptr_t>(p) + bytes, i, w});
    };
    add(t[i].out, true);
    add(t[i].a, false);
    add(t[i].b, false);
    add(t[i].c, false);
  }
  std::sort(iv.begin(), iv.end(), [](const Interval& x, const Interval& y) { return x.lo < y.lo; });
  std::vector<int64_t> conf(size_t(n), -1);
  for (size_t x = 0; x < iv.size(); ++x)
    for (size_t y = x + 1; y < iv.size() && iv[y].lo < iv[x].hi; ++y) {
      if (iv[x].entry == iv[y].entry || !(iv[x].written || iv[y].written)) continue;
      const int64_t lo = std::min(iv[x].entry, iv[y].entry), hi = std::max(iv[x].entry, iv[y].entry);
      conf[size_t(hi)] = std::max(conf[size_t(hi)], lo);
    }
  return conf;
}

template <int OP>
void launch(const FeEntry* dtab, int ntens, int64_t chunks, hipStream_t s) {
  const int64_t grid = std::max<int64_t>(1, std::min<int64_t>(chunks, int64_t(cu_count()) * 16));
  hipLaunchKernelGGL(foreach_kernel<OP>, dim3(unsigned(grid)), dim3(256), 0, s, dtab, ntens, chunks);
}

int dispatch(int op, const FeEntry* dtab, int ntens, int64_t chunks, hipStream_t s) {
  switch (op) {
    case MX_FOREACH_MUL_SCALAR: launch<MX_FOREACH_MUL_SCALAR>(dtab, ntens, chunks, s); break;
    case MX_FOREACH_ADD_SCALAR: launch<MX_FOREACH_ADD_SCALAR>(dtab, ntens, chunks, s); break;
    case MX_FOREACH_DIV_SCALAR: launch<MX_FOREACH_DIV_SCALAR>(dtab, ntens, chunks, s); break;
    case MX_FOREACH_LERP_SCALAR: launch<MX_FOREACH_LERP_SCALAR>(dtab, ntens, chunks, s); break;
    case MX_FOREACH_LERP_TENSOR: launch<MX_FOREACH_LERP_TENSOR>(dtab, ntens, chunks, s); break;
    case MX_FOREACH_ADDCMUL: launch<MX_FOREACH_ADDCMUL>(dtab, ntens, chunks, s); break;
    case MX_FOREACH_ADDCDIV: launch<MX_FOREACH_ADDCDIV>(dtab, ntens, chunks, s); break;
    case MX_FOREACH_MAXIMUM: launch<MX_FOREACH_MAXIMUM>(dtab, ntens, chunks, s); break;
    case MX_FOREACH_MINIMUM: launch<MX_FOREACH_MINIMUM>(dtab, ntens, chunks, s); break;
    case MX_FOREACH_SQRT: launch<MX_FOREACH_SQRT>(dtab, ntens, chunks, s); break;
    case MX_FOREACH_ADD_LIST: launch<MX_FOREACH_ADD_LIST>(dtab, ntens, chunks, s); break;
    default: return set_error(MX_ERR_INVALID, cat("mx_foreach_f32: unknown op ", op));
  }
  MX_HIP(hipGetLastError());
  return MX_OK;
}

bool op_reads_b(int op) {
  return op == MX_FOREACH_LERP_SCALAR || op == MX_FOREACH_LERP_TENSOR || op == MX_FOREACH_ADDCMUL ||
         op == MX_FOREACH_ADDCDIV || op == MX_FOREACH_MAXIMUM || op == MX_FOREACH_MINIMUM ||
         op == MX_FOREACH_ADD_LIST;
}
bool op_reads_c(int op) {
  return op == MX_FOREACH_LERP_TENSOR || op == MX_FOREACH_ADDCMUL || op == MX_FOREACH_ADDCDIV;
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" int mx_foreach_f32(int op, const mx_foreach_tensor* tensors, int64_t count, int64_t* launches,
                              void* stream) {
  MX_ABI_BEGIN
  if (launches) *launches = 0;
  MX_REQUIRE(op >= MX_FOREACH_MUL_SCALAR && op <= MX_FOREACH_ADD_LIST, MX_ERR_INVALID, "mx_foreach_f32: unknown op ",
             op);
  MX_REQUIRE(count >= 0, MX_ERR_INVALID, "mx_foreach_f32: negative tensor count");
  if (count == 0) return MX_OK;
  MX_REQUIRE(tensors, MX_ERR_INVALID, "mx_foreach_f32: null tensor list");
  const bool rb = op_reads_b(op), rc = op_reads_c(op);
  for (int64_t i = 0; i < count; ++i) {
    const mx_foreach_tensor& t = tensors[i];
    MX_REQUIRE(t.numel >= 0, MX_ERR_INVALID, "mx_foreach_f32: negative numel at ", i);
    if (t.numel == 0) continue;
    MX_REQUIRE(t.out && t.a && (!rb || t.b) && (!rc || t.c), MX_ERR_INVALID, "mx_foreach_f32: null buffer at ", i);
  }
  hipStream_t s = resolve_stream(stream);
  const std::vector<int64_t> conf = latest_conflict(tensors, count);
  std::vector<FeEntry> tab;
  int64_t first = 0;
  while (first < count) {
    int64_t last = first + 1;
    while (last < count && conf[size_t(last)] < first) ++last;
    tab.clear();
    int64_t chunks = 0;
    for (int64_t i = first; i < last; ++i) {
      const mx_foreach_tensor& t = tensors[i];
      if (t.numel == 0) continue;
      FeEntry e{};
      e.out = t.out;
      e.a = t.a;
      e.b = rb ? t.b : nullptr;
      e.c = rc ? t.c : nullptr;
      e.numel = t.numel;
      e.chunk_begin = chunks;
      e.s = float(t.scalar);
      e.vec = aligned16(e.out) && aligned16(e.a) && (!rb || aligned16(e.b)) && (!rc || aligned16(e.c));
      chunks += (t.numel + kChunk - 1) / kChunk;
      tab.push_back(e);
    }
    if (!tab.empty()) {
      Scratch dtab;
      MX_TRY(upload(tab.data(), tab.size() * sizeof(FeEntry), s, dtab));
      MX_TRY(dispatch(op, dtab.as<FeEntry>(), int(tab.size()), chunks, s));
      if (launches) ++*launches;
    }
    first = last;
  }
  return MX_OK;
  MX_ABI_END
}
