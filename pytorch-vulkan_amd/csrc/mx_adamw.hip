// Multi-tensor fused AdamW (decoupled weight decay), optional AMSGrad.
//
// Replaces the reference's per-group Vulkan dispatches
// (fused_adamw_step_batch_impl csrc/ops/adamw.cpp:78-284,
// adamw_multitensor{4,8}[_amsgrad].comp, multitensor::partition
// csrc/ops/multitensor_plan.h:22-48): one persistent launch walks a device
// table of every tensor in 4096-element chunks dealt round-robin to the
// workgroups.  Where the four (five) streams are 16-byte aligned a thread issues
// all 16 (20) of its 128-bit loads for a chunk before any arithmetic, and the
// next chunk's loads before this chunk's stores -- the kernel is HBM-bound,
// so bytes in flight per CU set its speed -- and every access is
// non-temporal (each byte is touched once per step).  There is no 8-tensor
// or 65,535-workgroup cap; a new launch starts only where an entry writes
// memory an earlier entry of the same launch uses
// (the reference's alias-conflict predicate, csrc/ops/adamw.cpp:207-215).
//
// Per-element arithmetic follows torch.optim.AdamW's single-tensor update
// (the CPU oracle the reference tests against, tests/test_fused_adamw.py):
//   p = p * (1 - lr*wd)
//   m = lerp(m, g, 1 - beta1)            (one fused multiply-add, as torch's CPU lerp)
//   v = v * beta2 + ((1 - beta2) * g) * g
//   p = p + (-lr/bc1 * m) / (sqrt(v) / sqrt(bc2) + eps)
// with bc1 = 1 - beta1^step and bc2 = 1 - beta2^step in double, in that
// order, and no multiply-add contraction other than the lerp's.  With a
// grad_scale (torch's GradScaler through aten::_fused_adamw_) the gradient is
// divided by it first and the unscaled gradient is written back, before
// maximize negates it, as torch's fused AdamW does; a non-zero found_inf
// skips the whole step.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <vector>

#include "mx_internal.hpp"

namespace mx {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kVec = 4;                    // float4 per stream per thread per chunk
constexpr int kChunk = 256 * 4 * kVec;      // elements per chunk

struct AdamEntry {
  float* p;
  float* g;  // written only with a grad_scale (the unscaled gradient)
  float* m;
  float* v;
  float* vmax;
  const float* step_dev;
  int64_t numel;
  int64_t chunk_begin;
  float neg_step_size;  // -lr / bc1 (host steps)
  float bc2_sqrt;       // sqrt(bc2)  (host steps)
  int vec;              // all streams 16-byte aligned
  int pad;
};

struct AdamHP {
  double lr, beta1, beta2, eps, wd;
  const float* lr_dev;
  const float* grad_scale;
  const float* found_inf;
  int maximize;
  int ntens;
  int64_t total_chunks;
};

struct Coef {
  float wdf, b1c, omb1c, b2, b2c, eps, nss, bc2s;
};

__device__ __forceinline__ Coef coefficients(const AdamEntry& e, const AdamHP& hp) {
  Coef c;
  const double lr = hp.lr_dev ? double(*hp.lr_dev) : hp.lr;
  c.wdf = float(1.0 - lr * hp.wd);
  c.b1c = float(1.0 - hp.beta1);
  c.omb1c = 1.f - c.b1c;
  c.b2 = float(hp.beta2);
  c.b2c = float(1.0 - hp.beta2);
  c.eps = float(hp.eps);
  if (e.step_dev) {
    const double step = double(*e.step_dev);
    const double bc1 = 1.0 - pow(hp.beta1, step);
    const double bc2 = 1.0 - pow(hp.beta2, step);
    c.nss = float(-(lr / bc1));
    c.bc2s = float(sqrt(bc2));
  } else if (hp.lr_dev) {
    // neg_step_size carries -1/bc1 when the learning rate lives on the device.
    c.nss = float(lr * double(e.neg_step_size));
    c.bc2s = e.bc2_sqrt;
  } else {
    c.nss = e.neg_step_size;
    c.bc2s = e.bc2_sqrt;
  }
  return c;
}

__device__ __forceinline__ float nan_max(float a, float b) {
  return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b);
}

// g is the (already unscaled) gradient.
template <bool AMS>
__device__ __forceinline__ void update(float& p, float g, float& m, float& v, float* vmax_slot, const Coef& c,
                                       const AdamHP& hp) {
#pragma clang fp contract(off)
  if (hp.maximize) g = -g;
  p = p * c.wdf;
  // torch's vectorised lerp: one fused multiply-add, fma(w, end-self, self)
  // for small weights, fma(w-1, end-self, end) otherwise.
  m = (c.b1c < 0.5f) ? fmaf(c.b1c, g - m, m) : fmaf(c.b1c - 1.f, g - m, g);
  v = v * c.b2;
  v = v + (c.b2c * g) * g;
  float vd = v;
  if constexpr (AMS) {
    vd = nan_max(*vmax_slot, v);
    *vmax_slot = vd;
  }
  const float denom = sqrtf(vd) / c.bc2s + c.eps;
  p = p + (c.nss * m) / denom;
}

// Loads of one full vector chunk: element base + u * 1024 + (0..3), each
// load instruction 4 KiB contiguous per wave.
struct ChunkRegs {
  f32x4 p[kVec], g[kVec], m[kVec], v[kVec], x[kVec];
};

template <bool AMS>
__device__ __forceinline__ void load_chunk(ChunkRegs& r, const AdamEntry& e, int64_t base) {
#pragma unroll
  for (int u = 0; u < kVec; ++u) {
    const int64_t i = base + u * 1024;
    r.p[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(e.p + i));
    r.g[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(e.g + i));
    r.m[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(e.m + i));
    r.v[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(e.v + i));
    if constexpr (AMS) r.x[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(e.vmax + i));
  }
}

template <bool AMS>
__global__ __launch_bounds__(256) void adamw_kernel(const AdamEntry* __restrict__ tab, AdamHP hp) {
  if (hp.found_inf && *hp.found_inf != 0.f) return;
  const float scale = hp.grad_scale ? *hp.grad_scale : 1.f;
  const int64_t total = hp.total_chunks, stride = gridDim.x;
  // Chunks are dealt round-robin (chunk = blockIdx.x + i * gridDim.x), so the
  // workgroups in flight stream through neighbouring memory; each finds a
  // chunk's tensor by binary search over the table's chunk offsets (kept
  // when the next chunk is in the same tensor).
  auto locate = [&](int64_t ch, AdamEntry& e, int64_t& e_end, Coef& c) {
    if (ch < e_end && ch >= e.chunk_begin) return;
    int lo = 0, hi = hp.ntens - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tab[mid].chunk_begin <= ch) lo = mid;
      else hi = mid - 1;
    }
    e = tab[lo];
    e_end = e.chunk_begin + (e.numel + kChunk - 1) / kChunk;
    c = coefficients(e, hp);
  };
  auto chunk_base = [&](const AdamEntry& e, int64_t ch) {
    return (ch - e.chunk_begin) * kChunk + int64_t(threadIdx.x) * 4;
  };
  auto vector_ok = [&](const AdamEntry& e, int64_t base) { return e.vec && base + (kVec - 1) * 1024 + 3 < e.numel; };
  int64_t ch = blockIdx.x;
  if (ch >= total) return;
  AdamEntry e = tab[0];
  int64_t e_end = (e.numel + kChunk - 1) / kChunk;
  Coef c = coefficients(e, hp);
  locate(ch, e, e_end, c);
  int64_t base = chunk_base(e, ch);
  bool full = vector_ok(e, base);
  // A full chunk's loads are issued one chunk ahead: the next chunk's (of
  // whatever tensor) go out after this chunk's arithmetic and before its
  // stores, so they are in flight while the stores drain.  Entries of one
  // launch never share memory (the host splits launches where they would),
  // so the early loads cannot read what the pending stores write.
  ChunkRegs r;
  if (full) load_chunk<AMS>(r, e, base);
  for (; ch < total; ch += stride) {
    const int64_t nch = ch + stride;
    if (full) {
      // The unscaled gradient goes out first: only the new p, m, v (and
      // vmax) stay live across the next chunk's loads.
      if (hp.grad_scale) {
#pragma unroll
        for (int u = 0; u < kVec; ++u) {
#pragma unroll
          for (int j = 0; j < 4; ++j) r.g[u][j] = r.g[u][j] / scale;
          __builtin_nontemporal_store(r.g[u], reinterpret_cast<f32x4*>(e.g + base + u * 1024));
        }
      }
      f32x4 np[kVec], nm[kVec], nv[kVec], nx[kVec];
#pragma unroll
      for (int u = 0; u < kVec; ++u) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float pp = r.p[u][j], mm = r.m[u][j], vv = r.v[u][j], xx = AMS ? r.x[u][j] : 0.f;
          update<AMS>(pp, r.g[u][j], mm, vv, &xx, c, hp);
          np[u][j] = pp;
          nm[u][j] = mm;
          nv[u][j] = vv;
          if constexpr (AMS) nx[u][j] = xx;
        }
      }
      const AdamEntry ce = e;
      const int64_t cbase = base;
      if (nch < total) {
        locate(nch, e, e_end, c);
        base = chunk_base(e, nch);
        full = vector_ok(e, base);
        if (full) load_chunk<AMS>(r, e, base);
      }
#pragma unroll
      for (int u = 0; u < kVec; ++u) {
        const int64_t i = cbase + u * 1024;
        __builtin_nontemporal_store(np[u], reinterpret_cast<f32x4*>(ce.p + i));
        __builtin_nontemporal_store(nm[u], reinterpret_cast<f32x4*>(ce.m + i));
        __builtin_nontemporal_store(nv[u], reinterpret_cast<f32x4*>(ce.v + i));
        if constexpr (AMS) __builtin_nontemporal_store(nx[u], reinterpret_cast<f32x4*>(ce.vmax + i));
      }
    } else {
      // A tensor's last (partial) chunk, or unaligned streams: element loads,
      // a group of four elements per stream issued before its stores (a store
      // between them would order every later load after it, one memory round
      // trip per element); the groups run one after another to keep the
      // register count of the vector path.
#pragma unroll 1
      for (int u = 0; u < kVec; ++u) {
        float pp[4], gg[4], mm[4], vv[4], xx[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t i = base + u * 1024 + j;
          const bool in = i < e.numel;
          pp[j] = in ? e.p[i] : 0.f;
          gg[j] = in ? e.g[i] : 0.f;
          mm[j] = in ? e.m[i] : 0.f;
          vv[j] = in ? e.v[i] : 0.f;
          xx[j] = (AMS && in) ? e.vmax[i] : 0.f;
        }
        if (hp.grad_scale) {
#pragma unroll
          for (int j = 0; j < 4; ++j) gg[j] = gg[j] / scale;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) update<AMS>(pp[j], gg[j], mm[j], vv[j], &xx[j], c, hp);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t i = base + u * 1024 + j;
          if (i < e.numel) {
            if (hp.grad_scale) e.g[i] = gg[j];
            e.p[i] = pp[j];
            e.m[i] = mm[j];
            e.v[i] = vv[j];
            if constexpr (AMS) e.vmax[i] = xx[j];
          }
        }
      }
      if (nch < total) {
        locate(nch, e, e_end, c);
        base = chunk_base(e, nch);
        full = vector_ok(e, base);
        if (full) load_chunk<AMS>(r, e, base);
      }
    }
  }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

struct Interval {
  uintptr_t lo, hi;
  int64_t entry;
  bool written;
};

// For each entry j, the latest earlier entry i whose memory conflicts with j
// (one of them writes bytes the other reads or writes), or -1.  Gradients are
// written when `grads_written` (a grad_scale unscales them in place).
std::vector<int64_t> latest_conflict(const mx_adamw_tensor* t, int64_t n, bool ams, bool grads_written) {
  std::vector<Interval> iv;
  iv.reserve(size_t(n) * 5);
  for (int64_t i = 0; i < n; ++i) {
    if (t[i].numel <= 0) continue;
    const uintptr_t bytes = uintptr_t(t[i].numel) * 4;
    auto add = [&](const void* ptr, bool w) {
      if (ptr) iv.push_back({reinterpret_cast<uintptr_t>(ptr), reinterpret_cast<uintptr_t>(ptr) + bytes, i, w});
    };
    add(t[i].param, true);
    add(t[i].grad, grads_written);
    add(t[i].exp_avg, true);
    add(t[i].exp_avg_sq, true);
    if (ams) add(t[i].max_exp_avg_sq, true);
  }
  std::sort(iv.begin(), iv.end(), [](const Interval& a, const Interval& b) { return a.lo < b.lo; });
  std::vector<int64_t> conf(size_t(n), -1);
  // Sweep: compare each interval with the following ones that start before it ends.
  for (size_t a = 0; a < iv.size(); ++a)
    for (size_t b = a + 1; b < iv.size() && iv[b].lo < iv[a].hi; ++b) {
      if (iv[a].entry == iv[b].entry || !(iv[a].written || iv[b].written)) continue;
      const int64_t lo = std::min(iv[a].entry, iv[b].entry), hi = std::max(iv[a].entry, iv[b].entry);
      conf[size_t(hi)] = std::max(conf[size_t(hi)], lo);
    }
  return conf;
}

}  // namespace
}  // namespace mx

using namespace mx;

extern "C" int mx_adamw_step(const mx_adamw_tensor* tensors, int64_t count, const mx_adamw_hparams* hp_in,
                             int64_t* launches, void* stream) {
  MX_ABI_BEGIN
  if (launches) *launches = 0;
  MX_REQUIRE(hp_in, MX_ERR_INVALID, "fused AdamW: null hyperparameters");
  MX_REQUIRE(count >= 0, MX_ERR_INVALID, "fused AdamW: negative tensor count");
  const mx_adamw_hparams& h = *hp_in;
  MX_REQUIRE(h.lr >= 0 && h.beta1 >= 0 && h.beta1 < 1 && h.beta2 >= 0 && h.beta2 < 1 && h.eps >= 0 &&
                 h.weight_decay >= 0,
             MX_ERR_INVALID, "fused AdamW batch: invalid hyperparameters");
  if (count == 0) return MX_OK;
  MX_REQUIRE(tensors, MX_ERR_INVALID, "fused AdamW: null tensor list");
  const bool ams = h.amsgrad != 0;
  for (int64_t i = 0; i < count; ++i) {
    const mx_adamw_tensor& t = tensors[i];
    MX_REQUIRE(t.numel >= 0, MX_ERR_INVALID, "fused AdamW batch: negative numel at ", i);
    if (t.numel == 0) continue;
    MX_REQUIRE(t.param && t.grad && t.exp_avg && t.exp_avg_sq && (!ams || t.max_exp_avg_sq), MX_ERR_INVALID,
               "fused AdamW batch: null buffer at ", i);
    MX_REQUIRE(t.step_dev || t.step >= 1, MX_ERR_INVALID, "fused AdamW batch: step must be positive");
  }
  hipStream_t s = resolve_stream(stream);
  const std::vector<int64_t> conf = latest_conflict(tensors, count, ams, h.grad_scale != nullptr);
  AdamHP hp{};
  hp.lr = h.lr;
  hp.beta1 = h.beta1;
  hp.beta2 = h.beta2;
  hp.eps = h.eps;
  hp.wd = h.weight_decay;
  hp.lr_dev = h.lr_dev;
  hp.grad_scale = h.grad_scale;
  hp.found_inf = h.found_inf;
  hp.maximize = h.maximize;
  std::vector<AdamEntry> tab;
  int64_t first = 0;
  while (first < count) {
    // Extend the launch while no entry conflicts with one already in it.
    int64_t last = first + 1;
    while (last < count && conf[size_t(last)] < first) ++last;
    tab.clear();
    int64_t chunks = 0;
    for (int64_t i = first; i < last; ++i) {
      const mx_adamw_tensor& t = tensors[i];
      if (t.numel == 0) continue;
      AdamEntry e{};
      e.p = t.param;
      e.g = t.grad;
      e.m = t.exp_avg;
      e.v = t.exp_avg_sq;
      e.vmax = ams ? t.max_exp_avg_sq : nullptr;
      e.step_dev = t.step_dev;
      e.numel = t.numel;
      e.chunk_begin = chunks;
      if (!t.step_dev) {
        const double bc1 = 1.0 - std::pow(h.beta1, double(t.step));
        const double bc2 = 1.0 - std::pow(h.beta2, double(t.step));
        e.neg_step_size = h.lr_dev ? float(-1.0 / bc1) : float(-(h.lr / bc1));
        e.bc2_sqrt = float(std::sqrt(bc2));
      }
      e.vec = aligned16(e.p) && aligned16(e.g) && aligned16(e.m) && aligned16(e.v) && (!ams || aligned16(e.vmax));
      chunks += (t.numel + kChunk - 1) / kChunk;
      tab.push_back(e);
    }
    if (!tab.empty()) {
      hp.ntens = int(tab.size());
      hp.total_chunks = chunks;
      Scratch dtab;
      MX_TRY(upload(tab.data(), tab.size() * sizeof(AdamEntry), s, dtab));
      // 32 workgroups per CU: measured best for the 4-read / 3-write stream mix
      // (5.64 TB/s vs 5.59 at 16 and 5.56 at 4, one 125M-element tensor).
      const int64_t grid = std::max<int64_t>(1, std::min<int64_t>(chunks, int64_t(cu_count()) * 32));
      if (ams)
        hipLaunchKernelGGL(adamw_kernel<true>, dim3(unsigned(grid)), dim3(256), 0, s, dtab.as<AdamEntry>(), hp);
      else
        hipLaunchKernelGGL(adamw_kernel<false>, dim3(unsigned(grid)), dim3(256), 0, s, dtab.as<AdamEntry>(), hp);
      MX_HIP(hipGetLastError());
      if (launches) ++*launches;
    }
    first = last;
  }
  return MX_OK;
  MX_ABI_END
}
