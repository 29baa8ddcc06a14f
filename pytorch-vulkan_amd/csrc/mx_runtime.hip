// HIP runtime layer: errors, device selection, streams, events, the
// stream-ordered caching device allocator and the pinned upload ring.
//
// Replaces the reference's Vulkan runtime (VulkanContext,
// csrc/vulkan_context.cpp; VulkanAllocator, csrc/vulkan_allocator.cpp).  HIP
// launches are already asynchronous and device memory needs no host mirror,
// so only the ordering and safe-reuse semantics carry over: a freed block is
// reused on its own stream immediately (stream order protects it) and on other
// streams only after the events recorded at free time have completed.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <set>
#include <unordered_map>
#include <vector>

#include "mx_internal.hpp"

namespace mx {

static thread_local std::string g_last_error;

int set_error(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}
void clear_error() { g_last_error.clear(); }

static constexpr int kMaxDevices = 64;

int current_device() {
  int d = 0;
  if (hipGetDevice(&d) != hipSuccess) return 0;
  return d;
}

// ---------------------------------------------------------------- streams
static std::mutex g_stream_mu;
static hipStream_t g_default_stream[kMaxDevices] = {};

static int default_stream_for(int dev, hipStream_t* out) {
  std::lock_guard<std::mutex> lock(g_stream_mu);
  if (!g_default_stream[dev]) {
    int prev = 0;
    MX_HIP(hipGetDevice(&prev));
    if (prev != dev) MX_HIP(hipSetDevice(dev));
    hipStream_t s = nullptr;
    // Default priority only; non-blocking so it never serialises with the
    // legacy NULL stream used by other libraries in the process.
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (prev != dev) (void)hipSetDevice(prev);
    if (e != hipSuccess) return set_error(MX_ERR_HIP, cat("hipStreamCreateWithFlags: ", hipGetErrorString(e)));
    g_default_stream[dev] = s;
  }
  *out = g_default_stream[dev];
  return MX_OK;
}

// NULL is HIP's own null (legacy default) stream, as in the HIP API itself,
// so callers that use the null stream stay ordered with their own work.
hipStream_t resolve_stream(void* s) { return static_cast<hipStream_t>(s); }

int cu_count() {
  static int cached[kMaxDevices] = {};
  const int dev = current_device();
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// -------------------------------------------------------------- allocator
namespace {

constexpr size_t kSmallLimit = size_t(1) << 20;  // <= 1 MiB: 512 B classes
constexpr size_t kSmallRound = 512;
constexpr size_t kLargeRound = size_t(2) << 20;  // > 1 MiB: 2 MiB granules

size_t round_size(size_t bytes) {
  if (bytes <= kSmallLimit) return (bytes + kSmallRound - 1) / kSmallRound * kSmallRound;
  return (bytes + kLargeRound - 1) / kLargeRound * kLargeRound;
}

struct Block {
  void* ptr = nullptr;
  size_t size = 0;
  int device = 0;
  hipStream_t stream = nullptr;
  std::vector<hipStream_t> uses;  // other streams that touched the block
};

struct FreeKey {
  bool operator()(const Block* a, const Block* b) const {
    if (a->stream != b->stream) return std::less<hipStream_t>()(a->stream, b->stream);
    if (a->size != b->size) return a->size < b->size;
    return std::less<void*>()(a->ptr, b->ptr);
  }
};

struct Pending {
  Block* block;
  std::vector<hipEvent_t> events;
};

struct DevicePool {
  std::set<Block*, FreeKey> free_blocks;
  std::vector<Pending> pending;
};

std::mutex g_alloc_mu;
std::unordered_map<void*, Block*> g_live;
DevicePool g_pools[kMaxDevices];
mx_memory_stats g_stats = {};

// Moves pending blocks whose cross-stream events completed into the free set.
void process_pending(DevicePool& pool) {
  auto& pend = pool.pending;
  for (size_t i = 0; i < pend.size();) {
    bool done = true;
    for (auto ev : pend[i].events)
      if (hipEventQuery(ev) != hipSuccess) {
        done = false;
        break;
      }
    if (done) {
      for (auto ev : pend[i].events) (void)hipEventDestroy(ev);
      pend[i].block->uses.clear();
      pool.free_blocks.insert(pend[i].block);
      pend[i] = pend.back();
      pend.pop_back();
    } else {
      ++i;
    }
  }
}

// Releases every cached (free) block of `dev` back to HIP.  Caller holds the lock.
void release_cached(int dev) {
  auto& pool = g_pools[dev];
  for (Block* b : pool.free_blocks) {
    (void)hipFree(b->ptr);
    g_stats.reserved_bytes -= b->size;
    delete b;
  }
  pool.free_blocks.clear();
}

}  // namespace

void release_host_cache();  // the page-locked host block cache, below

}  // namespace mx

using namespace mx;

extern "C" {

const char* mx_last_error(void) { return g_last_error.c_str(); }
int mx_abi_version(void) { return 3; }

int mx_init(int ordinal) {
  MX_ABI_BEGIN
  int count = 0;
  MX_HIP(hipGetDeviceCount(&count));
  MX_REQUIRE(ordinal >= 0 && ordinal < count && ordinal < kMaxDevices, MX_ERR_INVALID,
             "mx_init: invalid device ordinal ", ordinal, " (", count, " devices)");
  MX_HIP(hipSetDevice(ordinal));
  hipStream_t s;
  MX_TRY(default_stream_for(ordinal, &s));
  return MX_OK;
  MX_ABI_END
}

int mx_device_count(int* count) {
  MX_ABI_BEGIN
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  *count = e == hipSuccess ? n : 0;
  return MX_OK;
  MX_ABI_END
}

int mx_get_device(int* ordinal) {
  MX_ABI_BEGIN
  MX_HIP(hipGetDevice(ordinal));
  return MX_OK;
  MX_ABI_END
}

int mx_set_device(int ordinal) {
  MX_ABI_BEGIN
  MX_REQUIRE(ordinal >= 0 && ordinal < kMaxDevices, MX_ERR_INVALID, "invalid device ", ordinal);
  MX_HIP(hipSetDevice(ordinal));
  return MX_OK;
  MX_ABI_END
}

int mx_device_name(int ordinal, char* buf, size_t len) {
  MX_ABI_BEGIN
  hipDeviceProp_t prop;
  MX_HIP(hipGetDeviceProperties(&prop, ordinal));
  std::string name = cat(prop.name, " (", prop.gcnArchName, ", ", prop.multiProcessorCount, " CUs)");
  if (len) {
    std::strncpy(buf, name.c_str(), len - 1);
    buf[len - 1] = 0;
  }
  return MX_OK;
  MX_ABI_END
}

int mx_device_synchronize(void) {
  MX_ABI_BEGIN
  MX_HIP(hipDeviceSynchronize());
  return MX_OK;
  MX_ABI_END
}

int mx_default_stream(void** stream) {
  MX_ABI_BEGIN
  hipStream_t s;
  MX_TRY(default_stream_for(current_device(), &s));
  *stream = s;
  return MX_OK;
  MX_ABI_END
}

int mx_stream_create(void** stream) {
  MX_ABI_BEGIN
  hipStream_t s;
  MX_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = s;
  return MX_OK;
  MX_ABI_END
}

int mx_stream_destroy(void* stream) {
  MX_ABI_BEGIN
  if (stream) MX_HIP(hipStreamDestroy(static_cast<hipStream_t>(stream)));
  return MX_OK;
  MX_ABI_END
}

int mx_stream_synchronize(void* stream) {
  MX_ABI_BEGIN
  MX_HIP(hipStreamSynchronize(resolve_stream(stream)));
  return MX_OK;
  MX_ABI_END
}

int mx_stream_query(void* stream, int* done) {
  MX_ABI_BEGIN
  hipError_t e = hipStreamQuery(resolve_stream(stream));
  if (e == hipSuccess) *done = 1;
  else if (e == hipErrorNotReady) *done = 0;
  else return set_error(MX_ERR_HIP, cat("hipStreamQuery: ", hipGetErrorString(e)));
  return MX_OK;
  MX_ABI_END
}

int mx_stream_wait_event(void* stream, void* event) {
  MX_ABI_BEGIN
  MX_HIP(hipStreamWaitEvent(resolve_stream(stream), static_cast<hipEvent_t>(event), 0));
  return MX_OK;
  MX_ABI_END
}

int mx_event_create(void** event, int enable_timing) {
  MX_ABI_BEGIN
  hipEvent_t e;
  MX_HIP(hipEventCreateWithFlags(&e, enable_timing ? hipEventDefault : hipEventDisableTiming));
  *event = e;
  return MX_OK;
  MX_ABI_END
}

int mx_event_destroy(void* event) {
  MX_ABI_BEGIN
  if (event) MX_HIP(hipEventDestroy(static_cast<hipEvent_t>(event)));
  return MX_OK;
  MX_ABI_END
}

int mx_event_record(void* event, void* stream) {
  MX_ABI_BEGIN
  MX_HIP(hipEventRecord(static_cast<hipEvent_t>(event), resolve_stream(stream)));
  return MX_OK;
  MX_ABI_END
}

int mx_event_query(void* event, int* done) {
  MX_ABI_BEGIN
  hipError_t e = hipEventQuery(static_cast<hipEvent_t>(event));
  if (e == hipSuccess) *done = 1;
  else if (e == hipErrorNotReady) *done = 0;
  else return set_error(MX_ERR_HIP, cat("hipEventQuery: ", hipGetErrorString(e)));
  return MX_OK;
  MX_ABI_END
}

int mx_event_synchronize(void* event) {
  MX_ABI_BEGIN
  MX_HIP(hipEventSynchronize(static_cast<hipEvent_t>(event)));
  return MX_OK;
  MX_ABI_END
}

int mx_event_elapsed_ms(void* start, void* end, float* ms) {
  MX_ABI_BEGIN
  MX_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end)));
  return MX_OK;
  MX_ABI_END
}

int mx_malloc(void** ptr, size_t bytes, void* stream) {
  MX_ABI_BEGIN
  *ptr = nullptr;
  if (bytes == 0) return MX_OK;
  const int dev = current_device();
  MX_REQUIRE(dev >= 0 && dev < kMaxDevices, MX_ERR_INVALID, "device out of range");
  hipStream_t s = resolve_stream(stream);
  const size_t size = round_size(bytes);
  std::lock_guard<std::mutex> lock(g_alloc_mu);
  auto& pool = g_pools[dev];
  if (!pool.pending.empty()) process_pending(pool);
  // Best fit on the same stream.  Small classes must match exactly; large
  // blocks may exceed the request by at most a quarter.
  Block probe;
  probe.stream = s;
  probe.size = size;
  probe.ptr = nullptr;
  auto it = pool.free_blocks.lower_bound(&probe);
  if (it != pool.free_blocks.end() && (*it)->stream == s &&
      ((*it)->size == size || (size > kSmallLimit && (*it)->size <= size + size / 4))) {
    Block* b = *it;
    pool.free_blocks.erase(it);
    g_live[b->ptr] = b;
    g_stats.allocated_bytes += b->size;
    g_stats.cache_hits++;
    g_stats.cached_blocks = pool.free_blocks.size();
    *ptr = b->ptr;
    return MX_OK;
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, size);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    // Out of memory: wait for in-flight work, release the cache and retry.
    (void)hipDeviceSynchronize();
    process_pending(pool);
    release_cached(dev);
    e = hipMalloc(&p, size);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return set_error(MX_ERR_OOM, cat("mx_malloc: out of device memory allocating ", bytes, " bytes"));
    }
  }
  Block* b = new Block();
  b->ptr = p;
  b->size = size;
  b->device = dev;
  b->stream = s;
  g_live[p] = b;
  g_stats.allocated_bytes += size;
  g_stats.reserved_bytes += size;
  g_stats.device_mallocs++;
  *ptr = p;
  return MX_OK;
  MX_ABI_END
}

int mx_free(void* ptr) {
  MX_ABI_BEGIN
  if (!ptr) return MX_OK;
  std::lock_guard<std::mutex> lock(g_alloc_mu);
  auto it = g_live.find(ptr);
  MX_REQUIRE(it != g_live.end(), MX_ERR_INVALID, "mx_free: pointer not owned by the allocator");
  Block* b = it->second;
  g_live.erase(it);
  g_stats.allocated_bytes -= b->size;
  auto& pool = g_pools[b->device];
  if (b->uses.empty()) {
    pool.free_blocks.insert(b);
  } else {
    Pending p{b, {}};
    for (hipStream_t s : b->uses) {
      hipEvent_t ev;
      if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) continue;
      (void)hipEventRecord(ev, s);
      p.events.push_back(ev);
    }
    pool.pending.push_back(std::move(p));
  }
  g_stats.cached_blocks = pool.free_blocks.size();
  return MX_OK;
  MX_ABI_END
}

int mx_record_stream(void* ptr, void* stream) {
  MX_ABI_BEGIN
  if (!ptr) return MX_OK;
  hipStream_t s = resolve_stream(stream);
  std::lock_guard<std::mutex> lock(g_alloc_mu);
  auto it = g_live.find(ptr);
  MX_REQUIRE(it != g_live.end(), MX_ERR_INVALID, "mx_record_stream: pointer not owned by the allocator");
  Block* b = it->second;
  if (s != b->stream && std::find(b->uses.begin(), b->uses.end(), s) == b->uses.end()) b->uses.push_back(s);
  return MX_OK;
  MX_ABI_END
}

int mx_empty_cache(void) {
  MX_ABI_BEGIN
  std::lock_guard<std::mutex> lock(g_alloc_mu);
  const int dev = current_device();
  (void)hipDeviceSynchronize();
  process_pending(g_pools[dev]);
  release_cached(dev);
  g_stats.cached_blocks = 0;
  release_host_cache();
  return MX_OK;
  MX_ABI_END
}

int mx_memory_stats_get(mx_memory_stats* out) {
  MX_ABI_BEGIN
  std::lock_guard<std::mutex> lock(g_alloc_mu);
  *out = g_stats;
  return MX_OK;
  MX_ABI_END
}

int mx_memcpy(void* dst, const void* src, size_t bytes, int kind, void* stream) {
  MX_ABI_BEGIN
  if (!bytes) return MX_OK;
  hipStream_t s = resolve_stream(stream);
  hipMemcpyKind k;
  switch (kind) {
    case MX_COPY_H2D: k = hipMemcpyHostToDevice; break;
    case MX_COPY_D2H: k = hipMemcpyDeviceToHost; break;
    case MX_COPY_D2D: k = hipMemcpyDeviceToDevice; break;
    default: return set_error(MX_ERR_INVALID, cat("mx_memcpy: bad kind ", kind));
  }
  MX_HIP(hipMemcpyAsync(dst, src, bytes, k, s));
  // Host buffers may be pageable and are reused by the caller on return.
  if (kind != MX_COPY_D2D) MX_HIP(hipStreamSynchronize(s));
  return MX_OK;
  MX_ABI_END
}

}  // extern "C"

namespace mx {
namespace {
// Page-locked host blocks, cached by rounded size.  A freed block is reusable
// at once: the PyTorch layer keeps a host storage alive until every
// asynchronous copy that reads or writes it has completed, and host code is
// synchronous.
std::mutex g_host_mu;
std::unordered_map<void*, size_t> g_host_live;        // pointer -> rounded size
std::multimap<size_t, void*> g_host_free;             // rounded size -> cached block

size_t host_round(size_t bytes) {
  if (bytes <= (size_t(1) << 20)) {
    size_t r = 512;
    while (r < bytes) r <<= 1;
    return r;
  }
  const size_t g = size_t(2) << 20;
  return (bytes + g - 1) / g * g;
}
}  // namespace

void release_host_cache() {
  std::lock_guard<std::mutex> lock(g_host_mu);
  for (auto& kv : g_host_free) (void)hipHostFree(kv.second);
  g_host_free.clear();
}
}  // namespace mx

extern "C" {

int mx_host_malloc(void** ptr, size_t bytes) {
  MX_ABI_BEGIN
  *ptr = nullptr;
  if (bytes == 0) return MX_OK;
  const size_t r = host_round(bytes);
  std::lock_guard<std::mutex> lock(g_host_mu);
  auto it = g_host_free.find(r);
  void* p = nullptr;
  if (it != g_host_free.end()) {
    p = it->second;
    g_host_free.erase(it);
  } else {
    MX_HIP(hipHostMalloc(&p, r, hipHostMallocDefault));
  }
  g_host_live[p] = r;
  *ptr = p;
  return MX_OK;
  MX_ABI_END
}

int mx_host_free(void* ptr) {
  MX_ABI_BEGIN
  if (!ptr) return MX_OK;
  std::lock_guard<std::mutex> lock(g_host_mu);
  auto it = g_host_live.find(ptr);
  MX_REQUIRE(it != g_host_live.end(), MX_ERR_INVALID, "mx_host_free: pointer not from mx_host_malloc");
  g_host_free.emplace(it->second, ptr);
  g_host_live.erase(it);
  return MX_OK;
  MX_ABI_END
}

int mx_host_is_pinned(const void* ptr, int* pinned) {
  MX_ABI_BEGIN
  *pinned = 0;
  if (!ptr) return MX_OK;
  hipPointerAttribute_t attr;
  std::memset(&attr, 0, sizeof(attr));
  if (hipPointerGetAttributes(&attr, ptr) != hipSuccess) {
    (void)hipGetLastError();  // memory HIP does not know: pageable, not an error
    return MX_OK;
  }
  *pinned = attr.type == hipMemoryTypeHost ? 1 : 0;
  return MX_OK;
  MX_ABI_END
}

int mx_memcpy_async(void* dst, const void* src, size_t bytes, int kind, void* stream) {
  MX_ABI_BEGIN
  if (!bytes) return MX_OK;
  if (kind != MX_COPY_H2D && kind != MX_COPY_D2H)
    return set_error(MX_ERR_INVALID, cat("mx_memcpy_async: kind must be H2D or D2H, got ", kind));
  const char* host = static_cast<const char*>(kind == MX_COPY_H2D ? src : dst);
  int first = 0, last = 0;
  int rc = mx_host_is_pinned(host, &first);
  if (rc != MX_OK) return rc;
  rc = mx_host_is_pinned(host + bytes - 1, &last);
  if (rc != MX_OK) return rc;
  if (!first || !last)
    return set_error(MX_ERR_INVALID, "mx_memcpy_async: the host buffer is not page-locked (hipHostMalloc) memory");
  MX_HIP(hipMemcpyAsync(dst, src, bytes, kind == MX_COPY_H2D ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost,
                        resolve_stream(stream)));
  return MX_OK;
  MX_ABI_END
}

}  // extern "C"

namespace mx {

// ----------------------------------------------------------- pinned upload ring
namespace {
constexpr size_t kRingBytes = size_t(8) << 20;
struct RingSlot {
  size_t off, size;
  hipEvent_t ev;
};
std::mutex g_ring_mu;
char* g_ring = nullptr;      // host address of the page-locked ring
char* g_ring_dev = nullptr;  // the same memory as the device addresses it
size_t g_ring_head = 0;
std::vector<RingSlot> g_ring_slots;  // FIFO of in-flight regions

// Device-side copy of a staged table out of the page-locked ring.  A kernel on
// the caller's stream starts a few microseconds after the previous one; a
// DMA-engine copy (hipMemcpyAsync) costs its ~6 us transfer plus a ~30 us
// hand-over between the copy engine and the compute queue before the kernel
// that reads the table can start.
__global__ __launch_bounds__(256) void ring_copy_kernel(const char* __restrict__ src, char* __restrict__ dst,
                                                        size_t bytes) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const size_t n16 = bytes / 16;
  for (size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += size_t(gridDim.x) * blockDim.x)
    reinterpret_cast<u32x4*>(dst)[i] = reinterpret_cast<const u32x4*>(src)[i];
  if (blockIdx.x == 0 && threadIdx.x < bytes % 16) dst[n16 * 16 + threadIdx.x] = src[n16 * 16 + threadIdx.x];
}
}  // namespace

int upload(const void* host, size_t bytes, hipStream_t s, Scratch& holder) {
  MX_REQUIRE(bytes <= kRingBytes / 2, MX_ERR_INVALID, "upload: table of ", bytes, " bytes too large");
  MX_TRY(holder.alloc(bytes, s));
  std::lock_guard<std::mutex> lock(g_ring_mu);
  if (!g_ring) {
    char* ring = nullptr;
    MX_HIP(hipHostMalloc(reinterpret_cast<void**>(&ring), kRingBytes, hipHostMallocMapped | hipHostMallocPortable));
    void* dev = nullptr;
    const hipError_t e = hipHostGetDevicePointer(&dev, ring, 0);
    if (e != hipSuccess) {
      (void)hipHostFree(ring);
      return set_error(MX_ERR_HIP, cat("hipHostGetDevicePointer (upload ring): ", hipGetErrorString(e)));
    }
    g_ring = ring;
    g_ring_dev = static_cast<char*>(dev);
  }
  const size_t sz = (bytes + 255) / 256 * 256;
  size_t off = g_ring_head;
  if (off + sz > kRingBytes) off = 0;
  // Wait for older copies that still read the region we are about to overwrite.
  for (size_t i = 0; i < g_ring_slots.size();) {
    auto& sl = g_ring_slots[i];
    bool overlap = sl.off < off + sz && off < sl.off + sl.size;
    bool done = hipEventQuery(sl.ev) == hipSuccess;
    if (overlap && !done) {
      MX_HIP(hipEventSynchronize(sl.ev));
      done = true;
    }
    if (done) {
      (void)hipEventDestroy(sl.ev);
      g_ring_slots.erase(g_ring_slots.begin() + i);
    } else {
      ++i;
    }
  }
  std::memcpy(g_ring + off, host, bytes);
  // Ring offsets are 256-byte aligned and device blocks 512-byte aligned, so
  // both ends of the copy are 16-byte aligned.
  const unsigned blocks = unsigned(std::min<size_t>((bytes / 16 + 255) / 256, 64));
  hipLaunchKernelGGL(ring_copy_kernel, dim3(std::max(blocks, 1u)), dim3(256), 0, s, g_ring_dev + off,
                     static_cast<char*>(holder.ptr), bytes);
  MX_HIP(hipGetLastError());
  hipEvent_t ev;
  MX_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  MX_HIP(hipEventRecord(ev, s));
  g_ring_slots.push_back({off, sz, ev});
  g_ring_head = off + sz;
  return MX_OK;
}

}  // namespace mx
