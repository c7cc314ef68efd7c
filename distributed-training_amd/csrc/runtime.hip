// libdtmi runtime: device selection, the library stream, a caching device-memory
// pool, pinned staging for host-to-device uploads, fills, events and
// per-kernel-family launch timing.
//
// One process drives one GPU on one stream. Device memory handed back with
// dtmi_free goes to a per-size free list and is reused by later allocations;
// because every kernel and copy of the library is ordered on the same stream,
// a block freed on the host can be reused at once without a wait.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "common.h"

namespace dtmi {

static thread_local char g_err[1024] = "";
static int g_device = -1;
static hipStream_t g_stream = nullptr;
static int g_num_cus = 0;
static std::mutex g_mu;

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int fail_hip(hipError_t e, const char* what, const char* file, int line) {
  const char* base = strrchr(file, '/');
  snprintf(g_err, sizeof(g_err), "HIP error %d (%s) in %s at %s:%d", (int)e, hipGetErrorString(e), what,
           base ? base + 1 : file, line);
  return e == hipErrorOutOfMemory ? DTMI_ERR_OOM : DTMI_ERR_HIP;
}

hipStream_t stream() { return g_stream; }
bool initialized() { return g_stream != nullptr; }
int num_cus() { return g_num_cus; }
int device_id() { return g_device; }

// ------------------------------------------------------------------ pool
// Sizes are rounded up (256 B granules below 1 MiB, 64 KiB granules below
// 64 MiB, 2 MiB above) and freed blocks are kept on exact-size free lists.
static std::map<size_t, std::vector<void*>> g_free;
static std::unordered_map<void*, size_t> g_live;
static size_t g_in_use = 0, g_cached = 0, g_peak = 0;

static size_t round_size(size_t b) {
  if (b == 0) b = 1;
  if (b < (1u << 20)) return (b + 255) & ~size_t(255);
  if (b < (64u << 20)) return (b + 65535) & ~size_t(65535);
  return (b + (2u << 20) - 1) & ~size_t((2u << 20) - 1);
}

static void release_cached_locked() {
  for (auto& kv : g_free)
    for (void* p : kv.second) {
      (void)hipFree(p);
      g_cached -= kv.first;
    }
  g_free.clear();
}

int pool_alloc(void** out, size_t bytes) {
  std::lock_guard<std::mutex> lk(g_mu);
  size_t sz = round_size(bytes);
  auto it = g_free.find(sz);
  void* p = nullptr;
  if (it != g_free.end() && !it->second.empty()) {
    p = it->second.back();
    it->second.pop_back();
    g_cached -= sz;
  } else {
    hipError_t e = hipMalloc(&p, sz);
    if (e == hipErrorOutOfMemory) {
      (void)hipGetLastError();
      // Blocks on the free lists may still be read by queued kernels; wait
      // for the stream before handing them back to HIP.
      (void)hipStreamSynchronize(g_stream);
      release_cached_locked();
      e = hipMalloc(&p, sz);
    }
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return fail(DTMI_ERR_OOM, "dtmi_malloc: out of device memory allocating %zu bytes (in use %zu)", sz, g_in_use);
    }
  }
  g_live[p] = sz;
  g_in_use += sz;
  if (g_in_use > g_peak) g_peak = g_in_use;
  *out = p;
  return DTMI_OK;
}

int pool_free(void* p) {
  if (!p) return DTMI_OK;
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_live.find(p);
  if (it == g_live.end()) return fail(DTMI_ERR_INVALID, "dtmi_free: %p was not allocated by dtmi_malloc", p);
  size_t sz = it->second;
  g_live.erase(it);
  g_in_use -= sz;
  g_free[sz].push_back(p);
  g_cached += sz;
  return DTMI_OK;
}

// --------------------------------------------------------- pinned staging
// Host-to-device uploads are copied into a pinned ring and sent with an async
// copy, so an upload does not stall the stream. A ring region is reused only
// after the event recorded behind its copy has completed.
static const size_t kStageBytes = size_t(64) << 20;
static char* g_stage = nullptr;
static size_t g_stage_head = 0;
struct StageRegion {
  size_t begin, end;
  hipEvent_t ev;
};
static std::vector<StageRegion> g_stage_regions;

static int stage_wait_overlap(size_t begin, size_t end) {
  for (size_t i = 0; i < g_stage_regions.size();) {
    StageRegion& r = g_stage_regions[i];
    bool overlap = r.begin < end && begin < r.end;
    bool done = hipEventQuery(r.ev) == hipSuccess;
    if (overlap && !done) HIP_TRY(hipEventSynchronize(r.ev));
    if (overlap || done) {
      HIP_TRY(hipEventDestroy(r.ev));
      g_stage_regions.erase(g_stage_regions.begin() + i);
    } else {
      ++i;
    }
  }
  return DTMI_OK;
}

static int staged_h2d(void* dst, const void* src, size_t bytes) {
  if (bytes > kStageBytes / 2 || g_stage == nullptr) {
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
    HIP_TRY(hipStreamSynchronize(g_stream));
    return DTMI_OK;
  }
  size_t need = (bytes + 255) & ~size_t(255);
  if (g_stage_head + need > kStageBytes) g_stage_head = 0;
  size_t begin = g_stage_head, end = begin + need;
  int rc = stage_wait_overlap(begin, end);
  if (rc) return rc;
  memcpy(g_stage + begin, src, bytes);
  HIP_TRY(hipMemcpyAsync(dst, g_stage + begin, bytes, hipMemcpyHostToDevice, g_stream));
  hipEvent_t ev;
  HIP_TRY(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  HIP_TRY(hipEventRecord(ev, g_stream));
  g_stage_regions.push_back({begin, end, ev});
  g_stage_head = end;
  return DTMI_OK;
}

int upload_table(const void* host, size_t bytes, void** dev) {
  int rc = pool_alloc(dev, bytes);
  if (rc) return rc;
  rc = staged_h2d(*dev, host, bytes);
  if (rc) {
    pool_free(*dev);
    return rc;
  }
  return DTMI_OK;
}

// ------------------------------------------------------------------ timing
static bool g_timing = false;
struct FamStats {
  int64_t launches = 0;
  double ms = 0, work = 0;
};
static FamStats g_fam[DTMI_FAM_COUNT];
struct PendingTiming {
  int family;
  double work;
  hipEvent_t a, b;
};
static std::vector<PendingTiming> g_pending;

static void drain_pending(bool wait) {
  size_t keep = 0;
  for (size_t i = 0; i < g_pending.size(); ++i) {
    PendingTiming& t = g_pending[i];
    if (!wait && hipEventQuery(t.b) != hipSuccess) {
      g_pending[keep++] = t;
      continue;
    }
    float ms = 0;
    if (hipEventSynchronize(t.b) == hipSuccess && hipEventElapsedTime(&ms, t.a, t.b) == hipSuccess) {
      g_fam[t.family].launches += 1;
      g_fam[t.family].ms += ms;
      g_fam[t.family].work += t.work;
    }
    (void)hipEventDestroy(t.a);
    (void)hipEventDestroy(t.b);
  }
  g_pending.resize(keep);
}

TimedLaunch::TimedLaunch(int fam, double w) : family(fam), work(w), slot(-1) {
  if (!g_timing || fam < 0) return;  // family -1: never timed (creates no events)
  if (g_pending.size() > 4096) drain_pending(false);
  PendingTiming t{fam, w, nullptr, nullptr};
  // timing-only events: no system-scope cache writeback and invalidate when
  // recorded, which would otherwise add to the bracketed launch and leave the
  // next kernel with a cold L2
  if (hipEventCreateWithFlags(&t.a, hipEventDisableSystemFence) != hipSuccess) return;
  if (hipEventCreateWithFlags(&t.b, hipEventDisableSystemFence) != hipSuccess) {
    (void)hipEventDestroy(t.a);
    return;
  }
  (void)hipEventRecord(t.a, g_stream);
  g_pending.push_back(t);
  slot = (int)g_pending.size() - 1;
}

TimedLaunch::~TimedLaunch() {
  if (slot < 0) return;
  (void)hipEventRecord(g_pending[slot].b, g_stream);
}

// ----------------------------------------------------------------- kernels
template <typename T>
__global__ void fill_kernel(T* __restrict__ x, T value, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) x[i] = value;
}

__global__ void zero_bytes_kernel(uint8_t* __restrict__ x, size_t nbytes) {
  // 16-byte body when aligned (checked on the host), byte tail.
  size_t nvec = nbytes / 16;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  uint4 z = {0, 0, 0, 0};
  for (size_t k = i; k < nvec; k += stride) reinterpret_cast<uint4*>(x)[k] = z;
  for (size_t k = nvec * 16 + i; k < nbytes; k += stride) x[k] = 0;
}

__global__ void zero_bytes_unaligned_kernel(uint8_t* __restrict__ x, size_t nbytes) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < nbytes; i += stride) x[i] = 0;
}

static int grid_for(int64_t n, int per_thread = 4) {
  int64_t b = cdiv(n, 256LL * per_thread);
  if (b < 1) b = 1;
  int64_t cap = (int64_t)g_num_cus * 16;
  if (cap < 1) cap = 1024;
  return (int)(b < cap ? b : cap);
}

}  // namespace dtmi

using namespace dtmi;

DTMI_EXPORT const char* dtmi_last_error(void) { return dtmi::g_err; }

DTMI_EXPORT int dtmi_init(int device) {
  DTMI_BODY_BEGIN
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_stream != nullptr) {
    DTMI_CHECK(device == g_device, "dtmi_init: already initialised on device %d (asked for %d)", g_device, device);
    return DTMI_OK;
  }
  int count = 0;
  HIP_TRY(hipGetDeviceCount(&count));
  DTMI_CHECK(device >= 0 && device < count, "dtmi_init: device %d out of range (%d devices)", device, count);
  HIP_TRY(hipSetDevice(device));
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, device));
  g_num_cus = prop.multiProcessorCount;
  {
    int rc = ln_scratch_setup(device);
    if (rc) return rc;
  }
  HIP_TRY(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
  void* stage = nullptr;
  if (hipHostMalloc(&stage, kStageBytes, hipHostMallocDefault) == hipSuccess) {
    g_stage = static_cast<char*>(stage);
  } else {
    (void)hipGetLastError();
    g_stage = nullptr;  // uploads fall back to synchronous copies
  }
  g_device = device;
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_device_info(int* num_cus, size_t* hbm_bytes, char* name, int name_len) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, g_device));
  if (num_cus) *num_cus = prop.multiProcessorCount;
  if (hbm_bytes) *hbm_bytes = prop.totalGlobalMem;
  if (name && name_len > 0) {
    snprintf(name, (size_t)name_len, "%s (%s)", prop.name, prop.gcnArchName);
  }
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_malloc(void** ptr, size_t bytes) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_CHECK(ptr != nullptr, "dtmi_malloc: ptr is NULL");
  return pool_alloc(ptr, bytes);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_free(void* ptr) {
  DTMI_BODY_BEGIN
  if (!initialized()) return DTMI_OK;  // interpreter shutdown after the runtime went away
  return pool_free(ptr);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_empty_cache(void) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  HIP_TRY(hipStreamSynchronize(g_stream));
  std::lock_guard<std::mutex> lk(g_mu);
  release_cached_locked();
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_memory_stats(size_t* in_use, size_t* cached, size_t* peak) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (in_use) *in_use = g_in_use;
  if (cached) *cached = g_cached;
  if (peak) *peak = g_peak;
  return DTMI_OK;
}

DTMI_EXPORT int dtmi_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  if (bytes == 0) return DTMI_OK;
  DTMI_CHECK(dst && src, "dtmi_memcpy_h2d: NULL pointer");
  return staged_h2d(dst, src, bytes);
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  if (bytes == 0) return DTMI_OK;
  DTMI_CHECK(dst && src, "dtmi_memcpy_d2h: NULL pointer");
  HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
  HIP_TRY(hipStreamSynchronize(g_stream));
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_memcpy_d2d(void* dst, const void* src, size_t bytes) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  if (bytes == 0) return DTMI_OK;
  DTMI_CHECK(dst && src, "dtmi_memcpy_d2d: NULL pointer");
  TimedLaunch tl(DTMI_FAM_OTHER, 2.0 * (double)bytes);
  HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream));
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_fill(int dtype, void* x, double value, int64_t n) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_DTYPE_OK(dtype);
  DTMI_CHECK(n >= 0, "dtmi_fill: negative size");
  if (n == 0) return DTMI_OK;
  DTMI_CHECK(x != nullptr, "dtmi_fill: NULL pointer");
  TimedLaunch tl(DTMI_FAM_OTHER, (double)n * (dtype == DTMI_F32 ? 4 : 8));
  int grid = grid_for(n);
  if (dtype == DTMI_F32)
    fill_kernel<float><<<grid, 256, 0, g_stream>>>(static_cast<float*>(x), (float)value, n);
  else
    fill_kernel<double><<<grid, 256, 0, g_stream>>>(static_cast<double*>(x), value, n);
  LAUNCH_CHECK("fill_kernel");
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_zero_bytes(void* x, size_t bytes) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  if (bytes == 0) return DTMI_OK;
  DTMI_CHECK(x != nullptr, "dtmi_zero_bytes: NULL pointer");
  TimedLaunch tl(DTMI_FAM_OTHER, (double)bytes);
  int grid = grid_for((int64_t)(bytes / 16 + 1));
  if (aligned(x, 16))
    zero_bytes_kernel<<<grid, 256, 0, g_stream>>>(static_cast<uint8_t*>(x), bytes);
  else
    zero_bytes_unaligned_kernel<<<grid_for((int64_t)bytes), 256, 0, g_stream>>>(static_cast<uint8_t*>(x), bytes);
  LAUNCH_CHECK("zero_bytes_kernel");
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_sync(void) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  HIP_TRY(hipStreamSynchronize(g_stream));
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_event_create(void** ev) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_CHECK(ev != nullptr, "dtmi_event_create: NULL");
  hipEvent_t e;
  HIP_TRY(hipEventCreate(&e));
  *ev = (void*)e;
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_event_record(void* ev) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  HIP_TRY(hipEventRecord((hipEvent_t)ev, g_stream));
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_event_elapsed_ms(void* start, void* stop, float* ms) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  HIP_TRY(hipEventSynchronize((hipEvent_t)stop));
  HIP_TRY(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_event_destroy(void* ev) {
  DTMI_BODY_BEGIN
  HIP_TRY(hipEventDestroy((hipEvent_t)ev));
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_timing_enable(int enable) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  HIP_TRY(hipStreamSynchronize(g_stream));
  drain_pending(true);
  if (enable)
    for (auto& f : g_fam) f = FamStats();
  g_timing = enable != 0;
  return DTMI_OK;
  DTMI_BODY_END
}

DTMI_EXPORT int dtmi_timing_read(int family, int64_t* launches, double* ms, double* work) {
  DTMI_BODY_BEGIN
  DTMI_REQUIRE_INIT();
  DTMI_CHECK(family >= 0 && family < DTMI_FAM_COUNT, "dtmi_timing_read: bad family %d", family);
  HIP_TRY(hipStreamSynchronize(g_stream));
  drain_pending(true);
  if (launches) *launches = g_fam[family].launches;
  if (ms) *ms = g_fam[family].ms;
  if (work) *work = g_fam[family].work;
  return DTMI_OK;
  DTMI_BODY_END
}
