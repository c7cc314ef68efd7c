// Shared definitions for libdtmi: status codes, error reporting, the library
// stream, the device-memory pool and the per-kernel-family timing hooks.
//
// Every exported entry point returns an int status (0 = ok). A failure stores a
// thread-local message that dtmi_last_error() returns. No C++ exception crosses
// the C ABI: bodies run inside DTMI_BODY_BEGIN / DTMI_BODY_END.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "dtmi.h"

#define DTMI_EXPORT extern "C" __attribute__((visibility("default")))

namespace dtmi {

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail_hip(hipError_t e, const char* what, const char* file, int line);

// The one HIP stream every kernel, copy and fill of the library is ordered on.
hipStream_t stream();
bool initialized();
int num_cus();
int device_id();  // the device dtmi_init selected (-1 before)

// Set-up of the allocation-free LayerNorm backward's device scratch array on
// `device` (which must be current); called once per device by dtmi_init.
int ln_scratch_setup(int device);

// Pooled device allocation (stream-ordered reuse on the single library stream).
int pool_alloc(void** p, size_t bytes);
int pool_free(void* p);

// Timing hooks: when timing is enabled the launch wrappers bracket each launch
// of a kernel family with events on the library stream.
struct TimedLaunch {
  int family;
  double work;  // algorithmic FLOP or bytes of this launch
  int slot;
  TimedLaunch(int fam, double w);
  ~TimedLaunch();
};

// Multi-tensor tables are uploaded to a pooled device buffer; the buffer is
// returned to the pool right after the launch that reads it (stream order).
int upload_table(const void* host, size_t bytes, void** dev);

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
__host__ __device__ inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace dtmi

#define DTMI_BODY_BEGIN try {
#define DTMI_BODY_END                                                  \
  }                                                                    \
  catch (...) {                                                        \
    return dtmi::fail(DTMI_ERR_INTERNAL, "%s: C++ exception", __func__); \
  }

#define DTMI_REQUIRE_INIT()                                                                \
  do {                                                                                     \
    if (!dtmi::initialized()) return dtmi::fail(DTMI_ERR_NOT_INITIALIZED, "%s: call dtmi_init first", __func__); \
  } while (0)

#define HIP_TRY(expr)                                                 \
  do {                                                                \
    hipError_t _e = (expr);                                           \
    if (_e != hipSuccess) return dtmi::fail_hip(_e, #expr, __FILE__, __LINE__); \
  } while (0)

#define LAUNCH_CHECK(name)                                            \
  do {                                                                \
    hipError_t _e = hipGetLastError();                                \
    if (_e != hipSuccess) return dtmi::fail_hip(_e, name, __FILE__, __LINE__); \
  } while (0)

#define DTMI_CHECK(cond, ...)                                         \
  do {                                                                \
    if (!(cond)) return dtmi::fail(DTMI_ERR_INVALID, __VA_ARGS__);    \
  } while (0)

#define DTMI_DTYPE_OK(dt) DTMI_CHECK((dt) == DTMI_F32 || (dt) == DTMI_F64, "%s: dtype must be DTMI_F32 or DTMI_F64 (got %d)", __func__, (int)(dt))
