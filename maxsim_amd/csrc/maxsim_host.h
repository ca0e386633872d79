// Host-side helpers shared by the C-ABI entry points: error reporting and
// argument checks.  The error message is thread-local; every entry point
// clears it on entry.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "../../include/maxsim_amd.h"

namespace maxsim {

void clear_error();
// Records a printf-style message and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// hipGetLastError() after a launch -> MAXSIM_ERR_LAUNCH with the kernel name.
int check_launch(const char* what);

inline int check_dtype(maxsim_dtype dt) {
  if (dt != MAXSIM_FLOAT32 && dt != MAXSIM_FLOAT16 && dt != MAXSIM_BFLOAT16)
    return fail(MAXSIM_ERR_INVALID, "unknown dtype tag %d", (int)dt);
  return MAXSIM_OK;
}

inline int check_dim(int64_t dim) {
  if (dim <= 0) return fail(MAXSIM_ERR_INVALID, "dim must be > 0; got %lld", (long long)dim);
  if (dim > MAXSIM_AMD_MAX_DIM)
    return fail(MAXSIM_ERR_UNSUPPORTED,
                "dim %lld exceeds the largest supported embedding dim (%d)",
                (long long)dim, MAXSIM_AMD_MAX_DIM);
  return MAXSIM_OK;
}

// Compute units of the current device (256 on MI355X), cached per device
// (every thread that fills a slot writes the same value).
inline int device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 256;
  }
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        v <= 0) {
      (void)hipGetLastError();
      v = 256;
    }
    cached[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// Raise a kernel's dynamic-LDS limit to `bytes` on the current device, once
// per device.  `raised` is the calling kernel instantiation's own per-device
// flag array; a flag is set only after hipFuncSetAttribute succeeded, so a
// failure is reported (MAXSIM_ERR_LAUNCH, nothing launched) and tried again
// on the next call.  Two threads launching at once may both set the
// attribute, which is idempotent; the flags are atomic.
constexpr int kMaxDevices = 64;
inline int raise_lds_limit(const void* kern, size_t bytes, const char* what,
                           std::atomic<bool> (&raised)[kMaxDevices]) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
    (void)hipGetLastError();
    return fail(MAXSIM_ERR_LAUNCH, "%s: no current HIP device", what);
  }
  if (dev < kMaxDevices && raised[dev].load(std::memory_order_acquire)) return MAXSIM_OK;
  const hipError_t e =
      hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(MAXSIM_ERR_LAUNCH, "%s: raising the LDS limit to %zu bytes failed: %s", what,
                bytes, hipGetErrorString(e));
  }
  if (dev < kMaxDevices) raised[dev].store(true, std::memory_order_release);
  return MAXSIM_OK;
}

// Workgroups of `kern` (with `threads` threads and `lds` bytes of dynamic
// LDS) that one CU holds at once, cached per device in the calling
// instantiation's own array; 1 if the runtime cannot tell.
inline int resident_per_cu(const void* kern, int threads, size_t lds,
                           std::atomic<int> (&cached)[kMaxDevices]) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
    (void)hipGetLastError();
    return 1;
  }
  int v = dev < kMaxDevices ? cached[dev].load(std::memory_order_relaxed) : 0;
  if (v == 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, kern, threads, lds) != hipSuccess ||
        v <= 0) {
      (void)hipGetLastError();
      v = 1;
    }
    if (dev < kMaxDevices) cached[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

}  // namespace maxsim
