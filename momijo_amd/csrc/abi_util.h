// Internal helpers of the C ABI (api.hip, api_host.hip): status codes with a
// per-thread message, argument checks, and the device staging used by the
// host-pointer (_h) entry points.  Not part of the public header.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "../../include/momijo_hip.h"

namespace mj_abi {

// message of the last non-OK status on this host thread (mj_last_error)
inline thread_local char g_err[512] = "";

inline int32_t fail(int32_t code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

inline int32_t hip_status(hipError_t e, const char *what) {
  if (e == hipSuccess) return MJ_OK;
  return fail(MJ_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

inline bool valid_epi(int32_t e) { return e >= MJ_EPI_NONE && e <= MJ_EPI_RELU_UNARY; }

constexpr int64_t kMaxDim = (int64_t)1 << 31;

inline int32_t check_dims(int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N < 0 || K < 0)
    return fail(MJ_ERR_ARG, "negative size (M=%lld N=%lld K=%lld)", (long long)M, (long long)N,
                (long long)K);
  if (M >= kMaxDim || N >= kMaxDim || K >= kMaxDim)
    return fail(MJ_ERR_UNSUPPORTED, "dimension exceeds 2^31");
  return MJ_OK;
}

inline hipStream_t S(void *stream) { return (hipStream_t)stream; }

// Number of elements a (rows x cols) view with element strides (s0, s1)
// spans from its first element: the extent a host copy must cover.
inline int64_t span2(int64_t rows, int64_t cols, int64_t s0, int64_t s1) {
  if (rows <= 0 || cols <= 0) return 0;
  return (rows - 1) * s0 + (cols - 1) * s1 + 1;
}

// One host array staged on the device for a host-pointer call.  `host` is
// copied in (if set), `host_out` is copied back after the run (if set).
// rows > 0 makes the copy-out two-dimensional: `rows` rows of `width` bytes
// at a pitch of `pitch` bytes, so padding between rows is left untouched.
struct HostArg {
  const void *host;
  void *host_out;
  size_t bytes;
  int64_t rows = 0;
  size_t width = 0, pitch = 0;
};

// Allocates one device block holding every array, copies the inputs in,
// runs body(device pointers) on the null stream, waits, and copies the
// outputs back: the reference seam's ownership model (runtime.mojo:556-604),
// synchronous, the caller keeping its host buffers.
template <typename Body>
int32_t with_device_copies(HostArg *args, int n, Body body) {
  constexpr int kMaxArgs = 10;
  if (n > kMaxArgs) return fail(MJ_ERR_ARG, "too many staged arrays");
  size_t total = 0;
  for (int i = 0; i < n; ++i) total += (args[i].bytes + 255) & ~(size_t)255;
  char *dev = nullptr;
  if (total && hipMalloc((void **)&dev, total) != hipSuccess) {
    (void)hipGetLastError();
    return fail(MJ_ERR_ALLOC, "hipMalloc(%zu) failed", total);
  }
  void *d[kMaxArgs];
  size_t off = 0;
  int32_t st = MJ_OK;
  for (int i = 0; i < n; ++i) {
    d[i] = args[i].bytes ? dev + off : nullptr;
    off += (args[i].bytes + 255) & ~(size_t)255;
    if (!st && args[i].host && args[i].bytes)
      st = hip_status(hipMemcpy(d[i], args[i].host, args[i].bytes, hipMemcpyHostToDevice),
                      "copy in");
  }
  if (!st) st = body(d);
  if (!st) st = hip_status(hipStreamSynchronize(nullptr), "device run");
  for (int i = 0; i < n && !st; ++i) {
    if (!args[i].host_out || !args[i].bytes) continue;
    if (args[i].rows > 0)
      st = hip_status(hipMemcpy2D(args[i].host_out, args[i].pitch, d[i], args[i].pitch,
                                  args[i].width, (size_t)args[i].rows, hipMemcpyDeviceToHost),
                      "copy out");
    else
      st = hip_status(hipMemcpy(args[i].host_out, d[i], args[i].bytes, hipMemcpyDeviceToHost),
                      "copy out");
  }
  if (dev) (void)hipFree(dev);
  return st;
}

}  // namespace mj_abi
