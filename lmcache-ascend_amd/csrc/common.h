// Internal helpers shared by the liblmcache_amd translation units: status
// codes carried as C++ exceptions inside the library, tensor descriptor
// accessors, device selection and host->device address translation.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "../../include/lmcache_amd.h"

namespace lmc {

// An error that crosses the C ABI as `status` plus a message.
struct Error : std::runtime_error {
  int status;
  Error(int s, const std::string &m) : std::runtime_error(m), status(s) {}
};

[[noreturn]] inline void fail(int status, const std::string &msg) {
  throw Error(status, msg);
}
inline void check(bool ok, const std::string &msg) {
  if (!ok) fail(LMC_ERR_RUNTIME, msg);
}
inline void check_value(bool ok, const std::string &msg) {
  if (!ok) fail(LMC_ERR_VALUE, msg);
}
inline void hip_check(hipError_t e, const char *what) {
  if (e != hipSuccess)
    fail(LMC_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

void set_last_error(const std::string &msg);

// Runs `body`, converting library errors into a status code + message.
template <typename F> int guarded(F &&body) {
  try {
    body();
    return LMC_OK;
  } catch (const Error &e) {
    set_last_error(e.what());
    return e.status;
  } catch (const std::exception &e) {
    set_last_error(e.what());
    return LMC_ERR_RUNTIME;
  }
}

inline int64_t dtype_size(int32_t dt) {
  switch (dt) {
  case LMC_U8:
  case LMC_I8:
    return 1;
  case LMC_I16:
  case LMC_F16:
  case LMC_BF16:
    return 2;
  case LMC_I32:
  case LMC_F32:
    return 4;
  case LMC_I64:
    return 8;
  default:
    fail(LMC_ERR_RUNTIME, "unsupported dtype code " + std::to_string(dt));
  }
}

inline const lmc_tensor &deref(const lmc_tensor *t, const char *name) {
  if (t == nullptr) fail(LMC_ERR_VALUE, std::string(name) + " is null");
  if (t->ndim < 0 || t->ndim > LMC_MAX_DIMS)
    fail(LMC_ERR_VALUE, std::string(name) + ": bad ndim");
  return *t;
}

// size(d) with Python-style negative indices.
inline int64_t size(const lmc_tensor &t, int d) {
  if (d < 0) d += t.ndim;
  if (d < 0 || d >= t.ndim)
    fail(LMC_ERR_RUNTIME, "dimension out of range (ndim=" +
                              std::to_string(t.ndim) + ", dim=" +
                              std::to_string(d) + ")");
  return t.sizes[d];
}
inline int64_t stride(const lmc_tensor &t, int d) {
  if (d < 0) d += t.ndim;
  if (d < 0 || d >= t.ndim)
    fail(LMC_ERR_RUNTIME, "dimension out of range");
  return t.strides[d];
}
inline int64_t numel(const lmc_tensor &t) {
  int64_t n = 1;
  for (int i = 0; i < t.ndim; ++i) n *= t.sizes[i];
  return n;
}
inline int64_t elem_size(const lmc_tensor &t) { return dtype_size(t.dtype); }
inline int64_t nbytes(const lmc_tensor &t) { return numel(t) * elem_size(t); }

// Bytes from element 0 to one past the last addressable element of a
// (possibly strided, non-negative-stride) tensor.
inline int64_t extent_bytes(const lmc_tensor &t) {
  if (numel(t) == 0) return 0;
  int64_t last = 0;
  for (int i = 0; i < t.ndim; ++i) {
    if (t.strides[i] < 0) fail(LMC_ERR_RUNTIME, "negative strides unsupported");
    last += (t.sizes[i] - 1) * t.strides[i];
  }
  return (last + 1) * elem_size(t);
}

// One pinned host allocation: [host, host + size) is mapped at dev.
struct PinnedRange {
  uintptr_t host;
  size_t size;
  uintptr_t dev;
};

// The pinned allocation holding `host`: a recorded range, or one HIP
// reports as mapped host memory with its extent.  False for pageable or
// unknown addresses.
bool pinned_range(uintptr_t host, PinnedRange *out);

// Host -> device address translation registry (pinned host memory).
// Returns 0 when `host` is not inside a recorded or HIP-mapped host range of
// at least `required` bytes.
uintptr_t translate_host_ptr(uintptr_t host, size_t required);

// Kernel-visible address of a tensor: device tensors pass through, host
// tensors must be pinned and mapped (the reference's get_kernel_ptr,
// csrc/utils.h:32-51).
inline uint8_t *kernel_ptr(const lmc_tensor &t) {
  if (t.device >= 0) return static_cast<uint8_t *>(t.data);
  uintptr_t dev = translate_host_ptr(reinterpret_cast<uintptr_t>(t.data),
                                     static_cast<size_t>(
                                         extent_bytes(t) > 0 ? extent_bytes(t) : 1));
  if (dev == 0)
    fail(LMC_ERR_RUNTIME, "host tensor is not in pinned, device-mapped memory: "
                          "no device address for it");
  return reinterpret_cast<uint8_t *>(dev);
}

// Makes `device` current on this thread for the duration of a call.
struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int device) {
    if (device < 0) return;
    hip_check(hipGetDevice(&prev), "hipGetDevice");
    if (prev != device) hip_check(hipSetDevice(device), "hipSetDevice");
    else prev = -1;
  }
  ~DeviceGuard() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

} // namespace lmc
