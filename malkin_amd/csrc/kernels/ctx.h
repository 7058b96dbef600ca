// Library-internal context, error plumbing and launch helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <stdexcept>
#include <string>

#include "../../../include/malkin_hip.h"

struct mk_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  int n_cu = 0;
  char name[64] = {0};
  void* scratch = nullptr;  // per-context device scratch (partial reductions), allocated once at init
  size_t scratch_bytes = 0;
  int32_t* meta = nullptr;  // 64 bytes of per-call metadata (mk_attend_gqa's token layout), allocated at init
};

namespace mk {

void set_error(const char* fmt, ...);
// Counts one host wait on the device (a stream or event synchronization), for mk_host_waits().
void count_host_wait();
// Records the HIP error and returns MK_ERR_HIP.
int hip_fail(hipError_t e, const char* what);

// Errors raised inside library code; the extern "C" wrappers turn them into status codes.
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

inline void check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw Error(MK_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// The launch's own error (bad configuration) and any asynchronous fault reported so far.
inline void check_launch(const char* what) { check(hipGetLastError(), what); }

// Compute units of the current device (queried once: the library runs one device per process).
inline int device_cus() {
  static int n = 0;
  if (n == 0) {
    int dev = 0;
    check(hipGetDevice(&dev), "hipGetDevice");
    check(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev), "hipDeviceGetAttribute");
  }
  return n;
}

template <typename F>
int guard(F&& f) {
  try {
    f();
    return MK_OK;
  } catch (const Error& e) {
    set_error("%s", e.what());
    return e.code;
  } catch (const std::exception& e) {
    set_error("%s", e.what());
    return MK_ERR_INVALID;
  }
}

inline void require(bool ok, const char* msg) {
  if (!ok) throw Error(MK_ERR_INVALID, msg);
}

}  // namespace mk
