// pk_abi_internal.h - pieces shared by the C ABI translation units: the
// context object, the thread-local error message and status helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "pk_palette.h"

struct pk_context {
  int device = 0;
  hipStream_t stream = nullptr;
};

namespace pk_abi {

extern thread_local std::string g_error;

// Sets the calling thread's last error message and returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
inline int ok() { return PK_OK; }
int check_ctx(const pk_context* ctx);

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline hipStream_t stream_or_default(pk_context* ctx, void* stream) {
  return stream ? static_cast<hipStream_t>(stream) : ctx->stream;
}

}  // namespace pk_abi

#define PK_HIP(call, what)                                                                       \
  do {                                                                                           \
    const hipError_t pk_e_ = (call);                                                             \
    if (pk_e_ != hipSuccess)                                                                     \
      return ::pk_abi::fail(PK_DEVICE_ERROR, "%s failed: %s", (what), hipGetErrorString(pk_e_)); \
  } while (0)
