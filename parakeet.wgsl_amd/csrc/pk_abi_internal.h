// pk_abi_internal.h - pieces shared by the C ABI translation units: the
// context object, the thread-local error message and status helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <string>

#include "pk_palette.h"

// A context is reference counted: pk_context_destroy drops the owner's
// reference, and every op, prepared weight, graph or encoder made on it
// holds one more until it is freed. The stream and the object go away with
// the last reference, so an object released after its context (a
// finalizer that runs late) still finds the device id and the stream.
struct pk_context {
  int device = 0;
  hipStream_t stream = nullptr;
  std::atomic<int> refs{1};
  std::atomic<bool> destroyed{false};
};

namespace pk_abi {

extern thread_local std::string g_error;

// Sets the calling thread's last error message and returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
inline int ok() { return PK_OK; }
// Null check for calls that take a context; a destroyed context is refused
// with PK_DESTROYED.
int check_ctx(const pk_context* ctx);

// Device bytes of the prepared codes a GEMM op reads (its own layout and
// the copies in other layouts that its prepared row plans read).
uint64_t gemm_weight_bytes(const pk_gemm_op* op);

// Reference counting of contexts (see pk_context).
pk_context* ctx_retain(pk_context* ctx);
void ctx_release(pk_context* ctx);

// The context member of an op: holds a reference from assignment until the
// op is deleted.
class CtxRef {
 public:
  CtxRef() = default;
  CtxRef(const CtxRef&) = delete;
  CtxRef& operator=(const CtxRef&) = delete;
  ~CtxRef() { ctx_release(p_); }
  CtxRef& operator=(pk_context* c) {
    ctx_retain(c);
    ctx_release(p_);
    p_ = c;
    return *this;
  }
  pk_context* operator->() const { return p_; }
  operator pk_context*() const { return p_; }

 private:
  pk_context* p_ = nullptr;
};

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline hipStream_t stream_or_default(pk_context* ctx, void* stream) {
  return stream ? static_cast<hipStream_t>(stream) : ctx->stream;
}

// Frees device memory that launches on any stream may still read (an op's
// buffers, a weight shared by ops enqueued on callers' streams): the
// device drains first, since hipFree alone is not ordered after work
// enqueued on other streams.
inline void free_after_drain(int device, void* p) {
  if (!p) return;
  (void)hipSetDevice(device);
  (void)hipDeviceSynchronize();
  (void)hipFree(p);
}

}  // namespace pk_abi

#define PK_HIP(call, what)                                                                       \
  do {                                                                                           \
    const hipError_t pk_e_ = (call);                                                             \
    if (pk_e_ != hipSuccess)                                                                     \
      return ::pk_abi::fail(PK_DEVICE_ERROR, "%s failed: %s", (what), hipGetErrorString(pk_e_)); \
  } while (0)
