// Execution context and device workspace (MetalContext + BufferPool analog,
// AnimaXS/Runtime/Metal/MetalContext.swift:14-104).
#pragma once

#include "common.hpp"

struct anima_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
};

namespace anima {

// RAII guard making the context's device current for the duration of a call.
struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(const anima_ctx* ctx) {
    ANIMA_HIP(hipGetDevice(&prev));
    if (prev != ctx->device) ANIMA_HIP(hipSetDevice(ctx->device));
  }
  ~DeviceGuard() {
    int cur = -1;
    if (hipGetDevice(&cur) == hipSuccess && cur != prev && prev >= 0) (void)hipSetDevice(prev);
  }
};

// A device scratch buffer that grows on demand and is freed on destruction
// (the reference's BufferPool grows and never frees, MetalContext.swift:86-104).
// Growing synchronises the stream first so in-flight kernels never see the old
// allocation freed under them.
class Workspace {
 public:
  Workspace() = default;
  Workspace(const Workspace&) = delete;
  Workspace& operator=(const Workspace&) = delete;
  ~Workspace() { release(); }

  void* get(int64_t bytes, hipStream_t stream) {
    if (bytes <= capacity_) return ptr_;
    if (ptr_) {
      ANIMA_HIP(hipStreamSynchronize(stream));
      release();
    }
    int64_t cap = bytes + (bytes >> 3);
    cap = (cap + 4095) & ~int64_t(4095);
    void* p = nullptr;
    ANIMA_HIP(hipMalloc(&p, static_cast<size_t>(cap)));
    ptr_ = p;
    capacity_ = cap;
    return ptr_;
  }
  int64_t capacity() const { return capacity_; }

 private:
  void release() {
    if (ptr_) (void)hipFree(ptr_);
    ptr_ = nullptr;
    capacity_ = 0;
  }
  void* ptr_ = nullptr;
  int64_t capacity_ = 0;
};

}  // namespace anima
