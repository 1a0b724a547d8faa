// Shared definitions of the MI355X (gfx950) decode-step library.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>

namespace hb {

// bf16 is carried as raw 16-bit patterns in device buffers.
using bf16_t = uint16_t;

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

inline void check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw Error(std::string(what) + ": " + hipGetErrorString(e));
}
#define HB_CHECK(call) ::hb::check((call), #call)

inline void require(bool ok, const char* message) {
  if (!ok) throw std::invalid_argument(message);
}

// Timing events for the next launch_timed() of this host thread: `start` takes
// that kernel's start time, `stop` its end time, from the kernel's own dispatch
// (no marker packets join the stream). A launch consumes what is set.
struct LaunchEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};
inline LaunchEvents& launch_events() {
  static thread_local LaunchEvents pending;
  return pending;
}
// hipLaunchKernelGGL, or hipExtLaunchKernelGGL with the pending timing events.
template <typename F, typename... Args>
inline void launch_timed(F kernel, dim3 grid, dim3 block, size_t shmem, hipStream_t stream, Args... args) {
  LaunchEvents& ev = launch_events();
  if (ev.start || ev.stop) {
    const LaunchEvents use = ev;
    ev = LaunchEvents{};
    hipExtLaunchKernelGGL(kernel, grid, block, uint32_t(shmem), stream, use.start, use.stop, 0u, args...);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, shmem, stream, args...);
  }
}

// Copies `message` into the caller's error buffer, truncated and NUL-terminated.
inline void report(char* error, size_t capacity, const char* message) noexcept {
  if (error && capacity) {
    size_t n = std::strlen(message);
    if (n > capacity - 1) n = capacity - 1;
    std::memcpy(error, message, n);
    error[n] = 0;
  }
}

// Runs f; any exception becomes -1 plus a message. No exception crosses the ABI.
template <class F>
int guarded(char* error, size_t capacity, F&& f) noexcept {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    report(error, capacity, e.what());
  } catch (...) {
    report(error, capacity, "unknown native HIP exception");
  }
  return -1;
}

__host__ __device__ inline float bf16_to_f32(bf16_t v) {
  uint32_t u = uint32_t(v) << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

// Round-to-nearest-even; NaN stays NaN.
__host__ __device__ inline bf16_t f32_to_bf16(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return bf16_t((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return bf16_t(u >> 16);
}

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

}  // namespace hb
