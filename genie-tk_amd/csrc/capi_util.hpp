// Host-side helpers shared by the extern "C" entry points: error reporting,
// launch checks and argument validation.  Every entry point returns 0 on
// success or a GTK_E* code; the message is available from gtk_last_error().
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string>

#include "../../include/genie_tk.h"

namespace gtk {

void set_error(const char* fmt, ...);

#define GTK_REQUIRE(cond, code, ...)        \
  do {                                      \
    if (!(cond)) {                          \
      ::gtk::set_error(__VA_ARGS__);        \
      return (code);                        \
    }                                       \
  } while (0)

#define GTK_HIP_CHECK(expr)                                                         \
  do {                                                                              \
    hipError_t _e = (expr);                                                         \
    if (_e != hipSuccess) {                                                         \
      ::gtk::set_error("HIP error %s at %s:%d: %s", hipGetErrorName(_e), __FILE__, \
                       __LINE__, hipGetErrorString(_e));                            \
      return GTK_EHIP;                                                              \
    }                                                                               \
  } while (0)

// Check the launch that was just enqueued.
#define GTK_LAUNCH_CHECK() GTK_HIP_CHECK(hipGetLastError())

inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// |f| <= lim and not NaN, tested on the bits (some sources are compiled
// without NaN semantics, where a float compare may assume a non-NaN value).
inline bool abs_at_most(float f, float lim) {
  uint32_t u, l;
  __builtin_memcpy(&u, &f, 4);
  __builtin_memcpy(&l, &lim, 4);
  return (u & 0x7fffffffu) <= l;
}

// Compute units of the current device (cached per device; persistent kernels
// launch one block per CU).
int device_cus();

// Per-kernel timing (gtk_timing_enable / gtk_timing_report): when enabled, a
// StageTimer records one HIP event before and one after the launch it
// scopes, on the launch stream.  Disabled, it costs one relaxed load.
class StageTimer {
 public:
  StageTimer(const char* name, hipStream_t st);
  ~StageTimer();
  StageTimer(const StageTimer&) = delete;
  StageTimer& operator=(const StageTimer&) = delete;

 private:
  const char* name_;
  hipStream_t st_;
  hipEvent_t begin_ = nullptr;
};

}  // namespace gtk
