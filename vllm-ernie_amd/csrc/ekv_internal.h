// Host-side plumbing shared by the C-ABI entry points: argument checks that
// turn into an error code plus a thread-local message, and launch status.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ekv {

constexpr int kSpan = 128;       // HCA compression ratio (compress_ratios default)
constexpr int kWindow = 128;     // sliding_window (config.py:27)
constexpr int kStateRing = 256;  // compressor state rows kept per sequence

enum Status : int {
  kOk = 0,
  kInvalidArgument = 1,
  kLaunchFailed = 2,
  kWorkspaceTooSmall = 3,
};

void set_error(const char* msg);
int launch_status();

inline bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }
inline bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace ekv

#define EKV_CHECK(cond, msg)                   \
  do {                                         \
    if (!(cond)) {                             \
      ::ekv::set_error(msg);                   \
      return ::ekv::kInvalidArgument;          \
    }                                          \
  } while (0)

#define ekv_launch_status() ::ekv::launch_status()
