// Host-side runtime shared by the entry points: thread-local error text,
// argument checks, workspace carving, launch counters and event timing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include <string>

#include "../../include/opendde_amd.h"

namespace odde {

int set_error(int code, const std::string& msg);
int check_launch(const char* what);
// Workgroups of `threads` threads of `kernel` resident on the current device
// at once (occupancy x CUs): the grid of a persistent kernel, whose
// workgroups must all be resident or the late ones finish a whole pass late.
int resident_grid(const void* kernel, int threads);

// Launch bookkeeping: counts every launch; when timing is on (and `events`),
// records a pair of events around it on `stream` (creating events the first
// time; callers that must not allocate pass events = false).
struct LaunchScope {
  LaunchScope(int kernel_id, hipStream_t stream, bool events = true);
  ~LaunchScope();
  int id;
  hipStream_t stream;
  int slot;
};

// Sequential carving of a caller-provided workspace, 256-byte aligned.
struct Carver {
  char* base;
  uint64_t size;
  uint64_t used = 0;
  Carver(void* b, uint64_t s) : base(static_cast<char*>(b)), size(s) {}
  template <typename T> T* take(uint64_t count) {
    used = (used + 255) & ~uint64_t(255);
    T* p = base ? reinterpret_cast<T*>(base + used) : nullptr;
    used += count * sizeof(T);
    return p;
  }
};

inline int round_up(int x, int m) { return (x + m - 1) / m * m; }

// Output-channel split (gridDim.z) for the fp32 projections, whose
// workgroups each walk all output channels: the smallest power of two s
// dividing `max_split` with wgs * s >= 1024 (four workgroups per CU of an
// MI355X), so small problems still keep two or more waves on every SIMD.
// ODDE_PROJ_SPLIT fixes s (tuning; clamped to those divisors).
int proj_split(int64_t wgs, int max_split);
inline int dtype_size(int dt) { return dt == ODDE_BF16 ? 2 : 4; }
inline bool valid_dtype(int dt) { return dt == ODDE_F32 || dt == ODDE_BF16; }


}  // namespace odde
