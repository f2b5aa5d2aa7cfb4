// Host-side helpers shared by the C-ABI entry points: the thread-local error
// string behind mi355_dsa_last_error() and argument/launch checking.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/mi355_dsa.h"

namespace mi355dsa {

// Records a formatted error message for mi355_dsa_last_error(); returns code.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the thread's error message (every entry point starts with this).
void clear_error();

// Converts a pending HIP launch error (if any) into MI355_DSA_EHIP.
int check_launch(const char* what);

// Raises a kernel's dynamic LDS limit to `bytes` on the current device (once
// per device and kernel; thread-safe); MI355_DSA_EHIP on failure.
int reserve_lds(const void* kernel, size_t bytes, const char* what);

// Arrival counters for launches whose last workgroup of a group finishes
// the group's work (one device atomic add per workgroup, no waiting): a slot
// of kArriveRows counters in a per-device pool that is zero at load, each
// call's last workgroups leaving their counters zero again.  An eager call
// gets its stream's slot (calls on one stream never overlap, so every op of
// a stream can share it); a call being captured into a graph gets a slot of
// its own, kept by the graph's replays.  nullptr when the pool is spent or
// unavailable: the caller then takes a path without counters.
constexpr int kArriveRows = 64;
uint32_t* arrive_slot(hipStream_t st);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned_to(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

}  // namespace mi355dsa

// Argument check that mirrors the reference's TORCH_CHECK: on failure the
// entry point returns MI355_DSA_EINVAL with the message recorded.
#define DSA_CHECK(cond, ...)                                            \
  do {                                                                  \
    if (!(cond)) return ::mi355dsa::set_error(MI355_DSA_EINVAL, __VA_ARGS__); \
  } while (0)

#define DSA_LAUNCH_CHECK(what)                                 \
  do {                                                         \
    int _rc = ::mi355dsa::check_launch(what);                  \
    if (_rc != MI355_DSA_OK) return _rc;                       \
  } while (0)
