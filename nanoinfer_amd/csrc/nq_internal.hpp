// Host-side helpers shared by the entry points: status/error text, argument
// validation, launch checking.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/nq.h"

namespace nq {

// Records the calling thread's last error message and returns the status.
nq_status fail(nq_status st, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Checks hipGetLastError after a launch: a failed launch is NQ_HIP_ERROR.
nq_status launch_status(const char* what);

// Raises kernel `fn`'s dynamic LDS limit to `bytes` on the current device, once
// per (kernel, device) pair (the attribute is a property of the kernel on each
// device).
nq_status set_dynamic_lds(const void* fn, size_t bytes, const char* who);

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

constexpr int64_t kMaxIndex = (int64_t(1) << 31) - 1;

inline size_t dtype_size(nq_dtype d) { return d == NQ_F16 ? 2 : 4; }
inline bool dtype_ok(int d) { return d == NQ_F32 || d == NQ_F16; }

inline size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace nq

#define NQ_REQUIRE(cond, st, ...)                          \
    do {                                                   \
        if (!(cond)) return ::nq::fail((st), __VA_ARGS__); \
    } while (0)
