// Shared host-side plumbing of libtbn_hip: error reporting, argument checks,
// device validation and launch checking.  Device code lives in the .hip files.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "tbn_hip.h"

namespace tbn_hip {

// Records `msg` as this thread's last error and returns `code`.
int fail(int code, const std::string& msg);
// Clears the thread's last error and returns TBN_SUCCESS.
int ok();
// Verifies the current device is a gfx950 (cached per device id).
int ensure_device();
// Maps the result of hipGetLastError() after a launch to a status.
int check_launch(const char* what);

inline hipStream_t stream_of(tbn_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Device scratch for split-K partial sums on stream s: a per-device buffer
// reused by consecutive calls on one stream, else (another stream) a
// stream-ordered temporary; release_workspace frees only the latter.  Refused
// (TBN_NOT_IMPLEMENTED) while s captures.  `counters`, if given, receives
// kWorkspaceCounters int32 counters that are zero when the call starts and
// that the call's kernels must leave zero.
constexpr int kWorkspaceCounters = 16384;
int stream_workspace(hipStream_t s, size_t bytes, void*& ptr, bool& temporary, int** counters = nullptr);
void release_workspace(void* ptr, bool temporary, hipStream_t s);

// Current value of a tuning control (TBN_TUNE_*), the environment read once.
int tuning(int option);

// Compute units of the current device (cached per device; 256 if the query
// fails).
int cu_count();

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace tbn_hip

#define TBN_REQUIRE(cond, code, msg)                         \
    do {                                                     \
        if (!(cond)) return ::tbn_hip::fail((code), (msg));  \
    } while (0)

#define TBN_DEVICE_GUARD()                             \
    do {                                               \
        int _rc = ::tbn_hip::ensure_device();          \
        if (_rc != TBN_SUCCESS) return _rc;            \
    } while (0)
