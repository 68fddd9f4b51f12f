// Library-level C ABI: error strings, version, device check, synchronisation.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <mutex>
#include <string>
#include <unordered_map>

#include "common.hpp"

namespace tbn_hip {

namespace {
thread_local std::string g_last_error;
std::mutex g_device_mutex;
std::unordered_map<int, int> g_device_status;  // device id -> status
}  // namespace

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int ok() {
    g_last_error.clear();
    return TBN_SUCCESS;
}

// Stream workspace for split-K partial sums.  A free followed by a new
// allocation on a stream makes the GPU wait on the allocator between kernels
// (about 6 us per call), so each device keeps one buffer for the stream that
// last used it, grown as needed; consecutive users on that stream are
// ordered by the stream.  Calls on another stream get a stream-ordered
// temporary.  Every allocation starts with kWorkspaceCounters int32 counters,
// zeroed when it is made; kernels that use them leave them zero again.  No
// allocation is recorded into a captured graph: such calls are refused.
namespace {
struct Workspace {
    hipStream_t stream = nullptr;
    void* ptr = nullptr;
    size_t bytes = 0;  // data bytes after the counters
};
std::mutex g_ws_mutex;
Workspace g_ws[64];

constexpr size_t kCounterBytes = kWorkspaceCounters * sizeof(int);

// Allocates counters + `bytes` on stream s and zeroes the counters.
int alloc_async(void*& base, size_t bytes, hipStream_t s) {
    hipError_t e = hipMallocAsync(&base, kCounterBytes + bytes, s);
    if (e == hipSuccess) {
        e = hipMemsetAsync(base, 0, kCounterBytes, s);
        if (e != hipSuccess) (void)hipFreeAsync(base, s);
    }
    if (e != hipSuccess) {
        (void)hipGetLastError();
        base = nullptr;
        return fail(e == hipErrorOutOfMemory ? TBN_OUT_OF_MEMORY : TBN_RUNTIME_ERROR,
                    std::string("workspace allocation failed: ") + hipGetErrorString(e));
    }
    return TBN_SUCCESS;
}
}  // namespace

int stream_workspace(hipStream_t s, size_t bytes, void*& ptr, bool& temporary, int** counters) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    const bool capturing = hipStreamIsCapturing(s, &st) != hipSuccess || st != hipStreamCaptureStatusNone;
    // A replay of a graph holding split-K temporaries as graph allocations
    // ended in a memory fault once (DESIGN notes what was examined), so no
    // allocation is recorded into a graph: such calls are refused while the
    // stream captures (the Session then runs that plan eagerly).
    if (capturing)
        return fail(TBN_NOT_IMPLEMENTED, "split-K workspace: no allocation while the stream is being captured");
    void* base = nullptr;
    temporary = true;
    int dev = 0;
    if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) {
        std::lock_guard<std::mutex> lock(g_ws_mutex);
        Workspace& w = g_ws[dev];
        if (w.ptr && w.stream == s && w.bytes >= bytes) {
            base = w.ptr;
            temporary = false;
        } else if (!w.ptr || w.stream == s) {
            if (w.ptr) (void)hipFreeAsync(w.ptr, w.stream);
            w = Workspace{};
            const size_t grown = bytes + bytes / 4;
            const int rc = alloc_async(base, grown, s);
            if (rc) return rc;
            w = Workspace{s, base, grown};
            temporary = false;
        }
    }
    if (temporary) {
        const int rc = alloc_async(base, bytes, s);
        if (rc) return rc;
    }
    ptr = static_cast<uint8_t*>(base) + kCounterBytes;
    if (counters) *counters = static_cast<int*>(base);
    return TBN_SUCCESS;
}

void release_workspace(void* ptr, bool temporary, hipStream_t s) {
    if (temporary && ptr) (void)hipFreeAsync(static_cast<uint8_t*>(ptr) - kCounterBytes, s);
}

// Tuning controls: read from the environment once (TBN_CONV_TILE,
// TBN_CONV_SPLITS, TBN_GEMM_SPLITS, TBN_GEMM_TILE, TBN_TBN_CONV), then changed only through
// tbn_hip_set_tuning.  Relaxed atomics: a value is a launch-shape choice, so a
// call that races with a change simply sees the old or the new one.
namespace {
std::atomic<int> g_tuning[6];
std::once_flag g_tuning_once;

void tuning_init() {
    auto env = [](const char* name, int dflt) {
        const char* e = std::getenv(name);
        return e && *e ? std::atoi(e) : dflt;
    };
    g_tuning[TBN_TUNE_CONV_TILE].store(env("TBN_CONV_TILE", -1), std::memory_order_relaxed);
    g_tuning[TBN_TUNE_CONV_SPLITS].store(std::max(0, env("TBN_CONV_SPLITS", 0)), std::memory_order_relaxed);
    g_tuning[TBN_TUNE_GEMM_SPLITS].store(std::max(0, env("TBN_GEMM_SPLITS", 0)), std::memory_order_relaxed);
    g_tuning[TBN_TUNE_GEMM_TILE].store(env("TBN_GEMM_TILE", -1), std::memory_order_relaxed);
    g_tuning[TBN_TUNE_TBN_CONV].store(std::max(0, std::min(2, env("TBN_TBN_CONV", 0))), std::memory_order_relaxed);
}
}  // namespace

int tuning(int option) {
    std::call_once(g_tuning_once, tuning_init);
    return g_tuning[option].load(std::memory_order_relaxed);
}

int ensure_device() {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        return fail(TBN_DEVICE_NOT_SUPPORTED,
                    std::string("no HIP device available: ") + hipGetErrorString(e));
    }
    std::lock_guard<std::mutex> lock(g_device_mutex);
    auto it = g_device_status.find(dev);
    if (it != g_device_status.end()) {
        if (it->second != TBN_SUCCESS)
            return fail(it->second, "device " + std::to_string(dev) + " is not a gfx950 (MI355X)");
        return TBN_SUCCESS;
    }
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) {
        return fail(TBN_DEVICE_NOT_SUPPORTED,
                    std::string("hipGetDeviceProperties failed: ") + hipGetErrorString(e));
    }
    const std::string arch(prop.gcnArchName);
    const int status = (arch.rfind("gfx950", 0) == 0) ? TBN_SUCCESS : TBN_DEVICE_NOT_SUPPORTED;
    g_device_status[dev] = status;
    if (status != TBN_SUCCESS)
        return fail(status, "device " + std::to_string(dev) + " is " + arch +
                                "; this library is built for gfx950 (MI355X) only");
    return TBN_SUCCESS;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) return ok();
    if (e == hipErrorNoBinaryForGpu || e == hipErrorInvalidDeviceFunction)
        return fail(TBN_DEVICE_NOT_SUPPORTED, std::string(what) + ": " + hipGetErrorString(e));
    if (e == hipErrorOutOfMemory)
        return fail(TBN_OUT_OF_MEMORY, std::string(what) + ": " + hipGetErrorString(e));
    return fail(TBN_RUNTIME_ERROR, std::string(what) + ": " + hipGetErrorString(e));
}

int cu_count() {
    static std::mutex mu;
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if (!cached[dev]) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}

}  // namespace tbn_hip

extern "C" {

const char* tbn_hip_last_error(void) { return tbn_hip::g_last_error.c_str(); }

int tbn_hip_version(void) { return 100; /* 0.1.0 */ }

int tbn_hip_device_check(void) {
    int rc = tbn_hip::ensure_device();
    return rc == TBN_SUCCESS ? tbn_hip::ok() : rc;
}

int tbn_hip_set_tuning(int option, int value) {
    TBN_REQUIRE(option >= TBN_TUNE_CONV_TILE && option <= TBN_TUNE_TBN_CONV, TBN_INVALID_ARGUMENT,
                "unknown tuning option");
    TBN_REQUIRE(option == TBN_TUNE_CONV_TILE
                    ? value >= -1
                    : (option == TBN_TUNE_GEMM_TILE ? value >= -1 && value <= 2
                                                    : (option == TBN_TUNE_TBN_CONV ? value >= 0 && value <= 2
                                                                                   : value >= 0)),
                TBN_INVALID_ARGUMENT, "tuning value out of range");
    (void)tbn_hip::tuning(option);  // the environment is read before the first change
    tbn_hip::g_tuning[option].store(value, std::memory_order_relaxed);
    return tbn_hip::ok();
}

int tbn_hip_get_tuning(int option, int* value) {
    TBN_REQUIRE(option >= TBN_TUNE_CONV_TILE && option <= TBN_TUNE_TBN_CONV, TBN_INVALID_ARGUMENT,
                "unknown tuning option");
    TBN_REQUIRE(value != nullptr, TBN_INVALID_ARGUMENT, "null pointer");
    *value = tbn_hip::tuning(option);
    return tbn_hip::ok();
}

int tbn_hip_synchronize(tbn_stream_t stream) {
    hipError_t e = hipStreamSynchronize(tbn_hip::stream_of(stream));
    if (e != hipSuccess)
        return tbn_hip::fail(TBN_RUNTIME_ERROR, std::string("device error: ") + hipGetErrorString(e));
    return tbn_hip::ok();
}

}  // extern "C"
