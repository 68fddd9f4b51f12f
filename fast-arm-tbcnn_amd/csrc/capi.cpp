// Library-level C ABI: error strings, version, device check, synchronisation.
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

}  // namespace tbn_hip

extern "C" {

const char* tbn_hip_last_error(void) { return tbn_hip::g_last_error.c_str(); }

int tbn_hip_version(void) { return 100; /* 0.1.0 */ }

int tbn_hip_device_check(void) {
    int rc = tbn_hip::ensure_device();
    return rc == TBN_SUCCESS ? tbn_hip::ok() : rc;
}

int tbn_hip_synchronize(tbn_stream_t stream) {
    hipError_t e = hipStreamSynchronize(tbn_hip::stream_of(stream));
    if (e != hipSuccess)
        return tbn_hip::fail(TBN_RUNTIME_ERROR, std::string("device error: ") + hipGetErrorString(e));
    return tbn_hip::ok();
}

}  // extern "C"
