// Device plumbing, errors, types and Tensor of the tbn host runtime.
#include <hip/hip_runtime_api.h>

#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "tbn/device.hpp"
#include "tbn/errors.hpp"
#include "tbn/tensor.hpp"
#include "tbn/types.hpp"
#include "tbn_hip.h"

namespace tbn {

// ---- errors --------------------------------------------------------------------

void throw_status(int status, const std::string& what) {
    std::string msg = what + ": " + tbn_hip_last_error();
    switch (status) {
        case TBN_INVALID_ARGUMENT: throw InvalidArgumentError(msg);
        case TBN_OUT_OF_MEMORY: throw OutOfMemoryError(msg);
        case TBN_NOT_IMPLEMENTED: throw NotImplementedError(msg);
        case TBN_INVALID_MODEL: throw InvalidModelError(msg);
        case TBN_QUANTIZATION_ERROR: throw QuantizationError(msg);
        case TBN_INVALID_SHAPE: throw InvalidShapeError(msg);
        case TBN_DEVICE_NOT_SUPPORTED: throw DeviceNotSupportedError(msg);
        case TBN_OPERATOR_NOT_SUPPORTED: throw OperatorNotSupportedError(msg);
        default: throw RuntimeError(msg);
    }
}

namespace {
void check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return;
    const std::string msg = std::string(what) + ": " + hipGetErrorString(e);
    if (e == hipErrorOutOfMemory) throw OutOfMemoryError(msg);
    throw RuntimeError(msg);
}
}  // namespace

// ---- types ----------------------------------------------------------------------

std::string shape_to_string(const Shape& s) {
    std::string r = "[";
    for (size_t i = 0; i < s.dims.size(); ++i) {
        if (i) r += ", ";
        r += std::to_string(s.dims[i]);
    }
    return r + "]";
}

size_t element_size(DataType dtype) {
    switch (dtype) {
        case DataType::FLOAT32: case DataType::INT32: case DataType::UINT32: return 4;
        case DataType::FLOAT16: case DataType::BFLOAT16: case DataType::INT16: case DataType::UINT16: return 2;
        case DataType::INT8: case DataType::UINT8: case DataType::BOOL: case DataType::TERNARY:
        case DataType::BINARY: return 1;
        case DataType::INT64: case DataType::UINT64: return 8;
    }
    throw InvalidArgumentError("Unknown data type");
}

bool is_host(DeviceType d) { return d != DeviceType::HIP; }

// ---- device -------------------------------------------------------------------------

namespace device {
namespace {

thread_local Stream t_stream = nullptr;

// Size classes: 512-byte granules below 1 MiB, 2 MiB granules above.
size_t size_class(size_t bytes) {
    if (bytes == 0) bytes = 1;
    if (bytes < (1u << 20)) return (bytes + 511) & ~size_t(511);
    return (bytes + (2u << 20) - 1) & ~((size_t(2) << 20) - 1);
}

// A freed block is reused on the stream that released it right away (stream
// order covers the kernels that used it), and on any other stream only once
// the event recorded on the releasing stream at release time has completed.
struct FreeBlock {
    void* ptr;
    Stream stream;      // current stream of the releasing thread
    hipEvent_t ready;   // recorded there at release; null: nothing pending
};

struct Pool {
    std::mutex mu;
    std::map<std::pair<int, size_t>, std::vector<FreeBlock>> free_blocks;  // (device, class) -> blocks
    std::unordered_map<void*, std::pair<int, size_t>> live;                  // block -> (device, class)
    size_t cached = 0, allocated = 0;
};

Pool& pool() {
    static Pool* p = new Pool();  // never destroyed: blocks may be released during exit
    return *p;
}

int current_device() {
    int dev = 0;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    return dev;
}

void free_cached_locked(Pool& p, int dev) {
    for (auto it = p.free_blocks.begin(); it != p.free_blocks.end();) {
        if (dev >= 0 && it->first.first != dev) { ++it; continue; }
        for (FreeBlock& b : it->second) {
            if (b.ready) {
                (void)hipEventSynchronize(b.ready);
                (void)hipEventDestroy(b.ready);
            }
            (void)hipFree(b.ptr);
            p.cached -= it->first.second;
        }
        it = p.free_blocks.erase(it);
    }
}

}  // namespace

Stream current_stream() { return t_stream; }

void set_current_stream(Stream s) {
    if (s == t_stream) return;
    check_hip(hipStreamSynchronize(static_cast<hipStream_t>(t_stream)), "hipStreamSynchronize");
    t_stream = s;
}

void* allocate(size_t bytes) {
    const int dev = current_device();
    const size_t cls = size_class(bytes);
    Pool& p = pool();
    std::lock_guard<std::mutex> lock(p.mu);
    auto it = p.free_blocks.find({dev, cls});
    if (it != p.free_blocks.end()) {
        std::vector<FreeBlock>& v = it->second;
        for (size_t i = v.size(); i-- > 0;) {
            FreeBlock& fb = v[i];
            const bool usable = fb.stream == t_stream || !fb.ready || hipEventQuery(fb.ready) == hipSuccess;
            if (!usable) continue;
            void* b = fb.ptr;
            if (fb.ready) (void)hipEventDestroy(fb.ready);
            v.erase(v.begin() + static_cast<std::ptrdiff_t>(i));
            p.cached -= cls;
            p.live[b] = {dev, cls};
            p.allocated += cls;
            (void)hipGetLastError();  // a pending hipEventQuery status is not an error
            return b;
        }
    }
    void* b = nullptr;
    hipError_t e = hipMalloc(&b, cls);
    if (e == hipErrorOutOfMemory) {
        (void)hipGetLastError();
        free_cached_locked(p, dev);
        e = hipMalloc(&b, cls);
    }
    check_hip(e, ("hipMalloc(" + std::to_string(cls) + " bytes)").c_str());
    p.live[b] = {dev, cls};
    p.allocated += cls;
    return b;
}

void release(void* b) noexcept {
    if (!b) return;
    Pool& p = pool();
    std::lock_guard<std::mutex> lock(p.mu);
    auto it = p.live.find(b);
    if (it == p.live.end()) return;
    hipEvent_t ev = nullptr;
    bool recorded = false;
    if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) == hipSuccess) {
        recorded = hipEventRecord(ev, static_cast<hipStream_t>(t_stream)) == hipSuccess;
        if (!recorded) (void)hipEventDestroy(ev);
    }
    if (!recorded) {
        // no event: wait for the device, so the block is free for any stream
        ev = nullptr;
        (void)hipDeviceSynchronize();
    }
    (void)hipGetLastError();
    p.free_blocks[it->second].push_back(FreeBlock{b, t_stream, ev});
    p.cached += it->second.second;
    p.allocated -= it->second.second;
    p.live.erase(it);
}

void empty_cache() {
    Pool& p = pool();
    std::lock_guard<std::mutex> lock(p.mu);
    free_cached_locked(p, -1);
}

size_t cached_bytes() {
    std::lock_guard<std::mutex> lock(pool().mu);
    return pool().cached;
}

size_t allocated_bytes() {
    std::lock_guard<std::mutex> lock(pool().mu);
    return pool().allocated;
}

void copy_to_device(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return;
    check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(t_stream)),
              "hipMemcpyAsync(host to device)");
    // The host buffer belongs to the caller and may be reused as soon as this
    // returns, so the copy is complete before returning.
    synchronize();
}

void copy_to_host(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return;
    check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, static_cast<hipStream_t>(t_stream)),
              "hipMemcpyAsync(device to host)");
    synchronize();
}

void copy_on_device(void* dst, const void* src, size_t bytes) {
    if (bytes == 0 || dst == src) return;
    check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(t_stream)),
              "hipMemcpyAsync(device to device)");
}

void synchronize() { check_status(tbn_hip_synchronize(t_stream), "synchronize"); }

}  // namespace device

// ---- Tensor ------------------------------------------------------------------------------

namespace {
std::shared_ptr<void> alloc_storage(size_t bytes, DeviceType device) {
    if (device == DeviceType::HIP) {
        check_status(tbn_hip_device_check(), "device check");
        return std::shared_ptr<void>(device::allocate(bytes), [](void* p) { device::release(p); });
    }
    return std::shared_ptr<void>(new uint8_t[bytes > 0 ? bytes : 1], std::default_delete<uint8_t[]>());
}

size_t checked_bytes(const Shape& shape, DataType dtype) {
    for (auto d : shape.dims)
        TBN_CHECK(d >= 0, InvalidShapeError, "negative dimension in " + shape_to_string(shape));
    return static_cast<size_t>(shape.size()) * element_size(dtype);
}
}  // namespace

Tensor Tensor::empty(const Shape& shape, DataType dtype, DeviceType device) {
    Tensor t;
    t.shape_ = shape;
    t.dtype_ = dtype;
    t.device_ = device;
    t.data_size_ = checked_bytes(shape, dtype);
    t.data_ = alloc_storage(t.data_size_, device);
    return t;
}

Tensor::Tensor(const Shape& shape, DataType dtype, DeviceType device) {
    *this = empty(shape, dtype, device);
    if (device == DeviceType::HIP) {
        if (data_size_)
            check_hip(hipMemsetAsync(data_.get(), 0, data_size_,
                                     static_cast<hipStream_t>(device::current_stream())),
                      "hipMemsetAsync");
    } else {
        std::memset(data_.get(), 0, data_size_);
    }
}

Tensor::Tensor(const Shape& shape, DataType dtype, const void* data, DeviceType device) {
    *this = empty(shape, dtype, device);
    if (device == DeviceType::HIP)
        device::copy_to_device(data_.get(), data, data_size_);
    else if (data_size_)
        std::memcpy(data_.get(), data, data_size_);
}

Tensor Tensor::wrap(const Shape& shape, DataType dtype, void* data, DeviceType device) {
    Tensor t;
    t.shape_ = shape;
    t.dtype_ = dtype;
    t.device_ = device;
    t.data_size_ = checked_bytes(shape, dtype);
    t.data_ = std::shared_ptr<void>(data, [](void*) {});
    return t;
}

Tensor Tensor::reshaped(const Shape& shape) const {
    TBN_CHECK(shape.size() == shape_.size(), InvalidShapeError,
              "reshape " + shape_to_string(shape_) + " -> " + shape_to_string(shape) +
                  " changes the element count");
    Tensor t = *this;
    t.shape_ = shape;
    return t;
}

Tensor Tensor::copy() const {
    Tensor t = empty(shape_, dtype_, device_);
    t.qparams_ = qparams_;
    if (device_ == DeviceType::HIP)
        device::copy_on_device(t.data_.get(), data_.get(), data_size_);
    else if (data_size_)
        std::memcpy(t.data_.get(), data_.get(), data_size_);
    return t;
}

Tensor Tensor::to_device(DeviceType device) const {
    const bool src_dev = device_ == DeviceType::HIP, dst_dev = device == DeviceType::HIP;
    if (src_dev == dst_dev) {
        Tensor t = copy();
        t.device_ = device;
        return t;
    }
    Tensor t = empty(shape_, dtype_, device);
    t.qparams_ = qparams_;
    if (dst_dev)
        device::copy_to_device(t.data_.get(), data_.get(), data_size_);
    else
        device::copy_to_host(t.data_.get(), data_.get(), data_size_);
    return t;
}

void Tensor::read_bytes(void* host_dst) const {
    if (device_ == DeviceType::HIP)
        device::copy_to_host(host_dst, data_.get(), data_size_);
    else if (data_size_)
        std::memcpy(host_dst, data_.get(), data_size_);
}

Tensor make_tensor(const Shape& shape, const std::vector<float>& data) {
    TBN_CHECK(static_cast<int64_t>(data.size()) == shape.size(), InvalidShapeError,
              "Data size doesn't match shape");
    return Tensor(shape, DataType::FLOAT32, data.data());
}

Tensor make_tensor(const Shape& shape, const std::vector<TernaryWeight>& data) {
    TBN_CHECK(static_cast<int64_t>(data.size()) == shape.size(), InvalidShapeError,
              "Data size doesn't match shape");
    return Tensor(shape, DataType::TERNARY, data.data());
}

Tensor make_tensor(const Shape& shape, const std::vector<BinaryWeight>& data) {
    TBN_CHECK(static_cast<int64_t>(data.size()) == shape.size(), InvalidShapeError,
              "Data size doesn't match shape");
    return Tensor(shape, DataType::BINARY, data.data());
}

}  // namespace tbn
