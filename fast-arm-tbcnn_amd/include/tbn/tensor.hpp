// tbn::Tensor (tbn-runtime/include/tbn/runtime/tensor.hpp:11-110) with device
// residency: the bytes live either in host memory (DeviceType::CPU) or in the
// MI355X's HBM (DeviceType::HIP).  Storage is shared between shallow copies,
// as in the reference; copy() is deep; to_device() moves between host and
// device (the reference throws there).  typed_data<T>() of a HIP tensor is a
// device pointer.
#pragma once

#include <cstring>
#include <memory>
#include <vector>

#include "errors.hpp"
#include "types.hpp"

namespace tbn {

class Tensor {
public:
    Tensor() = default;
    // Zero-filled tensor on `device`.
    Tensor(const Shape& shape, DataType dtype, DeviceType device = DeviceType::CPU);
    // Tensor on `device` initialised from HOST memory `data` (shape.size() elements).
    Tensor(const Shape& shape, DataType dtype, const void* data, DeviceType device = DeviceType::CPU);

    // Uninitialised tensor (device tensors skip the zero fill).
    static Tensor empty(const Shape& shape, DataType dtype, DeviceType device);
    // Non-owning view of existing memory (host or device); the caller keeps
    // the memory alive for the view's lifetime.
    static Tensor wrap(const Shape& shape, DataType dtype, void* data, DeviceType device);

    const Shape& shape() const { return shape_; }
    DataType dtype() const { return dtype_; }
    DeviceType device() const { return device_; }
    bool on_device() const { return device_ == DeviceType::HIP; }
    bool defined() const { return data_ != nullptr || data_size_ == 0; }
    void* data() { return data_.get(); }
    const void* data() const { return data_.get(); }
    size_t data_size() const { return data_size_; }

    const QuantizationParams& quantization_params() const { return qparams_; }
    void set_quantization_params(const QuantizationParams& p) { qparams_ = p; }

    int64_t num_elements() const { return shape_.size(); }
    int64_t dim(int idx) const {
        TBN_CHECK(idx >= 0 && static_cast<size_t>(idx) < shape_.dims.size(), InvalidArgumentError,
                  "Dimension index out of range");
        return shape_.dims[idx];
    }

    template <typename T>
    T* typed_data() { return static_cast<T*>(data_.get()); }
    template <typename T>
    const T* typed_data() const { return static_cast<const T*>(data_.get()); }

    // Same storage, new shape (element count must match).
    Tensor reshaped(const Shape& shape) const;

    Tensor copy() const;
    Tensor to_device(DeviceType device) const;
    // Host copy of the elements (waits for the device when on_device()).
    template <typename T>
    std::vector<T> to_vector() const {
        std::vector<T> out(data_size_ / sizeof(T));
        read_bytes(out.data());
        return out;
    }

private:
    void read_bytes(void* host_dst) const;

    Shape shape_;
    DataType dtype_ = DataType::FLOAT32;
    DeviceType device_ = DeviceType::CPU;
    std::shared_ptr<void> data_;
    size_t data_size_ = 0;
    QuantizationParams qparams_;
};

Tensor make_tensor(const Shape& shape, const std::vector<float>& data);
Tensor make_tensor(const Shape& shape, const std::vector<TernaryWeight>& data);
Tensor make_tensor(const Shape& shape, const std::vector<BinaryWeight>& data);

}  // namespace tbn
