// Element types, devices, shapes and quantization parameters of the tbn
// runtime (tbn-runtime/include/tbn/runtime/types.hpp:11-106).  DeviceType gains
// HIP: a tensor whose bytes live in the MI355X's HBM.
#pragma once

#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <string>
#include <vector>

namespace tbn {

enum class DataType {
    FLOAT32,
    FLOAT16,
    BFLOAT16,
    INT8,
    INT16,
    INT32,
    INT64,
    UINT8,
    UINT16,
    UINT32,
    UINT64,
    BOOL,
    TERNARY,  // one int8 per element: -1, 0, +1
    BINARY    // one byte per element: 1 = +1, anything else = -1
};

enum class DeviceType {
    CPU,
    ARM_NEON,
    ARM_SVE,
    HIP  // device memory of the current HIP device (gfx950)
};

struct Shape {
    std::vector<int64_t> dims;

    Shape() = default;
    Shape(std::initializer_list<int64_t> d) : dims(d) {}
    Shape(const std::vector<int64_t>& d) : dims(d) {}

    int64_t size() const {
        int64_t s = 1;
        for (auto d : dims) s *= d;
        return s;
    }
    size_t rank() const { return dims.size(); }
    bool operator==(const Shape& o) const { return dims == o.dims; }
    bool operator!=(const Shape& o) const { return dims != o.dims; }
};

std::string shape_to_string(const Shape& s);
size_t element_size(DataType dtype);
bool is_host(DeviceType d);

struct QuantizationParams {
    float scale = 1.0f;
    int32_t zero_point = 0;
    int32_t bit_width = 8;
    QuantizationParams() = default;
    QuantizationParams(float s, int32_t z, int32_t bits = 8) : scale(s), zero_point(z), bit_width(bits) {}
};

using TernaryWeight = int8_t;
using BinaryWeight = uint8_t;

constexpr TernaryWeight TERNARY_MINUS_ONE = -1;
constexpr TernaryWeight TERNARY_ZERO = 0;
constexpr TernaryWeight TERNARY_PLUS_ONE = 1;
constexpr BinaryWeight BINARY_ZERO = 0;
constexpr BinaryWeight BINARY_ONE = 1;

}  // namespace tbn
