// Core enums and shape aliases.  Enum values are ABI: they match the
// reference's include/velomind/types.h:20-37, with DeviceType::HIP appended.
#pragma once

#include <cstddef>
#include <cstdint>
#include <ostream>
#include <string>
#include <vector>

namespace velomind {

using index_t = std::int64_t;
using dim_t = std::int64_t;
using shape_t = std::vector<dim_t>;
using stride_t = std::vector<dim_t>;
using strides_t = stride_t;

// Values must stay contiguous; Last sizes the per-dtype tables.
enum class DataType : std::uint8_t {
    Float32 = 0,
    Int32 = 1,
    Int8 = 2,
    Bool = 3,
    Float16 = 4,
    BFloat16 = 5,
    Last = BFloat16,
};

// Values must stay contiguous; Last sizes the per-device registries.
enum class DeviceType : std::uint8_t {
    CPU = 0,
    CUDA = 1,
    ISPC = 2,
    HIP = 3,
    Last = HIP,
};

constexpr std::size_t MAX_DEVICE_TYPES = static_cast<std::size_t>(DeviceType::Last) + 1;

constexpr std::size_t data_type_size(DataType dtype) {
    switch (dtype) {
        case DataType::Float32: return 4;
        case DataType::Int32: return 4;
        case DataType::Int8: return 1;
        case DataType::Bool: return sizeof(bool);
        case DataType::Float16: return 2;
        case DataType::BFloat16: return 2;
    }
    return 0;
}

constexpr const char* data_type_name(DataType dtype) {
    switch (dtype) {
        case DataType::Float32: return "Float32";
        case DataType::Int32: return "Int32";
        case DataType::Int8: return "Int8";
        case DataType::Bool: return "Bool";
        case DataType::Float16: return "Float16";
        case DataType::BFloat16: return "BFloat16";
    }
    return "Unknown";
}

constexpr const char* device_type_name(DeviceType device) {
    switch (device) {
        case DeviceType::CPU: return "CPU";
        case DeviceType::CUDA: return "CUDA";
        case DeviceType::ISPC: return "ISPC";
        case DeviceType::HIP: return "HIP";
    }
    return "Unknown";
}

inline std::string to_string(const shape_t& shape) {
    std::string out = "[";
    for (std::size_t i = 0; i < shape.size(); ++i) {
        if (i) out += ", ";
        out += std::to_string(shape[i]);
    }
    return out + "]";
}

inline std::string to_string(DataType dtype) { return data_type_name(dtype); }
inline std::string to_string(DeviceType device) { return device_type_name(device); }

inline std::ostream& operator<<(std::ostream& os, DataType dtype) { return os << data_type_name(dtype); }
inline std::ostream& operator<<(std::ostream& os, DeviceType device) { return os << device_type_name(device); }
inline std::ostream& operator<<(std::ostream& os, const shape_t& shape) { return os << to_string(shape); }

}  // namespace velomind

#include "velomind/dtype.h"
