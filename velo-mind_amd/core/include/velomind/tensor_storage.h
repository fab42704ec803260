// Physical storage (or view) of one tensor: shape, element strides, byte
// offset into the owning allocation and the device pointer.  Field set and
// meaning follow the reference's include/velomind/tensor_storage.h:50-80;
// `data` already includes the view offset.
#pragma once

#include <algorithm>
#include <cstddef>
#include <limits>
#include <memory>
#include <ostream>
#include <stdexcept>
#include <string>

#include "velomind/ptr.h"
#include "velomind/types.h"
#include "velomind_core_export.h"

namespace velomind {

// Row-major element strides of `shape` (saturating on overflow).
inline auto default_strides(const shape_t& shape) -> stride_t {
    if (shape.empty()) return {};
    stride_t st(shape.size(), 1);
    for (std::size_t i = shape.size() - 1; i > 0; --i) {
        const dim_t extent = std::max<dim_t>(0, shape[i]);
        dim_t next = 0;
        if (__builtin_mul_overflow(st[i], extent, &next)) next = std::numeric_limits<dim_t>::max();
        st[i - 1] = next;
    }
    return st;
}

// True when `strides` (empty = default) describe a row-major layout;
// size-1 dimensions may carry any stride.
inline auto is_shape_contiguous(const shape_t& shape, const stride_t& strides) -> bool {
    if (strides.empty() || shape.empty()) return true;
    if (strides.size() != shape.size()) return false;
    dim_t expect = 1;
    for (std::size_t i = shape.size(); i-- > 0;) {
        if (shape[i] <= 0) return true;
        if (shape[i] == 1) continue;
        if (strides[i] != expect) return false;
        if (__builtin_mul_overflow(expect, shape[i], &expect)) return false;
    }
    return true;
}

struct TensorStorage {
    shape_t shape;
    stride_t strides;                       // element strides; empty means row-major
    std::size_t offset_bytes = 0;           // view offset inside the owning allocation
    std::size_t capacity_bytes = 0;         // bytes of the owning allocation
    DataType dtype = DataType::Float32;
    DeviceType device = DeviceType::CPU;
    void* data = nullptr;                   // first element (offset already applied)
    std::size_t size_bytes = 0;             // logical bytes of this tensor
    std::shared_ptr<void> external_owner;   // keeps the allocation of a view alive

    // Allocates `bytes` through the storage creator registered for `device`
    // (nullptr when none is registered).
    VELOMIND_CORE_EXPORT static auto allocate(std::size_t bytes, DeviceType device)
        -> std::shared_ptr<TensorStorage>;
    VELOMIND_CORE_EXPORT static auto is_available(DeviceType device) noexcept -> bool;

    auto effective_strides() const -> stride_t { return strides.empty() ? default_strides(shape) : strides; }
    auto is_contiguous() const -> bool { return is_shape_contiguous(shape, strides); }
    auto is_alias() const noexcept -> bool { return external_owner != nullptr; }
};

inline auto storage_numel(const TensorStorage& s) -> std::size_t {
    std::size_t n = 1;
    bool empty = false;
    for (dim_t d : s.shape) {
        if (d < 0) throw std::invalid_argument("Tensor: negative dimension");
        if (d == 0) empty = true;
    }
    if (empty) return 0;
    for (dim_t d : s.shape) {
        if (static_cast<std::uint64_t>(d) > std::numeric_limits<std::size_t>::max() / n)
            throw std::invalid_argument("Tensor: element count overflow");
        n *= static_cast<std::size_t>(d);
    }
    return n;
}

inline auto storage_nbytes(const TensorStorage& s) -> std::size_t {
    const std::size_t width = data_type_size(s.dtype);
    if (width == 0) throw std::invalid_argument("Tensor: invalid dtype");
    const std::size_t n = storage_numel(s);
    if (n > std::numeric_limits<std::size_t>::max() / width) throw std::invalid_argument("Tensor: byte count overflow");
    return n * width;
}

inline auto to_string(const TensorStorage& s) -> std::string {
    std::string out = "TensorStorage(shape=" + to_string(s.shape) + ", dtype=" + data_type_name(s.dtype) +
                      ", device=" + device_type_name(s.device);
    if (!s.strides.empty()) out += ", strides=" + to_string(s.strides);
    if (s.offset_bytes) out += ", offset_bytes=" + std::to_string(s.offset_bytes);
    if (s.is_alias()) out += ", alias=true";
    out += s.data ? ", allocated)" : ", unallocated)";
    return out;
}

inline auto operator<<(std::ostream& os, const TensorStorage& s) -> std::ostream& { return os << to_string(s); }

VELOMIND_EXPORT_PTR(TensorStorage);

}  // namespace velomind
