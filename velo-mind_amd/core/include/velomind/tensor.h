// Lightweight handle to a tensor owned by a Graph (graph pointer + index,
// guarded by the graph's lifetime token).
#pragma once

#include <cstddef>
#include <memory>
#include <ostream>
#include <span>
#include <string>

#include "velomind/ptr.h"
#include "velomind/tensor_storage.h"
#include "velomind/types.h"
#include "velomind_core_export.h"

namespace velomind {

class Graph;

class VELOMIND_CORE_EXPORT Tensor {
public:
    Tensor() = default;
    Tensor(Graph* graph, std::size_t index) noexcept;

    auto shape() const -> const shape_t&;
    auto dtype() const -> DataType;
    auto device() const -> DeviceType;
    auto numel() const -> std::size_t;
    auto nbytes() const -> std::size_t;
    auto strides() const -> stride_t;
    auto offset_bytes() const -> std::size_t;
    auto capacity_bytes() const -> std::size_t;
    auto is_contiguous() const -> bool;
    auto is_alias() const -> bool;

    // First element (device address for HIP tensors).
    auto data() const -> const void*;
    auto data() -> void*;

    auto storage() const -> pConstTensorStorage;
    auto storage() -> pTensorStorage;
    auto shared_storage() const -> std::shared_ptr<TensorStorage>;
    auto has_storage() const -> bool { return storage() != nullptr; }
    auto index() const noexcept -> std::size_t { return _index; }
    auto graph() const noexcept -> Graph* { return _graph; }
    explicit operator bool() const noexcept { return storage() != nullptr; }

    // Synchronous host <-> device copies through the device's MemoryTransfer.
    auto copy_from_host(std::span<const std::byte> data) -> void;
    auto copy_from_host(std::span<const std::byte> data, std::size_t dst_offset_bytes) -> void;
    auto copy_to_host(std::span<std::byte> data) const -> void;
    auto copy_to_host(std::span<std::byte> data, std::size_t src_offset_bytes) const -> void;

    auto to_string(bool print_data = false) const -> std::string;

    friend bool operator==(const Tensor& a, const Tensor& b) noexcept { return a._graph == b._graph && a._index == b._index; }
    friend bool operator!=(const Tensor& a, const Tensor& b) noexcept { return !(a == b); }

private:
    friend class Graph;
    Graph* _graph = nullptr;
    std::size_t _index = 0;
    std::weak_ptr<void> _graph_lifetime;
};

inline auto to_string(const Tensor& t, bool print_data = false) -> std::string { return t.to_string(print_data); }
inline auto operator<<(std::ostream& os, const Tensor& t) -> std::ostream& { return os << t.to_string(); }

VELOMIND_EXPORT_PTR(Tensor);

}  // namespace velomind
