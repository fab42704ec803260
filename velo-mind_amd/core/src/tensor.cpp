// Tensor handle accessors and host transfers (the reference's src/tensor.cpp).
#include "velomind/tensor.h"

#include <sstream>
#include <stdexcept>

#include "internal/registry/memory_transfer.h"
#include "internal/registry/storage.h"
#include "velomind/graph.h"

namespace velomind {

Tensor::Tensor(Graph* graph, std::size_t index) noexcept
    : _graph(graph), _index(index), _graph_lifetime(graph ? graph->lifetime_token() : std::weak_ptr<void>{}) {}

auto Tensor::storage() const -> pConstTensorStorage {
    return (_graph && !_graph_lifetime.expired()) ? _graph->tensor_storage_at(_index) : nullptr;
}
auto Tensor::storage() -> pTensorStorage {
    return (_graph && !_graph_lifetime.expired()) ? _graph->tensor_storage_at(_index) : nullptr;
}
auto Tensor::shared_storage() const -> std::shared_ptr<TensorStorage> {
    return (_graph && !_graph_lifetime.expired()) ? _graph->shared_storage_at(_index) : nullptr;
}

auto Tensor::shape() const -> const shape_t& {
    static const shape_t empty;
    auto* s = storage();
    return s ? s->shape : empty;
}
auto Tensor::dtype() const -> DataType { auto* s = storage(); return s ? s->dtype : DataType::Float32; }
auto Tensor::device() const -> DeviceType { auto* s = storage(); return s ? s->device : DeviceType::CPU; }
auto Tensor::numel() const -> std::size_t { auto* s = storage(); return s ? storage_numel(*s) : 0; }
auto Tensor::nbytes() const -> std::size_t { auto* s = storage(); return s ? s->size_bytes : 0; }
auto Tensor::strides() const -> stride_t { auto* s = storage(); return s ? s->effective_strides() : stride_t{}; }
auto Tensor::offset_bytes() const -> std::size_t { auto* s = storage(); return s ? s->offset_bytes : 0; }
auto Tensor::capacity_bytes() const -> std::size_t { auto* s = storage(); return s ? s->capacity_bytes : 0; }
auto Tensor::is_contiguous() const -> bool { auto* s = storage(); return s ? s->is_contiguous() : true; }
auto Tensor::is_alias() const -> bool { auto* s = storage(); return s ? s->is_alias() : false; }
auto Tensor::data() const -> const void* { auto* s = storage(); return s ? s->data : nullptr; }
auto Tensor::data() -> void* { auto* s = storage(); return s ? s->data : nullptr; }

void Tensor::copy_from_host(std::span<const std::byte> data) {
    auto* s = storage();
    if (!s) throw std::runtime_error("Tensor::copy_from_host: handle not bound (call Graph::build first)");
    if (data.size() != s->size_bytes) throw std::runtime_error("Tensor::copy_from_host: size mismatch");
    copy_from_host(data, 0);
}

void Tensor::copy_from_host(std::span<const std::byte> data, std::size_t dst_offset) {
    auto* s = storage();
    if (!s) throw std::runtime_error("Tensor::copy_from_host: handle not bound (call Graph::build first)");
    if (dst_offset > s->size_bytes || data.size() > s->size_bytes - dst_offset)
        throw std::runtime_error("Tensor::copy_from_host: offset and size exceed tensor bounds");
    if (data.empty()) return;
    if (!s->data) throw std::logic_error("Tensor::copy_from_host: tensor buffer is not allocated");
    const auto t = internal::get_memory_transfer(s->device);
    if (!t.copy_h2d) throw std::runtime_error("Tensor::copy_from_host: no host->device transfer for device");
    t.copy_h2d(static_cast<char*>(s->data) + dst_offset, data.data(), data.size());
}

void Tensor::copy_to_host(std::span<std::byte> data) const {
    auto* s = storage();
    if (!s) throw std::runtime_error("Tensor::copy_to_host: handle not bound (call Graph::build first)");
    if (data.size() != s->size_bytes) throw std::runtime_error("Tensor::copy_to_host: size mismatch");
    copy_to_host(data, 0);
}

void Tensor::copy_to_host(std::span<std::byte> data, std::size_t src_offset) const {
    auto* s = storage();
    if (!s) throw std::runtime_error("Tensor::copy_to_host: handle not bound (call Graph::build first)");
    if (src_offset > s->size_bytes || data.size() > s->size_bytes - src_offset)
        throw std::runtime_error("Tensor::copy_to_host: offset and size exceed tensor bounds");
    if (data.empty()) return;
    if (!s->data) throw std::logic_error("Tensor::copy_to_host: tensor buffer is not allocated");
    const auto t = internal::get_memory_transfer(s->device);
    if (!t.copy_d2h) throw std::runtime_error("Tensor::copy_to_host: no device->host transfer for device");
    t.copy_d2h(data.data(), static_cast<const char*>(s->data) + src_offset, data.size());
}

auto Tensor::to_string(bool) const -> std::string {
    auto* s = storage();
    if (!s) return "Tensor(unbound)";
    std::ostringstream os;
    os << "Tensor(shape=" << velomind::to_string(s->shape) << ", dtype=" << data_type_name(s->dtype)
       << ", device=" << device_type_name(s->device) << ")";
    return os.str();
}

auto TensorStorage::is_available(DeviceType device) noexcept -> bool { return internal::is_device_available(device); }

auto TensorStorage::allocate(std::size_t bytes, DeviceType device) -> std::shared_ptr<TensorStorage> {
    auto fn = internal::get_storage_creator(device);
    return fn ? fn(bytes) : nullptr;
}

}  // namespace velomind
