// DeviceType::CPU storage: zero-initialised host memory and memcpy
// transfers, so graphs and quantized weights can hold host tensors.  No
// compute kernels are registered for CPU in this library: the operator
// kernels of this build run on HIP.
#include <cstdlib>
#include <cstring>
#include <memory>
#include <new>

#include "internal/registry/memory_transfer.h"
#include "internal/registry/storage.h"

namespace {

std::shared_ptr<velomind::TensorStorage> host_allocate(std::size_t bytes) {
    void* p = nullptr;
    if (bytes > 0) {
        // 256-byte alignment, like the arena slots.
        p = std::aligned_alloc(256, (bytes + 255) / 256 * 256);
        if (!p) throw std::bad_alloc();
        std::memset(p, 0, bytes);
    }
    auto s = std::shared_ptr<velomind::TensorStorage>(new velomind::TensorStorage{}, [p](velomind::TensorStorage* t) {
        std::free(p);
        delete t;
    });
    s->size_bytes = bytes;
    s->capacity_bytes = bytes;
    s->device = velomind::DeviceType::CPU;
    s->data = p;
    return s;
}

void host_copy(void* dst, const void* src, std::size_t bytes) {
    if (bytes) std::memcpy(dst, src, bytes);
}

bool host_available() noexcept { return true; }

}  // namespace

VELOMIND_REGISTER_STORAGE_CREATOR(::velomind::DeviceType::CPU, &host_allocate)
VELOMIND_REGISTER_MEMORY_TRANSFER(::velomind::DeviceType::CPU, &host_copy, &host_copy)
VELOMIND_REGISTER_DEVICE_AVAILABILITY(::velomind::DeviceType::CPU, &host_available)
