// Per-device host<->device copy functions; both are synchronous on return
// (the reference's src/internal/registry/memory_transfer.h:11-39).
#pragma once

#include "internal/registry/macros.h"

#include <array>
#include <cstddef>

#include "velomind/types.h"

namespace velomind::internal {

struct MemoryTransfer {
    void (*copy_h2d)(void* dst, const void* src, std::size_t bytes) = nullptr;
    void (*copy_d2h)(void* dst, const void* src, std::size_t bytes) = nullptr;
};

auto memory_transfers() -> std::array<MemoryTransfer, MAX_DEVICE_TYPES>&;
void register_memory_transfer(DeviceType device, MemoryTransfer t);
auto get_memory_transfer(DeviceType device) -> MemoryTransfer;

}  // namespace velomind::internal

#define VELOMIND_REGISTER_MEMORY_TRANSFER(DEVICE, H2D_FN, D2H_FN)                                 \
    namespace {                                                                                   \
    [[maybe_unused]] const bool VELOMIND_CONCAT_(_velomind_mt_, __LINE__) = [] {                  \
        ::velomind::internal::register_memory_transfer(                                           \
            (DEVICE), ::velomind::internal::MemoryTransfer{(H2D_FN), (D2H_FN)});                  \
        return true;                                                                              \
    }();                                                                                          \
    }
