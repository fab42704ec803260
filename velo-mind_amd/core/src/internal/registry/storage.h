// Per-device storage creators and availability checks (the reference's
// src/internal/registry/storage.h:13-48).
#pragma once

#include "internal/registry/macros.h"

#include <array>
#include <cstddef>
#include <memory>

#include "velomind/tensor_storage.h"
#include "velomind/types.h"

namespace velomind::internal {

// Allocates `bytes` on the device; the returned storage's deleter frees the
// original allocation even if `data` is later rebound.
using StorageCreatorFn = std::shared_ptr<velomind::TensorStorage> (*)(std::size_t bytes);
using DeviceAvailabilityFn = bool (*)() noexcept;

auto storage_creaters() -> std::array<StorageCreatorFn, MAX_DEVICE_TYPES>&;
auto register_storage_creator(DeviceType device, StorageCreatorFn fn) -> void;
auto get_storage_creator(DeviceType device) -> StorageCreatorFn;
auto register_device_availability(DeviceType device, DeviceAvailabilityFn fn) -> void;
auto is_device_available(DeviceType device) noexcept -> bool;
auto create_tensor_storage(std::size_t bytes, DeviceType device) -> std::shared_ptr<velomind::TensorStorage>;

}  // namespace velomind::internal

#define VELOMIND_REGISTER_STORAGE_CREATOR(DEVICE, FN)                                             \
    namespace {                                                                                   \
    [[maybe_unused]] const bool VELOMIND_CONCAT_(_velomind_sc_, __LINE__) = [] {                  \
        ::velomind::internal::register_storage_creator(DEVICE, FN);                               \
        return true;                                                                              \
    }();                                                                                          \
    }

#define VELOMIND_REGISTER_DEVICE_AVAILABILITY(DEVICE, FN)                                         \
    namespace {                                                                                   \
    [[maybe_unused]] const bool VELOMIND_CONCAT_(_velomind_av_, __LINE__) = [] {                  \
        ::velomind::internal::register_device_availability(DEVICE, FN);                           \
        return true;                                                                              \
    }();                                                                                          \
    }
