// Per-device execution-context hooks.  A backend that runs asynchronously
// registers how to create its context (e.g. a HIP stream) for an
// Executable, how to make it current for the calling thread while
// execute() runs, and how to synchronize it.  The graph compiler and the
// executor call these instead of naming any backend, which replaces the
// reference's `#ifdef VELOMIND_ENABLE_CUDA` blocks
// (src/internal/graph_compiler.cpp:669-673, src/executable.cpp:9-23,44-81).
#pragma once

#include "internal/registry/macros.h"

#include <memory>

#include "velomind/types.h"

namespace velomind::internal {

struct DeviceContextHooks {
    // New context for one Executable (nullptr if the device needs none).
    std::shared_ptr<void> (*create)() = nullptr;
    // Makes `ctx` current on this thread; returns the previous one.
    void* (*activate)(void* ctx) = nullptr;
    // Restores the context returned by activate().
    void (*deactivate)(void* previous) = nullptr;
    // Waits for all work enqueued on `ctx`; throws on device errors.
    void (*synchronize)(void* ctx) = nullptr;
};

void register_device_context_hooks(DeviceType device, DeviceContextHooks hooks);
auto get_device_context_hooks(DeviceType device) -> DeviceContextHooks;

// RAII: activates an Executable's context for the duration of a scope.
class ScopedDeviceContext {
public:
    ScopedDeviceContext(DeviceType device, void* ctx);
    ~ScopedDeviceContext();
    ScopedDeviceContext(const ScopedDeviceContext&) = delete;
    ScopedDeviceContext& operator=(const ScopedDeviceContext&) = delete;

private:
    DeviceContextHooks _hooks;
    void* _previous = nullptr;
    bool _active = false;
};

}  // namespace velomind::internal

#define VELOMIND_REGISTER_DEVICE_CONTEXT(DEVICE, HOOKS)                                           \
    namespace {                                                                                   \
    [[maybe_unused]] const bool VELOMIND_CONCAT_(_velomind_dc_, __LINE__) = [] {                  \
        ::velomind::internal::register_device_context_hooks(DEVICE, HOOKS);                       \
        return true;                                                                              \
    }();                                                                                          \
    }
