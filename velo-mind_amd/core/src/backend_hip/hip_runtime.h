// HIP backend internals shared by its translation units.
#pragma once

#include <stdexcept>
#include <string>

#include "velomind/ops.h"
#include "velomind/tensor_storage.h"
#include "vm_hip.h"

namespace velomind::backend::hip {

// Stream of the HIP context active on this thread (nullptr = null stream).
void* current_stream() noexcept;

// Makes the storage blocks freed so far on the current device reusable (one
// device-wide synchronization when any are waiting).  For callers that know
// the device is idle and are about to allocate from another thread while
// new work runs: the allocations then need no synchronization of their own.
void reclaim_freed_blocks();

// "<op> on HIP output shape=[a,b] at <stage>" (the reference's CUDA
// message format, src/cuda/ops/backend_error.h:15-23).
std::string error_context(Op op, const TensorStorage& output, const char* stage);

// Throws for a failed libvmhip status: std::invalid_argument for argument
// errors, std::runtime_error otherwise; the message carries `context` and
// vm_hip_last_error().
[[noreturn]] void throw_status(int status, const std::string& context);

inline void check_status(int status, const std::string& context) {
    if (status != VM_HIP_OK) throw_status(status, context);
}

}  // namespace velomind::backend::hip
