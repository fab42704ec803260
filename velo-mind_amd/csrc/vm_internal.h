// Internal helpers shared by the libvmhip translation units: error state,
// fault injection, per-stream workspace and launch checks.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "vm_hip.h"

namespace vmhip {

// Thread-local message returned by vm_hip_last_error().
void set_error(const std::string& msg);
void clear_error();

// Records a hipError_t failure "<what>: <name> (<string>)"; returns err.
int fail_hip(hipError_t err, const char* what);
// Records an argument failure "<what>"; returns VM_HIP_EINVAL.
int fail_inval(const std::string& what);

// VELOMIND_FAIL_BACKEND="HIP:<op>:<stage>" makes the named stage fail, the
// HIP analogue of the reference's CUDA hook (src/cuda/ops/backend_error.h:
// 31-47).  Returns VM_HIP_EINJECTED after recording the message.
int injected_failure(const char* op, const char* stage);

// VELOMIND_HIP_SYNC=1 synchronizes the stream after every launch
// (the reference's VELOMIND_CUDA_SYNC, src/cuda/cuda_context.cu:115-118).
bool sync_debug_enabled();

// Checks the launch of `op` on `stream`: launch error, injected faults and
// the optional debug synchronization.  Returns 0 or an error status.
int check_launch(const char* op, hipStream_t stream);

// Split-K workspace bound to (device, stream).  Calls on one stream are
// ordered by the stream, so they may share it; different streams get
// different workspaces.  `counters` (one u32 per column tile) are zero
// whenever no kernel is running: the last workgroup of a tile resets its
// counter before exiting.
struct Workspace {
    float*    partials = nullptr;
    unsigned* counters = nullptr;
};
// Returns a workspace with at least `partial_floats` floats and
// `counter_slots` counters for `stream`, growing it if needed.
int get_workspace(hipStream_t stream, std::size_t partial_floats, std::size_t counter_slots,
                  Workspace* out);
// Frees the workspace of `stream` (called when the stream is destroyed).
void release_workspace(hipStream_t stream);

// Per-stream staging buffer for dtype conversions (grows on demand; the
// previous contents are not preserved across growth).
int get_staging(hipStream_t stream, std::size_t bytes, void** out);

// Per-stream buffer for operands a kernel prepares for the next kernel of
// the same call (the MFMA GEMM's fp16 copy of A with its row exponents).
// Grows like the workspace; refused during capture.
int get_aux(hipStream_t stream, std::size_t bytes, void** out);

// While an instance is alive, get_workspace() on this thread hands out the
// caller's fixed region (counters first, then partials) instead of the
// per-stream allocation, get_aux() hands out the end of the partials area,
// and either fails with a message naming `who` when a call needs more than
// the region holds; get_staging() fails.  Used by the entry points that
// must not allocate.
struct FixedRegion {
    void*       base = nullptr;
    std::size_t counter_slots = 0;
    std::size_t partial_floats = 0;
    const char* who = "";
    std::size_t aux_bytes = 0;   // taken from the end of the partials area
};

class FixedWorkspaceScope {
public:
    FixedWorkspaceScope(void* base, std::size_t counter_slots, std::size_t partial_floats, const char* who);
    ~FixedWorkspaceScope();
    FixedWorkspaceScope(const FixedWorkspaceScope&) = delete;
    FixedWorkspaceScope& operator=(const FixedWorkspaceScope&) = delete;

private:
    FixedRegion _region;
    FixedRegion* _previous;
};

// Number of compute units of the current device (cached per device).
int cu_count();

}  // namespace vmhip

// Status-propagating helpers for entry points.
#define VM_TRY_HIP(expr, what)                                   \
    do {                                                         \
        hipError_t vm_err_ = (expr);                             \
        if (vm_err_ != hipSuccess) return ::vmhip::fail_hip(vm_err_, what); \
    } while (0)

#define VM_TRY(expr)                    \
    do {                                \
        int vm_rc_ = (expr);            \
        if (vm_rc_ != 0) return vm_rc_; \
    } while (0)
