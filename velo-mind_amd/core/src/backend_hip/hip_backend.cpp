// DeviceType::HIP registration: storage creator (one device block per
// storage, so a graph's arena is a single device allocation), synchronous
// transfers on the thread's current stream, availability, and the
// execution context (one non-blocking stream per Executable, made current
// on the executing thread and synchronized at the end of execute()).
// Replaces the reference's src/cuda/storage.cu and cuda_context.{h,cu}.
//
// The reference's engine builds a new Graph for every call
// (llama_engine.cpp:395-455), so a decode token allocates and frees the
// arena, the inputs and every layer's grown K/V cache, and creates and
// destroys the Executable's stream.  On HIP those calls cost more than the
// token's kernels (hipFree synchronizes the device; a stream creation
// takes ~0.7 ms), so the backend keeps them:
//   * storages come from a per-device block cache in size classes
//     (block_cache.h): a freed block is parked, and becomes reusable only
//     after a device-wide synchronization that began after it was freed --
//     the guarantee hipFree gives; when the device allocator fails, the
//     cache gives its blocks back and the allocation is tried again;
//   * Executable streams come from a per-device pool and return to it
//     (synchronized) when the Executable is destroyed, keeping the
//     stream's split-K and staging workspaces;
//   * the device count is read once per process.
#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "backend_hip/block_cache.h"
#include "backend_hip/hip_runtime.h"
#include "internal/registry/device_context.h"
#include "internal/registry/memory_transfer.h"
#include "internal/registry/storage.h"

namespace velomind::backend::hip {

namespace {

thread_local void* t_current_stream = nullptr;

int current_device_or_zero() {
    int d = 0;
    return vm_hip_get_device(&d) == VM_HIP_OK ? d : 0;
}

// ---- storage block cache (block_cache.h)
constexpr std::size_t kMaxCachedBytes = std::size_t(8) << 30;   // parked + idle, per process

BlockCache& block_cache() {
    static BlockCache* c = new BlockCache(   // outlives every storage (never destroyed)
        BlockOps{[](void** p, std::size_t n) { return vm_hip_malloc(p, n); }, [](void* p) { return vm_hip_free(p); },
                 [] { return vm_hip_device_synchronize(); }},
        kMaxCachedBytes);
    return *c;
}

std::shared_ptr<TensorStorage> hip_allocate(std::size_t bytes) {
    void* block = nullptr;
    const std::size_t cls = bytes > 0 ? block_size_class(bytes) : 0;
    const int d = current_device_or_zero();
    if (cls > 0) {
        block = block_cache().allocate(d, cls);
        if (!block) throw std::runtime_error(vm_hip_last_error());
    }
    // The deleter keeps the original pointer: bind_input may rebind data.
    auto s = std::shared_ptr<TensorStorage>(new TensorStorage{}, [block, cls, d](TensorStorage* p) {
        if (block) (void)block_cache().park(d, cls, block);
        delete p;
    });
    s->size_bytes = bytes;
    s->capacity_bytes = cls;
    s->device = DeviceType::HIP;
    s->data = block;
    return s;
}

// ---- Executable streams
struct StreamPool {
    std::mutex mu;
    std::map<int, std::vector<void*>> idle;
    static StreamPool& get() {
        static StreamPool* p = new StreamPool();   // pooled streams live until the process ends
        return *p;
    }
    void* take(int d) {
        {
            std::lock_guard<std::mutex> lock(mu);
            auto& v = idle[d];
            if (!v.empty()) {
                void* s = v.back();
                v.pop_back();
                return s;
            }
        }
        void* s = nullptr;
        const int rc = vm_hip_stream_create(&s);
        if (rc != VM_HIP_OK) throw std::runtime_error(std::string("HIP context: ") + vm_hip_last_error());
        return s;
    }
    void give(int d, void* s) {
        if (vm_hip_stream_synchronize(s) != VM_HIP_OK) {
            (void)vm_hip_stream_destroy(s);
            return;
        }
        std::lock_guard<std::mutex> lock(mu);
        idle[d].push_back(s);
    }
};

struct HipContext {
    void* stream = nullptr;
    int device = 0;
    ~HipContext() {
        if (stream) StreamPool::get().give(device, stream);
    }
};

void hip_h2d(void* dst, const void* src, std::size_t bytes) {
    const int rc = vm_hip_memcpy_h2d(dst, src, bytes, t_current_stream);
    if (rc != VM_HIP_OK) throw std::runtime_error(vm_hip_last_error());
}

void hip_d2h(void* dst, const void* src, std::size_t bytes) {
    const int rc = vm_hip_memcpy_d2h(dst, src, bytes, t_current_stream);
    if (rc != VM_HIP_OK) throw std::runtime_error(vm_hip_last_error());
}

bool hip_available() noexcept {
    static const bool available = [] {
        int n = 0;
        return vm_hip_device_count(&n) == VM_HIP_OK && n > 0;
    }();
    return available;
}

std::shared_ptr<void> context_create() {
    auto ctx = std::make_shared<HipContext>();
    ctx->device = current_device_or_zero();
    ctx->stream = StreamPool::get().take(ctx->device);
    return ctx;
}

void* context_activate(void* ctx) {
    void* prev = t_current_stream;
    t_current_stream = static_cast<HipContext*>(ctx)->stream;
    return prev;
}

void context_deactivate(void* prev) { t_current_stream = prev; }

void context_synchronize(void* ctx) {
    const int rc = vm_hip_stream_synchronize(static_cast<HipContext*>(ctx)->stream);
    if (rc != VM_HIP_OK) throw std::runtime_error(std::string("HIP stream synchronize: ") + vm_hip_last_error());
}

}  // namespace

void* current_stream() noexcept { return t_current_stream; }

void reclaim_freed_blocks() { block_cache().reclaim(current_device_or_zero()); }

std::string error_context(Op op, const TensorStorage& output, const char* stage) {
    std::string msg = std::string(op_name(op)) + " on HIP output shape=[";
    for (std::size_t i = 0; i < output.shape.size(); ++i) {
        if (i) msg += ',';
        msg += std::to_string(output.shape[i]);
    }
    return msg + "] at " + stage;
}

void throw_status(int status, const std::string& context) {
    const std::string msg = context + ": " + vm_hip_last_error();
    if (status == VM_HIP_EINVAL) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

}  // namespace velomind::backend::hip

namespace {
using namespace velomind::backend::hip;
constexpr velomind::internal::DeviceContextHooks kHipHooks{&context_create, &context_activate, &context_deactivate,
                                                           &context_synchronize};
}  // namespace

VELOMIND_REGISTER_STORAGE_CREATOR(::velomind::DeviceType::HIP, &hip_allocate)
VELOMIND_REGISTER_MEMORY_TRANSFER(::velomind::DeviceType::HIP, &hip_h2d, &hip_d2h)
VELOMIND_REGISTER_DEVICE_AVAILABILITY(::velomind::DeviceType::HIP, &hip_available)
VELOMIND_REGISTER_DEVICE_CONTEXT(::velomind::DeviceType::HIP, kHipHooks)
