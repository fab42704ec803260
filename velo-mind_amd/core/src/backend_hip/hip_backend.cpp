// DeviceType::HIP registration: storage creator (one vm_hip_malloc per
// storage, so a graph's arena is a single device allocation), synchronous
// transfers on the thread's current stream, availability, and the
// execution context (one non-blocking stream per Executable, made current
// on the executing thread and synchronized at the end of execute()).
// Replaces the reference's src/cuda/storage.cu and cuda_context.{h,cu}.
#include <memory>
#include <string>

#include "backend_hip/hip_runtime.h"
#include "internal/registry/device_context.h"
#include "internal/registry/memory_transfer.h"
#include "internal/registry/storage.h"

namespace velomind::backend::hip {

namespace {

thread_local void* t_current_stream = nullptr;

struct HipContext {
    void* stream = nullptr;
    ~HipContext() {
        if (stream) (void)vm_hip_stream_destroy(stream);
    }
};

std::shared_ptr<TensorStorage> hip_allocate(std::size_t bytes) {
    void* dev = nullptr;
    if (bytes > 0) {
        const int rc = vm_hip_malloc(&dev, bytes);
        if (rc != VM_HIP_OK) throw std::runtime_error(vm_hip_last_error());
    }
    // The deleter keeps the original pointer: bind_input may rebind data.
    auto s = std::shared_ptr<TensorStorage>(new TensorStorage{}, [dev](TensorStorage* p) {
        if (dev) (void)vm_hip_free(dev);
        delete p;
    });
    s->size_bytes = bytes;
    s->capacity_bytes = bytes;
    s->device = DeviceType::HIP;
    s->data = dev;
    return s;
}

void hip_h2d(void* dst, const void* src, std::size_t bytes) {
    const int rc = vm_hip_memcpy_h2d(dst, src, bytes, t_current_stream);
    if (rc != VM_HIP_OK) throw std::runtime_error(vm_hip_last_error());
}

void hip_d2h(void* dst, const void* src, std::size_t bytes) {
    const int rc = vm_hip_memcpy_d2h(dst, src, bytes, t_current_stream);
    if (rc != VM_HIP_OK) throw std::runtime_error(vm_hip_last_error());
}

bool hip_available() noexcept {
    int n = 0;
    return vm_hip_device_count(&n) == VM_HIP_OK && n > 0;
}

std::shared_ptr<void> context_create() {
    auto ctx = std::make_shared<HipContext>();
    const int rc = vm_hip_stream_create(&ctx->stream);
    if (rc != VM_HIP_OK) throw std::runtime_error(std::string("HIP context: ") + vm_hip_last_error());
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
