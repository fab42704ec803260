// Runtime half of the C ABI: error state, devices, memory, streams,
// events and the per-stream split-K workspace.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "vm_internal.h"

namespace vmhip {

namespace {
thread_local std::string t_last_error;

// A grown workspace or staging buffer is retired, not freed: HIP graphs
// captured earlier on the stream hold its address and may be replayed
// later.  Retired buffers are freed with the stream (vm_hip_stream_destroy).
struct WsEntry {
    void*       base = nullptr;
    std::size_t partial_floats = 0;
    std::size_t counter_slots = 0;
    std::vector<void*> retired;
};


struct StagingEntry {
    void*       base = nullptr;
    std::size_t bytes = 0;
    std::vector<void*> retired;
};

thread_local FixedRegion* t_fixed = nullptr;

struct AuxEntry {
    void*       base = nullptr;
    std::size_t bytes = 0;
    std::vector<void*> retired;
};
// The per-(device, stream) buffers and their lock, created on first use and
// never destroyed: streams can be destroyed from finalizers that run while
// the process exits (Python objects, static destructors of other
// libraries), after namespace-scope objects of this library would already
// be gone.  The buffers themselves are freed with their stream, and the
// driver reclaims whatever is left at exit.
struct Registries {
    std::mutex mutex;
    std::map<std::pair<int, hipStream_t>, WsEntry> ws;
    std::map<std::pair<int, hipStream_t>, StagingEntry> staging;
    std::map<std::pair<int, hipStream_t>, AuxEntry> aux;
};

Registries& registries() {
    static Registries* r = new Registries;
    return *r;
}

int current_device() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    return dev;
}
}  // namespace

void set_error(const std::string& msg) { t_last_error = msg; }
void clear_error() { t_last_error.clear(); }

int fail_hip(hipError_t err, const char* what) {
    set_error(std::string(what) + ": " + hipGetErrorName(err) + " (" + hipGetErrorString(err) + ")");
    return static_cast<int>(err);
}

int fail_inval(const std::string& what) {
    set_error(what);
    return VM_HIP_EINVAL;
}

int injected_failure(const char* op, const char* stage) {
    const char* spec = std::getenv("VELOMIND_FAIL_BACKEND");
    if (!spec) return 0;
    const std::string key = std::string("HIP:") + op + ":" + stage;
    if (key != spec) return 0;
    set_error(std::string(op) + " on HIP at " + stage + ": injected failure");
    return VM_HIP_EINJECTED;
}

bool sync_debug_enabled() {
    const char* v = std::getenv("VELOMIND_HIP_SYNC");
    return v && v[0] == '1';
}

int check_launch(const char* op, hipStream_t stream) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        set_error(std::string(op) + " on HIP at launch: " + hipGetErrorName(err) + " (" +
                  hipGetErrorString(err) + ")");
        return static_cast<int>(err);
    }
    VM_TRY(injected_failure(op, "launch"));
    VM_TRY(injected_failure(op, "sync"));
    if (sync_debug_enabled()) {
        err = hipStreamSynchronize(stream);
        if (err != hipSuccess) {
            set_error(std::string(op) + " on HIP at sync: " + hipGetErrorName(err) + " (" +
                      hipGetErrorString(err) + ")");
            return static_cast<int>(err);
        }
    }
    return 0;
}

FixedWorkspaceScope::FixedWorkspaceScope(void* base, std::size_t counter_slots, std::size_t partial_floats,
                                         const char* who)
    : _region{base, counter_slots, partial_floats, who}, _previous(t_fixed) {
    t_fixed = &_region;
}

FixedWorkspaceScope::~FixedWorkspaceScope() { t_fixed = _previous; }

int get_workspace(hipStream_t stream, std::size_t partial_floats, std::size_t counter_slots,
                  Workspace* out) {
    if (const FixedRegion* f = t_fixed) {
        const std::size_t counter_bytes = f->counter_slots * sizeof(unsigned);
        const std::size_t room = f->partial_floats - (f->aux_bytes + sizeof(float) - 1) / sizeof(float);
        if (counter_slots > f->counter_slots || partial_floats > room)
            return fail_inval(std::string(f->who) + ": this shape's split-K scratch needs " +
                              std::to_string(counter_slots * sizeof(unsigned)) + " bytes of counters and " +
                              std::to_string(partial_floats * sizeof(float)) + " bytes of partials; the static scratch holds " +
                              std::to_string(counter_bytes) + " and " + std::to_string(room * sizeof(float)) +
                              (f->aux_bytes ? " (after " + std::to_string(f->aux_bytes) + " bytes of staged A)" : std::string()));
        out->counters = static_cast<unsigned*>(f->base);
        out->partials = reinterpret_cast<float*>(static_cast<char*>(f->base) + counter_bytes);
        return 0;
    }
    const int dev = current_device();
    Registries& reg = registries();
    std::lock_guard<std::mutex> lock(reg.mutex);
    WsEntry& e = reg.ws[{dev, stream}];
    if (e.base == nullptr || e.partial_floats < partial_floats || e.counter_slots < counter_slots) {
        if (stream != nullptr) {
            hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing(stream, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone)
                return fail_inval("QuantizedMatMul: split-K workspace must be sized by an eager call "
                                  "on this stream before graph capture");
        }
        // Grow geometrically so that a sweep of shapes settles quickly.
        std::size_t pf = std::max(partial_floats, e.partial_floats * 2);
        std::size_t cs = std::max(counter_slots, e.counter_slots * 2);
        pf = std::max<std::size_t>(pf, 1 << 16);
        cs = std::max<std::size_t>(cs, 1024);
        if (e.base) {
            // Queued kernels and captured graphs may still use the old buffer.
            e.retired.push_back(e.base);
            e.base = nullptr;
        }
        const std::size_t counter_bytes = ((cs * sizeof(unsigned)) + 255) & ~std::size_t(255);
        void* base = nullptr;
        VM_TRY_HIP(hipMalloc(&base, counter_bytes + pf * sizeof(float)), "workspace: hipMalloc");
        // Zero the counters on the stream that will use them: a plain
        // hipMemset runs on the null stream, which is not ordered with the
        // non-blocking streams the kernels are launched on.  (Growth is
        // refused during capture, so this memset is never captured.)
        hipError_t err = hipMemsetAsync(base, 0, counter_bytes, stream);
        if (err != hipSuccess) {
            (void)hipFree(base);
            return fail_hip(err, "workspace: hipMemsetAsync");
        }
        e.base = base;
        e.partial_floats = pf;
        e.counter_slots = cs;
    }
    const std::size_t counter_bytes = ((e.counter_slots * sizeof(unsigned)) + 255) & ~std::size_t(255);
    out->counters = static_cast<unsigned*>(e.base);
    out->partials = reinterpret_cast<float*>(static_cast<char*>(e.base) + counter_bytes);
    return 0;
}

int get_aux(hipStream_t stream, std::size_t bytes, void** out) {
    bytes = (bytes + 255) & ~std::size_t(255);
    if (FixedRegion* f = t_fixed) {
        const std::size_t area = f->partial_floats * sizeof(float);
        if (bytes > area)
            return fail_inval(std::string(f->who) + ": staging A for the MFMA path needs " + std::to_string(bytes) +
                              " bytes; the static scratch holds " + std::to_string(area));
        f->aux_bytes = bytes;
        *out = static_cast<char*>(f->base) + f->counter_slots * sizeof(unsigned) + (area - bytes);
        return 0;
    }
    const int dev = current_device();
    Registries& reg = registries();
    std::lock_guard<std::mutex> lock(reg.mutex);
    AuxEntry& e = reg.aux[{dev, stream}];
    if (e.base == nullptr || e.bytes < bytes) {
        if (stream != nullptr) {
            hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing(stream, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone)
                return fail_inval("QuantizedMatMul: the staged-A buffer must be sized by an eager call "
                                  "on this stream before graph capture");
        }
        const std::size_t want = std::max<std::size_t>(std::max(bytes, e.bytes * 2), 1 << 20);
        if (e.base) {
            e.retired.push_back(e.base);
            e.base = nullptr;
        }
        VM_TRY_HIP(hipMalloc(&e.base, want), "staged A: hipMalloc");
        e.bytes = want;
    }
    *out = e.base;
    return 0;
}

void release_workspace(hipStream_t stream) {
    const int dev = current_device();
    Registries& reg = registries();
    std::lock_guard<std::mutex> lock(reg.mutex);
    auto it = reg.ws.find({dev, stream});
    if (it != reg.ws.end()) {
        if (it->second.base) (void)hipFree(it->second.base);
        for (void* p : it->second.retired) (void)hipFree(p);
        reg.ws.erase(it);
    }
    auto ax = reg.aux.find({dev, stream});
    if (ax != reg.aux.end()) {
        if (ax->second.base) (void)hipFree(ax->second.base);
        for (void* p : ax->second.retired) (void)hipFree(p);
        reg.aux.erase(ax);
    }
    auto st = reg.staging.find({dev, stream});
    if (st != reg.staging.end()) {
        if (st->second.base) (void)hipFree(st->second.base);
        for (void* p : st->second.retired) (void)hipFree(p);
        reg.staging.erase(st);
    }
}

int get_staging(hipStream_t stream, std::size_t bytes, void** out) {
    if (const FixedRegion* f = t_fixed)
        return fail_inval(std::string(f->who) + ": dtype staging would allocate; only fp32 operands are accepted");
    const int dev = current_device();
    Registries& reg = registries();
    std::lock_guard<std::mutex> lock(reg.mutex);
    StagingEntry& e = reg.staging[{dev, stream}];
    if (e.base == nullptr || e.bytes < bytes) {
        if (stream != nullptr) {
            hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing(stream, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone)
                return fail_inval("QuantizedMatMul: staging buffer must be sized by an eager call "
                                  "on this stream before graph capture");
        }
        const std::size_t want = std::max<std::size_t>(std::max(bytes, e.bytes * 2), 1 << 20);
        if (e.base) {
            e.retired.push_back(e.base);
            e.base = nullptr;
        }
        VM_TRY_HIP(hipMalloc(&e.base, want), "staging: hipMalloc");
        e.bytes = want;
    }
    *out = e.base;
    return 0;
}

int cu_count() {
    // never destroyed, like the buffer registries (usable during exit)
    static std::mutex& m = *new std::mutex;
    static std::map<int, int>& cache = *new std::map<int, int>;
    const int dev = current_device();
    std::lock_guard<std::mutex> lock(m);
    auto it = cache.find(dev);
    if (it != cache.end()) return it->second;
    int cus = 256;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    cache[dev] = cus;
    return cus;
}

}  // namespace vmhip

using namespace vmhip;

extern "C" {

int vm_hip_abi_version(void) { return VM_HIP_ABI_VERSION; }

const char* vm_hip_last_error(void) { return t_last_error.c_str(); }

int vm_hip_device_count(int* count) {
    if (!count) return fail_inval("vm_hip_device_count: null count");
    *count = 0;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    int usable = 0;
    for (int d = 0; d < n; ++d) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, d) != hipSuccess) continue;
        if (std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) ++usable;
    }
    *count = usable;
    return 0;
}

int vm_hip_set_device(int device) {
    VM_TRY_HIP(hipSetDevice(device), "hipSetDevice");
    return 0;
}

int vm_hip_get_device(int* device) {
    if (!device) return fail_inval("vm_hip_get_device: null device");
    VM_TRY_HIP(hipGetDevice(device), "hipGetDevice");
    return 0;
}

int vm_hip_device_synchronize(void) {
    VM_TRY_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
    return 0;
}

int vm_hip_malloc(void** ptr, size_t bytes) {
    if (!ptr) return fail_inval("vm_hip_malloc: null ptr");
    *ptr = nullptr;
    if (bytes == 0) return 0;
    hipError_t err = hipMalloc(ptr, bytes);
    if (err != hipSuccess) {
        *ptr = nullptr;
        set_error("velomind: hipMalloc failed for " + std::to_string(bytes) + " bytes (" +
                  hipGetErrorName(err) + "): " + hipGetErrorString(err));
        return static_cast<int>(err);
    }
    return 0;
}

int vm_hip_free(void* ptr) {
    if (!ptr) return 0;
    VM_TRY_HIP(hipFree(ptr), "hipFree");
    return 0;
}

static int copy_sync(void* dst, const void* src, size_t bytes, void* stream, hipMemcpyKind kind,
                     const char* what) {
    if (bytes == 0) return 0;
    if (!dst || !src) return fail_inval(std::string(what) + ": null pointer");
    auto s = static_cast<hipStream_t>(stream);
    hipError_t err = hipMemcpyAsync(dst, src, bytes, kind, s);
    if (err != hipSuccess) {
        set_error(std::string("velomind: ") + what + " failed for " + std::to_string(bytes) +
                  " bytes (" + hipGetErrorName(err) + "): " + hipGetErrorString(err));
        return static_cast<int>(err);
    }
    err = hipStreamSynchronize(s);
    if (err != hipSuccess) {
        set_error(std::string("velomind: hipStreamSynchronize (") + what + ") failed (" +
                  hipGetErrorName(err) + "): " + hipGetErrorString(err));
        return static_cast<int>(err);
    }
    return 0;
}

int vm_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    return copy_sync(dst, src, bytes, stream, hipMemcpyHostToDevice, "hipMemcpyAsync (H2D)");
}

int vm_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    return copy_sync(dst, src, bytes, stream, hipMemcpyDeviceToHost, "hipMemcpyAsync (D2H)");
}

int vm_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return 0;
    if (!dst || !src) return fail_inval("vm_hip_memcpy_d2d: null pointer");
    VM_TRY_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream)),
               "hipMemcpyAsync (D2D)");
    return 0;
}

int vm_hip_memcpy_2d_d2d(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width, size_t rows,
                         void* stream) {
    if (width == 0 || rows == 0) return 0;
    if (!dst || !src) return fail_inval("vm_hip_memcpy_2d_d2d: null pointer");
    if (width > dpitch || width > spitch) return fail_inval("vm_hip_memcpy_2d_d2d: width exceeds a pitch");
    VM_TRY_HIP(hipMemcpy2DAsync(dst, dpitch, src, spitch, width, rows, hipMemcpyDeviceToDevice,
                                static_cast<hipStream_t>(stream)),
               "hipMemcpy2DAsync (D2D)");
    return 0;
}

int vm_hip_stream_create(void** stream) {
    if (!stream) return fail_inval("vm_hip_stream_create: null stream");
    hipStream_t s = nullptr;
    // Default priority and non-blocking w.r.t. the null stream, like the
    // reference's CudaStream (src/cuda/cuda_context.h:19).
    VM_TRY_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags");
    *stream = s;
    return 0;
}

int vm_hip_stream_destroy(void* stream) {
    if (!stream) return 0;
    auto s = static_cast<hipStream_t>(stream);
    VM_TRY_HIP(hipStreamSynchronize(s), "hipStreamSynchronize");
    release_workspace(s);
    VM_TRY_HIP(hipStreamDestroy(s), "hipStreamDestroy");
    return 0;
}

int vm_hip_stream_synchronize(void* stream) {
    VM_TRY_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "hipStreamSynchronize");
    return 0;
}

int vm_hip_event_create(void** event) {
    if (!event) return fail_inval("vm_hip_event_create: null event");
    hipEvent_t e = nullptr;
    VM_TRY_HIP(hipEventCreate(&e), "hipEventCreate");
    *event = e;
    return 0;
}

int vm_hip_event_destroy(void* event) {
    if (!event) return 0;
    VM_TRY_HIP(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
    return 0;
}

int vm_hip_event_record(void* event, void* stream) {
    VM_TRY_HIP(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)),
               "hipEventRecord");
    return 0;
}

int vm_hip_event_synchronize(void* event) {
    VM_TRY_HIP(hipEventSynchronize(static_cast<hipEvent_t>(event)), "hipEventSynchronize");
    return 0;
}

int vm_hip_event_elapsed_ms(float* ms, void* start, void* end) {
    if (!ms) return fail_inval("vm_hip_event_elapsed_ms: null ms");
    VM_TRY_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end)),
               "hipEventElapsedTime");
    return 0;
}

int vm_hip_stream_begin_capture(void* stream) {
    if (!stream) return fail_inval("vm_hip_stream_begin_capture: capture needs a non-null stream");
    VM_TRY_HIP(hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal),
               "hipStreamBeginCapture");
    return 0;
}

int vm_hip_stream_end_capture(void* stream, void** graph_exec) {
    if (!stream || !graph_exec) return fail_inval("vm_hip_stream_end_capture: null argument");
    *graph_exec = nullptr;
    hipGraph_t graph = nullptr;
    VM_TRY_HIP(hipStreamEndCapture(static_cast<hipStream_t>(stream), &graph), "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    hipError_t err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (err != hipSuccess) return fail_hip(err, "hipGraphInstantiate");
    *graph_exec = exec;
    return 0;
}

int vm_hip_graph_launch(void* graph_exec, void* stream) {
    if (!graph_exec) return fail_inval("vm_hip_graph_launch: null graph");
    VM_TRY_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), static_cast<hipStream_t>(stream)),
               "hipGraphLaunch");
    return 0;
}

int vm_hip_graph_destroy(void* graph_exec) {
    if (!graph_exec) return 0;
    VM_TRY_HIP(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)), "hipGraphExecDestroy");
    return 0;
}

}  // extern "C"
