// vm_hip_qmm_f32_noalloc: vm_hip_qmm_f32 for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  It has no counterpart in the
// reference.
//
// The only device memory vm_hip_qmm_f32 allocates is its split-K scratch:
// the GEMV's pair-word tree (one 64-bit word per output and tree node) and
// the MFMA GEMM's partial tiles and tile tickets, normally a per-stream
// buffer grown on demand.  Here that scratch is `scratch`, a file-scope
// device array of kScratchBytes: the first kCounterBytes hold the counters
// and pair words (zero between calls: the kernels that use them reset them
// before they exit), the rest the fp32 partials.  The kernels are the same
// as vm_hip_qmm_f32's, so both entry points give identical results.
//
// Each GPU the library runs on holds its own copy of the array, at its own
// address, until the process ends.  Every call on one GPU shares it: calls
// that overlap on one GPU (different streams, or host threads) race and
// must be serialized by the caller.  Shapes whose scratch would exceed the
// array are rejected with VM_HIP_EINVAL and leave the output unwritten; a
// refused MFMA GEMM call (more than 4 rows) may already have launched its
// A-staging kernel into the array's staging area, whose contents no call
// relies on (every call stages its own A before reading it).
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <mutex>

#include "qmm_kernels.h"
#include "vm_internal.h"

namespace vmhip {
namespace {

constexpr std::size_t kScratchBytes = VM_HIP_QMM_NOALLOC_SCRATCH_BYTES;   // 16 MiB per GPU
constexpr std::size_t kCounterBytes = VM_HIP_QMM_NOALLOC_COUNTER_BYTES;   // 2 MiB of it: counters, pair words
static_assert(kCounterBytes % 256 == 0 && kCounterBytes < kScratchBytes, "scratch layout");
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

// Device address of `scratch` per device.  In host code the array's name
// only stands in for the symbol; kernels and copies get this address.
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

__global__ void zero_words_kernel(unsigned* __restrict__ p, int count) {
    const int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
    if (i < count) p[i] = 0u;
}

// Resolves this device's copy of `scratch` on the first call made with the
// device current, and clears its counter region on `stream` with a kernel
// (not a memset, so that a first call under graph capture records a kernel
// node).  Later calls find the counters at zero: every kernel that takes a
// ticket or pair word resets it before exiting.
int scratch_for_current_device(hipStream_t stream, void** out) {
    int dev = 0;
    VM_TRY_HIP(hipGetDevice(&dev), "vm_hip_qmm_f32_noalloc: hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail_inval("vm_hip_qmm_f32_noalloc: device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        VM_TRY_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "vm_hip_qmm_f32_noalloc: hipGetSymbolAddress");
        if (!ptr) return fail_inval("vm_hip_qmm_f32_noalloc: hipGetSymbolAddress returned null");
        const int words = static_cast<int>(kCounterBytes / sizeof(unsigned));
        hipLaunchKernelGGL(zero_words_kernel, dim3((words + 255) / 256), dim3(256), 0, stream,
                           static_cast<unsigned*>(ptr), words);
        VM_TRY(check_launch("QuantizedMatMul", stream));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

}  // namespace
}  // namespace vmhip

using namespace vmhip;

extern "C" {

int vm_hip_qmm_f32_noalloc(const float* a, const int8_t* wq, const float* scale, float* c, int64_t rows_m,
                           int64_t k, int64_t n, int quant_type, int block_size, void* stream) {
    clear_error();
    VM_TRY(validate_qmm(a, wq, scale, c, rows_m, k, n, quant_type, block_size));
    VM_TRY(injected_failure("QuantizedMatMul", "launch"));
    auto s = static_cast<hipStream_t>(stream);
    void* base = nullptr;
    VM_TRY(scratch_for_current_device(s, &base));
    FixedWorkspaceScope fixed(base, kCounterBytes / sizeof(unsigned), (kScratchBytes - kCounterBytes) / sizeof(float),
                              "vm_hip_qmm_f32_noalloc");
    return qmm_f32_impl(a, wq, scale, c, rows_m, k, n, quant_type, block_size, s);
}

}  // extern "C"
