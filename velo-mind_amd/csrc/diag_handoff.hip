// Platform diagnostic (no reference counterpart): the cost of handing data
// from every workgroup to every other inside one launch, the primitive a
// one-launch decode step is built from.  One workgroup per compute unit
// (cooperative launch, 96 KB of LDS each); every participant stores 8
// tagged 64-bit words {round, value} per round and polls all participants'
// words with agent-scope loads until each carries the round's tag
// (double-buffered by round parity; every poll is bounded).  Variants:
//   VM_HIP_DIAG_ALONE        the participants alone;
//   VM_HIP_DIAG_STREAM_CUS   the other compute units stream a 1 GiB buffer
//                            from HBM meanwhile (16-byte loads, 8 per lane
//                            in flight);
//   VM_HIP_DIAG_STREAM_FIRST each participant first streams `kb` KiB of
//                            its own and then polls (a phase that loads its
//                            weights before waiting for its inputs);
//   VM_HIP_DIAG_STREAM_WAVES waves 4 .. 3 + kb of each participant stream
//                            continuously while waves 0-3 run the rounds
//                            (one compute unit serving both).
// Results: microseconds per round (slowest participant, 100 MHz wall
// clock) and the streaming rate of the variant's loads.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <vector>

#include "vm_device.h"
#include "vm_internal.h"

namespace vmhip {
namespace {

typedef unsigned long long u64;
constexpr int kDiagThreads = 512;
constexpr unsigned kDiagSpin = 1u << 20;
constexpr int kDiagLds = 96 * 1024;   // one workgroup per compute unit
constexpr int kDiagFailed = static_cast<int>(hipErrorUnknown);

struct DiagArgs {
    u64* words;          // [2][participants * 8]
    const uint4* buf;    // streaming buffer
    u64 buf16;           // its 16-byte pieces
    unsigned* status;    // bit 0: a poll timed out
    unsigned* stop;      // set when participant 0 is done
    u64* ticks;          // [participants]
    u64* streamed;       // bytes streamed
    float* sink;
    int rounds, mode, participants, kb;
};

// Streams this wave's share until *stop (bounded); returns bytes read.
template <int U>
__device__ u64 stream_until_stop(const DiagArgs& a, u64 base, u64 span, float& acc) {
    const int lane = threadIdx.x & 63;
    u64 i = lane, n = 0;
    for (unsigned it = 0; it < (1u << 22); ++it) {
        uint4 v[U];
#pragma unroll
        for (int k = 0; k < U; ++k) v[k] = a.buf[base + (i + k * 64) % span];
#pragma unroll
        for (int k = 0; k < U; ++k) acc += __uint_as_float(v[k].x ^ v[k].w);
        i += U * 64;
        n += U * 64 * 16;
        if ((it & 7) == 0 && __hip_atomic_load(a.stop, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
    }
    return n;
}

__global__ __launch_bounds__(kDiagThreads) void diag_handoff_kernel(DiagArgs a) {
    extern __shared__ int lds_pad[];   // occupancy only
    __shared__ int ctr;
    const int g = blockIdx.x, t = threadIdx.x, wave = t >> 6;
    const int P = a.participants;
    float acc = 0.0f;
    if (t == 0) ctr = 0;
    __syncthreads();
    if (g >= P) {   // a streaming compute unit (STREAM_CUS) or idle
        if (a.mode == VM_HIP_DIAG_STREAM_CUS) {
            const u64 per = a.buf16 / static_cast<u64>(static_cast<int>(gridDim.x) - P);
            const u64 span = per / 8;
            const u64 n = stream_until_stop<8>(a, per * static_cast<u64>(g - P) + span * wave, span, acc);
            if ((t & 63) == 0) atomicAdd(a.streamed, n);
        }
        if (acc == 12345.0f) a.sink[g * kDiagThreads + t] = acc + lds_pad[0];
        return;
    }
    if (wave >= 4) {   // STREAM_WAVES: waves 4 .. 3 + kb stream
        if (a.mode == VM_HIP_DIAG_STREAM_WAVES && wave - 4 < a.kb) {
            const u64 per = a.buf16 / static_cast<u64>(P * a.kb);
            const u64 n = stream_until_stop<8>(a, per * static_cast<u64>(g * a.kb + wave - 4), per, acc);
            if ((t & 63) == 0) atomicAdd(a.streamed, n);
        }
        if (acc == 12345.0f) a.sink[g * kDiagThreads + t] = acc;
        return;
    }
    // waves 0-3: the rounds
    const int nw = P * 8;   // 16-byte piece j = t + 256 k holds words 2 j, 2 j + 1
    const uint32_t wbytes = static_cast<uint32_t>(nw) * 8u;
    u64 t0 = 0;
    bool dead = false;
    int bar = 0;
    for (int r = 0; r < a.rounds; ++r) {
        if (r == 1 && t == 0) t0 = wall_clock64();
        u64* w = a.words + static_cast<int64_t>(r & 1) * nw;
        const unsigned tag = static_cast<unsigned>(r) + 1u;
        if (t < 8)
            __hip_atomic_store(w + g * 8 + t, (static_cast<u64>(tag) << 32) | __float_as_uint(static_cast<float>(g)),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (a.mode == VM_HIP_DIAG_STREAM_FIRST && a.kb > 0) {
            const u64 n16 = static_cast<u64>(a.kb) * 64;
            const u64 off = (static_cast<u64>(g) * a.rounds + r) * n16 % (a.buf16 - n16);
            for (u64 i = t; i < n16; i += 256) {
                const uint4 q = a.buf[off + i];
                acc += __uint_as_float(q.x ^ q.z);
            }
            if (t == 0 && g == 0) atomicAdd(a.streamed, n16 * 16 * P);
        }
        const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(w, wbytes);
        u32x4 v[4];
        auto poll = [&]() {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                v[k] = coherent_load16(rs, 2 * (t + k * 256) < nw ? static_cast<uint32_t>(t + k * 256) * 16u : wbytes);
        };
        poll();
        unsigned spins = 0;
        for (;;) {
            bool ok = true;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const bool live = 2 * (t + k * 256) < nw;
                ok = ok && (!live || (v[k][1] == tag && v[k][3] == tag));
            }
            if (ok || dead) break;
            if (++spins > kDiagSpin) {
                dead = true;
                __hip_atomic_fetch_or(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            poll();
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) acc += __uint_as_float(v[k][0]);
        // barrier of waves 0-3 in LDS (waves 4-7 do not take part)
        ++bar;
        if ((t & 63) == 0) __hip_atomic_fetch_add(&ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        unsigned s2 = 0;
        while (__hip_atomic_load(&ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < bar * 4) {
            if (++s2 > (1u << 26)) {
                __hip_atomic_fetch_or(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
    }
    if (t == 0) {
        a.ticks[g] = wall_clock64() - t0;
        if (g == 0) __hip_atomic_store(a.stop, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (acc == 12345.0f) a.sink[g * kDiagThreads + t] = acc;
}

}  // namespace
}  // namespace vmhip

using namespace vmhip;

extern "C" int vm_hip_diag_handoff(int mode, int participants, int kb, int rounds, double* us_per_round,
                                   double* stream_gb_s, void* stream) {
    clear_error();
    if (!us_per_round) return fail_inval("vm_hip_diag_handoff: null result");
    if (mode < VM_HIP_DIAG_ALONE || mode > VM_HIP_DIAG_STREAM_WAVES || rounds < 2 || rounds > 100000 || kb < 0)
        return fail_inval("vm_hip_diag_handoff: bad mode, rounds or kb");
    if (mode == VM_HIP_DIAG_STREAM_WAVES && (kb < 1 || kb > 4))
        return fail_inval("vm_hip_diag_handoff: STREAM_WAVES takes 1 to 4 streaming waves");
    if (mode == VM_HIP_DIAG_STREAM_FIRST && kb > 1024) return fail_inval("vm_hip_diag_handoff: kb above 1024");
    int dev = 0, cus = 0, coop = 0;
    VM_TRY_HIP(hipGetDevice(&dev), "diag: hipGetDevice");
    VM_TRY_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "diag: CU count");
    VM_TRY_HIP(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev), "diag: attribute");
    if (!coop) return VM_HIP_EUNSUPPORTED;
    if (participants < 2 || participants > cus || participants > 256 || (mode == VM_HIP_DIAG_STREAM_CUS && participants == cus))
        return fail_inval("vm_hip_diag_handoff: participants must be in [2, min(256, CUs)) (below the CU count "
                          "when other CUs stream)");
    const int grid = mode == VM_HIP_DIAG_STREAM_CUS ? cus : participants;
    auto s = static_cast<hipStream_t>(stream);
    const std::size_t buf_bytes = std::size_t(1) << 30;
    char* mem = nullptr;
    const std::size_t words_bytes = 2 * std::size_t(participants) * 8 * 8;
    const std::size_t small = 4096 + words_bytes + std::size_t(cus) * 8 + std::size_t(cus) * kDiagThreads * 4;
    VM_TRY_HIP(hipMalloc(&mem, buf_bytes + small), "diag: hipMalloc");
    DiagArgs a{};
    a.buf = reinterpret_cast<const uint4*>(mem);
    a.buf16 = buf_bytes / 16;
    char* p = mem + buf_bytes;
    a.status = reinterpret_cast<unsigned*>(p);
    a.stop = reinterpret_cast<unsigned*>(p + 256);
    a.streamed = reinterpret_cast<u64*>(p + 512);
    a.words = reinterpret_cast<u64*>(p + 4096);
    a.ticks = reinterpret_cast<u64*>(p + 4096 + words_bytes);
    a.sink = reinterpret_cast<float*>(p + 4096 + words_bytes + std::size_t(cus) * 8);
    a.rounds = rounds;
    a.mode = mode;
    a.participants = participants;
    a.kb = kb;
    int rc = 0;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    do {
        if (hipMemsetAsync(mem, 1, buf_bytes, s) != hipSuccess || hipMemsetAsync(p, 0, small, s) != hipSuccess ||
            hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
            rc = kDiagFailed;
            set_error("diag: set-up failed");
            break;
        }
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(diag_handoff_kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kDiagLds);
        void* args[] = {&a};
        (void)hipEventRecord(e0, s);
        if (hipLaunchCooperativeKernel(reinterpret_cast<const void*>(diag_handoff_kernel), dim3(grid),
                                       dim3(kDiagThreads), args, kDiagLds, s) != hipSuccess) {
            rc = VM_HIP_EUNSUPPORTED;
            set_error("diag: hipLaunchCooperativeKernel failed (one workgroup per CU must fit)");
            (void)hipGetLastError();
            break;
        }
        (void)hipEventRecord(e1, s);
        if (hipStreamSynchronize(s) != hipSuccess) {
            rc = kDiagFailed;
            set_error("diag: kernel failed");
            break;
        }
        unsigned status = 0;
        u64 streamed = 0;
        std::vector<u64> ticks(participants);
        (void)hipMemcpy(&status, a.status, 4, hipMemcpyDeviceToHost);
        (void)hipMemcpy(&streamed, a.streamed, 8, hipMemcpyDeviceToHost);
        (void)hipMemcpy(ticks.data(), a.ticks, participants * 8, hipMemcpyDeviceToHost);
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, e0, e1);
        if (status) {
            rc = kDiagFailed;
            set_error("diag: a poll timed out");
            break;
        }
        const u64 slowest = *std::max_element(ticks.begin(), ticks.end());
        *us_per_round = static_cast<double>(slowest) * 0.01 / (rounds - 1);
        if (stream_gb_s) *stream_gb_s = ms > 0.0f ? static_cast<double>(streamed) / (ms * 1e-3) / 1e9 : 0.0;
    } while (false);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipFree(mem);
    return rc;
}
