// Weight packing on the device, bit-exact with the reference's host
// packers (src/quant.cpp:74-104 INT8, :125-175 INT4), plus the inverse
// maps and half->fp32 widening.
//
// Exactness: the scale is a correctly rounded fp32 division (max / 127 or
// max / 7; built with -fhip-fp32-correctly-rounded-divide-sqrt and without
// fast-math), the reciprocal is a correctly rounded 1 / scale that is then
// multiplied, roundf() rounds half away from zero, and the clamp and the
// int8 cast follow.  Only finite inputs are in the contract (the
// reference's float->int8 cast of NaN/Inf is undefined).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "vm_internal.h"

namespace vmhip {
namespace {

constexpr int kColsPerWg = 64;
constexpr int kRowGroups = 4;

// One workgroup owns 64 columns; 4 row groups find the column maxima
// together, then every thread quantizes its own rows.
__global__ __launch_bounds__(kColsPerWg * kRowGroups) void pack_int8_kernel(
    const float* __restrict__ w, int8_t* __restrict__ q, float* __restrict__ scale, int64_t rows,
    int64_t cols) {
    __shared__ float smax[kRowGroups][kColsPerWg];
    const int tx = threadIdx.x % kColsPerWg;
    const int ty = threadIdx.x / kColsPerWg;
    const int64_t c = static_cast<int64_t>(blockIdx.x) * kColsPerWg + tx;
    float m = 0.0f;
    if (c < cols) {
        for (int64_t r = ty; r < rows; r += kRowGroups) {
            const float v = fabsf(w[r * cols + c]);
            if (v > m) m = v;
        }
    }
    smax[ty][tx] = m;
    __syncthreads();
    float amax = smax[0][tx];
    for (int g = 1; g < kRowGroups; ++g) amax = smax[g][tx] > amax ? smax[g][tx] : amax;
    if (c >= cols) return;
    const float s = amax > 0.0f ? amax / 127.0f : 1.0f;
    const float inv = 1.0f / s;
    if (ty == 0) scale[c] = s;
    for (int64_t r = ty; r < rows; r += kRowGroups) {
        float v = roundf(w[r * cols + c] * inv);
        v = v < -127.0f ? -127.0f : (127.0f < v ? 127.0f : v);
        q[r * cols + c] = static_cast<int8_t>(v);
    }
}

// Two-pass INT8 packing for wide matrices (cols % 4 == 0, aligned): one
// workgroup of the single-pass kernel scans all rows of 64 columns, a
// serial chain of loads that leaves the GPU mostly idle (2048 x 5632:
// 350 us).  Here thread (x, chunk) owns four adjacent columns:
//   pass 1: the maximum |w| of its columns over one chunk of rows
//           (16-byte loads, kPackUnroll in flight), one partial per chunk;
//   pass 2: the column maxima from the partials (max is exact in any
//           order), then quant.cpp's scale / reciprocal / round / clamp for
//           its columns over one chunk of rows, four codes per 4-byte store.
// The comparison `v > m` skips NaN, as the single-pass kernel does.
constexpr int kPackThreads = 256;
constexpr int kPackUnroll = 8;

__global__ __launch_bounds__(kPackThreads) void pack_int8_colmax_kernel(const float* __restrict__ w,
                                                                        float* __restrict__ part, int64_t rows,
                                                                        int64_t cols, int64_t rows_per_chunk) {
    const int64_t c4 = (static_cast<int64_t>(blockIdx.x) * kPackThreads + threadIdx.x) * 4;
    if (c4 >= cols) return;
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * rows_per_chunk;
    const int64_t r1 = min(rows, r0 + rows_per_chunk);
    float m[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t r = r0; r < r1; r += kPackUnroll) {
        float4 v[kPackUnroll];
#pragma unroll
        for (int u = 0; u < kPackUnroll; ++u)
            v[u] = r + u < r1 ? *reinterpret_cast<const float4*>(w + (r + u) * cols + c4)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int u = 0; u < kPackUnroll; ++u) {
            const float a[4] = {fabsf(v[u].x), fabsf(v[u].y), fabsf(v[u].z), fabsf(v[u].w)};
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (a[e] > m[e]) m[e] = a[e];
        }
    }
    *reinterpret_cast<float4*>(part + static_cast<int64_t>(blockIdx.y) * cols + c4) = make_float4(m[0], m[1], m[2], m[3]);
}

__device__ __forceinline__ uint32_t int8_code(float x, float inv) {
    float v = roundf(x * inv);
    v = v < -127.0f ? -127.0f : (127.0f < v ? 127.0f : v);
    return static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(v)));
}

__global__ __launch_bounds__(kPackThreads) void pack_int8_quantize_kernel(
    const float* __restrict__ w, const float* __restrict__ part, int chunks, int8_t* __restrict__ q,
    float* __restrict__ scale, int64_t rows, int64_t cols, int64_t rows_per_chunk) {
    const int64_t c4 = (static_cast<int64_t>(blockIdx.x) * kPackThreads + threadIdx.x) * 4;
    if (c4 >= cols) return;
    float amax[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i0 = 0; i0 < chunks; i0 += kPackUnroll) {
        float4 pv[kPackUnroll];
#pragma unroll
        for (int u = 0; u < kPackUnroll; ++u)
            pv[u] = i0 + u < chunks ? *reinterpret_cast<const float4*>(part + static_cast<int64_t>(i0 + u) * cols + c4)
                                    : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int u = 0; u < kPackUnroll; ++u) {
            const float a[4] = {pv[u].x, pv[u].y, pv[u].z, pv[u].w};
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (a[e] > amax[e]) amax[e] = a[e];
        }
    }
    float inv[4];
    float sc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        sc[e] = amax[e] > 0.0f ? amax[e] / 127.0f : 1.0f;   // quant.cpp:94-96
        inv[e] = 1.0f / sc[e];
    }
    if (blockIdx.y == 0) *reinterpret_cast<float4*>(scale + c4) = make_float4(sc[0], sc[1], sc[2], sc[3]);
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * rows_per_chunk;
    const int64_t r1 = min(rows, r0 + rows_per_chunk);
    for (int64_t r = r0; r < r1; r += kPackUnroll) {
        float4 v[kPackUnroll];
#pragma unroll
        for (int u = 0; u < kPackUnroll; ++u)
            v[u] = r + u < r1 ? *reinterpret_cast<const float4*>(w + (r + u) * cols + c4)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int u = 0; u < kPackUnroll; ++u) {
            if (r + u >= r1) break;
            const uint32_t word = int8_code(v[u].x, inv[0]) | (int8_code(v[u].y, inv[1]) << 8) |
                                  (int8_code(v[u].z, inv[2]) << 16) | (int8_code(v[u].w, inv[3]) << 24);
            *reinterpret_cast<uint32_t*>(q + (r + u) * cols + c4) = word;
        }
    }
}

__device__ __forceinline__ unsigned int4_code(float x, float inv) {
    float v = roundf(x * inv);
    v = v < -8.0f ? -8.0f : (7.0f < v ? 7.0f : v);
    return static_cast<unsigned>(static_cast<int8_t>(v)) & 0xFu;
}

// One thread per (scale block, column); blocks are even, so every packed
// byte belongs to exactly one thread.
__global__ __launch_bounds__(256) void pack_int4_kernel(const float* __restrict__ w,
                                                        uint8_t* __restrict__ packed,
                                                        float* __restrict__ scale, int64_t rows,
                                                        int64_t cols, int64_t block) {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t b = blockIdx.y;
    if (c >= cols) return;
    const int64_t r0 = b * block;
    const int64_t r1 = r0 + block < rows ? r0 + block : rows;
    float amax = 0.0f;
    for (int64_t r = r0; r < r1; ++r) {
        const float v = fabsf(w[r * cols + c]);
        if (v > amax) amax = v;
    }
    const float s = amax > 0.0f ? amax / 7.0f : 1.0f;
    const float inv = 1.0f / s;
    scale[b * cols + c] = s;
    for (int64_t r = r0; r < r1; r += 2) {
        const unsigned lo = int4_code(w[r * cols + c], inv);
        const unsigned hi = (r + 1 < r1) ? int4_code(w[(r + 1) * cols + c], inv) : 0u;
        packed[(r / 2) * cols + c] = static_cast<uint8_t>(lo | (hi << 4));
    }
}

__global__ void dequant_int8_kernel(const int8_t* __restrict__ q, const float* __restrict__ scale,
                                    float* __restrict__ w, int64_t rows, int64_t cols) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= rows * cols) return;
    w[idx] = static_cast<float>(q[idx]) * scale[idx % cols];
}

__device__ __forceinline__ int nib(unsigned v) {
    v &= 0xFu;
    return (v & 8u) ? static_cast<int>(v) - 16 : static_cast<int>(v);
}

// Row r of block b reads the pair that the reference's block-local pair
// loop assigns to it (src/quant.cpp:197-205); for even blocks that is byte
// row r/2, nibble r%2.
__global__ void dequant_int4_kernel(const uint8_t* __restrict__ packed,
                                    const float* __restrict__ scale, float* __restrict__ w,
                                    int64_t rows, int64_t cols, int64_t block) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= rows * cols) return;
    const int64_t r = idx / cols;
    const int64_t c = idx - r * cols;
    const int64_t b = r / block;
    const int64_t r0 = b * block;
    const int64_t pair_row = r0 + ((r - r0) & ~int64_t(1));
    const unsigned byte = packed[(pair_row / 2) * cols + c];
    const int code = ((r - r0) & 1) ? nib(byte >> 4) : nib(byte);
    w[idx] = static_cast<float>(code) * scale[b * cols + c];
}

// dtype.h:21-51 (exact widening, NaN made quiet) and :91-95.
__global__ void half_to_f32_kernel(const uint16_t* __restrict__ src, float* __restrict__ dst,
                                   int64_t count, int is_bf16) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const uint32_t h = src[i];
    uint32_t f;
    if (is_bf16) {
        f = h << 16;
    } else {
        const uint32_t sign = (h & 0x8000u) << 16;
        const uint32_t e = (h >> 10) & 0x1Fu;
        uint32_t m = h & 0x3FFu;
        if (e == 0) {
            if (m == 0) {
                f = sign;
            } else {
                int ex = -14;
                while (!(m & 0x400u)) { m <<= 1; --ex; }
                f = sign | (static_cast<uint32_t>(ex + 127) << 23) | ((m & 0x3FFu) << 13);
            }
        } else if (e == 0x1F) {
            f = sign | 0x7F800000u | (m << 13) | (m ? 0x400000u : 0u);
        } else {
            f = sign | ((e + 112u) << 23) | (m << 13);
        }
    }
    dst[i] = __uint_as_float(f);
}

unsigned grid_1d(int64_t count, int threads) {
    return static_cast<unsigned>((count + threads - 1) / threads);
}

}  // namespace
}  // namespace vmhip

using namespace vmhip;

extern "C" {

int vm_hip_pack_int8(const float* w, int8_t* q, float* scale, int64_t rows, int64_t cols,
                     void* stream) {
    if (rows < 0 || cols < 0) return fail_inval("vm_hip_pack_int8: negative shape");
    if (rows == 0 || cols == 0) return 0;  // quant.cpp:81-83
    if (!w || !q || !scale) return fail_inval("vm_hip_pack_int8: null pointer");
    VM_TRY(injected_failure("QuantizePack", "launch"));
    auto s = static_cast<hipStream_t>(stream);
    // Two passes for matrices wide and tall enough to fill the GPU, when
    // 16-byte loads apply and the stream is not being captured (the row
    // partials use the stream's workspace, sized here).
    const bool vec = cols % 4 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(q) % 4 == 0 && reinterpret_cast<uintptr_t>(scale) % 16 == 0;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (s) (void)hipStreamIsCapturing(s, &cap);
    if (vec && rows >= 64 && cols >= 256 && cap == hipStreamCaptureStatusNone) {
        const int64_t col_groups = (cols / 4 + kPackThreads - 1) / kPackThreads;
        // about 512 workgroups per pass, at least 32 rows and at most 64 chunks
        int64_t chunks = std::max<int64_t>(1, std::min<int64_t>((512 + col_groups - 1) / col_groups, rows / 32));
        chunks = std::min<int64_t>(chunks, 64);   // pass 2 reads every chunk's partial
        const int64_t rpc = (rows + chunks - 1) / chunks;
        chunks = (rows + rpc - 1) / rpc;
        Workspace ws{};
        VM_TRY(get_workspace(s, static_cast<std::size_t>(chunks * cols), 0, &ws));
        const dim3 grid(static_cast<unsigned>(col_groups), static_cast<unsigned>(chunks));
        hipLaunchKernelGGL(pack_int8_colmax_kernel, grid, dim3(kPackThreads), 0, s, w, ws.partials, rows, cols, rpc);
        hipLaunchKernelGGL(pack_int8_quantize_kernel, grid, dim3(kPackThreads), 0, s, w, ws.partials,
                           static_cast<int>(chunks), q, scale, rows, cols, rpc);
        return check_launch("QuantizePack", s);
    }
    hipLaunchKernelGGL(pack_int8_kernel, dim3(grid_1d(cols, kColsPerWg)), dim3(kColsPerWg * kRowGroups),
                       0, s, w, q, scale, rows, cols);
    return check_launch("QuantizePack", s);
}

int vm_hip_pack_int4(const float* w, uint8_t* packed, float* scale, int64_t rows, int64_t cols,
                     int64_t block, void* stream) {
    if (rows < 0 || cols < 0) return fail_inval("vm_hip_pack_int4: negative shape");
    if (block <= 0) return fail_inval("vm_hip_pack_int4: block_size must be positive");
    if (block % 2 != 0) return fail_inval("vm_hip_pack_int4: block_size must be even");
    if (rows == 0 || cols == 0) return 0;
    if (!w || !packed || !scale) return fail_inval("vm_hip_pack_int4: null pointer");
    const int64_t nblk = (rows + block - 1) / block;
    if (nblk > 65535) return fail_inval("vm_hip_pack_int4: too many scale blocks");
    auto s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(pack_int4_kernel, dim3(grid_1d(cols, 256), static_cast<unsigned>(nblk)), dim3(256),
                       0, s, w, packed, scale, rows, cols, block);
    return check_launch("QuantizePack", s);
}

int vm_hip_dequant_int8(const int8_t* q, const float* scale, float* w, int64_t rows, int64_t cols,
                        void* stream) {
    if (rows < 0 || cols < 0) return fail_inval("vm_hip_dequant_int8: negative shape");
    if (rows == 0 || cols == 0) return 0;
    if (!q || !scale || !w) return fail_inval("vm_hip_dequant_int8: null pointer");
    auto s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(dequant_int8_kernel, dim3(grid_1d(rows * cols, 256)), dim3(256), 0, s, q, scale,
                       w, rows, cols);
    return check_launch("Dequantize", s);
}

int vm_hip_dequant_int4(const uint8_t* packed, const float* scale, float* w, int64_t rows,
                        int64_t cols, int64_t block, void* stream) {
    if (rows < 0 || cols < 0) return fail_inval("vm_hip_dequant_int4: negative shape");
    if (block <= 0) return fail_inval("vm_hip_dequant_int4: block_size must be positive");
    if (rows == 0 || cols == 0) return 0;
    if (!packed || !scale || !w) return fail_inval("vm_hip_dequant_int4: null pointer");
    auto s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(dequant_int4_kernel, dim3(grid_1d(rows * cols, 256)), dim3(256), 0, s, packed,
                       scale, w, rows, cols, block);
    return check_launch("Dequantize", s);
}

int vm_hip_half_to_f32(const uint16_t* src, int src_dtype, float* dst, int64_t count, void* stream) {
    if (src_dtype != VM_HIP_DTYPE_F16 && src_dtype != VM_HIP_DTYPE_BF16)
        return fail_inval("vm_hip_half_to_f32: source dtype must be Float16 or BFloat16");
    if (count < 0) return fail_inval("vm_hip_half_to_f32: negative count");
    if (count == 0) return 0;
    if (!src || !dst) return fail_inval("vm_hip_half_to_f32: null pointer");
    auto s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(half_to_f32_kernel, dim3(grid_1d(count, 256)), dim3(256), 0, s, src, dst, count,
                       src_dtype == VM_HIP_DTYPE_BF16 ? 1 : 0);
    return check_launch("ConvertDtype", s);
}

}  // extern "C"
