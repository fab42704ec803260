// Decode-shaped (rows_m <= 4) quantized matmul for gfx950: an HBM-bound
// GEMV that streams the reference's [K, N] code layout (N contiguous) with
// 128-bit loads, dequantizes in registers and accumulates in fp32.
//
// Work decomposition
//   lane  : VEC consecutive columns (VEC bytes of one code row per load)
//   wave  : 64 lanes -> 64*VEC columns ("column tile")
//   unit  : 32 logical K rows (INT4: 16 packed byte rows)
//   WG    : 4 waves on one column tile; wave w takes units w, w+4, ...
//           of the WG's K range; the 4 waves reduce through LDS
//   split : grid.y splits K across workgroups; partial sums go to a
//           per-stream workspace and the last workgroup of a tile (atomic
//           ticket) adds them in split order, so results are deterministic
//
// Dequantization: INT8 codes are sign-extended bytes (v_cvt_f32_i32 with
// an SDWA byte select).  An INT4 byte holds the even row in its low nibble;
// moving each nibble to the top of a byte ((w << 4) & 0xF0.. and
// w & 0xF0..) makes the signed byte equal 16*code, so the same SDWA
// convert applies and the factor 1/16 is folded (exactly) into the scale.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "qmm_kernels.h"
#include "vm_internal.h"

namespace vmhip {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kUnitK = 32;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int VEC>
__device__ __forceinline__ void load_codes(uint32_t (&dst)[VEC / 4], const uint8_t* p) {
    if constexpr (VEC == 16) {
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
        dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
    } else if constexpr (VEC == 8) {
        const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
        dst[0] = v.x; dst[1] = v.y;
    } else {
        dst[0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
    }
}

template <int VEC>
__device__ __forceinline__ void load_scales(float (&dst)[VEC], const float* p) {
#pragma unroll
    for (int i = 0; i < VEC; i += 4) {
        const float4 v = *reinterpret_cast<const float4*>(p + i);
        dst[i] = v.x; dst[i + 1] = v.y; dst[i + 2] = v.z; dst[i + 3] = v.w;
    }
}

// KIND: 0 = INT8 per-column scale, 1 = INT8 blockwise, 2 = INT4 blockwise.
template <int KIND, int VEC, int MR>
__global__ __launch_bounds__(kThreads) void qmm_gemv_kernel(
    const float* __restrict__ a, const uint8_t* __restrict__ wq, const float* __restrict__ scale,
    float* __restrict__ c, int m, int k, int n, int units_per_block, int units_per_split,
    float* __restrict__ partials, unsigned* __restrict__ counters) {
    constexpr bool kInt4 = KIND == 2;
    constexpr int kRows = kInt4 ? kUnitK / 2 : kUnitK;  // byte rows per unit
    constexpr int kWords = VEC / 4;

    __shared__ float red[kWaves][MR][64 * VEC];
    __shared__ unsigned ticket;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tile = blockIdx.x;
    const int split = blockIdx.y;
    const int splits = gridDim.y;
    const int col0 = tile * 64 * VEC + lane * VEC;
    const bool col_ok = col0 < n;

    const int total_units = (k + kUnitK - 1) / kUnitK;
    const int byte_rows = kInt4 ? (k + 1) / 2 : k;
    const int u_begin = split * units_per_split;
    const int u_end = min(total_units, u_begin + units_per_split);

    float total[MR][VEC];
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int j = 0; j < VEC; ++j) total[r][j] = 0.0f;

    for (int u = u_begin + wave; u < u_end; u += kWaves) {
        const int row0 = u * kRows;
        uint32_t w[kRows][kWords];
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            if (col_ok && row0 + r < byte_rows) {
                load_codes<VEC>(w[r], wq + static_cast<int64_t>(row0 + r) * n + col0);
            } else {
#pragma unroll
                for (int d = 0; d < kWords; ++d) w[r][d] = 0u;
            }
        }
        float sc[VEC];
        if constexpr (KIND != 0) {
            const int blk = (u * kUnitK) / units_per_block;  // units_per_block holds block_size
            if (col_ok) load_scales<VEC>(sc, scale + static_cast<int64_t>(blk) * n + col0);
        }

        float acc[MR][VEC];
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
            for (int j = 0; j < VEC; ++j) acc[r][j] = 0.0f;

        const int kbase = u * kUnitK;
        if constexpr (kInt4) {
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                const int ke = kbase + 2 * r;
                float xe[MR], xo[MR];
#pragma unroll
                for (int i = 0; i < MR; ++i) {
                    xe[i] = (i < m && ke < k) ? a[static_cast<int64_t>(i) * k + ke] : 0.0f;
                    xo[i] = (i < m && ke + 1 < k) ? a[static_cast<int64_t>(i) * k + ke + 1] : 0.0f;
                }
#pragma unroll
                for (int d = 0; d < kWords; ++d) {
                    const uint32_t lo8 = (w[r][d] << 4) & 0xF0F0F0F0u;
                    const uint32_t hi8 = w[r][d] & 0xF0F0F0F0u;
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const float fl = static_cast<float>(static_cast<int8_t>(lo8 >> (8 * b)));
                        const float fh = static_cast<float>(static_cast<int8_t>(hi8 >> (8 * b)));
#pragma unroll
                        for (int i = 0; i < MR; ++i) {
                            acc[i][4 * d + b] = fmaf(xe[i], fl, acc[i][4 * d + b]);
                            acc[i][4 * d + b] = fmaf(xo[i], fh, acc[i][4 * d + b]);
                        }
                    }
                }
            }
        } else {
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                const int kr = kbase + r;
                float x[MR];
#pragma unroll
                for (int i = 0; i < MR; ++i)
                    x[i] = (i < m && kr < k) ? a[static_cast<int64_t>(i) * k + kr] : 0.0f;
#pragma unroll
                for (int d = 0; d < kWords; ++d) {
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const float f = static_cast<float>(static_cast<int8_t>(w[r][d] >> (8 * b)));
#pragma unroll
                        for (int i = 0; i < MR; ++i) acc[i][4 * d + b] = fmaf(x[i], f, acc[i][4 * d + b]);
                    }
                }
            }
        }

        if constexpr (KIND == 0) {
#pragma unroll
            for (int i = 0; i < MR; ++i)
#pragma unroll
                for (int j = 0; j < VEC; ++j) total[i][j] += acc[i][j];
        } else {
            const float f = kInt4 ? 0.0625f : 1.0f;  // INT4 accumulated 16*code
#pragma unroll
            for (int i = 0; i < MR; ++i)
#pragma unroll
                for (int j = 0; j < VEC; ++j) total[i][j] = fmaf(sc[j] * f, acc[i][j], total[i][j]);
        }
    }

    // Reduce the 4 waves of the workgroup through LDS.
#pragma unroll
    for (int i = 0; i < MR; ++i)
#pragma unroll
        for (int j = 0; j < VEC; ++j) red[wave][i][lane * VEC + j] = total[i][j];
    __syncthreads();

    const int tile_cols = 64 * VEC;
    const int tile_col0 = tile * tile_cols;
    // Each thread finishes (MR * tile_cols) / kThreads outputs.
    for (int o = threadIdx.x; o < MR * tile_cols; o += kThreads) {
        const int i = o / tile_cols;
        const int cc = o - i * tile_cols;
        float s = red[0][i][cc] + red[1][i][cc] + red[2][i][cc] + red[3][i][cc];
        red[0][i][cc] = s;
    }

    const int64_t col_base = tile_col0;
    if (splits == 1) {
        __syncthreads();
        for (int o = threadIdx.x; o < MR * tile_cols; o += kThreads) {
            const int i = o / tile_cols;
            const int cc = o - i * tile_cols;
            const int col = tile_col0 + cc;
            if (i < m && col < n) {
                float v = red[0][i][cc];
                if constexpr (KIND == 0) v *= scale[col];
                c[static_cast<int64_t>(i) * n + col] = v;
            }
        }
        return;
    }

    // Split-K: publish this split's partial, take a ticket; the last
    // workgroup of the tile sums all splits in order and writes C.
    float* my_part = partials + (static_cast<int64_t>(split) * MR) * n;
    __syncthreads();
    for (int o = threadIdx.x; o < MR * tile_cols; o += kThreads) {
        const int i = o / tile_cols;
        const int cc = o - i * tile_cols;
        const int col = tile_col0 + cc;
        if (col < n) my_part[static_cast<int64_t>(i) * n + col] = red[0][i][cc];
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) ticket = atomicAdd(&counters[tile], 1u);
    __syncthreads();
    if (ticket != static_cast<unsigned>(splits - 1)) return;
    __threadfence();

    for (int o = threadIdx.x; o < MR * tile_cols; o += kThreads) {
        const int i = o / tile_cols;
        const int cc = o - i * tile_cols;
        const int col = tile_col0 + cc;
        if (i < m && col < n) {
            float v = 0.0f;
            for (int s = 0; s < splits; ++s)
                v += __builtin_nontemporal_load(partials + (static_cast<int64_t>(s) * MR + i) * n + col);
            if constexpr (KIND == 0) v *= scale[col];
            c[static_cast<int64_t>(i) * n + col] = v;
        }
    }
    (void)col_base;
    if (threadIdx.x == 0) counters[tile] = 0u;  // ready for the next call on this stream
}

template <int KIND, int VEC, int MR>
int launch_gemv(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k,
                int n, int block_size, hipStream_t stream) {
    const int tile_cols = 64 * VEC;
    const int tiles = (n + tile_cols - 1) / tile_cols;
    const int total_units = (k + kUnitK - 1) / kUnitK;
    // Aim for about two workgroups per CU, with at least one unit per wave.
    const int target_wgs = 2 * cu_count();
    int splits = std::max(1, target_wgs / std::max(tiles, 1));
    splits = std::min(splits, std::max(1, total_units / kWaves));
    splits = std::min(splits, 64);
    int units_per_split = (total_units + splits - 1) / splits;
    // Keep the four waves of a workgroup busy on whole rounds of units.
    units_per_split = ((units_per_split + kWaves - 1) / kWaves) * kWaves;
    splits = (total_units + units_per_split - 1) / units_per_split;

    Workspace ws{};
    if (splits > 1) {
        VM_TRY(get_workspace(stream, static_cast<std::size_t>(splits) * MR * n,
                             static_cast<std::size_t>(tiles), &ws));
    }
    dim3 grid(tiles, splits);
    hipLaunchKernelGGL((qmm_gemv_kernel<KIND, VEC, MR>), grid, dim3(kThreads), 0, stream, a, wq,
                       scale, c, m, k, n, block_size, units_per_split, ws.partials, ws.counters);
    return check_launch("QuantizedMatMul", stream);
}

template <int KIND, int MR>
int dispatch_vec(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k,
                 int n, int block_size, hipStream_t stream) {
    const auto aligned = [&](int v) {
        return n % v == 0 && (reinterpret_cast<uintptr_t>(wq) % v) == 0 &&
               (reinterpret_cast<uintptr_t>(scale) % 16) == 0;
    };
    if (n >= 1024 && aligned(16)) return launch_gemv<KIND, 16, MR>(a, wq, scale, c, m, k, n, block_size, stream);
    if (n >= 512 && aligned(8)) return launch_gemv<KIND, 8, MR>(a, wq, scale, c, m, k, n, block_size, stream);
    if (aligned(4)) return launch_gemv<KIND, 4, MR>(a, wq, scale, c, m, k, n, block_size, stream);
    return VM_HIP_EUNSUPPORTED;
}

template <int KIND>
int dispatch_mr(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k,
                int n, int block_size, hipStream_t stream) {
    if (m == 1) return dispatch_vec<KIND, 1>(a, wq, scale, c, m, k, n, block_size, stream);
    if (m == 2) return dispatch_vec<KIND, 2>(a, wq, scale, c, m, k, n, block_size, stream);
    return dispatch_vec<KIND, 4>(a, wq, scale, c, m, k, n, block_size, stream);
}

}  // namespace

int gemv_qmm_f32(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k,
                 int n, int quant_type, int block_size, hipStream_t stream) {
    if (m < 1 || m > 4) return VM_HIP_EUNSUPPORTED;
    if (quant_type == VM_HIP_QUANT_INT4) {
        if (block_size <= 0 || block_size % kUnitK != 0) return VM_HIP_EUNSUPPORTED;
        return dispatch_mr<2>(a, wq, scale, c, m, k, n, block_size, stream);
    }
    if (block_size > 0) {
        if (block_size % kUnitK != 0) return VM_HIP_EUNSUPPORTED;
        return dispatch_mr<1>(a, wq, scale, c, m, k, n, block_size, stream);
    }
    return dispatch_mr<0>(a, wq, scale, c, m, k, n, 0, stream);
}

}  // namespace vmhip
