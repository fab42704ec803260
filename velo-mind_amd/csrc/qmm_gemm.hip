// Prefill-shaped (rows_m > 4) quantized matmul on gfx950 MFMA.
//
// C[M, N] = A[M, K] * W[K, N] with W given as the reference's codes
// (INT8 [K, N] or INT4 packed [(K+1)/2, N]) and fp32 scales.
//
// Per K step of 32 (one INT4 scale block):
//   A tile  BM x 32 fp32 -> fp16 (round to nearest even) -> LDS [BM][32]
//   B tile  32 x BN codes -> fp16 (exact: |code| <= 127) -> LDS [BN][32],
//           i.e. K-contiguous per column, the B-operand layout of
//           v_mfma_f32_16x16x32_f16 (lane l: column l % 16, k 8*(l/16)..+7)
//   MFMA    each wave owns WM x WN outputs as 16x16 tiles
//   scales  INT8 per column: applied once in the epilogue; blockwise
//           (INT4, INT8 with block_size > 0): each step's MFMA result is
//           multiplied by its block's fp32 scale and added to an fp32
//           accumulator, so codes and scales are never rounded to fp16.
// LDS is double-buffered: the next step's global loads are in flight while
// the current step's MFMAs run; one barrier per step.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "qmm_kernels.h"
#include "vm_internal.h"

namespace vmhip {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kBK = 32;       // K per step
constexpr int kPad = 8;       // halves of padding per LDS row (80-byte rows)
constexpr int kRow = kBK + kPad;
constexpr int kThreads = 256;

// KIND: 0 = INT8 per-column, 1 = INT8 blockwise, 2 = INT4 blockwise.
// BM x BN output tile per workgroup; WAVES_M x WAVES_N = 4 waves.
template <int KIND, int BM, int BN, int WAVES_M, int WAVES_N>
__global__ __launch_bounds__(kThreads) void qmm_gemm_kernel(const float* __restrict__ a,
                                                            const uint8_t* __restrict__ wq,
                                                            const float* __restrict__ scale,
                                                            float* __restrict__ c, int m, int k, int n,
                                                            int block_size) {
    static_assert(WAVES_M * WAVES_N == 4, "four waves per workgroup");
    constexpr bool kInt4 = KIND == 2;
    constexpr bool kBlockScaled = KIND != 0;
    constexpr int WM = BM / WAVES_M;
    constexpr int WN = BN / WAVES_N;
    constexpr int TM = WM / 16;
    constexpr int TN = WN / 16;
    static_assert(TM >= 1 && TN >= 1, "wave tile must hold at least one 16x16 MFMA tile");
    constexpr int kAVec = BM * kBK / 4;           // float4 loads of A per step
    constexpr int kAPerThread = (kAVec + kThreads - 1) / kThreads;
    constexpr int kBQuads = BN / 4;               // 4-column groups
    constexpr int kBJobs = kBQuads * (kBK / 4);   // (column quad, k quad) pairs per step
    constexpr int kBPerThread = (kBJobs + kThreads - 1) / kThreads;

    __shared__ __attribute__((aligned(16))) _Float16 sA[2][BM][kRow];
    __shared__ __attribute__((aligned(16))) _Float16 sB[2][BN][kRow];
    __shared__ float sS[2][kBlockScaled ? BN : 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N;
    const int wn = wave % WAVES_N;
    const int n0 = blockIdx.x * BN;
    const int m0 = blockIdx.y * BM;
    const int steps = k / kBK;  // dispatch guarantees k % 32 == 0

    // Register staging of one step's global data.
    float4 ra[kAPerThread];
    uint32_t rb[kBPerThread][kInt4 ? 2 : 4];
    float4 rs = {0.f, 0.f, 0.f, 0.f};

    auto load_global = [&](int step) {
        const int k0 = step * kBK;
#pragma unroll
        for (int i = 0; i < kAPerThread; ++i) {
            const int f = tid + i * kThreads;
            const int row = f / (kBK / 4);
            const int c4 = f % (kBK / 4);
            ra[i] = float4{0.f, 0.f, 0.f, 0.f};
            if (f < kAVec && m0 + row < m)
                ra[i] = *reinterpret_cast<const float4*>(a + static_cast<int64_t>(m0 + row) * k + k0 + c4 * 4);
        }
#pragma unroll
        for (int i = 0; i < kBPerThread; ++i) {
            const int job = tid + i * kThreads;
            const int quad = job % kBQuads;
            const int kq = job / kBQuads;  // k rows 4*kq .. 4*kq+3 of the step
            const int col = n0 + quad * 4;
            const bool ok = job < kBJobs && col < n;
            if constexpr (kInt4) {
                const int prow = (k0 + kq * 4) / 2;  // two packed rows hold four k rows
#pragma unroll
                for (int r = 0; r < 2; ++r)
                    rb[i][r] = ok ? *reinterpret_cast<const uint32_t*>(wq + static_cast<int64_t>(prow + r) * n + col) : 0u;
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    rb[i][r] = ok ? *reinterpret_cast<const uint32_t*>(wq + static_cast<int64_t>(k0 + kq * 4 + r) * n + col) : 0u;
            }
        }
        if constexpr (kBlockScaled) {
            if (tid < BN / 4) {
                const int blk = k0 / block_size;
                const int col = n0 + tid * 4;
                rs = col < n ? *reinterpret_cast<const float4*>(scale + static_cast<int64_t>(blk) * n + col)
                             : float4{0.f, 0.f, 0.f, 0.f};
            }
        }
    };

    auto store_lds = [&](int buf) {
#pragma unroll
        for (int i = 0; i < kAPerThread; ++i) {
            const int f = tid + i * kThreads;
            if (f < kAVec) {
                const int row = f / (kBK / 4);
                const int c4 = f % (kBK / 4);
                half4 h = {static_cast<_Float16>(ra[i].x), static_cast<_Float16>(ra[i].y),
                           static_cast<_Float16>(ra[i].z), static_cast<_Float16>(ra[i].w)};
                *reinterpret_cast<half4*>(&sA[buf][row][c4 * 4]) = h;
            }
        }
#pragma unroll
        for (int i = 0; i < kBPerThread; ++i) {
            const int job = tid + i * kThreads;
            if (job >= kBJobs) continue;
            const int quad = job % kBQuads;
            const int kq = job / kBQuads;
            // codes[r][col] for the 4 k rows and 4 columns of this job
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                half4 h;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int code;
                    if constexpr (kInt4) {
                        const uint32_t byte = (rb[i][r >> 1] >> (8 * cc)) & 0xFFu;
                        const int nib = (r & 1) ? static_cast<int>(byte >> 4) : static_cast<int>(byte & 0xFu);
                        code = nib >= 8 ? nib - 16 : nib;
                    } else {
                        code = static_cast<int8_t>((rb[i][r] >> (8 * cc)) & 0xFFu);
                    }
                    h[r] = static_cast<_Float16>(code);
                }
                *reinterpret_cast<half4*>(&sB[buf][quad * 4 + cc][kq * 4]) = h;
            }
        }
        if constexpr (kBlockScaled) {
            if (tid < BN / 4) *reinterpret_cast<float4*>(&sS[buf][tid * 4]) = rs;
        }
    };

    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    load_global(0);
    store_lds(0);
    __syncthreads();

    const int frag_row = lane % 16;
    const int frag_k = 8 * (lane / 16);
    for (int step = 0; step < steps; ++step) {
        const int buf = step & 1;
        if (step + 1 < steps) load_global(step + 1);

        half8 bf[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j)
            bf[j] = *reinterpret_cast<const half8*>(&sB[buf][wn * WN + j * 16 + frag_row][frag_k]);
        float sv[TN];
        if constexpr (kBlockScaled) {
#pragma unroll
            for (int j = 0; j < TN; ++j) sv[j] = sS[buf][wn * WN + j * 16 + frag_row];
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const half8 af = *reinterpret_cast<const half8*>(&sA[buf][wm * WM + i * 16 + frag_row][frag_k]);
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                if constexpr (kBlockScaled) {
                    const floatx4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], floatx4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[i][j][e] = fmaf(sv[j], d[e], acc[i][j][e]);
                } else {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], acc[i][j], 0, 0, 0);
                }
            }
        }
        if (step + 1 < steps) store_lds(buf ^ 1);
        __syncthreads();
    }

    // D layout: lane l holds rows 4*(l/16)+e, column l%16 of each tile.
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn * WN + j * 16 + frag_row;
        if (col >= n) continue;
        const float s = KIND == 0 ? scale[col] : 1.0f;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = m0 + wm * WM + i * 16 + 4 * (lane / 16) + e;
                if (row < m) c[static_cast<int64_t>(row) * n + col] = acc[i][j][e] * s;
            }
        }
    }
}

template <int KIND, int BM, int BN, int WAVES_M, int WAVES_N>
int launch(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k, int n, int block_size,
           hipStream_t stream) {
    dim3 grid((n + BN - 1) / BN, (m + BM - 1) / BM);
    hipLaunchKernelGGL((qmm_gemm_kernel<KIND, BM, BN, WAVES_M, WAVES_N>), grid, dim3(kThreads), 0, stream, a, wq,
                       scale, c, m, k, n, block_size);
    return check_launch("QuantizedMatMul", stream);
}

template <int KIND>
int launch_kind(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k, int n,
                int block_size, hipStream_t stream) {
    if (m <= 16) return launch<KIND, 16, 128, 1, 4>(a, wq, scale, c, m, k, n, block_size, stream);
    if (m <= 32) return launch<KIND, 32, 128, 2, 2>(a, wq, scale, c, m, k, n, block_size, stream);
    if (m <= 64) return launch<KIND, 64, 128, 2, 2>(a, wq, scale, c, m, k, n, block_size, stream);
    return launch<KIND, 128, 128, 2, 2>(a, wq, scale, c, m, k, n, block_size, stream);
}

}  // namespace

int gemm_qmm_f32(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k, int n,
                 int quant_type, int block_size, hipStream_t stream) {
    // Whole 32-row steps, dword-aligned code rows and float4-aligned A/scales.
    if (k % kBK != 0 || n % 4 != 0 || reinterpret_cast<uintptr_t>(a) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(wq) % 4 != 0 || reinterpret_cast<uintptr_t>(scale) % 16 != 0)
        return VM_HIP_EUNSUPPORTED;
    if (static_cast<int64_t>(m) > 65535 * 128) return VM_HIP_EUNSUPPORTED;
    if (quant_type == VM_HIP_QUANT_INT4) {
        if (block_size <= 0 || block_size % kBK != 0) return VM_HIP_EUNSUPPORTED;
        return launch_kind<2>(a, wq, scale, c, m, k, n, block_size, stream);
    }
    if (block_size > 0) {
        if (block_size % kBK != 0) return VM_HIP_EUNSUPPORTED;
        return launch_kind<1>(a, wq, scale, c, m, k, n, block_size, stream);
    }
    return launch_kind<0>(a, wq, scale, c, m, k, n, 0, stream);
}

}  // namespace vmhip
