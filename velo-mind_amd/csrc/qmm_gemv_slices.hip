// Decode GEMV (one activation row) that leaves its split-K reduction to the
// consumer: workgroup split s writes its partial sums for its columns to
// out[s * n + j], and the kernel that reads the result adds the slices in
// split order (a fixed order, so results are reproducible).  Kernel
// boundaries order the slices before their reader, so no workgroup waits
// for another: the ticket handoff of a final-output split-K GEMV (partial
// stores, their acknowledgement, an atomic ticket and a reload, a chain of
// dependent memory round trips) disappears from every launch.
//
// Work decomposition (gfx950, wave64):
//   lane      16 consecutive columns x R consecutive byte rows of the codes
//             (R 16-byte loads)
//   wave      16 lanes across (256 columns = two 128-byte lines per byte
//             row) x 4 row-lanes (the wave's four 16-lane DPP rows) = 4R
//             byte rows, all inside one scale block
//   workgroup W waves stacked in K (4RW byte rows), on one 256-column tile
//   grid      (tiles, splits); tiles are renumbered so that each XCD owns a
//             contiguous run of columns
// The four row-lanes of a wave are reduced first with the gfx950
// permlane16/32 swaps (each lane is left with 4 of its 16 columns), so the
// block scale is one 16-byte load per lane and four FMAs; the waves of a
// workgroup add through LDS.
//
// Activation sources (the consumer side of the previous kernel):
//   PLAIN   x[k]: each lane loads its own 2R (INT4) or R (INT8) values
//   SLICES  x = sum of `in_slices` slices [in_slices][k], staged in LDS
//   SWIGLU  x[j] = silu(g[j]) * u[j] with g, u the sums of `in_slices`
//           slices of a fused gate|up projection [in_slices][2k], staged
//           in LDS (the Sigmoid, Mul, Mul of llama_graph.cpp:22-28)
//
// Dequantization matches the final-output GEMV: INT4 nibbles moved to the
// top of a byte give 16 * code (factor 1/16 folded into the scale), INT8
// codes are sign-extended bytes; fp32 FMA accumulation throughout.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "vm_device.h"
#include "vm_internal.h"

namespace vmhip {
namespace {

constexpr int kTileCols = 256;
constexpr int kGemvSrcPlain = VM_HIP_GEMV_SRC_PLAIN;
constexpr int kGemvSrcSlices = VM_HIP_GEMV_SRC_SLICES;
constexpr int kGemvSrcSwiglu = VM_HIP_GEMV_SRC_SWIGLU;

__device__ __forceinline__ float swap_rows_add(float a, float b) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    unsigned q[2];
    __builtin_memcpy(q, &p, sizeof q);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

__device__ __forceinline__ float swap_halves_add(float a, float b) {
    auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    unsigned q[2];
    __builtin_memcpy(q, &p, sizeof q);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

__device__ __forceinline__ float silu_mul(float g, float u) {
    const float sig = 1.0f / (1.0f + expf(-g));
    return (sig * g) * u;
}

// KIND: 0 = INT8 per-column scale, 1 = INT8 blockwise, 2 = INT4 blockwise.
template <int KIND, int R, int W, int SRC>
__global__ __launch_bounds__(W * 64) void qmm_gemv_slices_kernel(
    const float* __restrict__ act, int in_slices, const uint8_t* __restrict__ wq, const float* __restrict__ scale,
    float* __restrict__ out, int k, int n, int block_size, uint32_t code_bytes, uint32_t scale_bytes) {
    constexpr bool kInt4 = KIND == 2;
    constexpr int kRowsWave = 4 * R;                  // byte rows per wave
    constexpr int kRowsWg = W * kRowsWave;            // byte rows per workgroup
    constexpr int kKPerRow = kInt4 ? 2 : 1;           // K values per byte row
    constexpr int kXLane = R * kKPerRow;              // K values per lane
    constexpr int kXWg = kRowsWg * kKPerRow;          // K values per workgroup
    static_assert(kXLane % 4 == 0, "a lane's activations are whole float4s");
    __shared__ __align__(16) float red[W][kTileCols];
    __shared__ __align__(16) float xs[SRC == kGemvSrcPlain ? 4 : kXWg];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int cl = lane & 15;   // column lane
    const int rl = lane >> 4;   // row lane (DPP row)
    int tile = blockIdx.x;
    {
        const int full = static_cast<int>(gridDim.x) & ~7;
        if (tile < full) tile = (tile & 7) * (full >> 3) + (tile >> 3);
    }
    const int split = blockIdx.y;
    const int col0 = tile * kTileCols + cl * 16;
    const bool col_ok = col0 < n;                          // n % 16 == 0: all 16 columns or none
    const int wg_row0 = split * kRowsWg;
    const int wave_row0 = wg_row0 + wave * kRowsWave;
    const int row0 = wave_row0 + rl * R;
    const int byte_rows = kInt4 ? (k + 1) / 2 : k;

    // Codes: rows past the matrix and columns past n read zeros.
    const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(wq, code_bytes);
    u32x4 w[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = row0 + r;
        const uint32_t off = (col_ok && row < byte_rows)
                                 ? static_cast<uint32_t>(row) * static_cast<uint32_t>(n) + static_cast<uint32_t>(col0)
                                 : code_bytes;
        w[r] = buffer_load16(wrs, off);
    }
    // After the row-lane reduction this lane keeps columns col0 + keep .. +3.
    const int keep = 8 * (rl & 1) + 4 * (rl >> 1);
    u32x4 sv;
    {
        const __amdgpu_buffer_rsrc_t srs = buffer_rsrc(scale, scale_bytes);
        uint32_t soff = scale_bytes;
        if (col_ok) {
            if constexpr (KIND == 0) {
                soff = static_cast<uint32_t>(col0 + keep) * 4u;
            } else {
                // The wave's byte rows lie in one block (checked by the host).
                const int blk = (wave_row0 * kKPerRow) / block_size;
                if (wave_row0 < byte_rows)
                    soff = (static_cast<uint32_t>(blk) * static_cast<uint32_t>(n) + static_cast<uint32_t>(col0 + keep)) * 4u;
            }
        }
        sv = buffer_load16(srs, soff);
    }

    // Activations for the lane's K range [row0 * kKPerRow, + kXLane).
    u32x4 xv[kXLane / 4];
    const int kk0 = row0 * kKPerRow;
    if constexpr (SRC == kGemvSrcPlain) {
        const __amdgpu_buffer_rsrc_t ars = buffer_rsrc(act, static_cast<uint32_t>(k) * 4u);
#pragma unroll
        for (int i = 0; i < kXLane / 4; ++i) xv[i] = buffer_load16(ars, static_cast<uint32_t>(kk0 + 4 * i) * 4u);
    } else {
        // Stage the workgroup's K range: thread t sums the slices of float4
        // group t (four consecutive K values), all loads issued at once.
        const int kw0 = wg_row0 * kKPerRow;
        constexpr int kSrcMult = SRC == kGemvSrcSwiglu ? 2 : 1;
        const uint32_t slice_stride = static_cast<uint32_t>(k) * kSrcMult;   // floats per slice
        const __amdgpu_buffer_rsrc_t ars =
            buffer_rsrc(act, static_cast<uint32_t>(in_slices) * slice_stride * 4u);
        for (int q = threadIdx.x; q < kXWg / 4; q += W * 64) {
            const int kk = kw0 + 4 * q;
            const bool ok = kk < k;
            float4 g = make_float4(0.f, 0.f, 0.f, 0.f), u = g;
            for (int s0 = 0; s0 < in_slices; s0 += 8) {
                u32x4 tg[8], tu[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const bool v = ok && s0 + e < in_slices;
                    const uint32_t base = static_cast<uint32_t>(s0 + e) * slice_stride + static_cast<uint32_t>(kk);
                    tg[e] = buffer_load16(ars, v ? base * 4u : 0xfffffff0u);
                    if constexpr (SRC == kGemvSrcSwiglu)
                        tu[e] = buffer_load16(ars, v ? (base + static_cast<uint32_t>(k)) * 4u : 0xfffffff0u);
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    if (s0 + e < in_slices) {   // slices added in order
                        g.x += __uint_as_float(tg[e][0]);
                        g.y += __uint_as_float(tg[e][1]);
                        g.z += __uint_as_float(tg[e][2]);
                        g.w += __uint_as_float(tg[e][3]);
                        if constexpr (SRC == kGemvSrcSwiglu) {
                            u.x += __uint_as_float(tu[e][0]);
                            u.y += __uint_as_float(tu[e][1]);
                            u.z += __uint_as_float(tu[e][2]);
                            u.w += __uint_as_float(tu[e][3]);
                        }
                    }
                }
            }
            if constexpr (SRC == kGemvSrcSwiglu) {
                if (ok) g = make_float4(silu_mul(g.x, u.x), silu_mul(g.y, u.y), silu_mul(g.z, u.z), silu_mul(g.w, u.w));
            }
            // K values past k stay zero (their codes are zero too).
            *reinterpret_cast<float4*>(xs + 4 * q) = ok ? g : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kXLane / 4; ++i)
            xv[i] = *reinterpret_cast<const u32x4*>(xs + (kk0 - kw0) + 4 * i);
    }

    // Dequantize and accumulate the lane's 16 columns.
    float acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if constexpr (kInt4) {
            const float xe = __uint_as_float(xv[(2 * r) / 4][(2 * r) % 4]);
            const float xo = __uint_as_float(xv[(2 * r + 1) / 4][(2 * r + 1) % 4]);
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint32_t wd = w[r][d];
                const uint32_t lo8 = (wd << 4) & 0xF0F0F0F0u;
                const uint32_t hi8 = wd & 0xF0F0F0F0u;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    acc[4 * d + b] = fmaf(xe, static_cast<float>(static_cast<int8_t>(lo8 >> (8 * b))), acc[4 * d + b]);
                    acc[4 * d + b] = fmaf(xo, static_cast<float>(static_cast<int8_t>(hi8 >> (8 * b))), acc[4 * d + b]);
                }
            }
        } else {
            const float x = __uint_as_float(xv[r / 4][r % 4]);
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint32_t wd = w[r][d];
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    acc[4 * d + b] =
                        fmaf(x, static_cast<float>(static_cast<int>(wd << (24 - 8 * b)) >> 24), acc[4 * d + b]);
            }
        }
    }

    // Row-lane reduction: row pairs (permlane16 swap), then wave halves
    // (permlane32 swap); the lane keeps columns keep .. keep + 3.
    float h[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = swap_rows_add(acc[j], acc[j + 8]);
    float z[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) z[j] = swap_halves_add(h[j], h[j + 4]);
    const float f = kInt4 ? 0.0625f : 1.0f;   // INT4 accumulated 16 * code
#pragma unroll
    for (int j = 0; j < 4; ++j) z[j] *= __uint_as_float(sv[j]) * f;
    *reinterpret_cast<float4*>(&red[wave][cl * 16 + keep]) = make_float4(z[0], z[1], z[2], z[3]);
    __syncthreads();

    float* dst = out + static_cast<int64_t>(split) * n;
    for (int o = threadIdx.x; o < kTileCols; o += W * 64) {
        const int col = tile * kTileCols + o;
        if (col < n) {
            float v = 0.0f;
#pragma unroll
            for (int ww = 0; ww < W; ++ww) v += red[ww][o];
            dst[col] = v;
        }
    }
}

struct SlicesConfig {
    int R = 4;
    int W = 4;
    int splits = 1;
};

int byte_rows_of(int kind, int64_t k) { return static_cast<int>(kind == 2 ? (k + 1) / 2 : k); }

// Whether a wave's 4R byte rows stay inside one scale block.
bool rows_fit_block(int kind, int R, int block) {
    if (kind == 0) return true;
    const int rows_per_block = kind == 2 ? block / 2 : block;
    return block > 0 && (kind != 2 || block % 2 == 0) && rows_per_block % (4 * R) == 0;
}

// Measured on MI355X (cold weights, graph replay) over the TinyLlama and
// SmolLM2 decode shapes: R = 4, W = 4 is within a few percent of the best
// everywhere; wider workgroups are used only to keep the slice count within
// what the consumer accepts, and R shrinks for blocks of fewer byte rows.
bool choose_slices_config(int kind, int64_t k, int64_t n, int block, int max_slices, SlicesConfig* cfg) {
    const int rows = byte_rows_of(kind, k);
    for (int R : {4, 2}) {
        if (!rows_fit_block(kind, R, block)) continue;
        for (int W : {4, 8, 16}) {
            const int splits = (rows + 4 * R * W - 1) / (4 * R * W);
            if (splits <= max_slices || W == 16) {
                if (splits > max_slices) break;
                cfg->R = R;
                cfg->W = W;
                cfg->splits = splits;
                return true;
            }
        }
    }
    (void)n;
    return false;
}

template <int KIND, int R, int W, int SRC>
void launch_slices(const float* act, int in_slices, const uint8_t* wq, const float* scale, float* out, int k, int n,
                   int block, int splits, hipStream_t stream) {
    const int tiles = (n + kTileCols - 1) / kTileCols;
    const int64_t rows = KIND == 2 ? (static_cast<int64_t>(k) + 1) / 2 : k;
    const int64_t nblk = KIND == 0 ? 1 : (static_cast<int64_t>(k) + block - 1) / block;
    const uint32_t code_bytes = static_cast<uint32_t>(rows * n);
    const uint32_t scale_bytes = static_cast<uint32_t>(KIND == 0 ? static_cast<int64_t>(n) * 4 : nblk * n * 4);
    hipLaunchKernelGGL((qmm_gemv_slices_kernel<KIND, R, W, SRC>), dim3(tiles, splits), dim3(W * 64), 0, stream, act,
                       in_slices, wq, scale, out, k, n, block, code_bytes, scale_bytes);
}

template <int KIND, int SRC>
void dispatch_rw(const SlicesConfig& c, const float* act, int in_slices, const uint8_t* wq, const float* scale,
                 float* out, int k, int n, int block, hipStream_t stream) {
#define VM_SLICES_CASE(RR, WW)                                                                              \
    if (c.R == RR && c.W == WW)                                                                             \
        return launch_slices<KIND, RR, WW, SRC>(act, in_slices, wq, scale, out, k, n, block, c.splits, stream);
    if constexpr (KIND == 2) {
        VM_SLICES_CASE(4, 4)
        VM_SLICES_CASE(4, 8)
        VM_SLICES_CASE(4, 16)
        VM_SLICES_CASE(2, 4)
        VM_SLICES_CASE(2, 8)
        VM_SLICES_CASE(2, 16)
    } else {
        // INT8: a lane's R K values must be whole float4s (R = 4).
        VM_SLICES_CASE(4, 4)
        VM_SLICES_CASE(4, 8)
        VM_SLICES_CASE(4, 16)
    }
#undef VM_SLICES_CASE
}

}  // namespace

int gemv_slices_plan(int quant_type, int64_t k, int64_t n, int block_size, int max_slices, int* splits, int* r,
                     int* w) {
    const int kind = quant_type == VM_HIP_QUANT_INT4 ? 2 : (block_size > 0 ? 1 : 0);
    const int block = kind == 2 ? (block_size > 0 ? block_size : 32) : block_size;
    SlicesConfig cfg;
    if (!choose_slices_config(kind, k, n, block, max_slices, &cfg)) return 0;
    if (kind != 2 && cfg.R != 4) return 0;
    *splits = cfg.splits;
    *r = cfg.R;
    *w = cfg.W;
    return 1;
}

}  // namespace vmhip

using namespace vmhip;

extern "C" {

int vm_hip_gemv_slices_count(int64_t k, int64_t n, int quant_type, int block_size, int max_slices, int* slices) {
    clear_error();
    if (!slices) return fail_inval("gemv_slices_count: null pointer");
    *slices = 0;
    if (k < 1 || n < 1 || n % 16 != 0) return fail_inval("gemv_slices: k >= 1 and n a multiple of 16 required");
    if (quant_type != VM_HIP_QUANT_INT8 && quant_type != VM_HIP_QUANT_INT4)
        return fail_inval("gemv_slices: quant_type must be INT8 or INT4");
    if (max_slices < 1) return fail_inval("gemv_slices: max_slices must be positive");
    int s = 0, r = 0, w = 0;
    if (!gemv_slices_plan(quant_type, k, n, block_size, max_slices, &s, &r, &w)) {
        set_error("gemv_slices: no configuration for this shape, block size and slice limit");
        return VM_HIP_EUNSUPPORTED;
    }
    *slices = s;
    return 0;
}

int vm_hip_qmm_gemv_slices_f32(const float* act, int act_kind, int64_t act_slices, const int8_t* wq,
                               const float* scale, float* out, int64_t k, int64_t n, int quant_type, int block_size,
                               int max_slices, void* stream) {
    int s = 0;
    VM_TRY(vm_hip_gemv_slices_count(k, n, quant_type, block_size, max_slices, &s));
    if (!act || !wq || !scale || !out) return fail_inval("gemv_slices: null pointer");
    if (act_kind != VM_HIP_GEMV_SRC_PLAIN && act_kind != VM_HIP_GEMV_SRC_SLICES && act_kind != VM_HIP_GEMV_SRC_SWIGLU)
        return fail_inval("gemv_slices: unknown activation source");
    if (act_kind != VM_HIP_GEMV_SRC_PLAIN && (act_slices < 1 || act_slices > 4096))
        return fail_inval("gemv_slices: act_slices must be in [1, 4096]");
    if (k % 4 != 0 || reinterpret_cast<uintptr_t>(act) % 16 != 0)
        return fail_inval("gemv_slices: k % 4 == 0 and a 16-byte aligned activation required");
    const int64_t rows = quant_type == VM_HIP_QUANT_INT4 ? (k + 1) / 2 : k;
    const int64_t src_floats = act_kind == VM_HIP_GEMV_SRC_PLAIN ? k : act_slices * k * (act_kind == VM_HIP_GEMV_SRC_SWIGLU ? 2 : 1);
    if (rows * n > 0x7fffffffLL || s * n > 0x7fffffffLL || src_floats * 4 > 0x7fffffffLL)
        return fail_inval("gemv_slices: operands must stay below 2 GiB");
    VM_TRY(injected_failure("QuantizedMatMul", "launch"));
    int r = 0, w = 0;
    gemv_slices_plan(quant_type, k, n, block_size, max_slices, &s, &r, &w);
    SlicesConfig cfg;
    cfg.R = r;
    cfg.W = w;
    cfg.splits = s;
    const int kind = quant_type == VM_HIP_QUANT_INT4 ? 2 : (block_size > 0 ? 1 : 0);
    const int block = kind == 2 ? (block_size > 0 ? block_size : 32) : block_size;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const auto* wb = reinterpret_cast<const uint8_t*>(wq);
    const int ki = static_cast<int>(k), ni = static_cast<int>(n), sl = static_cast<int>(act_slices);
#define VM_SLICES_SRC(KINDV)                                                                                    \
    do {                                                                                                      \
        if (act_kind == VM_HIP_GEMV_SRC_PLAIN)                                                                \
            dispatch_rw<KINDV, kGemvSrcPlain>(cfg, act, 0, wb, scale, out, ki, ni, block, st);                \
        else if (act_kind == VM_HIP_GEMV_SRC_SLICES)                                                          \
            dispatch_rw<KINDV, kGemvSrcSlices>(cfg, act, sl, wb, scale, out, ki, ni, block, st);              \
        else                                                                                                  \
            dispatch_rw<KINDV, kGemvSrcSwiglu>(cfg, act, sl, wb, scale, out, ki, ni, block, st);              \
    } while (0)
    if (kind == 2)
        VM_SLICES_SRC(2);
    else if (kind == 1)
        VM_SLICES_SRC(1);
    else
        VM_SLICES_SRC(0);
#undef VM_SLICES_SRC
    return check_launch("QuantizedMatMul", st);
}

}  // extern "C"
