// Decode-shaped (rows_m <= 4) quantized matmul for gfx950: an HBM-bound
// GEMV that streams the reference's [K, N] code layout (N contiguous) with
// 128-bit loads, dequantizes in registers and accumulates in fp32.
//
// Work decomposition
//   lane      : 16 consecutive columns (one 16-byte load per code row)
//   row group : L lanes side by side cover one 16*L-column row segment;
//               a wave holds G = 64/L row groups on consecutive chunks
//   chunk     : 8 logical K rows (INT4: 4 packed byte rows; INT8: 8 rows),
//               the unit a row group loads and reduces at a time
//   workgroup : W waves = W*G row groups on one 16*L-column tile; they walk
//               the workgroup's K range chunk by chunk, two chunks in
//               flight per row group (the next chunk's codes and scales are
//               loaded before the current chunk is reduced)
//   split     : grid.y splits K; the last workgroup of a tile to finish
//               (atomic ticket) adds the splits' partials in split order, so
//               results do not depend on scheduling
//
// Reduction: row groups of a wave combine with xor shuffles, the waves of
// a workgroup through LDS, splits through the per-stream workspace.  The
// split handoff uses agent-scope atomic stores/loads (coherent across XCDs,
// `sc1`) for the partials: each wave waits for its partial stores to be
// acknowledged (s_waitcnt) before the barrier that precedes the ticket
// increment, and the last workgroup reads the partials only after it has
// observed the final ticket.  No L2 write-back or invalidate is needed.
//
// Dequantization: INT8 codes are sign-extended bytes (v_cvt_f32_i32 with an
// SDWA byte select).  An INT4 byte holds the even K row in its low nibble;
// moving each nibble to the top of a byte ((w << 4) & 0xF0.. and w & 0xF0..)
// makes the signed byte equal 16*code, so the same SDWA convert applies and
// the factor 1/16 is folded (exactly) into the scale.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "qmm_kernels.h"
#include "vm_internal.h"

namespace vmhip {
namespace {

constexpr int kChunkK = 8;    // logical K rows per chunk
constexpr int kVec = 16;      // columns per lane
constexpr int kMaxSplits = 32;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int KIND>
struct ChunkShape {
    static constexpr bool kInt4 = KIND == 2;
    static constexpr int kRows = kInt4 ? kChunkK / 2 : kChunkK;  // byte rows per chunk
    static constexpr bool kScaled = KIND != 0;
};

// Raw buffer access (gfx9 descriptor word 3 = 0x00020000): loads past
// `num_records` bytes return zeros instead of faulting, so tails and idle
// chunks need no branches and every lane issues the same loads.
constexpr int kBufferFlags = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kBufferFlags);
}

__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t offset) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, static_cast<int>(offset), 0, 0));
}

__device__ __forceinline__ float coherent_load(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void coherent_store(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Codes and scales of one chunk for one lane.
template <int KIND>
struct Chunk {
    u32x4 w[ChunkShape<KIND>::kRows];
    u32x4 s[ChunkShape<KIND>::kScaled ? 4 : 1];
};

// KIND: 0 = INT8 per-column scale, 1 = INT8 blockwise, 2 = INT4 blockwise.
// MR: activation rows (1, 2 or 4); L: lanes per row segment; W: waves.
template <int KIND, int MR, int L, int W>
__global__ __launch_bounds__(W * 64) void qmm_gemv_kernel(
    const float* __restrict__ a, const uint8_t* __restrict__ wq, const float* __restrict__ scale,
    float* __restrict__ c, int m, int k, int n, int block_size, int chunks_per_split,
    uint32_t code_bytes, uint32_t scale_bytes, int blk_shift, float* __restrict__ partials,
    unsigned* __restrict__ counters) {
    using CS = ChunkShape<KIND>;
    constexpr int G = 64 / L;            // row groups per wave
    constexpr int RG = W * G;            // row groups per workgroup
    constexpr int kTileCols = kVec * L;

    extern __shared__ float smem[];
    float* xs = smem;                                     // [MR][chunks_per_split * 8]
    const int xs_len = chunks_per_split * kChunkK;
    float* red = smem + MR * xs_len;                      // [W][MR][kTileCols]
    __shared__ unsigned ticket;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int rg = wave * G + lane / L;                   // row group in the workgroup
    const int tile = blockIdx.x;
    const int split = blockIdx.y;
    const int splits = gridDim.y;
    const int col0 = tile * kTileCols + (lane % L) * kVec;

    const int total_chunks = (k + kChunkK - 1) / kChunkK;
    const int byte_rows = CS::kInt4 ? (k + 1) / 2 : k;
    const int c_begin = split * chunks_per_split;
    const int c_end = min(total_chunks, c_begin + chunks_per_split);
    const int k_begin = c_begin * kChunkK;

    const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(wq, code_bytes);
    const __amdgpu_buffer_rsrc_t srs = buffer_rsrc(scale, scale_bytes);
    (void)byte_rows;

    // Chunks outside [c_begin, c_end) read past the end of the buffers and
    // come back as zeros (codes and scales), contributing nothing.
    auto load_chunk = [&](int ch, Chunk<KIND>& dst) {
        const bool valid = ch < c_end;
        const uint32_t off = valid ? static_cast<uint32_t>(ch * CS::kRows) * static_cast<uint32_t>(n) + col0
                                   : code_bytes;
#pragma unroll
        for (int r = 0; r < CS::kRows; ++r) dst.w[r] = buffer_load16(wrs, off + static_cast<uint32_t>(r * n));
        if constexpr (CS::kScaled) {
            const uint32_t blk = blk_shift >= 0 ? static_cast<uint32_t>(ch) >> blk_shift
                                                : static_cast<uint32_t>(ch * kChunkK) / static_cast<uint32_t>(block_size);
            const uint32_t soff = valid ? (blk * static_cast<uint32_t>(n) + col0) * 4u : scale_bytes;
#pragma unroll
            for (int q = 0; q < 4; ++q) dst.s[q] = buffer_load16(srs, soff + 16u * q);
        }
    };

    auto compute_chunk = [&](const Chunk<KIND>& cur, int ch, float (&total)[MR][kVec]) {
        const float* xc = xs + (min(ch, c_end - 1) * kChunkK - k_begin);
        float acc[MR][kVec];
#pragma unroll
        for (int i = 0; i < MR; ++i)
#pragma unroll
            for (int j = 0; j < kVec; ++j) acc[i][j] = 0.0f;

        if constexpr (CS::kInt4) {
#pragma unroll
            for (int r = 0; r < CS::kRows; ++r) {
                float xe[MR], xo[MR];
#pragma unroll
                for (int i = 0; i < MR; ++i) {
                    const float2 xp = *reinterpret_cast<const float2*>(xc + i * xs_len + 2 * r);
                    xe[i] = xp.x;
                    xo[i] = xp.y;
                }
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const uint32_t wd = cur.w[r][d];
                    const uint32_t lo8 = (wd << 4) & 0xF0F0F0F0u;
                    const uint32_t hi8 = wd & 0xF0F0F0F0u;
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
            for (int r = 0; r < CS::kRows; ++r) {
                float x[MR];
#pragma unroll
                for (int i = 0; i < MR; ++i) x[i] = xc[i * xs_len + r];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const uint32_t wd = cur.w[r][d];
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const float f = static_cast<float>(static_cast<int>(wd << (24 - 8 * b)) >> 24);
#pragma unroll
                        for (int i = 0; i < MR; ++i) acc[i][4 * d + b] = fmaf(x[i], f, acc[i][4 * d + b]);
                    }
                }
            }
        }

        if constexpr (CS::kScaled) {
            const float f = CS::kInt4 ? 0.0625f : 1.0f;  // INT4 accumulated 16*code
            float sv[kVec];
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) sv[4 * q + e] = __uint_as_float(cur.s[q][e]) * f;
#pragma unroll
            for (int i = 0; i < MR; ++i)
#pragma unroll
                for (int j = 0; j < kVec; ++j) total[i][j] = fmaf(sv[j], acc[i][j], total[i][j]);
        } else {
#pragma unroll
            for (int i = 0; i < MR; ++i)
#pragma unroll
                for (int j = 0; j < kVec; ++j) total[i][j] += acc[i][j];
        }
    };

    // Issue the first chunk's loads, then stage this split's activations.
    Chunk<KIND> ca, cb;
    int ch = c_begin + rg;
    load_chunk(ch, ca);

    for (int i = threadIdx.x; i < MR * xs_len; i += W * 64) {
        const int r = i / xs_len;
        const int kk = k_begin + (i - r * xs_len);
        xs[i] = (r < m && kk < k) ? a[static_cast<int64_t>(r) * k + kk] : 0.0f;
    }
    __syncthreads();

    float total[MR][kVec];
#pragma unroll
    for (int i = 0; i < MR; ++i)
#pragma unroll
        for (int j = 0; j < kVec; ++j) total[i][j] = 0.0f;

    // Every row group runs the same number of steps; two buffers alternate
    // so one chunk's loads are in flight while the other is reduced (loads
    // past the split read zeros).  An odd last step runs after the loop.
    const int iters = (c_end - c_begin + RG - 1) / RG;
    for (int it = 0; it + 1 < iters; it += 2) {
        load_chunk(ch + RG, cb);
        compute_chunk(ca, ch, total);
        load_chunk(ch + 2 * RG, ca);
        compute_chunk(cb, ch + RG, total);
        ch += 2 * RG;
    }
    if (iters & 1) compute_chunk(ca, ch, total);

    // Row groups of a wave: lanes l and l ^ (L * 2^t) hold the same columns.
#pragma unroll
    for (int off = L; off < 64; off <<= 1)
#pragma unroll
        for (int i = 0; i < MR; ++i)
#pragma unroll
            for (int j = 0; j < kVec; ++j) total[i][j] += __shfl_xor(total[i][j], off, 64);

    // Waves of the workgroup through LDS.
    if (lane < L) {
#pragma unroll
        for (int i = 0; i < MR; ++i)
#pragma unroll
            for (int j = 0; j < kVec; ++j) red[(wave * MR + i) * kTileCols + lane * kVec + j] = total[i][j];
    }
    __syncthreads();

    const int tile_col0 = tile * kTileCols;
    if (splits == 1) {
        for (int o = threadIdx.x; o < MR * kTileCols; o += W * 64) {
            const int i = o / kTileCols;
            const int cc = o - i * kTileCols;
            const int col = tile_col0 + cc;
            if (i < m && col < n) {
                float v = 0.0f;
#pragma unroll
                for (int w = 0; w < W; ++w) v += red[(w * MR + i) * kTileCols + cc];
                if constexpr (KIND == 0) v *= scale[col];
                c[static_cast<int64_t>(i) * n + col] = v;
            }
        }
        return;
    }

    // Split-K handoff.
    float* my_part = partials + static_cast<int64_t>(split) * MR * n;
    for (int o = threadIdx.x; o < MR * kTileCols; o += W * 64) {
        const int i = o / kTileCols;
        const int cc = o - i * kTileCols;
        const int col = tile_col0 + cc;
        if (col < n) {
            float v = 0.0f;
#pragma unroll
            for (int w = 0; w < W; ++w) v += red[(w * MR + i) * kTileCols + cc];
            coherent_store(my_part + static_cast<int64_t>(i) * n + col, v);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // partial stores acknowledged before the ticket
    __syncthreads();
    if (threadIdx.x == 0)
        ticket = __hip_atomic_fetch_add(&counters[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (ticket != static_cast<unsigned>(splits - 1)) return;

    for (int o = threadIdx.x; o < MR * kTileCols; o += W * 64) {
        const int i = o / kTileCols;
        const int cc = o - i * kTileCols;
        const int col = tile_col0 + cc;
        if (i < m && col < n) {
            const float* p = partials + static_cast<int64_t>(i) * n + col;
            const int64_t stride = static_cast<int64_t>(MR) * n;
            float v = 0.0f;
            // Batches of independent loads, summed in split order.
            for (int s0 = 0; s0 < splits; s0 += 8) {
                float t[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) t[u] = (s0 + u < splits) ? coherent_load(p + (s0 + u) * stride) : 0.0f;
#pragma unroll
                for (int u = 0; u < 8; ++u) v += t[u];
            }
            if constexpr (KIND == 0) v *= scale[col];
            c[static_cast<int64_t>(i) * n + col] = v;
        }
    }
    if (threadIdx.x == 0)
        __hip_atomic_store(&counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct GemvConfig {
    int L = 16;
    int W = 4;
    int splits = 1;
    int chunks_per_split = 0;
};

int mr_for(int m) { return m <= 1 ? 1 : (m <= 2 ? 2 : 4); }

// Picks lanes-per-segment, waves and splits for a shape.  Measured on
// MI355X over the TinyLlama-1.1B and SmolLM2 shapes: 8 lanes per row segment
// (128-column tiles) is best everywhere; about 200 workgroups with at least
// 16 chunks per split balances split-K round trips against per-wave work;
// 8 waves pay off once a split holds more than 32 chunks.
GemvConfig choose_config(int kind, int m, int k, int n) {
    (void)kind;
    const int mr = mr_for(m);
    const int total_chunks = (k + kChunkK - 1) / kChunkK;
    GemvConfig cfg;
    cfg.L = 8;
    const int tiles = (n + kVec * cfg.L - 1) / (kVec * cfg.L);
    int S = 1;
    while (S * 2 <= 16 && S * 2 * tiles <= 200) S *= 2;
    while (S > 1 && (total_chunks + S - 1) / S < 16) S /= 2;
    int cps = (total_chunks + S - 1) / S;
    cfg.W = cps > 32 ? 8 : 4;
    // Activations of one split and the cross-wave buffer share 60 KB of LDS.
    while (S < kMaxSplits &&
           (static_cast<long>(mr) * cps * kChunkK + static_cast<long>(cfg.W) * mr * kVec * cfg.L) * 4 > 60 * 1024) {
        S *= 2;
        cps = (total_chunks + S - 1) / S;
    }
    cfg.chunks_per_split = cps;
    cfg.splits = (total_chunks + cps - 1) / cps;

    // Tuning override for measurement sweeps: VELOMIND_GEMV_CFG="L,W,S".
    if (const char* env = std::getenv("VELOMIND_GEMV_CFG")) {
        int L = 0, W = 0, Sx = 0;
        if (std::sscanf(env, "%d,%d,%d", &L, &W, &Sx) == 3 && (L == 8 || L == 16 || L == 64) &&
            (W == 4 || W == 8) && Sx >= 1 && Sx <= kMaxSplits) {
            const int c2 = (total_chunks + Sx - 1) / Sx;
            const long lds = (static_cast<long>(mr) * c2 * kChunkK + static_cast<long>(W) * mr * kVec * L) * 4;
            if (lds <= 60 * 1024) {
                cfg.L = L;
                cfg.W = W;
                cfg.chunks_per_split = c2;
                cfg.splits = (total_chunks + c2 - 1) / c2;
            }
        }
    }
    return cfg;
}

template <int KIND, int MR, int L, int W>
int launch_cfg(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k, int n,
               int block_size, const GemvConfig& cfg, hipStream_t stream) {
    const int tiles = (n + kVec * L - 1) / (kVec * L);
    Workspace ws{};
    if (cfg.splits > 1) {
        VM_TRY(get_workspace(stream, static_cast<std::size_t>(cfg.splits) * MR * n,
                             static_cast<std::size_t>(tiles), &ws));
    }
    const std::size_t lds = (static_cast<std::size_t>(MR) * cfg.chunks_per_split * kChunkK +
                             static_cast<std::size_t>(W) * MR * kVec * L) * sizeof(float);
    const int64_t byte_rows = KIND == 2 ? (static_cast<int64_t>(k) + 1) / 2 : k;
    const int64_t nblk = KIND == 0 ? 1 : (static_cast<int64_t>(k) + block_size - 1) / block_size;
    const uint32_t code_bytes = static_cast<uint32_t>(byte_rows * n);
    const uint32_t scale_bytes = static_cast<uint32_t>(KIND == 0 ? 0 : nblk * n * 4);
    // Chunk -> scale block is a shift when block_size / 8 is a power of two.
    int blk_shift = -1;
    if (KIND != 0) {
        const int cpb = block_size / kChunkK;
        if ((cpb & (cpb - 1)) == 0) blk_shift = __builtin_ctz(static_cast<unsigned>(cpb));
    }
    hipLaunchKernelGGL((qmm_gemv_kernel<KIND, MR, L, W>), dim3(tiles, cfg.splits), dim3(W * 64), lds,
                       stream, a, wq, scale, c, m, k, n, block_size, cfg.chunks_per_split, code_bytes,
                       scale_bytes, blk_shift, ws.partials, ws.counters);
    return check_launch("QuantizedMatMul", stream);
}

template <int KIND, int MR>
int launch_mr(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k, int n,
              int block_size, hipStream_t stream) {
    const GemvConfig cfg = choose_config(KIND, m, k, n);
#define VM_GEMV_CASE(LL, WW)                                                                    \
    if (cfg.L == LL && cfg.W == WW)                                                             \
        return launch_cfg<KIND, MR, LL, WW>(a, wq, scale, c, m, k, n, block_size, cfg, stream);
    VM_GEMV_CASE(8, 4)
    VM_GEMV_CASE(8, 8)
    VM_GEMV_CASE(16, 4)
    VM_GEMV_CASE(16, 8)
    VM_GEMV_CASE(64, 4)
    VM_GEMV_CASE(64, 8)
#undef VM_GEMV_CASE
    return VM_HIP_EUNSUPPORTED;
}

template <int KIND>
int launch_kind(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k, int n,
                int block_size, hipStream_t stream) {
    if (m == 1) return launch_mr<KIND, 1>(a, wq, scale, c, m, k, n, block_size, stream);
    if (m == 2) return launch_mr<KIND, 2>(a, wq, scale, c, m, k, n, block_size, stream);
    return launch_mr<KIND, 4>(a, wq, scale, c, m, k, n, block_size, stream);
}

}  // namespace

int gemv_qmm_f32(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k,
                 int n, int quant_type, int block_size, hipStream_t stream) {
    if (m < 1 || m > 4) return VM_HIP_EUNSUPPORTED;
    // Buffer offsets are 32-bit: codes and scales must stay below 2 GiB.
    if (static_cast<int64_t>(k) * n >= (int64_t(1) << 31)) return VM_HIP_EUNSUPPORTED;
    // 16-byte code loads need 16-byte aligned rows; scales are read as float4.
    if (n % kVec != 0 || reinterpret_cast<uintptr_t>(wq) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(scale) % 16 != 0)
        return VM_HIP_EUNSUPPORTED;
    if (quant_type == VM_HIP_QUANT_INT4) {
        if (block_size <= 0 || block_size % kChunkK != 0) return VM_HIP_EUNSUPPORTED;
        return launch_kind<2>(a, wq, scale, c, m, k, n, block_size, stream);
    }
    if (block_size > 0) {
        if (block_size % kChunkK != 0) return VM_HIP_EUNSUPPORTED;
        return launch_kind<1>(a, wq, scale, c, m, k, n, block_size, stream);
    }
    return launch_kind<0>(a, wq, scale, c, m, k, n, 0, stream);
}

}  // namespace vmhip
