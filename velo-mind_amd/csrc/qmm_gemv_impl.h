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
//   split     : grid.y splits K; the splits' sums meet in a binary tree of
//               64-bit pair words (atomic OR with return), summed in a fixed
//               grouping, so results do not depend on scheduling
//
// Reduction: row groups of a wave combine with VALU cross-lane operations
// (DPP row rotations inside 16-lane rows, then the gfx950 permlane16/32
// swaps across rows and wave halves), the waves of a workgroup through LDS,
// splits through the pair words in the per-stream workspace.  The pair
// words are agent-scope atomics (coherent across XCDs), so no L2 write-back,
// invalidate or barrier is needed, and no workgroup waits for another.
//
// Dequantization: INT8 codes are sign-extended bytes (v_cvt_f32_i32 with an
// SDWA byte select).  An INT4 byte holds the even K row in its low nibble;
// moving each nibble to the top of a byte ((w << 4) & 0xF0.. and w & 0xF0..)
// makes the signed byte equal 16*code, so the same SDWA convert applies; the
// sums then carry a factor 16, taken out (exactly, a power of two) once per
// output when the waves' sums are added, not once per chunk and column.
//
// Shared by qmm_gemv.hip (the plain kernels) and qmm_gemv_fx.hip (the
// fused ones: an addend, RMSNorm or SwiGLU activations); each translation
// unit instantiates its own half, so the two compile side by side.
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "qmm_kernels.h"
#include "vm_device.h"
#include "vm_internal.h"

namespace vmhip {
namespace {

constexpr int kChunkK = 8;    // logical K rows per chunk
constexpr int kVec = 16;      // columns per lane
constexpr int kMaxSplits = 32;
constexpr int kStageBatch = 4;  // activation loads in flight per thread while staging

// Phase timestamps, compiled in only with -DVM_GEMV_TRACE (build.py:
// VELOMIND_GEMV_TRACE=1): thread 0 of each of the first kGemvTraceWgs
// workgroups (linear id y * gridDim.x + x) keeps the 100 MHz wall clock at
//   0 kernel entry          1 first weight load issued
//   2 chunk and activations in (after the staging barrier)
//   3 its wave's chunks reduced   4 the waves' sums in LDS (barrier)
//   5 done: outputs or its pair words written and complete
// in registers and stores them when it ends (each launch overwrites the
// previous one's), read back with vm_hip_gemv_trace_read.  The traced
// build waits for its stores before the last mark.  Each translation unit
// holds its own copy of the buffer; the reader (qmm_gemv.hip) sees the plain
// kernels' marks only.
constexpr int kGemvTraceWgs = 4096;
constexpr int kGemvTraceEvents = 8;
#ifdef VM_GEMV_TRACE
__device__ unsigned long long g_gemv_trace[kGemvTraceWgs * kGemvTraceEvents];
#define VM_GEMV_MARKS unsigned long long gemv_ts[kGemvTraceEvents] = {}
#define VM_GEMV_MARK(ev) gemv_ts[ev] = wall_clock64()
#define VM_GEMV_END()                                                                               \
    do {                                                                                            \
        __builtin_amdgcn_s_waitcnt(0);                                                              \
        __syncthreads();                                                                            \
        gemv_ts[5] = wall_clock64();                                                                \
        const unsigned wg_ = blockIdx.y * gridDim.x + blockIdx.x;                                   \
        if (threadIdx.x == 0 && wg_ < kGemvTraceWgs)                                                \
            for (int e_ = 0; e_ < kGemvTraceEvents; ++e_) g_gemv_trace[wg_ * kGemvTraceEvents + e_] = gemv_ts[e_]; \
    } while (0)
#else
#define VM_GEMV_MARKS \
    do {              \
    } while (0)
#define VM_GEMV_MARK(ev) \
    do {                 \
    } while (0)
#define VM_GEMV_END() \
    do {              \
    } while (0)
#endif

template <int KIND>
struct ChunkShape {
    static constexpr bool kInt4 = KIND == 2;
    static constexpr int kRows = kInt4 ? kChunkK / 2 : kChunkK;  // byte rows per chunk
    static constexpr bool kScaled = KIND != 0;
};

// v rotated right by `off` lanes inside each 16-lane row (DPP row_ror).
__device__ __forceinline__ float dpp_row_ror(float v, int off) {
    const int ctrl = 0x120 | off;  // row_ror:off, off in 1..15
    int r = 0;
    switch (ctrl) {
        case 0x121: r = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x121, 0xf, 0xf, false); break;
        case 0x122: r = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x122, 0xf, 0xf, false); break;
        case 0x124: r = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x124, 0xf, 0xf, false); break;
        default: r = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xf, 0xf, false); break;
    }
    return __int_as_float(r);
}

// The matrices one launch multiplies by the same activations (a group of
// sibling projections such as q | k | v): their tiles are numbered one
// after the other, member g owning tiles [tile_end[g-1], tile_end[g]), and
// the split-K pair words index the members' columns side by side
// (col_base[g] + column, n_total in all).  A single matrix is a group of
// one.  Members are picked with selects on a workgroup-uniform index:
// indexing the argument arrays would copy them to scratch memory.
constexpr int kMaxMembers = 4;

struct GemvMembers {
    const uint8_t* wq[kMaxMembers];
    const float* scale[kMaxMembers];
    float* c[kMaxMembers];
    int n[kMaxMembers];
    int col_base[kMaxMembers];
    int tile_end[kMaxMembers];
    uint32_t code_bytes[kMaxMembers];
    uint32_t scale_bytes[kMaxMembers];
    int count;
    int n_total;
};

template <class T>
__device__ __forceinline__ T pick(const T (&v)[kMaxMembers], int g) {
    T r = v[0];
#pragma unroll
    for (int i = 1; i < kMaxMembers; ++i) r = g == i ? v[i] : r;
    return r;
}

// Codes and scales of one chunk for one lane.
template <int KIND>
struct Chunk {
    u32x4 w[ChunkShape<KIND>::kRows];
    u32x4 s[ChunkShape<KIND>::kScaled ? 4 : 1];
};

// KIND: 0 = INT8 per-column scale, 1 = INT8 blockwise, 2 = INT4 blockwise.
// MR: activation rows (1, 2 or 4); L: lanes per row segment; W: waves.
// GROUPED: several members (one launch for sibling projections); a single
// matrix runs the GROUPED = false copy, which reads member 0's fields only
// (each argument it reads is a scalar load on the path to the first code
// load: the member table costs ~0.6 us per launch when it is searched).
// What a fused launch adds to the product (FX kernels only): C = addend +
// product; A RMS-normalized first (norm_w); A the SwiGLU product of A (the
// gate) and a_up.  Not norm_w and a_up together.
struct GemvExtras {
    const float* addend = nullptr;   // [m, n] (a launch of one matrix only)
    const float* norm_w = nullptr;   // [k]
    float norm_eps = 0.0f;
    const float* a_up = nullptr;     // [m, k]
};

template <int KIND, int MR, int L, int W, bool GROUPED, bool FX>
__device__ __forceinline__ void gemv_body(
    const float* __restrict__ a, const GemvMembers& mb, int m, int k, int block_size, int chunks_per_split,
    uint32_t a_bytes, int a_vec, int blk_shift, unsigned long long* __restrict__ pairs, const GemvExtras& fx) {
    VM_GEMV_MARKS;
    VM_GEMV_MARK(0);
    using CS = ChunkShape<KIND>;
    constexpr int G = 64 / L;            // row groups per wave
    constexpr int RG = W * G;            // row groups per workgroup
    constexpr int kTileCols = kVec * L;

    extern __shared__ __align__(16) float smem[];
    float* xs = smem;                                     // [MR][chunks_per_split * 8]
    const int xs_len = chunks_per_split * kChunkK;
    float* red = smem + MR * xs_len;                      // [W][MR][kTileCols]
    float* spare = red + W * MR * kTileCols;              // [4], write-only

    // Every argument on the path to the first weight load, requested in one
    // batch of scalar loads: left to itself the compiler issues a second,
    // dependent batch after the tile renumbering below, one more kernel-
    // argument round trip (0.1-0.3 us when the weight stream has evicted the
    // arguments from L2) before any weight is requested.
    if constexpr (!GROUPED)
        asm volatile("" ::"s"(mb.wq[0]), "s"(mb.scale[0]), "s"(mb.n[0]), "s"(mb.code_bytes[0]),
                     "s"(mb.scale_bytes[0]), "s"(k), "s"(block_size), "s"(chunks_per_split), "s"(blk_shift),
                     "s"(gridDim.x));

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int rg = wave * G + lane / L;                   // row group in the workgroup
    // Workgroups are dispatched to the 8 XCDs round-robin by linear id, and
    // each XCD has its own L2.  Tiles are renumbered so that each XCD owns a
    // contiguous run of them: neighbouring tiles share 128-byte code and scale
    // lines, which are then fetched into one L2 instead of several.
    int tile = blockIdx.x;
    {
        const int full = static_cast<int>(gridDim.x) & ~7;
        if (tile < full) tile = (tile & 7) * (full >> 3) + (tile >> 3);
    }
    // the member this tile belongs to, and the tile within it
    int member = 0;
    if constexpr (GROUPED) {
#pragma unroll
        for (int g = 1; g < kMaxMembers; ++g) member += (g < mb.count && tile >= mb.tile_end[g - 1]) ? 1 : 0;
        int first = 0;
#pragma unroll
        for (int g = 1; g < kMaxMembers; ++g) first = member == g ? mb.tile_end[g - 1] : first;
        tile -= first;
    }
    const uint8_t* __restrict__ wq = pick(mb.wq, member);
    const float* __restrict__ scale = pick(mb.scale, member);
    float* __restrict__ c = pick(mb.c, member);
    const int n = pick(mb.n, member);
    const int col_base = pick(mb.col_base, member);
    const uint32_t code_bytes = pick(mb.code_bytes, member);
    const uint32_t scale_bytes = pick(mb.scale_bytes, member);
    const int n_total = GROUPED ? mb.n_total : n;
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
            float sv[kVec];
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) sv[4 * q + e] = __uint_as_float(cur.s[q][e]);
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

    // Memory requests in the order their results are needed: the RMSNorm
    // operands and the first batch of this split's activations (one batch of
    // kStageBatch buffer loads per thread covers 4 * 4 * W * 64 elements),
    // then the first chunk's codes and scales.  Loads complete in issue
    // order, so the staging, the norm and their barriers wait only for the
    // activations (an L2 hit when the producer just wrote them) and run while
    // the weights are still in flight from HBM.  Loads outside a row's
    // [0, k) use an offset past the buffer and read zeros.  With k % 4 == 0
    // and a 16-byte aligned A (a_vec) each load covers four elements that
    // all lie inside one row; otherwise each covers one element.
    Chunk<KIND> ca, cb;
    int ch = c_begin + rg;
    VM_GEMV_MARK(1);

    // RMSNorm (fx.norm_w non-null): the row's sum of squares over all k
    // with rmsnorm_kernel's arithmetic (256 threads striding the row with an
    // fma chain, xor butterflies, the four waves' sums in order), then each
    // staged element scaled as that kernel scales it, (x * inv) * w: bit for
    // bit the separate RMSNorm.  The first kNormRegs elements of this
    // thread's stride of each row are requested before everything else, the
    // sum is reduced while the weights are in flight, and the staging stores
    // write the scaled values (norm_w is loaded beside the activations).
    // 1024-thread workgroups (at most 128 VGPRs) keep no such registers:
    // they would spill, so they read the row in the sum's loop.
    constexpr int kNormRegs = W >= 16 ? 0 : 8;
    const bool norm = FX && fx.norm_w != nullptr;
    float nv[MR][kNormRegs > 0 ? kNormRegs : 1];
    if constexpr (FX) {
        if (norm) {
            const __amdgpu_buffer_rsrc_t ars = buffer_rsrc(a, a_bytes);
#pragma unroll
            for (int r = 0; r < MR; ++r)
#pragma unroll
                for (int j = 0; j < kNormRegs; ++j) {
                    const int i = static_cast<int>(threadIdx.x) + 256 * j;
                    const uint32_t off = (threadIdx.x < 256 && r < m && i < k)
                                             ? (static_cast<uint32_t>(r) * static_cast<uint32_t>(k) + i) * 4u
                                             : a_bytes;
                    nv[r][j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ars, static_cast<int>(off), 0, 0));
                }
        }
    }
    __shared__ float norm_part[FX ? MR : 1][4];
    // Each row's 1/rms once the waves' partial sums are in norm_part, in a
    // vector register: rows picked at run time read it without the array
    // going to scratch.
    float __attribute__((ext_vector_type(4))) inv = {0.0f, 0.0f, 0.0f, 0.0f};
    static_assert(MR <= 4, "one 1/rms lane per row");
    auto norm_sum = [&] {
        if constexpr (FX) {
#pragma unroll
            for (int r = 0; r < MR; ++r) {
                float sq = 0.0f;
                if (r < m && threadIdx.x < 256) {
#pragma unroll
                    for (int j = 0; j < kNormRegs; ++j)
                        if (static_cast<int>(threadIdx.x) + 256 * j < k) sq = fmaf(nv[r][j], nv[r][j], sq);
                    for (int i = threadIdx.x + 256 * kNormRegs; i < k; i += 256) {
                        const float v = a[static_cast<int64_t>(r) * k + i];
                        sq = fmaf(v, v, sq);
                    }
                }
                for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off, 64);
                if (r < m && threadIdx.x < 256 && lane == 0) norm_part[r][wave] = sq;
            }
        }
    };
    auto norm_inv = [&] {
        if constexpr (FX) {
#pragma unroll
            for (int r = 0; r < MR; ++r) {
                float tot = 0.0f;
                if (r < m)
#pragma unroll
                    for (int w = 0; w < 4; ++w) tot += norm_part[r][w];
                inv[r] = 1.0f / sqrtf(tot / static_cast<float>(k) + fx.norm_eps);
            }
        }
    };
    auto inv_of = [&](int r) { return MR == 1 ? inv[0] : inv[r]; };

    {
        // With a_up the staged activation is the SwiGLU product of a (gate)
        // and a_up, silu_mul_f32 per element (the elementwise kernels'
        // rounding); out-of-range reads give zeros for both, hence 0.
        const __amdgpu_buffer_rsrc_t ars = buffer_rsrc(a, a_bytes);
        const __amdgpu_buffer_rsrc_t urs = buffer_rsrc(FX && fx.a_up ? fx.a_up : a, a_bytes);
        // The second operand of each staged element, at most one: a_up (same
        // offset as a) or norm_w (the element's column).  One load from a
        // resource chosen here keeps the two from looking like competing
        // writes of one register, which would cost a wait for every load.
        const uint32_t nw_bytes = static_cast<uint32_t>(k) * 4u;
        const bool up = FX && fx.a_up;
        const bool two = up || norm;
        const __amdgpu_buffer_rsrc_t rs2 = norm ? buffer_rsrc(fx.norm_w, nw_bytes) : urs;
        constexpr int T = W * 64;
        // Prologue shared by both layouts: the weights requested after the
        // first batch, the norm's partial sums published with one barrier
        // and each row's 1/rms computed before any staged value is written.
        auto after_first_issue = [&] {
            load_chunk(ch, ca);
            if (norm) {
                norm_sum();
                __syncthreads();
                norm_inv();
            }
        };
        if (a_vec) {
            const int q_per_row = xs_len / 4;  // xs_len is a multiple of 8
            const int q_total = MR * q_per_row;
            u32x4 t[kStageBatch], tu[kStageBatch];
            int row[kStageBatch];
            auto issue = [&](int q0) {
#pragma unroll
                for (int u = 0; u < kStageBatch; ++u) {
                    const int q = q0 + u * T;
                    int r = 0;  // q / q_per_row for MR <= 4, without a division
#pragma unroll
                    for (int i = 1; i < MR; ++i) r += q >= i * q_per_row ? 1 : 0;
                    row[u] = r;
                    const int kk = k_begin + 4 * (q - r * q_per_row);
                    const bool in = q < q_total && r < m && kk < k;
                    const uint32_t off =
                        in ? (static_cast<uint32_t>(r) * static_cast<uint32_t>(k) + kk) * 4u : a_bytes;
                    // A wave whose lanes all lie past the slice requests
                    // nothing: its loads would only queue ahead of the
                    // weights' (plain kernels: TinyLlama gate/up 6.10 ->
                    // 5.86 us, down 6.81 -> 6.33; the fused ones measured
                    // 0.15-0.23 us slower with the branch and keep every load).
                    const bool live = FX || q - lane < q_total;
                    t[u] = live ? buffer_load16(ars, off) : u32x4{0u, 0u, 0u, 0u};
                    if (two)
                        tu[u] = live ? buffer_load16(rs2, norm ? (in ? static_cast<uint32_t>(kk) * 4u : nw_bytes) : off)
                                     : u32x4{0u, 0u, 0u, 0u};
                }
            };
            auto store = [&](int q0) {
                if (up)
#pragma unroll
                    for (int u = 0; u < kStageBatch; ++u)
#pragma unroll
                        for (int c = 0; c < 4; ++c)
                            t[u][c] = __float_as_uint(silu_mul_f32(__uint_as_float(t[u][c]), __uint_as_float(tu[u][c])));
                if (norm)
#pragma unroll
                    for (int u = 0; u < kStageBatch; ++u) {
                        const float ir = inv_of(row[u]);
#pragma unroll
                        for (int c = 0; c < 4; ++c)
                            t[u][c] = __float_as_uint((__uint_as_float(t[u][c]) * ir) * __uint_as_float(tu[u][c]));
                    }
                // Unconditional writes (surplus ones go to a spare LDS slot)
                // keep the compiler from sinking loads into per-write branches.
#pragma unroll
                for (int u = 0; u < kStageBatch; ++u) {
                    const int q = q0 + u * T;
                    *reinterpret_cast<u32x4*>(q < q_total ? xs + 4 * q : spare) = t[u];
                }
            };
            issue(threadIdx.x);
            after_first_issue();
            store(threadIdx.x);
            for (int q0 = threadIdx.x + kStageBatch * T; q0 < q_total; q0 += kStageBatch * T) {
                issue(q0);
                store(q0);
            }
        } else {
            const int e_total = MR * xs_len;
            uint32_t t[kStageBatch], tu[kStageBatch];
            int row[kStageBatch];
            auto issue = [&](int e0) {
#pragma unroll
                for (int u = 0; u < kStageBatch; ++u) {
                    const int e = e0 + u * T;
                    int r = 0;
#pragma unroll
                    for (int i = 1; i < MR; ++i) r += e >= i * xs_len ? 1 : 0;
                    row[u] = r;
                    const int kk = k_begin + (e - r * xs_len);
                    const bool in = e < e_total && r < m && kk < k;
                    const uint32_t off =
                        in ? (static_cast<uint32_t>(r) * static_cast<uint32_t>(k) + kk) * 4u : a_bytes;
                    t[u] = __builtin_amdgcn_raw_buffer_load_b32(ars, static_cast<int>(off), 0, 0);
                    if (two)
                        tu[u] = __builtin_amdgcn_raw_buffer_load_b32(
                            rs2, static_cast<int>(norm ? (in ? static_cast<uint32_t>(kk) * 4u : nw_bytes) : off), 0, 0);
                }
            };
            auto store = [&](int e0) {
                if (up)
#pragma unroll
                    for (int u = 0; u < kStageBatch; ++u)
                        t[u] = __float_as_uint(silu_mul_f32(__uint_as_float(t[u]), __uint_as_float(tu[u])));
                if (norm)
#pragma unroll
                    for (int u = 0; u < kStageBatch; ++u)
                        t[u] = __float_as_uint((__uint_as_float(t[u]) * inv_of(row[u])) * __uint_as_float(tu[u]));
#pragma unroll
                for (int u = 0; u < kStageBatch; ++u) {
                    const int e = e0 + u * T;
                    *(e < e_total ? xs + e : spare) = __uint_as_float(t[u]);
                }
            };
            issue(threadIdx.x);
            after_first_issue();
            store(threadIdx.x);
            for (int e0 = threadIdx.x + kStageBatch * T; e0 < e_total; e0 += kStageBatch * T) {
                issue(e0);
                store(e0);
            }
        }
    }
    __syncthreads();
    VM_GEMV_MARK(2);

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
    VM_GEMV_MARK(3);

    // Row groups of a wave (lanes that agree in lane % L) are summed with
    // VALU cross-lane operations, then each wave leaves one copy of its
    // tile's sums in LDS for the cross-wave step.
    static_assert(L == 1 || L == 2 || L == 4 || L == 8 || L == 16, "L must divide a 16-lane row");
    {
        // 1. inside each 16-lane row: rotations by L, 2L, .., 8 (DPP row_ror)
#pragma unroll
        for (int off = L; off < 16; off <<= 1)
#pragma unroll
            for (int i = 0; i < MR; ++i)
#pragma unroll
                for (int j = 0; j < kVec; ++j) total[i][j] += dpp_row_ror(total[i][j], off);
        // 2. row pairs: swapping columns j and j + 8 leaves even rows with
        //    the sum of column j and odd rows with the sum of column j + 8
        float h[MR][8];
#pragma unroll
        for (int i = 0; i < MR; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) h[i][j] = swap_rows_add(total[i][j], total[i][j + 8]);
        // 3. wave halves: columns j and j + 4 of step 2, same pattern
        float z[MR][4];
#pragma unroll
        for (int i = 0; i < MR; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) z[i][j] = swap_halves_add(h[i][j], h[i][j + 4]);
        // lane holds columns 8 * row-parity + 4 * half + (0..3) of its
        // 16-column group lane % L; one lane per group and row writes.
        if ((lane & 15) < L) {
            const int cc = (lane & 15) * kVec + 8 * ((lane >> 4) & 1) + 4 * (lane >> 5);
#pragma unroll
            for (int i = 0; i < MR; ++i)
                *reinterpret_cast<float4*>(red + (wave * MR + i) * kTileCols + cc) =
                    make_float4(z[i][0], z[i][1], z[i][2], z[i][3]);
        }
    }
    __syncthreads();
    VM_GEMV_MARK(4);

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
                if constexpr (CS::kInt4) v *= 0.0625f;  // INT4 sums carry 16 * code
                if constexpr (KIND == 0) v *= scale[col];
                if constexpr (FX)
                    if (fx.addend) v = fx.addend[static_cast<int64_t>(i) * n + col] + v;
                c[static_cast<int64_t>(i) * n + col] = v;
            }
        }
        VM_GEMV_END();
        return;
    }

    // Split-K handoff through a binary tree of pair words: one 64-bit word
    // per output and tree node, zero between launches.  At level l the
    // subtrees of 2^l splits are paired: each side ORs its sum, encoded as
    // its fp32 bits with the sign bit flipped (never 0 once -0 is turned
    // into +0), into its half of the node's word.  The side whose atomic
    // returns the other half already set adds the two in split order,
    // clears the word and moves up; the other side is done.  The root's
    // holder writes C.  One atomic round trip per level, no barrier and no
    // wait on another workgroup; the grouping of the sum is fixed by the
    // tree, so results do not depend on scheduling.
    for (int o = threadIdx.x; o < MR * kTileCols; o += W * 64) {
        const int i = o / kTileCols;
        const int cc = o - i * kTileCols;
        const int col = tile_col0 + cc;
        if (i >= m || col >= n) continue;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) v += red[(w * MR + i) * kTileCols + cc];
        if constexpr (CS::kInt4) v *= 0.0625f;
        bool last = true;
        int64_t level_base = 0;
        for (int lvl = 0; (1 << lvl) < splits; ++lvl) {
            const int node = split >> (lvl + 1);
            const int half = (split >> lvl) & 1;
            // A lower half whose upper partner lies past the last split
            // moves up alone.
            if (half == 1 || ((2 * node + 1) << lvl) < splits) {
                unsigned long long* word =
                    pairs + level_base + (static_cast<int64_t>(node) * MR + i) * n_total + col_base + col;
                const unsigned enc = __float_as_uint(v + 0.0f) ^ 0x80000000u;
                const unsigned long long mine = half ? static_cast<unsigned long long>(enc) << 32 : enc;
                const unsigned long long old =
                    __hip_atomic_fetch_or(word, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const unsigned other = half ? static_cast<unsigned>(old) : static_cast<unsigned>(old >> 32);
                if (other == 0u) {
                    last = false;
                    break;
                }
                __hip_atomic_store(word, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const float po = __uint_as_float(other ^ 0x80000000u);
                v = half ? po + v : v + po;
            }
            level_base += static_cast<int64_t>((splits + (2 << lvl) - 1) >> (lvl + 1)) * MR * n_total;
        }
        if (!last) continue;
        if constexpr (KIND == 0) v *= scale[col];
        if constexpr (FX)
            if (fx.addend) v = fx.addend[static_cast<int64_t>(i) * n + col] + v;
        c[static_cast<int64_t>(i) * n + col] = v;
    }
    VM_GEMV_END();
}

// The plain launch, and the fused one (FX: addend, RMSNorm or SwiGLU
// activations); the plain kernel carries none of the fused code.
template <int KIND, int MR, int L, int W, bool GROUPED>
__global__ __launch_bounds__(W * 64) void qmm_gemv_kernel(
    const float* __restrict__ a, const GemvMembers mb, int m, int k, int block_size, int chunks_per_split,
    uint32_t a_bytes, int a_vec, int blk_shift, unsigned long long* __restrict__ pairs) {
    gemv_body<KIND, MR, L, W, GROUPED, false>(a, mb, m, k, block_size, chunks_per_split, a_bytes, a_vec, blk_shift,
                                              pairs, GemvExtras{});
}

template <int KIND, int MR, int L, int W, bool GROUPED>
__global__ __launch_bounds__(W * 64) void qmm_gemv_fx_kernel(
    const float* __restrict__ a, const GemvMembers mb, int m, int k, int block_size, int chunks_per_split,
    uint32_t a_bytes, int a_vec, int blk_shift, unsigned long long* __restrict__ pairs, const GemvExtras fx) {
    gemv_body<KIND, MR, L, W, GROUPED, true>(a, mb, m, k, block_size, chunks_per_split, a_bytes, a_vec, blk_shift,
                                             pairs, fx);
}

// Pair words of every level of the split tree (level l has
// ceil(splits / 2^(l+1)) nodes), per activation row and column.
std::size_t tree_words(int splits, int mr, int n) {
    std::size_t nodes = 0;
    for (int lvl = 0; (1 << lvl) < splits; ++lvl)
        nodes += static_cast<std::size_t>((splits + (2 << lvl) - 1) >> (lvl + 1));
    return nodes * static_cast<std::size_t>(mr) * static_cast<std::size_t>(n);
}

struct GemvConfig {
    int L = 16;
    int W = 4;
    int splits = 1;
    int chunks_per_split = 0;
};

int mr_for(int m) { return m <= 1 ? 1 : (m <= 2 ? 2 : 4); }

// Largest wave count whose register budget (512 / W * 4 VGPRs per lane)
// holds the kernel without spilling: MR x 16 accumulators, two chunks of
// codes and scales in flight.
constexpr int max_waves(int kind, int mr) {
    return (kind == 0 && mr == 1) ? 16 : (kind == 1 && mr == 4) ? 4 : 8;
}

// (L, W) pairs the kernel is instantiated for.
constexpr int kShapes[][2] = {{1, 4}, {2, 4}, {2, 8}, {4, 4}, {4, 8}, {8, 4}, {8, 8}, {16, 4}, {16, 8}, {16, 16}};

bool instantiated(int L, int W) {
    for (const auto& lw : kShapes)
        if (lw[0] == L && lw[1] == W) return true;
    return false;
}

struct Geometry {
    int tiles, cps, splits, row_groups, iters, wgs;
    long lds_bytes;
};

Geometry geometry(int mr, int k, int n, int L, int W, int S) {
    Geometry g{};
    const int chunks = (k + kChunkK - 1) / kChunkK;
    g.tiles = (n + kVec * L - 1) / (kVec * L);
    g.cps = (chunks + S - 1) / S;
    g.splits = (chunks + g.cps - 1) / g.cps;
    g.row_groups = W * 64 / L;
    g.iters = (g.cps + g.row_groups - 1) / g.row_groups;
    g.wgs = g.tiles * g.splits;
    g.lds_bytes = (static_cast<long>(mr) * g.cps * kChunkK + static_cast<long>(W) * mr * kVec * L + 4) * 4;
    return g;
}

GemvConfig make_config(int mr, int k, int n, int L, int W, int S) {
    const Geometry g = geometry(mr, k, n, L, W, S);
    GemvConfig cfg;
    cfg.L = L;
    cfg.W = W;
    cfg.splits = g.splits;
    cfg.chunks_per_split = g.cps;
    return cfg;
}

constexpr long kLdsBudget = 60 * 1024;

// Picks lanes-per-segment L, waves W and K splits S for a shape.  The rule
// follows a sweep of every instantiated (L, W) and S in 1..32 over the
// TinyLlama-1.1B INT4 and SmolLM2 INT8 decode shapes on MI355X, where it
// lands within 0.25 us of the per-shape best:
//   - latency-bound shapes (every row group needs at most one chunk with
//     16- or 32-column tiles and no K split, at most 256 workgroups) run
//     unsplit on narrow tiles;
//   - wide outputs (N >= 192 * 128) run unsplit on 128- or 256-column tiles,
//     about one workgroup per CU or more, each row group streaming several
//     chunks;
//   - everything else splits K so that every row group holds exactly one
//     chunk (all loads in flight at once), on tiles of at least 64 (INT4) or
//     32 (INT8) columns, with at most 256 workgroups of at most 64 KB (INT4)
//     or 32 KB (INT8) of codes each, and takes the fewest tree levels, then
//     the fewest waves (idle row groups cost time), then the narrowest tile
//     (with 2-4 activation rows, four waves on those tiles and splits);
//   - larger shapes that none of these fit are bandwidth-bound: wide tiles
//     and enough workgroups to fill the GPU (70B-class projections, e.g.
//     28672 x 8192 INT4: 3.6 -> 4.1 TB/s against the previous fallback).
// The config depends only on the shape, so results are reproducible.
GemvConfig choose_config(int kind, int m, int k, int n) {
    const int mr = mr_for(m);
    const int chunks = (k + kChunkK - 1) / kChunkK;
    const int w_max = max_waves(kind, mr);
    const int min_cols = kind == 2 ? 64 : 32;
    const long max_wg_bytes = kind == 2 ? 64 * 1024 : 32 * 1024;
    const int rows_per_chunk = kind == 2 ? kChunkK / 2 : kChunkK;  // code byte rows
    GemvConfig cfg;
    bool found = false;

    for (int L : {1, 2}) {
        const Geometry g = geometry(mr, k, n, L, 4, 1);
        if (chunks <= g.row_groups && g.tiles <= 256 && g.lds_bytes <= kLdsBudget) {
            cfg = make_config(mr, k, n, L, 4, 1);
            found = true;
            break;
        }
    }
    if (!found && n >= 192 * 128) {
        const int L = (n + 127) / 128 <= 256 ? 8 : 16;
        // 256-column tiles over a long K stream best with four waves
        // (8192 x 128256 INT4: 5.1 -> 5.5 TB/s); short K keeps more waves.
        const int W = (L == 16 && k >= 4096) ? 4 : std::min(L, w_max);
        int S = 1;
        while (S < kMaxSplits && geometry(mr, k, n, L, W, S).lds_bytes > kLdsBudget) S *= 2;
        cfg = make_config(mr, k, n, L, W, S);
        found = true;
    }
    if (!found) {
        long best_key = 0;
        for (const auto& lw : kShapes) {
            const int L = lw[0], W = lw[1];
            if (W > std::min(8, w_max) || kVec * L < min_cols) continue;
            for (int S = 2, levels = 1; S <= kMaxSplits; S *= 2, ++levels) {
                const Geometry g = geometry(mr, k, n, L, W, S);
                const long wg_bytes = static_cast<long>(g.cps) * rows_per_chunk * kVec * L;
                if (g.splits != S || g.iters != 1 || g.wgs > 256 || g.lds_bytes > kLdsBudget ||
                    wg_bytes > max_wg_bytes)
                    continue;
                const long key = (static_cast<long>(levels) * 64 + W) * 64 + L;
                if (!found || key < best_key) {
                    best_key = key;
                    cfg = make_config(mr, k, n, L, W, S);
                    found = true;
                }
            }
        }
        // Two or four activation rows: the same tiles and splits on four
        // waves, each row group taking two chunks (M = 2 / 4, TinyLlama
        // gate 2048 x 5632: 7.49 -> 7.14 / 9.24 -> 8.64 us; down 5632 x 2048:
        // 8.15 -> 7.83 / 9.99 -> 9.40 us).
        if (found && mr >= 2 && cfg.W == 8 && geometry(mr, k, n, cfg.L, 4, cfg.splits).lds_bytes <= kLdsBudget)
            cfg = make_config(mr, k, n, cfg.L, 4, cfg.splits);
    }
    if (!found) {
        // Bandwidth-bound shapes (tens of MB and more): 128-column tiles
        // (256 for N >= 14336), four waves, and the fewest splits that give
        // at least 192 workgroups; each row group streams many chunks.
        const int L = n >= 14336 ? 16 : 8;
        const int W = 4;
        int S = 1;
        while (S < kMaxSplits && (geometry(mr, k, n, L, W, S).wgs < 192 ||
                                  geometry(mr, k, n, L, W, S).lds_bytes > kLdsBudget))
            S *= 2;
        if (geometry(mr, k, n, L, W, S).lds_bytes <= kLdsBudget) {
            cfg = make_config(mr, k, n, L, W, S);
            found = true;
        }
    }
    if (!found) cfg = make_config(mr, k, n, 8, 4, kMaxSplits);

    // Tuning override for measurement sweeps: VELOMIND_GEMV_CFG="L,W,S".
    if (const char* env = std::getenv("VELOMIND_GEMV_CFG")) {
        int L = 0, W = 0, Sx = 0;
        if (std::sscanf(env, "%d,%d,%d", &L, &W, &Sx) == 3 && instantiated(L, W) && W <= w_max &&
            Sx >= 1 && Sx <= kMaxSplits && geometry(mr, k, n, L, W, Sx).lds_bytes <= kLdsBudget)
            cfg = make_config(mr, k, n, L, W, Sx);
    }
    return cfg;
}

// One matrix of a group, as the launchers take it.
struct Member {
    const uint8_t* wq;
    const float* scale;
    float* c;
    int n;
};

template <int KIND, int MR, int L, int W, bool FX>
int launch_cfg(const float* a, const Member* members, int count, int m, int k, int block_size,
               const GemvConfig& cfg, const GemvExtras& fx, hipStream_t stream) {
    const int64_t byte_rows = KIND == 2 ? (static_cast<int64_t>(k) + 1) / 2 : k;
    const int64_t nblk = KIND == 0 ? 1 : (static_cast<int64_t>(k) + block_size - 1) / block_size;
    GemvMembers mb{};
    int tiles = 0, n_total = 0;
    for (int g = 0; g < count; ++g) {
        const int n = members[g].n;
        mb.wq[g] = members[g].wq;
        mb.scale[g] = members[g].scale;
        mb.c[g] = members[g].c;
        mb.n[g] = n;
        mb.col_base[g] = n_total;
        tiles += (n + kVec * L - 1) / (kVec * L);
        mb.tile_end[g] = tiles;
        mb.code_bytes[g] = static_cast<uint32_t>(byte_rows * n);
        mb.scale_bytes[g] = static_cast<uint32_t>(KIND == 0 ? 0 : nblk * n * 4);
        n_total += n;
    }
    mb.count = count;
    mb.n_total = n_total;
    Workspace ws{};
    if (cfg.splits > 1)  // two 32-bit counter slots per pair word
        VM_TRY(get_workspace(stream, 0, 2 * tree_words(cfg.splits, MR, n_total), &ws));
    unsigned long long* pairs = reinterpret_cast<unsigned long long*>(ws.counters);
    const std::size_t lds = (static_cast<std::size_t>(MR) * cfg.chunks_per_split * kChunkK +
                             static_cast<std::size_t>(W) * MR * kVec * L + 4) * sizeof(float);
    const uint32_t a_bytes = static_cast<uint32_t>(static_cast<int64_t>(m) * k * 4);
    // 16-byte activation loads: rows of a multiple of 4 elements and 16-byte
    // aligned operands (a_up and norm_w are read at the same offsets).
    const int a_vec = (k % 4 == 0 && reinterpret_cast<uintptr_t>(a) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(fx.a_up) % 16 == 0 && reinterpret_cast<uintptr_t>(fx.norm_w) % 16 == 0)
                          ? 1
                          : 0;
    // Chunk -> scale block is a shift when block_size / 8 is a power of two.
    int blk_shift = -1;
    if (KIND != 0) {
        const int cpb = block_size / kChunkK;
        if ((cpb & (cpb - 1)) == 0) blk_shift = __builtin_ctz(static_cast<unsigned>(cpb));
    }
    const dim3 grid(tiles, cfg.splits), block(W * 64);
    if constexpr (FX) {
        if (count == 1)
            hipLaunchKernelGGL((qmm_gemv_fx_kernel<KIND, MR, L, W, false>), grid, block, lds, stream, a, mb, m, k,
                               block_size, cfg.chunks_per_split, a_bytes, a_vec, blk_shift, pairs, fx);
        else
            hipLaunchKernelGGL((qmm_gemv_fx_kernel<KIND, MR, L, W, true>), grid, block, lds, stream, a, mb, m, k,
                               block_size, cfg.chunks_per_split, a_bytes, a_vec, blk_shift, pairs, fx);
    } else {
        (void)fx;
        if (count == 1)
            hipLaunchKernelGGL((qmm_gemv_kernel<KIND, MR, L, W, false>), grid, block, lds, stream, a, mb, m, k,
                               block_size, cfg.chunks_per_split, a_bytes, a_vec, blk_shift, pairs);
        else
            hipLaunchKernelGGL((qmm_gemv_kernel<KIND, MR, L, W, true>), grid, block, lds, stream, a, mb, m, k,
                               block_size, cfg.chunks_per_split, a_bytes, a_vec, blk_shift, pairs);
    }
    return check_launch("QuantizedMatMul", stream);
}

template <int KIND, int MR, bool FX>
int launch_mr(const float* a, const Member* members, int count, int m, int k, int n_total, int block_size,
              const GemvExtras& fx, hipStream_t stream) {
    const GemvConfig cfg = choose_config(KIND, m, k, n_total);
#define VM_GEMV_CASE(LL, WW)                                                                    \
    if constexpr (WW <= max_waves(KIND, MR))                                                    \
        if (cfg.L == LL && cfg.W == WW)                                                         \
            return launch_cfg<KIND, MR, LL, WW, FX>(a, members, count, m, k, block_size, cfg, fx, stream);
    VM_GEMV_CASE(1, 4)
    VM_GEMV_CASE(2, 4)
    VM_GEMV_CASE(2, 8)
    VM_GEMV_CASE(4, 4)
    VM_GEMV_CASE(4, 8)
    VM_GEMV_CASE(8, 4)
    VM_GEMV_CASE(8, 8)
    VM_GEMV_CASE(16, 4)
    VM_GEMV_CASE(16, 8)
    VM_GEMV_CASE(16, 16)
#undef VM_GEMV_CASE
    return VM_HIP_EUNSUPPORTED;
}

template <int KIND, bool FX>
int launch_kind(const float* a, const Member* members, int count, int m, int k, int n_total, int block_size,
                const GemvExtras& fx, hipStream_t stream) {
    if (m == 1) return launch_mr<KIND, 1, FX>(a, members, count, m, k, n_total, block_size, fx, stream);
    if (m == 2) return launch_mr<KIND, 2, FX>(a, members, count, m, k, n_total, block_size, fx, stream);
    return launch_mr<KIND, 4, FX>(a, members, count, m, k, n_total, block_size, fx, stream);
}

// One launch for `count` matrices sharing the activations; VM_HIP_EUNSUPPORTED
// when any member needs another kernel.
template <bool FX>
int gemv_group_f32(const float* a, const Member* members, int count, int m, int k, int quant_type,
                   int block_size, const GemvExtras& fx, hipStream_t stream) {
    if (m < 1 || m > 4 || count < 1 || count > kMaxMembers) return VM_HIP_EUNSUPPORTED;
    int64_t n_total = 0;
    for (int g = 0; g < count; ++g) {
        const Member& mm = members[g];
        // Buffer offsets are 32-bit: codes and scales must stay below 2 GiB.
        if (mm.n < 1 || static_cast<int64_t>(k) * mm.n >= (int64_t(1) << 31)) return VM_HIP_EUNSUPPORTED;
        // 16-byte code loads need 16-byte aligned rows; scales are read as float4.
        if (mm.n % kVec != 0 || reinterpret_cast<uintptr_t>(mm.wq) % 16 != 0 ||
            reinterpret_cast<uintptr_t>(mm.scale) % 16 != 0)
            return VM_HIP_EUNSUPPORTED;
        n_total += mm.n;
    }
    if (n_total >= (int64_t(1) << 30)) return VM_HIP_EUNSUPPORTED;
    const int nt = static_cast<int>(n_total);
    if (quant_type == VM_HIP_QUANT_INT4) {
        if (block_size <= 0 || block_size % kChunkK != 0) return VM_HIP_EUNSUPPORTED;
        return launch_kind<2, FX>(a, members, count, m, k, nt, block_size, fx, stream);
    }
    if (block_size > 0) {
        if (block_size % kChunkK != 0) return VM_HIP_EUNSUPPORTED;
        return launch_kind<1, FX>(a, members, count, m, k, nt, block_size, fx, stream);
    }
    return launch_kind<0, FX>(a, members, count, m, k, nt, 0, fx, stream);
}

}  // namespace
}  // namespace vmhip
