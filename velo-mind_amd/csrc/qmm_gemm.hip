// Prefill-shaped (rows_m > 4) quantized matmul on gfx950 MFMA
// (v_mfma_f32_16x16x32_f16, fp32 accumulation).
//
// C[M, N] = A[M, K] * W[K, N] with W given as the reference's codes (INT8
// [K, N] or INT4 packed [(K+1)/2, N], N contiguous) and fp32 scales.
//
// A is first split once per call (a_split_f16_kernel): each row r is
// multiplied by 2^x_r, the power of two that puts its largest magnitude in
// [2^14, 2^15), and written as two fp16 parts hi = fp16(a * 2^x_r) and
// lo = fp16(a * 2^x_r - hi), so that hi + lo carries 22 significant bits of
// any finite fp32 row without overflow or underflow.  Both parts go through
// the MFMAs (products with the exact fp16 codes are exact, accumulation is
// fp32), and the epilogue multiplies by 2^-x_r, which is exact: the
// activations are used at fp32-equivalent precision.
//
// Pipeline (per workgroup: a BM x BN output tile, four waves, K in steps of
// 64 rows):
//   global -> registers  raw buffer loads (zeros past the end), two steps
//                        ahead of the MFMAs;
//   registers -> LDS     A: the hi and lo parts as loaded, row-major [BM][64];
//                        B: codes -> fp16 with packed-half magic numbers
//                        (0x6400 | (code ^ 0x80..) is 1024 + 128 + code),
//                        times the block scale, stored in the codes' own
//                        layout [64][BN] (N contiguous, 16-byte writes);
//   LDS -> MFMA          A operand: ds_read_b128 of 8 consecutive k;
//                        B operand: two ds_read_b64_tr_b16 transposed reads
//                        give each lane 8 consecutive k of one column.
// Columns are kept in the order (c0, c2, c1, c3) inside every group of four
// in LDS (the order the magic-number unpacking produces); the epilogue
// writes each result to its true column.
//
// Scales.  INT8 per column: applied in the epilogue (fp32).  Blockwise
// (INT4, INT8 with block_size > 0): B is staged as fp16(code * s / 2^e),
// where 2^e is a per-column power of two with max_s / 2^e in [0.5, 1) over
// the workgroup's K range, and the fp32 result is multiplied by 2^e (exact).
// The normalisation keeps every staged weight inside fp16's normal range
// whatever the scales' magnitude.  Beyond fp32 accumulation the only
// rounding is then (code * s / 2^e) -> fp16 for blockwise weights (relative
// 2^-11, a fixed function of the weights) and A's split (relative 2^-22);
// INT8 per-column codes are exact and their scales apply in fp32.
//
// Split-K for small M: each split stores its scaled partial tile
// with agent-scope stores, the last split of a tile (atomic ticket) adds
// the partials in split order and writes C, so results are deterministic.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "qmm_kernels.h"
#include "vm_device.h"
#include "vm_internal.h"

namespace vmhip {
namespace {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));

constexpr int kBK = 64;         // K rows per pipeline step
constexpr int kThreads = 256;   // four waves
// LDS row padding (halves).  Measured on MI355X (M = 512, K = 2048, N =
// 5632): A rows padded by 16 halves have 20% fewer bank conflicts than by
// 8; B padding of 8, 16 or 32 makes no difference, none doubles the time.
constexpr int kApad = 16;       // halves of padding per LDS row of A
constexpr int kBpad = 16;       // halves of padding per LDS row of B
constexpr int kMaxSplits = 16;

typedef __attribute__((address_space(3))) short4v lds_short4;

__device__ __forceinline__ half4v lds_read_tr16(const _Float16* p) {
    // Generic -> LDS address space: the low 32 bits of a generic LDS pointer
    // are the LDS offset.
    auto* lp = (lds_short4*)(uintptr_t)(uint32_t)(uintptr_t)p;
    return __builtin_bit_cast(half4v, __builtin_amdgcn_ds_read_tr16_b64_v4i16(lp));
}

__device__ __forceinline__ uint32_t pk_f16(float lo, float hi) {
    const half2v h = {static_cast<_Float16>(lo), static_cast<_Float16>(hi)};
    return __builtin_bit_cast(uint32_t, h);
}

__device__ __forceinline__ uint32_t hmul2(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, a) * __builtin_bit_cast(half2v, b));
}

__device__ __forceinline__ uint32_t hsub2(uint32_t a, _Float16 b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, a) - half2v{b, b});
}

// KIND: 0 = INT8 per-column, 1 = INT8 blockwise, 2 = INT4 blockwise.
template <int KIND, int BM, int BN, int WAVES_M, int WAVES_N>
struct Tile {
    static constexpr bool kInt4 = KIND == 2;
    static constexpr bool kBlock = KIND != 0;
    static constexpr int WM = BM / WAVES_M;
    static constexpr int WN = BN / WAVES_N;
    static constexpr int TM = WM / 16;
    static constexpr int TN = WN / 16;
    static constexpr int kArow = kBK + kApad;                  // halves per A row
    static constexpr int kBrow = BN + kBpad;                   // halves per B k-row
    static constexpr int kAPieces = BM * (kBK / 8);            // 8 halves (16 bytes) each
    static constexpr int kAPass = (kAPieces + kThreads - 1) / kThreads;
    static constexpr int kBRows = kInt4 ? kBK / 2 : kBK;       // code byte rows per step
    static constexpr int kBPieces = kBRows * (BN / 16);        // 16 bytes each
    static constexpr int kBPass = (kBPieces + kThreads - 1) / kThreads;
    static constexpr int kQB = BN / 4;                         // column quads
    static constexpr int kRedRows = kThreads / kQB;
    static_assert(WAVES_M * WAVES_N == 4, "four waves");
    static_assert(TM >= 1 && TN >= 1 && WM % 16 == 0 && WN % 16 == 0, "16x16 MFMA tiles");
    static_assert(BN % 16 == 0 && kThreads % kQB == 0, "tile shape");
};

template <int KIND, int BM, int BN, int WAVES_M, int WAVES_N>
struct Stage {
    using T = Tile<KIND, BM, BN, WAVES_M, WAVES_N>;
    u32x4 a[T::kAPass];
    u32x4 al[T::kAPass];
    u32x4 b[T::kBPass];
    u32x4 s[T::kBlock ? T::kBPass : 1][T::kBlock ? 4 : 1];
};

// DEEP = 0: a two-step register pipeline over the split's K steps.
// DEEP > 0 (small M, at most DEEP steps per split): every step's loads are
// issued before the first MFMA, so the workgroup waits for one memory round
// trip instead of one per pipeline step.
template <int KIND, int BM, int BN, int WAVES_M, int WAVES_N, int DEEP>
__global__ __launch_bounds__(kThreads, BM >= 128 ? 1 : 2) void qmm_mfma_kernel(
    const _Float16* __restrict__ a, const int* __restrict__ row_exp, const uint8_t* __restrict__ wq,
    const float* __restrict__ scale, float* __restrict__ c, int m, int k, int n, int block_size,
    int steps_per_split, int tiles_n, int tiles_m,
    uint32_t a_bytes, uint32_t lo_offset, uint32_t code_bytes, uint32_t scale_bytes, float* __restrict__ partials,
    unsigned* __restrict__ counters) {
    using T = Tile<KIND, BM, BN, WAVES_M, WAVES_N>;
    using S = Stage<KIND, BM, BN, WAVES_M, WAVES_N>;

    __shared__ __attribute__((aligned(16))) _Float16 sA[2][BM * T::kArow];
    __shared__ __attribute__((aligned(16))) _Float16 sAl[2][BM * T::kArow];
    __shared__ __attribute__((aligned(16))) _Float16 sB[2][kBK * T::kBrow];
    __shared__ float sPow[T::kBlock ? BN : 1];   // 2^e per column (physical order)
    __shared__ float sInv[T::kBlock ? BN : 1];   // 2^-e
    // The scale-normalisation scratch lives in the second B buffer: it is
    // used (and released by a barrier) before any B step is written there.
    float* sRed = reinterpret_cast<float*>(sB[1]);
    static_assert(!T::kBlock || T::kRedRows * BN * 4 <= kBK * T::kBrow * 2, "sRed fits in a B buffer");
    __shared__ unsigned ticket;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N;
    const int wn = wave % WAVES_N;
    // One-dimensional grid over (split, tile row, tile column), column
    // fastest.  Workgroups go to the 8 XCDs round-robin by id; renumbering
    // gives each XCD a contiguous run, so the workgroups sharing one L2
    // mostly share one A panel (the operand every column tile re-reads).
    int lin = blockIdx.x;
    {
        const int full = static_cast<int>(gridDim.x) & ~7;
        if (lin < full) lin = (lin & 7) * (full >> 3) + (lin >> 3);
    }
    const int tile_x = lin % tiles_n;
    const int tile_y = (lin / tiles_n) % tiles_m;
    const int split = lin / (tiles_n * tiles_m);
    const int splits = static_cast<int>(gridDim.x) / (tiles_n * tiles_m);
    const int n0 = tile_x * BN;
    const int m0 = tile_y * BM;
    const int total_steps = (k + kBK - 1) / kBK;
    const int step0 = split * steps_per_split;
    const int nsteps = min(total_steps, step0 + steps_per_split) - step0;
    const int k_begin = step0 * kBK;
    const int k_end = min(k, k_begin + nsteps * kBK);

    const __amdgpu_buffer_rsrc_t ars = buffer_rsrc(a, a_bytes);
    const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(wq, code_bytes);
    const __amdgpu_buffer_rsrc_t srs = buffer_rsrc(scale, scale_bytes);

    // ---- per-column normalisation of block scales over this split's K range
    auto normalise_scales = [&]() {
        if constexpr (T::kBlock) {
            const int b0 = k_begin / block_size;
            const int b1 = (k_end + block_size - 1) / block_size;
            const int q = tid % T::kQB;
            float mx[4] = {0.f, 0.f, 0.f, 0.f};
            for (int b = b0 + tid / T::kQB; b < b1; b += 4 * T::kRedRows) {
                u32x4 v[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int bb = b + u * T::kRedRows;
                    const uint32_t off = bb < b1 ? (static_cast<uint32_t>(bb) * n + n0 + 4 * q) * 4u : scale_bytes;
                    v[u] = buffer_load16(srs, off);
                }
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int e = 0; e < 4; ++e) mx[e] = fmaxf(mx[e], fabsf(__uint_as_float(v[u][e])));
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) sRed[(tid / T::kQB) * BN + 4 * q + e] = mx[e];
            __syncthreads();
            if (tid < BN) {
                float mm = 0.f;
#pragma unroll
                for (int r = 0; r < T::kRedRows; ++r) mm = fmaxf(mm, sRed[r * BN + tid]);
                int e = 0;
                if (mm > 0.f && mm <= 3.0e38f) (void)frexpf(mm, &e);
                sPow[tid] = ldexpf(1.0f, e);
                sInv[tid] = ldexpf(1.0f, -e);
            }
            __syncthreads();
        }
    };
    if constexpr (DEEP == 0) normalise_scales();

    // ---- global -> registers for one step
    auto load_step = [&](int s, S& st) {
        const int k0 = (step0 + s) * kBK;
#pragma unroll
        for (int p = 0; p < T::kAPass; ++p) {
            const int piece = tid + p * kThreads;
            const int row = piece / (kBK / 8);
            const int kk = k0 + 8 * (piece % (kBK / 8));
            const bool ok = piece < T::kAPieces && m0 + row < m && kk < k_end;
            const uint32_t off = (static_cast<uint32_t>(m0 + row) * k + kk) * 2u;
            st.a[p] = buffer_load16(ars, ok ? off : a_bytes);
            st.al[p] = buffer_load16(ars, ok ? off + lo_offset : a_bytes);
        }
#pragma unroll
        for (int p = 0; p < T::kBPass; ++p) {
            const int piece = tid + p * kThreads;
            const int row = piece / (BN / 16);            // code byte row within the step
            const int col = n0 + 16 * (piece % (BN / 16));
            const int krow = T::kInt4 ? k0 / 2 + row : k0 + row;
            const int klog = T::kInt4 ? k0 + 2 * row : k0 + row;   // first logical K row of the piece
            const bool ok = piece < T::kBPieces && klog < k_end;
            st.b[p] = buffer_load16(wrs, ok ? static_cast<uint32_t>(krow) * n + col : code_bytes);
            if constexpr (T::kBlock) {
                const uint32_t blk = static_cast<uint32_t>(klog) / static_cast<uint32_t>(block_size);
                const uint32_t soff = ok ? (blk * n + col) * 4u : scale_bytes;
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) st.s[p][qd] = buffer_load16(srs, soff + 16u * qd);
            }
        }
    };

    // ---- registers -> fp16 registers (VALU only) -> LDS
    struct Packed {
        u32x4 a[T::kAPass];
        u32x4 al[T::kAPass];
        u32x4 b[T::kBPass][T::kInt4 ? 4 : 2];
    };
    auto convert_step = [&](const S& st, Packed& pk) {
#pragma unroll
        for (int p = 0; p < T::kAPass; ++p) {
            pk.a[p] = st.a[p];
            pk.al[p] = st.al[p];
        }
#pragma unroll
        for (int p = 0; p < T::kBPass; ++p) {
            const int piece = tid + p * kThreads;
            const int cl = 16 * (piece % (BN / 16));      // local column of the piece
            // normalised scales, paired in (c0, c2), (c1, c3) order per quad
            uint32_t sn[8];
            if constexpr (T::kBlock) {
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) {
                    const float* inv = sInv + cl + 4 * qd;
                    sn[2 * qd] = pk_f16(__uint_as_float(st.s[p][qd][0]) * inv[0], __uint_as_float(st.s[p][qd][2]) * inv[2]);
                    sn[2 * qd + 1] = pk_f16(__uint_as_float(st.s[p][qd][1]) * inv[1], __uint_as_float(st.s[p][qd][3]) * inv[3]);
                }
            }
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                if constexpr (T::kInt4) {
                    const uint32_t x = st.b[p][d] ^ 0x88888888u;
                    uint32_t e02 = hsub2((x & 0x000F000Fu) | 0x64006400u, static_cast<_Float16>(1032.0f));
                    uint32_t e13 = hsub2(((x >> 8) & 0x000F000Fu) | 0x64006400u, static_cast<_Float16>(1032.0f));
                    uint32_t o02 = hsub2(((x >> 4) & 0x000F000Fu) | 0x64006400u, static_cast<_Float16>(1032.0f));
                    uint32_t o13 = hsub2(((x >> 12) & 0x000F000Fu) | 0x64006400u, static_cast<_Float16>(1032.0f));
                    // b[p][0..1]: even K row, 16 columns; b[p][2..3]: odd K row
                    pk.b[p][d / 2][2 * (d % 2)] = hmul2(e02, sn[2 * d]);
                    pk.b[p][d / 2][2 * (d % 2) + 1] = hmul2(e13, sn[2 * d + 1]);
                    pk.b[p][2 + d / 2][2 * (d % 2)] = hmul2(o02, sn[2 * d]);
                    pk.b[p][2 + d / 2][2 * (d % 2) + 1] = hmul2(o13, sn[2 * d + 1]);
                } else {
                    const uint32_t x = st.b[p][d] ^ 0x80808080u;
                    uint32_t e02 = hsub2((x & 0x00FF00FFu) | 0x64006400u, static_cast<_Float16>(1152.0f));
                    uint32_t e13 = hsub2(((x >> 8) & 0x00FF00FFu) | 0x64006400u, static_cast<_Float16>(1152.0f));
                    if constexpr (T::kBlock) {
                        e02 = hmul2(e02, sn[2 * d]);
                        e13 = hmul2(e13, sn[2 * d + 1]);
                    }
                    pk.b[p][d / 2][2 * (d % 2)] = e02;
                    pk.b[p][d / 2][2 * (d % 2) + 1] = e13;
                }
            }
        }
    };
    auto write_step = [&](const Packed& pk, int buf) {
        _Float16* la = sA[buf];
        _Float16* lal = sAl[buf];
        _Float16* lb = sB[buf];
#pragma unroll
        for (int p = 0; p < T::kAPass; ++p) {
            const int piece = tid + p * kThreads;
            if (piece < T::kAPieces) {
                const int row = piece / (kBK / 8);
                const int kc = 8 * (piece % (kBK / 8));
                *reinterpret_cast<u32x4*>(la + row * T::kArow + kc) = pk.a[p];
                *reinterpret_cast<u32x4*>(lal + row * T::kArow + kc) = pk.al[p];
            }
        }
#pragma unroll
        for (int p = 0; p < T::kBPass; ++p) {
            const int piece = tid + p * kThreads;
            if (piece >= T::kBPieces) continue;
            const int row = piece / (BN / 16);
            const int cl = 16 * (piece % (BN / 16));
            if constexpr (T::kInt4) {
                _Float16* r0 = lb + (2 * row) * T::kBrow + cl;
                _Float16* r1 = r0 + T::kBrow;
                *reinterpret_cast<u32x4*>(r0) = pk.b[p][0];
                *reinterpret_cast<u32x4*>(r0 + 8) = pk.b[p][1];
                *reinterpret_cast<u32x4*>(r1) = pk.b[p][2];
                *reinterpret_cast<u32x4*>(r1 + 8) = pk.b[p][3];
            } else {
                _Float16* r0 = lb + row * T::kBrow + cl;
                *reinterpret_cast<u32x4*>(r0) = pk.b[p][0];
                *reinterpret_cast<u32x4*>(r0 + 8) = pk.b[p][1];
            }
        }
    };
    auto store_step = [&](const S& st, int buf) {
        Packed pk;
        convert_step(st, pk);
        write_step(pk, buf);
    };

    floatx4 acc[T::TM][T::TN];
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
        for (int j = 0; j < T::TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    const int fr = lane & 15;        // fragment row (A) / column (B)
    const int fg = lane >> 4;        // 8-k group
    struct Frags {
        half8v a[T::TM];
        half8v al[T::TM];
        half8v b[T::TN];
    };
    auto read_frags = [&](int buf, int kh, Frags& f) {
        const _Float16* la = sA[buf];
        const _Float16* lal = sAl[buf];
        const _Float16* lb = sB[buf];
#pragma unroll
        for (int i = 0; i < T::TM; ++i) {
            const int off = (wm * T::WM + i * 16 + fr) * T::kArow + kh * 32 + 8 * fg;
            f.a[i] = *reinterpret_cast<const half8v*>(la + off);
            f.al[i] = *reinterpret_cast<const half8v*>(lal + off);
        }
#pragma unroll
        for (int j = 0; j < T::TN; ++j) {
            // lane L of each 16-lane group points at row base + L/4,
            // columns 4 * (L % 4) .. + 3: the transposed read returns,
            // for lane i, rows base .. base + 3 of column i.
            const _Float16* p = lb + (kh * 32 + 8 * fg + (fr >> 2)) * T::kBrow + wn * T::WN + j * 16 + 4 * (fr & 3);
            const half4v lo = lds_read_tr16(p);
            const half4v hi = lds_read_tr16(p + 4 * T::kBrow);
            f.b[j] = half8v{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
    };
    auto mfma_frags = [&](const Frags& f) {
#pragma unroll
        for (int i = 0; i < T::TM; ++i)
#pragma unroll
            for (int j = 0; j < T::TN; ++j)
            {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.al[i], f.b[j], acc[i][j], 0, 0, 0);
            }
    };
    // One pipeline step: all fragment reads of the current buffer are issued
    // first, the next stage is converted in registers while they are in
    // flight, the MFMAs follow, and the converted stage is written to the
    // other buffer while the MFMAs drain.
    auto step = [&](int cur, const S& next_raw) {
        Frags f0, f1;
        read_frags(cur, 0, f0);
        read_frags(cur, 1, f1);
        Packed pk;
        convert_step(next_raw, pk);
        mfma_frags(f0);
        mfma_frags(f1);
        write_step(pk, cur ^ 1);
    };

    if constexpr (DEEP > 0) {
        // ---- all of the split's steps in flight (nsteps <= DEEP; steps past
        // the split read zeros), then the LDS double buffer as below.  The
        // vector-memory counter retires loads in issue order, so each step
        // is released as soon as its own loads are in.
        S st[DEEP];
#pragma unroll
        for (int s = 0; s < DEEP; ++s) load_step(s, st[s]);
        normalise_scales();   // its scale loads queue behind the steps' loads
        store_step(st[0], 0);
        __syncthreads();
#pragma unroll
        for (int s = 0; s < DEEP; ++s) {
            if (s >= nsteps) break;
            if (s + 1 < DEEP) {
                step(s & 1, st[s + 1]);
            } else {
                Frags f0, f1;
                read_frags(s & 1, 0, f0);
                read_frags(s & 1, 1, f1);
                mfma_frags(f0);
                mfma_frags(f1);
            }
            __syncthreads();
        }
    } else {
        // ---- main loop: LDS double buffer, register stages two steps ahead.
        // Loads and stores are unconditional (steps past the end read zeros):
        // with a fixed number of loads per iteration the compiler's vmcnt
        // waits release each stage as soon as its own loads are in, leaving
        // the next stage's loads in flight.
        S st0, st1;
        load_step(0, st0);
        load_step(1, st1);
        store_step(st0, 0);
        load_step(2, st0);
        __syncthreads();
        for (int s = 0; s < nsteps; s += 2) {
            step(0, st1);
            __syncthreads();
            load_step(s + 3, st1);
            if (s + 1 >= nsteps) break;
            step(1, st0);
            __syncthreads();
            load_step(s + 4, st0);
        }
    }

    // ---- epilogue.  D layout: lane holds rows 4 * (lane / 16) + e, column
    // lane % 16 of each 16x16 tile (LDS column order).
    auto col_of = [&](int j) {
        const int nl = wn * T::WN + j * 16 + fr;
        return (nl & ~3) | ((nl & 1) << 1) | ((nl >> 1) & 1);   // (c0, c2, c1, c3) -> physical
    };
    float colscale[T::TN];
#pragma unroll
    for (int j = 0; j < T::TN; ++j) {
        const int cp = col_of(j);
        if constexpr (T::kBlock) {
            colscale[j] = sPow[cp];
        } else {
            colscale[j] = __uint_as_float(buffer_load4(srs, (n0 + cp < n) ? static_cast<uint32_t>(n0 + cp) * 4u : scale_bytes));
        }
    }

    // 2^-x of each of the lane's rows undoes the staging scale (exact).
    int neg_exp[T::TM][4];
#pragma unroll
    for (int i = 0; i < T::TM; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int row = m0 + wm * T::WM + i * 16 + 4 * fg + e;
            neg_exp[i][e] = row < m ? -row_exp[row] : 0;
        }

    if (splits == 1) {
#pragma unroll
        for (int j = 0; j < T::TN; ++j) {
            const int col = n0 + col_of(j);
            if (col >= n) continue;
#pragma unroll
            for (int i = 0; i < T::TM; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int row = m0 + wm * T::WM + i * 16 + 4 * fg + e;
                    if (row < m)
                        c[static_cast<int64_t>(row) * n + col] = ldexpf(acc[i][j][e] * colscale[j], neg_exp[i][e]);
                }
        }
        return;
    }

    float* part = partials + static_cast<int64_t>(split) * m * n;
#pragma unroll
    for (int j = 0; j < T::TN; ++j) {
        const int col = n0 + col_of(j);
        if (col >= n) continue;
#pragma unroll
        for (int i = 0; i < T::TM; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int row = m0 + wm * T::WM + i * 16 + 4 * fg + e;
                if (row < m)
                    coherent_store(part + static_cast<int64_t>(row) * n + col,
                                   ldexpf(acc[i][j][e] * colscale[j], neg_exp[i][e]));
            }
    }
    publish_partials();
    __syncthreads();
    const int tile = tile_y * tiles_n + tile_x;
    if (tid == 0) ticket = ticket_take(&counters[tile], static_cast<unsigned>(splits));
    __syncthreads();
    if (ticket != static_cast<unsigned>(splits - 1)) return;
    const int64_t stride = static_cast<int64_t>(m) * n;
    for (int idx = tid; idx < BM * BN; idx += kThreads) {
        const int row = m0 + idx / BN;
        const int col = n0 + idx % BN;
        if (row >= m || col >= n) continue;
        const float* p = partials + static_cast<int64_t>(row) * n + col;
        float v = 0.f;
        for (int s0 = 0; s0 < splits; s0 += 8) {
            float t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) t[u] = s0 + u < splits ? coherent_load(p + (s0 + u) * stride) : 0.f;
#pragma unroll
            for (int u = 0; u < 8; ++u) v += t[u];
        }
        c[static_cast<int64_t>(row) * n + col] = v;
    }
    if (tid == 0) __hip_atomic_store(&counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// A [m, k] fp32 -> two fp16 parts with a power-of-two scale per row: x_r
// is chosen so that max_k |a[r, k]| * 2^x_r lies in [2^14, 2^15) (x_r = 0
// for an all-zero row, or one holding an infinity or NaN, which then
// reaches the output as the reference's fp32 arithmetic would propagate
// it); hi = fp16(a * 2^x_r) and lo = fp16(a * 2^x_r - hi), the difference
// being exact in fp32.  hi at ah[r * k + c], lo at ah[m * k + r * k + c].
// One workgroup per row.  Rows of up to kSplitHeld float4 groups per
// thread stay in registers between the maximum and the split (one read of
// A); longer rows are read a second time (from L2).
constexpr int kSplitHeld = 6;   // k <= 6144 in one read

__global__ __launch_bounds__(256) void a_split_f16_kernel(const float* __restrict__ a,
                                                          _Float16* __restrict__ ah,
                                                          int* __restrict__ row_exp, int m, int k, int vec) {
    __shared__ float wmax[4];
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const float* src = a + static_cast<int64_t>(row) * k;
    const int vecs = k >> 2;   // k % 32 == 0 on this path
    const bool held = vecs <= kSplitHeld * 256;
    auto load4 = [&](int v) {
        if (vec) return reinterpret_cast<const float4*>(src)[v];
        return make_float4(src[4 * v], src[4 * v + 1], src[4 * v + 2], src[4 * v + 3]);
    };
    float4 keep[kSplitHeld];
    float mx = 0.0f;
    bool special = false;
    auto scan = [&](const float4& x) {
        const float t = fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w)));
        special |= !(fabsf(x.x) <= 3.4028235e38f) || !(fabsf(x.y) <= 3.4028235e38f) ||
                   !(fabsf(x.z) <= 3.4028235e38f) || !(fabsf(x.w) <= 3.4028235e38f);
        mx = fmaxf(mx, t);
    };
    if (held) {
#pragma unroll
        for (int r = 0; r < kSplitHeld; ++r) {
            const int v = tid + r * 256;
            keep[r] = v < vecs ? load4(v) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int r = 0; r < kSplitHeld; ++r) scan(keep[r]);
    } else {
        for (int v = tid; v < vecs; v += 256) scan(load4(v));
    }
    // an infinity or NaN anywhere in the row disables the scaling
    if (special) mx = __builtin_inff();
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((tid & 63) == 0) wmax[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    int x = 0;
    if (mx > 0.0f && mx <= 3.4028235e38f) {
        int e = 0;
        (void)frexpf(mx, &e);   // mx = f * 2^e, f in [0.5, 1)
        x = 15 - e;
    }
    if (tid == 0) row_exp[row] = x;
    half4v* hi = reinterpret_cast<half4v*>(ah + static_cast<int64_t>(row) * k);
    half4v* lo = reinterpret_cast<half4v*>(ah + (static_cast<int64_t>(m) + row) * k);
    auto split = [&](int v, const float4& y) {
        const float s0 = ldexpf(y.x, x), s1 = ldexpf(y.y, x), s2 = ldexpf(y.z, x), s3 = ldexpf(y.w, x);
        const half4v h = {static_cast<_Float16>(s0), static_cast<_Float16>(s1), static_cast<_Float16>(s2),
                          static_cast<_Float16>(s3)};
        hi[v] = h;
        // an infinite part (|a| beyond fp16 in an unscaled row) leaves lo at 0
        auto rest = [](float s, _Float16 hh) {
            const float d = s - static_cast<float>(hh);
            return static_cast<_Float16>(d == d && fabsf(d) <= 65504.0f ? d : 0.0f);
        };
        lo[v] = half4v{rest(s0, h[0]), rest(s1, h[1]), rest(s2, h[2]), rest(s3, h[3])};
    };
    if (held) {
#pragma unroll
        for (int r = 0; r < kSplitHeld; ++r) {
            const int v = tid + r * 256;
            if (v < vecs) split(v, keep[r]);
        }
    } else {
        for (int v = tid; v < vecs; v += 256) split(v, load4(v));
    }
}

struct GemmConfig {
    int bm = 128, bn = 128, splits = 1, deep = 0;
};

// Tile and split choice, from sweeps of every tile variant and split count
// on MI355X over config-3 shapes (K = 2048, N = 5632, M = 16..512) and the
// TinyLlama / SmolLM2 prefill projections (M = 512: N = 2048..11264, K =
// 2048 and 5632; M = 128: K, N = 960..5120):
//   M <= 128: 32 x 64 tiles (many small workgroups hide load latency best);
//     K splits (at least four 64-row steps each) until about two workgroups
//     per CU, while the fp32 partials stay under a quarter of the code
//     bytes -- or, with fewer than 128 tiles, while each split keeps at
//     least eight steps; INT4 with M > 64 at least two splits;
//   M > 128: 64 x 128 tiles (M = 512, K = 2048, N = 5632, INT8, weights
//     cold: 51.2 us vs 64.2 with 64 x 64); K splits of at least twenty
//     64-row steps up to ~512 workgroups (K = 5632: 4 splits); 32 x 128
//     when an unsplit grid would hold fewer than 150 tiles (N = 2048).
GemmConfig choose_gemm(int kind, int m, int k, int n) {
    GemmConfig cfg;
    const int steps = (k + kBK - 1) / kBK;
    const double code_bytes = kind == 2 ? 0.5 * k * n : 1.0 * k * n;
    auto tiles_of = [&](int bm, int bn) {
        return static_cast<long>((m + bm - 1) / bm) * ((n + bn - 1) / bn);
    };
    int s = 1;
    if (m <= 128) {
        // M <= 16 (and INT8 M <= 32): 16-row tiles, no MFMA rows wasted on
        // padding.
        cfg.bm = (m <= 16 || (kind != 2 && m <= 32)) ? 16 : 32;
        cfg.bn = 64;
        const long tiles = tiles_of(cfg.bm, cfg.bn);
        while (s * 2 <= 8 && tiles * s * 2 <= 512 &&
               ((steps / (s * 2) >= 4 && 4.0 * s * 2 * m * n <= 0.25 * code_bytes) ||
                (tiles < 128 && steps / (s * 2) >= 8)))
            s *= 2;
        // INT4 with 64 < M <= 128: two K splits spread its heavier B
        // unpacking (K = 2048, N = 5632, M = 128, weights cold: 33.5 us vs
        // 38.1 unsplit, 38.4 with 64 x 64 tiles)
        if (kind == 2 && m > 64 && s == 1 && steps >= 16) s = 2;
    } else {
        cfg.bm = 64;
        cfg.bn = 128;
        const long tiles = tiles_of(cfg.bm, cfg.bn);
        while (s * 2 <= 4 && tiles * s * 2 <= 512 && steps / (s * 2) >= 20) s *= 2;
        if (s == 1 && tiles < 150) cfg.bm = 32;
    }
    cfg.splits = s;
    // M <= 32: every K step of a split in flight at once (8 steps INT8, 4
    // INT4, whose scale registers double a step's), with as many more splits
    // as that needs (at most kMaxSplits).  K = 2048, N = 5632: M = 16 INT8
    // 13.3 -> 10.9 us, INT4 15.5 -> 12.5; M = 32 INT8 15.7 -> 12.8.
    if (m <= 32) {
        const int deep = kind == 2 ? 4 : 8;
        const int need = (steps + deep - 1) / deep;
        if (need <= kMaxSplits) {
            cfg.deep = deep;
            cfg.splits = std::max(s, need);
        }
    }
    // Tuning override for measurement sweeps: VELOMIND_GEMM_CFG="BM,BN,S"
    // or "BM,BN,S,D" (D = steps in flight, 4 or 8, for 16 x 64 and 32 x 64).
    if (const char* env = std::getenv("VELOMIND_GEMM_CFG")) {
        int bm = 0, bn = 0, sx = 0, d = 0;
        const int got = std::sscanf(env, "%d,%d,%d,%d", &bm, &bn, &sx, &d);
        const bool deep_ok = d == 0 || ((d == 4 || d == 8) && bn == 64 && (bm == 16 || bm == 32) &&
                                        (steps + sx - 1) / sx <= d);
        if (got >= 3 && sx >= 1 && sx <= kMaxSplits && deep_ok &&
            ((bn == 128 && (bm == 16 || bm == 32 || bm == 64 || bm == 128)) ||
             (bn == 64 && (bm == 16 || bm == 32 || bm == 64)))) {
            cfg.bm = bm;
            cfg.bn = bn;
            cfg.splits = sx;
            cfg.deep = d;
        }
    }
    return cfg;
}

template <int KIND, int BM, int BN, int WAVES_M, int WAVES_N, int DEEP = 0>
int launch(const _Float16* a, const int* row_exp, const uint8_t* wq, const float* scale, float* c, int m, int k,
           int n, int block_size, int splits, hipStream_t stream) {
    const int tiles_n = (n + BN - 1) / BN;
    const int tiles_m = (m + BM - 1) / BM;
    const int steps = (k + kBK - 1) / kBK;
    const int sps = (steps + splits - 1) / splits;
    splits = (steps + sps - 1) / sps;
    Workspace ws{};
    if (splits > 1) {
        VM_TRY(get_workspace(stream, static_cast<std::size_t>(splits) * m * n,
                             static_cast<std::size_t>(tiles_m) * tiles_n, &ws));
    }
    const int64_t nblk = KIND == 0 ? 1 : (static_cast<int64_t>(k) + block_size - 1) / block_size;
    const uint32_t lo_offset = static_cast<uint32_t>(static_cast<int64_t>(m) * k * 2);
    const uint32_t a_bytes = 2u * lo_offset;   // hi, then lo
    const uint32_t code_bytes =
        static_cast<uint32_t>((KIND == 2 ? (static_cast<int64_t>(k) + 1) / 2 : static_cast<int64_t>(k)) * n);
    const uint32_t scale_bytes = static_cast<uint32_t>((KIND == 0 ? 1 : nblk) * n * 4);
    if (DEEP > 0 && sps > DEEP) return fail_inval("QuantizedMatMul: internal error: K steps per split exceed the pipeline depth");
    hipLaunchKernelGGL((qmm_mfma_kernel<KIND, BM, BN, WAVES_M, WAVES_N, DEEP>), dim3(tiles_n * tiles_m * splits),
                       dim3(kThreads), 0, stream, a, row_exp, wq, scale, c, m, k, n, block_size, sps, tiles_n, tiles_m,
                       a_bytes, lo_offset, code_bytes, scale_bytes, ws.partials, ws.counters);
    return check_launch("QuantizedMatMul", stream);
}

template <int KIND>
int launch_kind(const _Float16* a, const int* row_exp, const uint8_t* wq, const float* scale, float* c, int m,
                int k, int n, int block_size, hipStream_t stream) {
    const GemmConfig cfg = choose_gemm(KIND, m, k, n);
    if (cfg.deep == 8) {
        if (cfg.bm == 16) return launch<KIND, 16, 64, 1, 4, 8>(a, row_exp, wq, scale, c, m, k, n, block_size, cfg.splits, stream);
        return launch<KIND, 32, 64, 2, 2, 8>(a, row_exp, wq, scale, c, m, k, n, block_size, cfg.splits, stream);
    }
    if (cfg.deep == 4) {
        if (cfg.bm == 16) return launch<KIND, 16, 64, 1, 4, 4>(a, row_exp, wq, scale, c, m, k, n, block_size, cfg.splits, stream);
        return launch<KIND, 32, 64, 2, 2, 4>(a, row_exp, wq, scale, c, m, k, n, block_size, cfg.splits, stream);
    }
    if (cfg.bn == 64 && cfg.bm == 16) return launch<KIND, 16, 64, 1, 4>(a, row_exp, wq, scale, c, m, k, n, block_size, cfg.splits, stream);
    if (cfg.bn == 128) {
        if (cfg.bm == 16) return launch<KIND, 16, 128, 1, 4>(a, row_exp, wq, scale, c, m, k, n, block_size, cfg.splits, stream);
        if (cfg.bm == 32) return launch<KIND, 32, 128, 2, 2>(a, row_exp, wq, scale, c, m, k, n, block_size, cfg.splits, stream);
        if (cfg.bm == 64) return launch<KIND, 64, 128, 2, 2>(a, row_exp, wq, scale, c, m, k, n, block_size, cfg.splits, stream);
        return launch<KIND, 128, 128, 2, 2>(a, row_exp, wq, scale, c, m, k, n, block_size, cfg.splits, stream);
    }
    if (cfg.bm == 32) return launch<KIND, 32, 64, 2, 2>(a, row_exp, wq, scale, c, m, k, n, block_size, cfg.splits, stream);
    return launch<KIND, 64, 64, 2, 2>(a, row_exp, wq, scale, c, m, k, n, block_size, cfg.splits, stream);
}

}  // namespace

int gemm_qmm_f32(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k, int n,
                 int quant_type, int block_size, hipStream_t stream) {
    // 64-row steps may end half-way (k % 32 == 0); 16-byte code pieces need
    // whole 16-column groups; buffer offsets are 32-bit.
    if (k % 32 != 0 || n % 16 != 0) return VM_HIP_EUNSUPPORTED;
    // (A's two fp16 parts take m * k * 4 bytes, addressed with 32-bit offsets)
    if (static_cast<int64_t>(m) * k * 4 >= (int64_t(1) << 31) || static_cast<int64_t>(k) * n >= (int64_t(1) << 31) ||
        static_cast<int64_t>(m) * n * 4 * kMaxSplits >= (int64_t(1) << 40))
        return VM_HIP_EUNSUPPORTED;
    // one-dimensional grid of at most 2^30 workgroups
    if (((static_cast<int64_t>(m) + 15) / 16) * ((n + 63) / 64) * kMaxSplits >= (int64_t(1) << 30))
        return VM_HIP_EUNSUPPORTED;
    int kind = 0;
    if (quant_type == VM_HIP_QUANT_INT4) {
        if (block_size <= 0 || block_size % 32 != 0) return VM_HIP_EUNSUPPORTED;
        kind = 2;
    } else if (block_size > 0) {
        if (block_size % 32 != 0) return VM_HIP_EUNSUPPORTED;
        kind = 1;
    }
    // A's row-scaled fp16 parts (hi, lo) and row exponents, staged for this call.
    const std::size_t half_bytes = (static_cast<std::size_t>(m) * k * 4 + 255) & ~std::size_t(255);
    void* aux = nullptr;
    VM_TRY(get_aux(stream, half_bytes + static_cast<std::size_t>(m) * sizeof(int), &aux));
    auto* ah = static_cast<_Float16*>(aux);
    auto* row_exp = reinterpret_cast<int*>(static_cast<char*>(aux) + half_bytes);
    hipLaunchKernelGGL(a_split_f16_kernel, dim3(m), dim3(256), 0, stream, a, ah, row_exp, m, k,
                       reinterpret_cast<uintptr_t>(a) % 16 == 0 ? 1 : 0);
    VM_TRY(check_launch("QuantizedMatMul", stream));
    if (kind == 2) return launch_kind<2>(ah, row_exp, wq, scale, c, m, k, n, block_size, stream);
    if (kind == 1) return launch_kind<1>(ah, row_exp, wq, scale, c, m, k, n, block_size, stream);
    return launch_kind<0>(ah, row_exp, wq, scale, c, m, k, n, 0, stream);
}

}  // namespace vmhip
