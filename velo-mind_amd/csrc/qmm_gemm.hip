// Prefill-shaped (rows_m > 4) quantized matmul on gfx950 MFMA, fp32
// accumulation.
//
// C[M, N] = A[M, K] * W[K, N] with W given as the reference's codes (INT8
// [K, N] or INT4 packed [(K+1)/2, N], N contiguous) and fp32 scales.
//
// A is first split once per call (the prep kernels, or its producer, see
// a_split.h): each row r is multiplied by 2^x_r, the power of two that puts
// its largest magnitude in [2^14, 2^15), and written as two fp16 parts
// hi = fp16(a * 2^x_r) and lo = fp16(a * 2^x_r - hi), so that hi + lo
// carries 22 significant bits of any finite fp32 row without overflow or
// underflow.  Both parts go through the MFMAs (products with the exact fp16
// codes are exact, accumulation is fp32), and the epilogue multiplies by
// 2^-x_r, which is exact: the activations are used at fp32-equivalent
// precision.
//
// B: codes -> fp16 with packed-half magic numbers (0x6400 | (code ^ 0x80..)
// is 1024 + 128 + code), exact.  Scales: INT8 per column multiplies each
// fp32 result in the epilogue; blockwise scales (INT4, INT8 with block_size
// > 0) multiply each 32-row chunk's fp32 sum, which the wide kernel keeps in
// an accumulator of its own (the reference's per-block sum times the block
// scale, quantized_matmul.cpp:76-90).  Beyond fp32 accumulation the only
// rounding is A's split (relative 2^-22).
//
// Two kernels:
//   qmm_mfma_kernel (small tiles, v_mfma_f32_16x16x32_f16) takes per-column
//     INT8 with few rows;
//   wide::qmm_mfma_wide_kernel (v_mfma_f32_32x32x16_f16) takes more rows
//     and every blockwise call.
// Small-tile pipeline (per workgroup: a BM x BN output tile, four waves, K
// in steps of 64 rows):
//   global -> registers  raw buffer loads (zeros past the end), two steps
//                        ahead of the MFMAs;
//   registers -> LDS     A: the hi and lo parts as loaded, row-major [BM][64];
//                        B: fp16 codes in the codes' own layout [64][BN]
//                        (N contiguous, 16-byte writes);
//   LDS -> MFMA          A operand: ds_read_b128 of 8 consecutive k;
//                        B operand: two ds_read_b64_tr_b16 transposed reads
//                        give each lane 8 consecutive k of one column.
// Columns are kept in the order (c0, c2, c1, c3) inside every group of four
// in LDS (the order the magic-number unpacking produces); the epilogue
// writes each result to its true column.
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

#include "a_split.h"
#include "qmm_kernels.h"
#include "vm_device.h"
#include "vm_internal.h"

namespace vmhip {
namespace {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
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

__device__ __forceinline__ uint32_t hsub2(uint32_t a, _Float16 b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, a) - half2v{b, b});
}

// KIND: 0 = INT8 per-column (the only kind this kernel takes).
template <int KIND, int BM, int BN, int WAVES_M, int WAVES_N>
struct Tile {
    static_assert(KIND == 0, "the small-tile kernel takes per-column INT8 (blockwise scales: the wide kernel)");
    static constexpr int WM = BM / WAVES_M;
    static constexpr int WN = BN / WAVES_N;
    static constexpr int TM = WM / 16;
    static constexpr int TN = WN / 16;
    static constexpr int kArow = kBK + kApad;                  // halves per A row
    static constexpr int kBrow = BN + kBpad;                   // halves per B k-row
    static constexpr int kAPieces = BM * (kBK / 8);            // 8 halves (16 bytes) each
    static constexpr int kAPass = (kAPieces + kThreads - 1) / kThreads;
    static constexpr int kBRows = kBK;                         // code byte rows per step
    static constexpr int kBPieces = kBRows * (BN / 16);        // 16 bytes each
    static constexpr int kBPass = (kBPieces + kThreads - 1) / kThreads;
    static constexpr int kQB = BN / 4;                         // column quads
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
            const int krow = k0 + row;
            const bool ok = piece < T::kBPieces && krow < k_end;
            st.b[p] = buffer_load16(wrs, ok ? static_cast<uint32_t>(krow) * n + col : code_bytes);
        }
    };

    // ---- registers -> fp16 registers (VALU only) -> LDS
    struct Packed {
        u32x4 a[T::kAPass];
        u32x4 al[T::kAPass];
        u32x4 b[T::kBPass][2];
    };
    auto convert_step = [&](const S& st, Packed& pk) {
#pragma unroll
        for (int p = 0; p < T::kAPass; ++p) {
            pk.a[p] = st.a[p];
            pk.al[p] = st.al[p];
        }
#pragma unroll
        for (int p = 0; p < T::kBPass; ++p) {
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint32_t x = st.b[p][d] ^ 0x80808080u;
                pk.b[p][d / 2][2 * (d % 2)] = hsub2((x & 0x00FF00FFu) | 0x64006400u, static_cast<_Float16>(1152.0f));
                pk.b[p][d / 2][2 * (d % 2) + 1] =
                    hsub2(((x >> 8) & 0x00FF00FFu) | 0x64006400u, static_cast<_Float16>(1152.0f));
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
            _Float16* r0 = lb + row * T::kBrow + cl;
            *reinterpret_cast<u32x4*>(r0) = pk.b[p][0];
            *reinterpret_cast<u32x4*>(r0 + 8) = pk.b[p][1];
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
        colscale[j] = __uint_as_float(buffer_load4(srs, (n0 + cp < n) ? static_cast<uint32_t>(n0 + cp) * 4u : scale_bytes));
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
// being exact in fp32.
// FRAG = false: row-major, hi at ah[r * k + c], lo at ah[m * k + r * k + c]
// (the small-tile kernel).
// FRAG = true (the wide kernel): in the operand order of
// v_mfma_f32_32x32x16_f16, so that one wave's operand for 32 rows and 16 k
// is 1 KB of consecutive memory: the 16 bytes lane l of the wave loads for
// row block b (rows 32b .. 32b + 31) and k block q (k 16q .. 16q + 15) --
// row 32b + l % 32, k 16q + 8 (l / 32) + 0..7 -- sit at half offset
// ((b * k / 16 + q) * 64 + l) * 8; lo follows hi after mp * k halves, mp =
// m rounded up to 32.  Inside each 16-byte piece the halves are stored in
// the order k = 0, 4, 1, 5, 2, 6, 3, 7, the order in which the wide
// kernel's weight unpacking produces B (a dot product does not depend on
// the order of its terms, so A and B only have to agree).
//
// Workgroup r splits row r; rows of up to kSplitHeld groups of eight per
// thread stay in registers between the maximum and the split (one read of
// A), longer rows are read a second time (from L2).
constexpr int kSplitHeld = 3;   // k <= 6144 in one read

template <bool FRAG>
__global__ __launch_bounds__(256) void gemm_prep_kernel(const float* __restrict__ a, _Float16* __restrict__ ah,
                                                        int* __restrict__ row_exp, int m, int k, int vec) {
    __shared__ float wmax[4];
    const int tid = threadIdx.x;
    const int row = static_cast<int>(blockIdx.x);
    const float* src = a + static_cast<int64_t>(row) * k;
    const int groups = k >> 3;   // k % 32 == 0 on this path
    const bool held = groups <= kSplitHeld * 256;
    auto load8 = [&](int g, float4& p, float4& q) {
        if (vec) {
            p = reinterpret_cast<const float4*>(src)[2 * g];
            q = reinterpret_cast<const float4*>(src)[2 * g + 1];
        } else {
            const float* s8 = src + 8 * g;
            p = make_float4(s8[0], s8[1], s8[2], s8[3]);
            q = make_float4(s8[4], s8[5], s8[6], s8[7]);
        }
    };
    float4 keep[kSplitHeld][2];
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
            const int g = tid + r * 256;
            if (g < groups) {
                load8(g, keep[r][0], keep[r][1]);
            } else {
                keep[r][0] = make_float4(0.f, 0.f, 0.f, 0.f);
                keep[r][1] = keep[r][0];
            }
        }
#pragma unroll
        for (int r = 0; r < kSplitHeld; ++r) {
            scan(keep[r][0]);
            scan(keep[r][1]);
        }
    } else {
        for (int g = tid; g < groups; g += 256) {
            float4 p, q;
            load8(g, p, q);
            scan(p);
            scan(q);
        }
    }
    // an infinity or NaN anywhere in the row disables the scaling
    if (special) mx = __builtin_inff();
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off));
    if ((tid & 63) == 0) wmax[tid >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const int x = a_row_exponent(mx);
    if (tid == 0) row_exp[row] = x;
    const int64_t mp = FRAG ? (static_cast<int64_t>(m) + 31) / 32 * 32 : m;
    half8v* hi = reinterpret_cast<half8v*>(ah);
    half8v* lo = reinterpret_cast<half8v*>(ah + mp * k);
    // 16-byte piece index of the row's 8-group g
    auto piece = [&](int g) -> int64_t {
        if constexpr (FRAG)
            return ((static_cast<int64_t>(row / 32) * (k / 16) + g / 2) * 64 + row % 32 + 32 * (g % 2));
        return static_cast<int64_t>(row) * (k / 8) + g;
    };
    auto split = [&](int g, const float4& p, const float4& q) {
        half8v h, l;
        a_split8<FRAG>(p, q, x, h, l);
        hi[piece(g)] = h;
        lo[piece(g)] = l;
    };
    if (held) {
#pragma unroll
        for (int r = 0; r < kSplitHeld; ++r) {
            const int g = tid + r * 256;
            if (g < groups) split(g, keep[r][0], keep[r][1]);
        }
    } else {
        for (int g = tid; g < groups; g += 256) {
            float4 p, q;
            load8(g, p, q);
            split(g, p, q);
        }
    }
}


// The wide kernel's prep for k <= 6144 (GT = ceil(k / 2048) groups of
// eight per thread and row): R = 8 / GT rows per workgroup, held in
// registers between their maxima and their split.  Operand order puts 32
// rows side by side in every 1 KB piece, so one row alone writes 16 bytes
// per 512-byte half-piece; R consecutive rows give each thread an R x
// 16-byte run.
template <int R, int GT>
__global__ __launch_bounds__(256) void gemm_prep_frag_kernel(const float* __restrict__ a, _Float16* __restrict__ ah,
                                                             int* __restrict__ row_exp, int m, int k, int vec) {
    __shared__ float wmax[4 * R];
    const int tid = threadIdx.x;
    const int wg = a_stage_wg(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
    const int row0 = wg * R;
    const int groups = k >> 3;
    float4 v[R][GT][2];
    float mx[R];
    bool special[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float* src = a + static_cast<int64_t>(row0 + r) * k;
#pragma unroll
        for (int u = 0; u < GT; ++u) {
            const int g = tid + u * 256;
            if (row0 + r < m && g < groups) {
                if (vec) {
                    v[r][u][0] = reinterpret_cast<const float4*>(src)[2 * g];
                    v[r][u][1] = reinterpret_cast<const float4*>(src)[2 * g + 1];
                } else {
                    const float* s8 = src + 8 * g;
                    v[r][u][0] = make_float4(s8[0], s8[1], s8[2], s8[3]);
                    v[r][u][1] = make_float4(s8[4], s8[5], s8[6], s8[7]);
                }
            } else {
                v[r][u][0] = make_float4(0.f, 0.f, 0.f, 0.f);
                v[r][u][1] = v[r][u][0];
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        mx[r] = 0.0f;
        special[r] = false;
#pragma unroll
        for (int u = 0; u < GT; ++u)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float4 x = v[r][u][h];
                mx[r] = fmaxf(mx[r], fmaxf(fmaxf(fabsf(x.x), fabsf(x.y)), fmaxf(fabsf(x.z), fabsf(x.w))));
                special[r] = special[r] || !(fabsf(x.x) <= 3.4028235e38f) || !(fabsf(x.y) <= 3.4028235e38f) ||
                             !(fabsf(x.z) <= 3.4028235e38f) || !(fabsf(x.w) <= 3.4028235e38f);
            }
        // an infinity or NaN anywhere in the row disables the scaling
        if (special[r]) mx[r] = __builtin_inff();
        for (int off = 32; off > 0; off >>= 1) mx[r] = fmaxf(mx[r], __shfl_xor(mx[r], off));
    }
    if ((tid & 63) == 0)
#pragma unroll
        for (int r = 0; r < R; ++r) wmax[(tid >> 6) * R + r] = mx[r];
    __syncthreads();
    int x[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
        x[r] = a_row_exponent(fmaxf(fmaxf(wmax[r], wmax[R + r]), fmaxf(wmax[2 * R + r], wmax[3 * R + r])));
    if (tid < R && row0 + tid < m) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (r == tid) row_exp[row0 + r] = x[r];
    }
    const int64_t mp = (static_cast<int64_t>(m) + 31) / 32 * 32;
    half8v* hi = reinterpret_cast<half8v*>(ah);
    half8v* lo = reinterpret_cast<half8v*>(ah + mp * k);
#pragma unroll
    for (int u = 0; u < GT; ++u) {
        const int g = tid + u * 256;
        if (g >= groups) break;
        // rows row0 .. row0 + R - 1 (one 32-row block) are consecutive 16-byte pieces
        const int64_t base = (static_cast<int64_t>(row0 / 32) * (k / 16) + g / 2) * 64 + row0 % 32 + 32 * (g % 2);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (row0 + r >= m) break;
            half8v h, l;
            a_split8<true>(v[r][u][0], v[r][u][1], x[r], h, l);
            hi[base + r] = h;
            lo[base + r] = l;
        }
    }
}

// ---------------------------------------------------------------------------
// Wide-tile MFMA GEMM (rows_m > 32).  A BM x BN tile per workgroup of four
// waves stacked in M (each wave BM/4 rows by all BN columns), K in steps of
// 64 rows.
//
// A (hi and lo fp16 parts, laid out in operand order by
// gemm_prep_kernel<true>) goes straight from global memory into MFMA
// operand registers: one wave's operand for 32 rows and 16 k is one 1 KB
// load of consecutive memory (rows scattered over 32 cache lines would
// take the vector memory pipeline 4x the line lookups, which measured as
// ~2000 cycles of load issue per step).  Each wave owns distinct rows, so
// A is read once per workgroup and never passes through LDS (with both fp16
// parts it is the larger operand: 4 bytes per element).
//
// B is unpacked once per tile and step and shared through LDS.  A thread
// takes "units" of 4 columns x 8 K rows: INT4 four dword loads (byte
// rows), INT8 eight, each a 128-byte run across 32 lanes.  v_perm_b32
// transposes the unit to one dword per column (INT4: its 8 nibbles in K
// order; INT8: rows {0,1,4,5} and {2,3,6,7}), the packed-half magic numbers
// turn the codes into fp16 in the order k = 0, 4, 1, 5, 2, 6, 3, 7 (the
// order A is stored in), and each column's 8 halves go to LDS as one
// 16-byte write.  B sits in LDS column-major ([column][k], 64 + 8 halves
// per row: 144-byte rows make both the writes and the fragment reads free
// of bank conflicts), and tile column 4q + c is stored at LDS row c * BN/4
// + q, so the 16 lanes of a write touch 16 consecutive rows; the epilogue
// maps rows back to columns.
//
// Pipeline: a ring of D register stages, stage t holding A's fragments of
// step t and B's raw codes of step t + 1; at step t the MFMAs use A(t) and
// B(t) from LDS while B(t + 1) is unpacked into the other LDS buffer, then
// stage t is refilled with step t + D.  One barrier per step.  The K loop
// runs whole rounds of D steps (steps past the split multiply zeros), so
// every iteration issues the same loads and the compiler's vmcnt waits
// release each stage as soon as its own loads are in.
namespace wide {

#ifndef VM_WIDE_SCHED
#define VM_WIDE_SCHED 1
#endif
#ifndef VM_WIDE_VALU
#define VM_WIDE_VALU 5
#endif

constexpr int kRow = kBK + 8;   // halves per LDS row of B (one column): 144 bytes

template <int KIND, int BM, int BN, int D, int G>
struct Cfg {
    static constexpr int kThreads = 256 * G;                          // G groups of four waves
    static constexpr int WAVES_N = 128 / BM;                          // BM 128: 4 x 1 waves; BM 64: 2 x 2
    static constexpr int WN = BN / WAVES_N;                           // columns per wave (32 rows each)
    static constexpr int TN = WN / 32;                                // 32 x 32 MFMA tiles per wave
    static constexpr int kQuads = BN / 4;
    static constexpr int kUnits = kQuads * (kBK / 8);                 // 4 columns x 8 K rows
    static constexpr int kBPer = (kUnits + 255) / 256;                // per thread of a group
    static constexpr int kWords = KIND == 2 ? 4 : 8;                  // code dwords per unit
    static constexpr bool kBlock = KIND != 0;
    static constexpr int kLdsB = BN * kRow;                           // halves per buffer
    static constexpr int kCRow = BN + 4;                              // epilogue tile row (floats)
    // blockwise scales of a step: [2 chunks of 32 K rows][BN] floats per
    // buffer, indexed like B's LDS rows, after the B buffers
    static constexpr int kLdsS = kBlock ? 2 * BN : 0;
    static constexpr int kLoopBytes = 2 * G * kLdsB * 2 + 2 * G * kLdsS * 4;
    static constexpr int kLdsBytes = kLoopBytes > BM * kCRow * 4 ? kLoopBytes : BM * kCRow * 4;
    // Two workgroups per CU when two fit in LDS and the registers a thread
    // holds (accumulators, D stages, B fragments, ~48 for addressing)
    // stay within the 256 that two waves per SIMD leave each; otherwise one,
    // with all 512.
    static constexpr int kRegEstimate =
        TN * 16 + (kBlock ? 32 : 0) + D * (32 + kBPer * (kWords + (kBlock ? 4 : 0))) + TN * 4 + 48;
    static constexpr int kWavesPerEu = G == 2 ? 2 : (2 * kLdsBytes <= 160 * 1024 && kRegEstimate <= 256) ? 2 : 1;
    static_assert((BM == 128 || BM == 64) && TN >= 1 && WN % 32 == 0, "32 x 32 MFMA tiles");
    static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
};

template <int KIND, int BM, int BN, int D, int G>
struct Raw {
    using C = Cfg<KIND, BM, BN, D, G>;
    half8v ah[4];   // A hi fragments of this step, one per 16-k sub-step
    half8v al[4];   // A lo fragments
    uint32_t w[C::kBPer][C::kWords];
    u32x4 s[C::kBlock ? C::kBPer : 1];
};

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}


template <int KIND, int BM, int BN, int D, int G>
__global__ __launch_bounds__(256 * G) __attribute__((amdgpu_waves_per_eu(Cfg<KIND, BM, BN, D, G>::kWavesPerEu,
                                                                         Cfg<KIND, BM, BN, D, G>::kWavesPerEu)))
void qmm_mfma_wide_kernel(const _Float16* __restrict__ a, const int* __restrict__ row_exp, const uint8_t* __restrict__ wq,
                          const float* __restrict__ scale, float* __restrict__ c, int m, int k, int n,
                          int block_size, int steps_per_split, int tiles_n, int tiles_m, uint32_t a_bytes,
                          uint32_t lo_offset, uint32_t code_bytes, uint32_t scale_bytes, float* __restrict__ partials,
                          unsigned* __restrict__ counters) {
    using C = Cfg<KIND, BM, BN, D, G>;
    using R = Raw<KIND, BM, BN, D, G>;
    extern __shared__ __attribute__((aligned(16))) _Float16 lds[];
    __shared__ unsigned ticket;

    // G = 2: two groups of four waves take alternate K steps of the tile
    // (group g the steps s with s % 2 == g), so each SIMD holds two waves and
    // one wave's stalls on load issue leave the MFMA pipe to the other; the
    // groups' accumulators are summed through LDS at the end.
    const int tid = threadIdx.x;
    const int grp = G == 2 ? tid >> 8 : 0;
    const int gtid = tid & 255;   // thread within the group
    const int lane = tid & 63;
    const int wave = gtid >> 6;
    const int wm = wave / C::WAVES_N;
    const int wn = wave % C::WAVES_N;
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
    const int k_end = min(k, (step0 + nsteps) * kBK);
    const int fr = lane & 31;   // operand row (A) / column (B) of a 32 x 32 x 16 MFMA
    const int fh = lane >> 5;   // which 8 of its 16 k

    const __amdgpu_buffer_rsrc_t ars = buffer_rsrc(a, a_bytes);
    const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(wq, code_bytes);
    const __amdgpu_buffer_rsrc_t srs = buffer_rsrc(scale, scale_bytes);

    // Scale block of a unit: with the loaded step's first row k0 = q0 *
    // block_size + r0, the unit's block is q0 + 0, 1 or 2 (block_size >= 32
    // > the unit's offset of at most 56 rows), found with compares.  (q0,
    // r0) advance by one step per load (each load fetches B for the step
    // after the previous load's), so no division sits in the loop.
    int q0 = 0, r0 = 0;
    if constexpr (C::kBlock) {
        const int kb = (step0 + G + grp) * kBK;   // the group's first load fetches B of its second step
        q0 = kb / block_size;
        r0 = kb - q0 * block_size;
    }
    // A pieces of this lane (out-of-range rows and steps read zeros): row
    // block (m0 / 32 + wm), k block q: byte offset ((b * k/16 + q) * 64 + lane) * 16
    const bool a_row_ok = m0 + wm * 32 + fr < m;
    const uint32_t a_blk_off = (static_cast<uint32_t>(m0 / 32 + wm) * static_cast<uint32_t>(k / 16) * 64u + lane) * 16u;

    // stage of the group's step t (K step G * t + grp): A of that step,
    // B codes and scales of the group's step t + 1
    auto load = [&](int t, R& r) {
        const int k0 = (step0 + G * t + grp) * kBK;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int kq = k0 / 16 + q;
            const bool ok = a_row_ok && 16 * kq < k_end;
            const uint32_t off = a_blk_off + static_cast<uint32_t>(kq) * 1024u;
            r.ah[q] = __builtin_bit_cast(half8v, buffer_load16(ars, ok ? off : a_bytes));
            r.al[q] = __builtin_bit_cast(half8v, buffer_load16(ars, ok ? off + lo_offset : a_bytes));
        }
        const int kb0 = k0 + G * kBK;
#pragma unroll
        for (int p = 0; p < C::kBPer; ++p) {
            const int u = gtid + p * 256;
            const int q = u % C::kQuads;
            const int kg = u / C::kQuads;
            const int col = n0 + 4 * q;
            const int klog = kb0 + 8 * kg;
            const bool ok = u < C::kUnits && klog < k_end && col < n;
            const uint32_t row0 = KIND == 2 ? static_cast<uint32_t>(klog) / 2u : static_cast<uint32_t>(klog);
#pragma unroll
            for (int i = 0; i < C::kWords; ++i)
                r.w[p][i] = buffer_load4(wrs, ok ? (row0 + i) * static_cast<uint32_t>(n) + col : code_bytes);
            if constexpr (C::kBlock) {
                const int tt = r0 + 8 * kg;
                const uint32_t blk = static_cast<uint32_t>(q0 + (tt >= block_size) + (tt >= 2 * block_size));
                r.s[p] = buffer_load16(srs, ok ? (blk * static_cast<uint32_t>(n) + col) * 4u : scale_bytes);
            }
        }
        if constexpr (C::kBlock) {   // r0 + 64 G < (2 G + 1) * block_size
            r0 += G * kBK;
#pragma unroll
            for (int i = 0; i < 2 * G; ++i) {
                const int c1 = r0 >= block_size ? 1 : 0;
                r0 -= c1 * block_size;
                q0 += c1;
            }
        }
    };

    // unit -> four columns of 8 fp16 weights (k order 0, 4, 1, 5, 2, 6, 3, 7)
    auto unpack = [&](const R& r, int p, u32x4 (&out)[4]) {
        uint32_t t[4][2];
        const uint32_t* w = r.w[p];
        if constexpr (KIND == 2) {
            const uint32_t a01 = perm(w[1], w[0], 0x05010400u), b01 = perm(w[1], w[0], 0x07030602u);
            const uint32_t a23 = perm(w[3], w[2], 0x05010400u), b23 = perm(w[3], w[2], 0x07030602u);
            t[0][0] = perm(a23, a01, 0x05040100u);
            t[1][0] = perm(a23, a01, 0x07060302u);
            t[2][0] = perm(b23, b01, 0x05040100u);
            t[3][0] = perm(b23, b01, 0x07060302u);
        } else {
            const uint32_t a01 = perm(w[1], w[0], 0x05010400u), b01 = perm(w[1], w[0], 0x07030602u);
            const uint32_t a23 = perm(w[3], w[2], 0x05010400u), b23 = perm(w[3], w[2], 0x07030602u);
            const uint32_t a45 = perm(w[5], w[4], 0x05010400u), b45 = perm(w[5], w[4], 0x07030602u);
            const uint32_t a67 = perm(w[7], w[6], 0x05010400u), b67 = perm(w[7], w[6], 0x07030602u);
            t[0][0] = perm(a45, a01, 0x05040100u);
            t[1][0] = perm(a45, a01, 0x07060302u);
            t[2][0] = perm(b45, b01, 0x05040100u);
            t[3][0] = perm(b45, b01, 0x07060302u);
            t[0][1] = perm(a67, a23, 0x05040100u);
            t[1][1] = perm(a67, a23, 0x07060302u);
            t[2][1] = perm(b67, b23, 0x05040100u);
            t[3][1] = perm(b67, b23, 0x07060302u);
        }
        // exact fp16 codes (the block scales multiply each 32-row chunk's
        // fp32 sum, see mfma_pair)
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
            if constexpr (KIND == 2) {
                const uint32_t x = t[cc][0] ^ 0x88888888u;
                const _Float16 bias = static_cast<_Float16>(1032.0f);
                out[cc][0] = hsub2((x & 0x000F000Fu) | 0x64006400u, bias);
                out[cc][1] = hsub2(((x >> 4) & 0x000F000Fu) | 0x64006400u, bias);
                out[cc][2] = hsub2(((x >> 8) & 0x000F000Fu) | 0x64006400u, bias);
                out[cc][3] = hsub2(((x >> 12) & 0x000F000Fu) | 0x64006400u, bias);
            } else {
                const _Float16 bias = static_cast<_Float16>(1152.0f);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t x = t[cc][h] ^ 0x80808080u;
                    out[cc][2 * h] = hsub2((x & 0x00FF00FFu) | 0x64006400u, bias);
                    out[cc][2 * h + 1] = hsub2(((x >> 8) & 0x00FF00FFu) | 0x64006400u, bias);
                }
            }
        }
    };
    // LDS B buffer `buf` (0, 1) of this group, and its chunk scales
    auto lds_b = [&](int buf) { return lds + (grp * 2 + buf) * C::kLdsB; };
    auto lds_s = [&](int buf) {
        return reinterpret_cast<float*>(lds + 2 * G * C::kLdsB) + (grp * 2 + buf) * C::kLdsS;
    };
    auto write_b = [&](const R& r, int buf) {
        _Float16* b = lds_b(buf);
#pragma unroll
        for (int p = 0; p < C::kBPer; ++p) {
            const int u = gtid + p * 256;
            if (C::kUnits % 256 == 0 || u < C::kUnits) {
                u32x4 out[4];
                unpack(r, p, out);
                const int q = u % C::kQuads;
                const int kg = u / C::kQuads;
#pragma unroll
                for (int cc = 0; cc < 4; ++cc)
                    *reinterpret_cast<u32x4*>(b + (cc * C::kQuads + q) * kRow + 8 * kg) = out[cc];
                if constexpr (C::kBlock) {
                    // the first unit of each 32-row chunk holds the chunk's block scales
                    if (kg % 4 == 0) {
                        float* ss = lds_s(buf) + (kg / 4) * BN;
#pragma unroll
                        for (int cc = 0; cc < 4; ++cc) ss[cc * C::kQuads + q] = __uint_as_float(r.s[p][cc]);
                    }
                }
            }
        }
    };

    floatx16 acc[C::TN];
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;

    // MFMAs of two 16-k sub-steps (one 32-row chunk of K): every tile's hi
    // product, then every tile's lo product (consecutive MFMAs rarely wait
    // for each other's accumulator).  Blockwise scales: the chunk lies in
    // one scale block, so its products go to a fresh accumulator that is
    // then multiplied by the block scale of its column and added to the
    // total in fp32 (quantized_matmul.cpp:76-90: a block's sum times its
    // scale), the codes themselves being exact in fp16.
    auto mfma_pair = [&](const R& r, int buf, int q0) {
        const _Float16* b = lds_b(buf);
        if constexpr (C::kBlock) {
            // tiles two at a time, so that two chunk accumulators are live
            constexpr int kPair = C::TN >= 2 ? 2 : 1;
            const float* ss = lds_s(buf) + (q0 / 2) * BN;
#pragma unroll
            for (int j0 = 0; j0 < C::TN; j0 += kPair) {
                floatx16 blk[kPair];
#pragma unroll
                for (int jj = 0; jj < kPair; ++jj)
#pragma unroll
                    for (int e = 0; e < 16; ++e) blk[jj][e] = 0.f;
#pragma unroll
                for (int q = q0; q < q0 + 2; ++q) {
                    half8v bf[kPair];
#pragma unroll
                    for (int jj = 0; jj < kPair; ++jj)
                        bf[jj] = *reinterpret_cast<const half8v*>(b + (wn * C::WN + (j0 + jj) * 32 + fr) * kRow +
                                                                  q * 16 + 8 * fh);
#pragma unroll
                    for (int jj = 0; jj < kPair; ++jj)
                        blk[jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(r.ah[q], bf[jj], blk[jj], 0, 0, 0);
#pragma unroll
                    for (int jj = 0; jj < kPair; ++jj)
                        blk[jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(r.al[q], bf[jj], blk[jj], 0, 0, 0);
                }
#pragma unroll
                for (int jj = 0; jj < kPair; ++jj) {
                    const float sj = ss[wn * C::WN + (j0 + jj) * 32 + fr];
#pragma unroll
                    for (int e = 0; e < 16; ++e) acc[j0 + jj][e] = fmaf(blk[jj][e], sj, acc[j0 + jj][e]);
                }
            }
        } else {
#pragma unroll
            for (int q = q0; q < q0 + 2; ++q) {
                half8v bf[C::TN];
#pragma unroll
                for (int j = 0; j < C::TN; ++j)
                    bf[j] = *reinterpret_cast<const half8v*>(b + (wn * C::WN + j * 32 + fr) * kRow + q * 16 + 8 * fh);
#pragma unroll
                for (int j = 0; j < C::TN; ++j)
                    acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(r.ah[q], bf[j], acc[j], 0, 0, 0);
#pragma unroll
                for (int j = 0; j < C::TN; ++j)
                    acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(r.al[q], bf[j], acc[j], 0, 0, 0);
            }
        }
    };

    // Instruction order inside a step (the compiler otherwise issues the
    // loads, the MFMAs and the B unpacking as separate runs, leaving the
    // MFMA pipe idle for more than half of the step): B fragment reads for
    // the first two 16-k sub-steps, then every MFMA followed by a share of
    // the VALU work and the loads, the remaining fragment reads halfway.
    auto interleave = [&]() {
#if VM_WIDE_SCHED
        // (per-column INT8 only: the blockwise loop's chunk accumulators
        // leave no registers for hoisting every fragment read)
        if constexpr (C::kBlock) return;
        constexpr int kMfma = 4 * C::TN * 2;
        constexpr int kLoads = 8 + C::kBPer * (C::kWords + (C::kBlock ? 1 : 0));
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * C::TN, 0);   // DS reads, sub-steps 0 and 1
#pragma unroll
        for (int i = 0; i < kMfma; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);        // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, VM_WIDE_VALU, 0);   // VALU
            if (i < kLoads) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // VMEM read
            if (i == kMfma / 2 - 2) __builtin_amdgcn_sched_group_barrier(0x100, 2 * C::TN, 0);   // DS reads 2, 3
        }
#endif
    };

    // ---- pipeline.  B(0) is loaded and unpacked on its own; stage t then
    // carries A(t) and B(t + 1).
    {
        R b0;
        const int kk0 = (step0 + grp) * kBK;
        // B of the group's first step: a stage whose B part is that step (its A part is unused)
#pragma unroll
        for (int p = 0; p < C::kBPer; ++p) {
            const int u = gtid + p * 256;
            const int q = u % C::kQuads;
            const int kg = u / C::kQuads;
            const int col = n0 + 4 * q;
            const int klog = kk0 + 8 * kg;
            const bool ok = u < C::kUnits && klog < k_end && col < n;
            const uint32_t row0 = KIND == 2 ? static_cast<uint32_t>(klog) / 2u : static_cast<uint32_t>(klog);
#pragma unroll
            for (int i = 0; i < C::kWords; ++i)
                b0.w[p][i] = buffer_load4(wrs, ok ? (row0 + i) * static_cast<uint32_t>(n) + col : code_bytes);
            if constexpr (C::kBlock) {
                const uint32_t blk = static_cast<uint32_t>(klog) / static_cast<uint32_t>(block_size);
                b0.s[p] = buffer_load16(srs, ok ? (blk * static_cast<uint32_t>(n) + col) * 4u : scale_bytes);
            }
        }
        write_b(b0, 0);
    }
    // Stage refills go into the stage of the previous step, at the start of
    // a step: a load into registers that MFMAs issued just before still
    // read waits for those MFMAs (measured: ~1800 cycles per step when the
    // stage just consumed was refilled right after its MFMAs).  So D stages
    // keep D - 1 steps in flight.  (The loader's scale-block state expects
    // the steps in order: the prologue loads steps 0 .. D - 2, step s loads
    // step s + D - 1.)
    R st[D];
#pragma unroll
    for (int d = 0; d + 1 < D; ++d) load(d, st[d]);
    __syncthreads();
    const int nloc = (nsteps + G - 1) / G;   // steps per group
    for (int s = 0; s < nloc; s += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            const int cur = u & 1;   // D is even: buffer parity is static
            load(s + u + D - 1, st[(u + D - 1) % D]);
            mfma_pair(st[u], cur, 0);
            write_b(st[u], cur ^ 1);
            mfma_pair(st[u], cur, 2);
            interleave();
            __syncthreads();
        }
    }

    // ---- epilogue.  The tile goes through LDS (free after the loop's last
    // barrier) so that C, or the split's partials, are written in whole
    // 16-byte pieces of rows.  32 x 32 D layout: element v of lane l is row
    // 8 * (v / 4) + 4 * (l / 32) + v % 4; its column is LDS B row rr = wn *
    // WN + j * 32 + l % 32, i.e. tile column 4 * (rr % BN/4) + rr / (BN/4).
    float* sc = reinterpret_cast<float*>(lds);
    if constexpr (G == 2) {
        // group 1's partial sums go through the tile (same positions as
        // group 0's), group 0 adds them in fixed order
        if (grp == 1) {
#pragma unroll
            for (int j = 0; j < C::TN; ++j) {
                const int rr = wn * C::WN + j * 32 + fr;
                const int tc = 4 * (rr % C::kQuads) + rr / C::kQuads;
#pragma unroll
                for (int v = 0; v < 16; ++v) sc[(wm * 32 + 8 * (v / 4) + 4 * fh + v % 4) * C::kCRow + tc] = acc[j][v];
            }
        }
        __syncthreads();
        if (grp == 0) {
#pragma unroll
            for (int j = 0; j < C::TN; ++j) {
                const int rr = wn * C::WN + j * 32 + fr;
                const int tc = 4 * (rr % C::kQuads) + rr / C::kQuads;
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[j][v] += sc[(wm * 32 + 8 * (v / 4) + 4 * fh + v % 4) * C::kCRow + tc];
            }
        }
        __syncthreads();
    }
    if (grp == 0) {
        // per-column INT8 scales multiply the fp32 sums here; blockwise
        // scales were applied chunk by chunk
        float colscale[C::TN];
        int tcol[C::TN];
#pragma unroll
        for (int j = 0; j < C::TN; ++j) {
            const int rr = wn * C::WN + j * 32 + fr;
            tcol[j] = 4 * (rr % C::kQuads) + rr / C::kQuads;
            const int col = n0 + tcol[j];
            colscale[j] = C::kBlock ? 1.0f
                                    : __uint_as_float(buffer_load4(srs, col < n ? static_cast<uint32_t>(col) * 4u
                                                                                : scale_bytes));
        }
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int trow = wm * 32 + 8 * (v / 4) + 4 * fh + v % 4;
            const int row = m0 + trow;
            const int nx = row < m ? -row_exp[row] : 0;   // 2^-x undoes the row's staging scale
#pragma unroll
            for (int j = 0; j < C::TN; ++j) sc[trow * C::kCRow + tcol[j]] = ldexpf(acc[j][v] * colscale[j], nx);
        }
    }
    __syncthreads();
    // The tile's rows of C (or of the split's partials) from a 64-bit base:
    // byte offsets within BM rows stay 32-bit for any C (gemm_plan bounds n).
    const uint32_t out_lim = static_cast<uint32_t>(static_cast<int64_t>(min(BM, m - m0)) * n * 4);
    const __amdgpu_buffer_rsrc_t out_rs =
        buffer_rsrc((splits == 1 ? c : partials + static_cast<int64_t>(split) * m * n) + static_cast<int64_t>(m0) * n,
                    out_lim);
    for (int idx = tid; idx < BM * (BN / 4); idx += C::kThreads) {
        const int trow = idx / (BN / 4);
        const int tc = 4 * (idx % (BN / 4));
        const int row = m0 + trow, col = n0 + tc;
        const u32x4 v = *reinterpret_cast<const u32x4*>(sc + trow * C::kCRow + tc);
        const uint32_t off = (row < m && col < n) ? (static_cast<uint32_t>(trow) * n + col) * 4u : out_lim;
        if (splits == 1) buffer_store16(out_rs, off, v);
        else coherent_store16(out_rs, off, v);   // read by another workgroup (XCD) after the ticket
    }
    if (splits == 1) return;

    publish_partials();
    __syncthreads();
    const int tile = tile_y * tiles_n + tile_x;
    if (tid == 0) ticket = ticket_take(&counters[tile], static_cast<unsigned>(splits));
    __syncthreads();
    if (ticket != static_cast<unsigned>(splits - 1)) return;
    // (split calls keep splits * m * n * 4 below 2^31, choose_wide)
    const int64_t stride = static_cast<int64_t>(m) * n;
    const __amdgpu_buffer_rsrc_t prs = buffer_rsrc(partials, 0x7fffffff);
    const __amdgpu_buffer_rsrc_t crs = buffer_rsrc(c, static_cast<uint32_t>(min(stride * 4, int64_t(0x7fffffff))));
    for (int idx = tid; idx < BM * (BN / 4); idx += C::kThreads) {
        const int row = m0 + idx / (BN / 4);
        const int col = n0 + 4 * (idx % (BN / 4));
        if (row >= m || col >= n) continue;
        const int64_t base = static_cast<int64_t>(row) * n + col;
        float v[4] = {0.f, 0.f, 0.f, 0.f};
        for (int s0 = 0; s0 < splits; s0 += 4) {
            u32x4 t[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int64_t e = base + (s0 + u) * stride;
                t[u] = s0 + u < splits ? coherent_load16(prs, static_cast<uint32_t>(e * 4)) : u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] += __uint_as_float(t[u][q]);
        }
        buffer_store16(crs, static_cast<uint32_t>(base * 4),
                       u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])});
    }
    if (tid == 0) __hip_atomic_store(&counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace wide

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

// ---- wide kernel: tile and split choice, launch
// Rows above this go to the wide kernel by default.
constexpr int kWideMinRows = 64;

// Which kernel takes rows_m > 4: the wide kernel above kWideMinRows rows;
// VELOMIND_GEMM_WIDE=0 or a forced small-tile configuration
// (VELOMIND_GEMM_CFG) keeps every shape on the small-tile kernel, a forced
// wide configuration (VELOMIND_GEMM_WIDE="BM,BN,S,D[,G]") sends every
// shape to the wide kernel (measurement sweeps and tests).
// By default the wide kernel also needs a grid of at least kWideMinWgs
// workgroups (tiles x K splits): short-K, narrow-N shapes such as
// SmolLM2-360M's 960 x 960 projections at 128 rows (15 tiles, K too short
// to split) keep the small-tile kernel's finer grid.
constexpr long kWideMinWgs = 96;

struct WideConfig;
WideConfig choose_wide(int kind, int m, int k, int n);

bool use_wide_kernel(int kind, int m, int k, int n);

struct WideConfig {
    int bm = 128, bn = 128, splits = 1, depth = 2, groups = 1;
};

// From sweeps on MI355X (config 3: K = 2048, N = 5632, M = 128 / 256 /
// 512, INT8 and INT4, and the TinyLlama prefill projections at M = 512,
// INT4; weights cold): 128-row tiles with two wave groups, 128 columns for
// M >= 256 and 64 below, and K splits until the grid holds at least ~150
// workgroups while every group keeps at least four steps (M = 512: 176
// tiles, no split; M = 256: 88 tiles x 2; M = 128: 88 x 2).  A split costs
// a write and a read of the fp32 partial tile, so it only pays where tiles
// alone leave most CUs idle.  Two refinements:
//   * when 128 columns would need splits that leave a group fewer than
//     eight steps, 64 columns with fewer splits (K = 2048, N = 2048:
//     27.6 us vs 29.8 with 128 columns and four splits);
//   * more tiles than CUs: one wave group per workgroup, so that two
//     workgroups share a CU and the whole grid is resident at once instead
//     of a second, partial round (K = 2048, N = 11264: 352 tiles, 66.1 us vs
//     75.0 with two groups).
WideConfig choose_wide(int kind, int m, int k, int n) {
    WideConfig cfg;
    const int steps = (k + kBK - 1) / kBK;
    cfg.bm = 128;
    cfg.groups = 2;
    auto tiles_of = [&](int bn) { return static_cast<long>((m + cfg.bm - 1) / cfg.bm) * ((n + bn - 1) / bn); };
    auto splits_of = [&](long tiles) {
        int s = 1;
        while (s * 2 <= kMaxSplits && tiles * s < 150 && steps / (s * 2 * cfg.groups) >= 4) s *= 2;
        return s;
    };
    // blockwise scales: 64-column tiles (two 32 x 32 tiles per wave, see
    // the kernel's chunk accumulators)
    cfg.bn = m >= 256 && kind == 0 ? 128 : 64;
    int s = splits_of(tiles_of(cfg.bn));
    if (cfg.bn == 128 && steps / (s * cfg.groups) < 8) {
        const int s64 = splits_of(tiles_of(64));
        if (s64 < s) {
            cfg.bn = 64;
            s = s64;
        }
    }
    if (s == 1 && tiles_of(cfg.bn) > 256) cfg.groups = 1;
    if (kind != 0 && (m <= 64 || m >= 256)) {
        // blockwise scales, few or many rows: 64 x 128 tiles, one wave
        // group (M = 512, K = 2048, N = 5632, INT4: 49.3 us, against 51.5
        // with 128 x 64 and 61.9 with 128 x 64 in two groups; M = 128 keeps
        // 128 x 64 in two groups with K splits, 25.8 against 28.0 us)
        cfg.bm = 64;
        cfg.bn = 128;
        cfg.groups = 1;
        s = splits_of(tiles_of(cfg.bn));
    }
    cfg.splits = s;
    // Tuning override for measurement sweeps: VELOMIND_GEMM_WIDE="BM,BN,S,D[,G]"
    if (const char* env = std::getenv("VELOMIND_GEMM_WIDE")) {
        int bm = 0, bn = 0, sx = 0, d = 0, g = 1;
        const int got = std::sscanf(env, "%d,%d,%d,%d,%d", &bm, &bn, &sx, &d, &g);
        const bool wide_ok = kind == 0;   // four tiles per wave, four stages: per-column INT8 only
        const bool known = (bm == 128 && bn == 128 && wide_ok && ((d == 2 && (g == 1 || g == 2)) || (d == 4 && g == 1))) ||
                           (bm == 128 && bn == 64 && d == 2 && (g == 1 || g == 2)) ||
                           (bm == 64 && bn == 128 && (d == 2 || (d == 4 && wide_ok)) && g == 1) ||
                           (bm == 64 && bn == 256 && d == 2 && g == 1 && wide_ok);
        if (got >= 4 && sx >= 1 && sx <= kMaxSplits && known) {
            cfg.bm = bm;
            cfg.bn = bn;
            cfg.splits = sx;
            cfg.depth = d;
            cfg.groups = g;
        }
    }
    // partial tiles are addressed with 32-bit byte offsets
    while (cfg.splits > 1 && static_cast<int64_t>(cfg.splits) * m * n * 4 >= (int64_t(1) << 31)) cfg.splits /= 2;
    return cfg;
}

bool use_wide_kernel(int kind, int m, int k, int n) {
    // Blockwise scales: only the wide kernel applies them to each 32-row
    // chunk's fp32 sum (the small-tile kernel folds them into fp16 weights,
    // 2^-11 relative rounding per weight), so it takes every such call.
    if (kind != 0) return true;
    if (std::getenv("VELOMIND_GEMM_CFG")) return false;
    const char* env = std::getenv("VELOMIND_GEMM_WIDE");
    if (env && env[0] == '0' && env[1] == '\0') return false;
    if (env && env[0] != '\0') return true;
    if (m <= kWideMinRows) return false;
    const WideConfig cfg = choose_wide(kind, m, k, n);
    const long tiles = static_cast<long>((m + cfg.bm - 1) / cfg.bm) * ((n + cfg.bn - 1) / cfg.bn);
    return tiles * cfg.splits >= kWideMinWgs;
}

template <int KIND, int BM, int BN, int D, int G>
int launch_wide(const _Float16* a, const int* row_exp, const uint8_t* wq, const float* scale,
                float* c, int m, int k, int n, int block_size, int splits, hipStream_t stream) {
    using C = wide::Cfg<KIND, BM, BN, D, G>;
    auto kernel = wide::qmm_mfma_wide_kernel<KIND, BM, BN, D, G>;
    static bool lds_set = false;   // per instantiation (LDS above the 64 KB default)
    if (!lds_set) {
        VM_TRY_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, C::kLdsBytes),
                   "QuantizedMatMul: hipFuncSetAttribute");
        lds_set = true;
    }
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
    // A in operand order: m rounded up to 32 rows per part
    const uint32_t lo_offset = static_cast<uint32_t>((static_cast<int64_t>(m) + 31) / 32 * 32 * k * 2);
    const uint32_t a_bytes = 2u * lo_offset;   // hi, then lo
    const uint32_t code_bytes =
        static_cast<uint32_t>((KIND == 2 ? (static_cast<int64_t>(k) + 1) / 2 : static_cast<int64_t>(k)) * n);
    const uint32_t scale_bytes = static_cast<uint32_t>((KIND == 0 ? 1 : nblk) * n * 4);
    hipLaunchKernelGGL(kernel, dim3(tiles_n * tiles_m * splits), dim3(C::kThreads), C::kLdsBytes, stream, a, row_exp,
                       wq, scale, c, m, k, n, block_size, sps, tiles_n, tiles_m, a_bytes, lo_offset,
                       code_bytes, scale_bytes, ws.partials, ws.counters);
    return check_launch("QuantizedMatMul", stream);
}

template <int KIND>
int launch_wide_kind(const _Float16* a, const int* row_exp, const uint8_t* wq,
                     const float* scale, float* c, int m, int k, int n, int block_size, hipStream_t stream) {
    const WideConfig cfg = choose_wide(KIND, m, k, n);
#define VM_WIDE(BMX, BNX, DX, GX)                                                                              \
    if (cfg.bm == BMX && cfg.bn == BNX && cfg.depth == DX && cfg.groups == GX)                                 \
        return launch_wide<KIND, BMX, BNX, DX, GX>(a, row_exp, wq, scale, c, m, k, n, block_size,               \
                                                   cfg.splits, stream);
    VM_WIDE(128, 64, 2, 1)
    VM_WIDE(128, 64, 2, 2)
    VM_WIDE(64, 128, 2, 1)
    // four 32 x 32 tiles per wave, and four register stages: per-column
    // INT8 only (blockwise scales hold a chunk accumulator per tile pair,
    // which leaves no registers for them)
    if constexpr (KIND == 0) {
        VM_WIDE(128, 128, 2, 1)
        VM_WIDE(128, 128, 2, 2)
        VM_WIDE(64, 256, 2, 1)
        VM_WIDE(128, 128, 4, 1)
        VM_WIDE(64, 128, 4, 1)
    }
#undef VM_WIDE
    return VM_HIP_EUNSUPPORTED;
}

}  // namespace

// Rows per workgroup of the operand-order prep: the most (up to 8 / GT,
// a power of two) that still leave at least kPrepMinWgs row workgroups.
// VELOMIND_PREP_MIN_WGS overrides the minimum (measurement sweeps).
constexpr int kPrepMinWgs = 256;

static int prep_rows_per_wg(int m, int gt) {
    if (gt > 3) return 0;
    int min_wgs = kPrepMinWgs;
    if (const char* env = std::getenv("VELOMIND_PREP_MIN_WGS")) min_wgs = std::max(0, std::atoi(env));
    int r = 8 / gt;
    if (r == 8 / 3) r = 2;
    while (r > 1 && (m + r - 1) / r < min_wgs) r /= 2;
    return r;
}

// Which MFMA path a call takes and how it stages A (VM_HIP_EUNSUPPORTED:
// another kernel takes the shape).
int gemm_plan(int m, int k, int n, int quant_type, int block_size, GemmPlan* plan) {
    // 64-row steps may end half-way (k % 32 == 0); 16-byte code pieces need
    // whole 16-column groups; buffer offsets are 32-bit.
    if (m <= 4 || k % 32 != 0 || n % 16 != 0) return VM_HIP_EUNSUPPORTED;
    // (A's two fp16 parts take m * k * 4 bytes, addressed with 32-bit offsets)
    if ((static_cast<int64_t>(m) + 31) / 32 * 32 * k * 4 >= (int64_t(1) << 31) ||
        static_cast<int64_t>(k) * n >= (int64_t(1) << 31) || static_cast<int64_t>(n) * 128 * 4 >= (int64_t(1) << 31) ||
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
    plan->kind = kind;
    plan->pieces = use_wide_kernel(kind, m, k, n);
    return 0;
}

int gemm_qmm_staged_f32(const GemmPlan& plan, const _Float16* ah, const int* row_exp,
                        const uint8_t* wq, const float* scale, float* c, int m, int k, int n, int block_size,
                        hipStream_t stream) {
    if (plan.pieces) {
        if (plan.kind == 2) return launch_wide_kind<2>(ah, row_exp, wq, scale, c, m, k, n, block_size, stream);
        if (plan.kind == 1) return launch_wide_kind<1>(ah, row_exp, wq, scale, c, m, k, n, block_size, stream);
        return launch_wide_kind<0>(ah, row_exp, wq, scale, c, m, k, n, 0, stream);
    }
    // (blockwise scales always take the wide kernel, gemm_plan)
    if (plan.kind != 0) return VM_HIP_EUNSUPPORTED;
    return launch_kind<0>(ah, row_exp, wq, scale, c, m, k, n, 0, stream);
}

int gemm_qmm_f32(const float* a, const uint8_t* wq, const float* scale, float* c, int m, int k, int n,
                 int quant_type, int block_size, hipStream_t stream) {
    GemmPlan plan;
    VM_TRY(gemm_plan(m, k, n, quant_type, block_size, &plan));
    // A's row-scaled fp16 parts (hi, lo) and row exponents
    const std::size_t half_bytes = a_stage_half_bytes(m, k, plan.pieces);
    void* aux = nullptr;
    VM_TRY(get_aux(stream, a_stage_bytes(m, k, plan.pieces), &aux));
    auto* ah = static_cast<_Float16*>(aux);
    auto* row_exp = reinterpret_cast<int*>(static_cast<char*>(aux) + half_bytes);
    const int vec = reinterpret_cast<uintptr_t>(a) % 16 == 0 ? 1 : 0;
    if (plan.pieces) {
        const int gt = (k / 8 + 255) / 256;
        const int rows_per_wg = prep_rows_per_wg(m, gt);
#define VM_PREP(RX, GX)                                                                                           \
    if (gt == GX && rows_per_wg == RX)                                                                            \
        hipLaunchKernelGGL((gemm_prep_frag_kernel<RX, GX>), dim3((m + RX - 1) / RX), dim3(256), 0, stream, a, ah, \
                           row_exp, m, k, vec);                                                                   \
    else
        VM_PREP(8, 1) VM_PREP(4, 1) VM_PREP(2, 1) VM_PREP(1, 1) VM_PREP(4, 2) VM_PREP(2, 2) VM_PREP(1, 2)
        VM_PREP(2, 3) VM_PREP(1, 3)
#undef VM_PREP
            hipLaunchKernelGGL(gemm_prep_kernel<true>, dim3(m), dim3(256), 0, stream, a, ah, row_exp, m, k, vec);
    } else {
        hipLaunchKernelGGL(gemm_prep_kernel<false>, dim3(m), dim3(256), 0, stream, a, ah, row_exp, m, k, vec);
    }
    VM_TRY(check_launch("QuantizedMatMul", stream));
    return gemm_qmm_staged_f32(plan, ah, row_exp, wq, scale, c, m, k, n, block_size, stream);
}

}  // namespace vmhip
