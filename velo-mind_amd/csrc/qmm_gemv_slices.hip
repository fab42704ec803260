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
//   grid      (tiles, splits), renumbered so that each XCD owns a
//             contiguous run of splits (K ranges)
// The four row-lanes of a wave are reduced first with the gfx950
// permlane16/32 swaps (each lane is left with 4 of its 16 columns), so the
// block scale is one 16-byte load per lane and four FMAs; the waves of a
// workgroup add through LDS.
//
// Activation sources (the consumer side of the previous kernel):
//   PLAIN    x[k]: each lane loads its own 2R (INT4) or R (INT8) values
//   SLICES   x = sum of `slices` slices [slices][k], staged in LDS
//   SWIGLU   x[j] = silu(g[j]) * u[j] with g, u the sums of `slices`
//            slices of a fused gate|up projection [slices][2k], staged in
//            LDS (the Sigmoid, Mul, Mul of llama_graph.cpp:22-28); with
//            per-split sums of squares `ss_in` from the producer, g and u
//            are first multiplied by that row's 1/rms (see NORMRES)
//   NORMRES  the residual Add and RMSNorm in front of a projection
//            (llama_graph.cpp:118-136): h = act + sum of `slices` delta
//            slices, x = h * w.  RMSNorm's 1/rms is a scalar, so it is
//            left to the consumer of this GEMV's output (the projection is
//            linear): each split writes the sum of squares of h over its K
//            range to ss_out[split], and workgroups of tile 0 write h to
//            h_out.  Every workgroup stages only its own K range.
//   ATTN     the output of decode attention, merged while staging: the
//            per-chunk softmax partials (m, l, o[head_dim]) of the
//            attention kernel are combined in chunk order (online softmax
//            rescaling) for the workgroup's heads
//
// Dequantization matches the final-output GEMV: INT4 nibbles moved to the
// top of a byte give 16 * code (factor 1/16 folded into the scale), INT8
// codes are sign-extended bytes; fp32 FMA accumulation throughout.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>

#include "vm_device.h"
#include "vm_internal.h"

namespace vmhip {
namespace {

constexpr int kTileCols = 256;
constexpr int kGemvSrcPlain = VM_HIP_GEMV_SRC_PLAIN;
constexpr int kGemvSrcSlices = VM_HIP_GEMV_SRC_SLICES;
constexpr int kGemvSrcSwiglu = VM_HIP_GEMV_SRC_SWIGLU;
constexpr int kGemvSrcNormRes = VM_HIP_GEMV_SRC_NORMRES;
constexpr int kGemvSrcAttn = VM_HIP_GEMV_SRC_ATTN;

__device__ __forceinline__ float silu_mul(float g, float u) {
    const float sig = 1.0f / (1.0f + expf(-g));
    return (sig * g) * u;
}

// KIND: 0 = INT8 per-column scale, 1 = INT8 blockwise, 2 = INT4 blockwise.
__device__ __forceinline__ float inv_rms(const float* __restrict__ ss, int count, float dim, float eps) {
    if (!ss || count <= 0) return 1.0f;
    float t = 0.0f;
    for (int i = 0; i < count; ++i) t += ss[i];
    return 1.0f / sqrtf(t / dim + eps);
}

template <int KIND, int R, int W, int SRC>
__global__ __launch_bounds__(W * 64) void qmm_gemv_slices_kernel(
    vm_hip_gemv_src src, const uint8_t* __restrict__ wq, const float* __restrict__ scale,
    float* __restrict__ out, int k, int n, int block_size, uint32_t code_bytes, uint32_t scale_bytes) {
    const float* __restrict__ act = src.act;
    const int in_slices = src.slices;
    constexpr bool kInt4 = KIND == 2;
    constexpr int kRowsWave = 4 * R;                  // byte rows per wave
    constexpr int kRowsWg = W * kRowsWave;            // byte rows per workgroup
    constexpr int kKPerRow = kInt4 ? 2 : 1;           // K values per byte row
    constexpr int kXLane = R * kKPerRow;              // K values per lane
    constexpr int kXWg = kRowsWg * kKPerRow;          // K values per workgroup
    static_assert(kXLane % 4 == 0, "a lane's activations are whole float4s");
    __shared__ __align__(16) float red[W][kTileCols];
    __shared__ __align__(16) float xs[SRC == kGemvSrcPlain ? 4 : kXWg];
    __shared__ __align__(16) float stage_g[SRC == kGemvSrcPlain ? 4 : W * 64 * 4];
    __shared__ __align__(16) float stage_u[(SRC == kGemvSrcSwiglu || SRC == kGemvSrcAttn) ? W * 64 * 4 : 4];
    __shared__ float ssp[W * 2];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int cl = lane & 15;   // column lane
    const int rl = lane >> 4;   // row lane (DPP row)
    // Workgroups are dealt to the 8 XCDs round-robin by linear id; each XCD
    // takes a contiguous run of (split, tile) pairs in split-major order, so
    // the workgroups that stage one K range of the activations share an L2
    // (tiles share no weight lines: a tile is whole 128-byte lines).
    int tile = blockIdx.x;
    int split = blockIdx.y;
    {
        const int gx = static_cast<int>(gridDim.x);
        const int lin = static_cast<int>(blockIdx.y) * gx + tile;
        const int full = (gx * static_cast<int>(gridDim.y)) & ~7;
        if (lin < full) {
            const int p = (lin & 7) * (full >> 3) + (lin >> 3);
            split = p / gx;
            tile = p - split * gx;
        }
    }
    const int col0 = tile * kTileCols + cl * 16;
    const bool col_ok = col0 < n;                          // n % 16 == 0: all 16 columns or none
    const int wg_row0 = split * kRowsWg;
    const int wave_row0 = wg_row0 + wave * kRowsWave;
    const int row0 = wave_row0 + rl * R;
    const int byte_rows = kInt4 ? (k + 1) / 2 : k;

    // Load order matters: vector memory counters retire in issue order, so
    // the staged activations (L2/MALL hits) are requested before the
    // weights (HBM) -- waiting for them then does not wait for the weight
    // stream, and staging overlaps it.
    //
    // Staging the workgroup's K range in LDS (sources other than PLAIN), in
    // two levels so that every thread has at most a few loads in flight:
    //   1. thread t = part * NQ + q takes float4 group q (four consecutive K
    //      values) and a contiguous range of the slices (attention chunks)
    //      of part `part`, and leaves the partial sum (partial softmax
    //      merge) in LDS;
    //   2. thread q < NQ combines the parts in order and applies the
    //      source's elementwise tail (residual, SwiGLU, norm weight).
    // The grouping of the additions is fixed, so results do not depend on
    // scheduling.
    constexpr int T = W * 64;
    constexpr int NQ = kXWg / 4;
    constexpr int P = T / NQ;
    static_assert(T % NQ == 0 && P >= 1, "staging parts");
    constexpr int kPer = 4;   // loads of one kind in flight per thread (one batch covers 4P slices)
    const int kw0 = wg_row0 * kKPerRow;
    const int q = threadIdx.x % NQ;
    const int part = threadIdx.x / NQ;
    const int kk = kw0 + 4 * q;
    const bool ok = kk < k;
    constexpr bool kNorm = SRC == kGemvSrcNormRes;
    constexpr bool kAttn = SRC == kGemvSrcAttn;
    constexpr int kSrcMult = SRC == kGemvSrcSwiglu ? 2 : 1;
    u32x4 tg[kPer], tu[kPer];
    u32x4 hres = {0u, 0u, 0u, 0u}, nwv = {0u, 0u, 0u, 0u};
    u32x4 w[R];
    u32x4 sv;
    const int keep = 8 * (rl & 1) + 4 * (rl >> 1);   // columns kept after the row-lane reduction
    auto issue_weights = [&]() {
        // Codes: rows past the matrix and columns past n read zeros.
        const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(wq, code_bytes);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = row0 + r;
            const uint32_t off = (col_ok && row < byte_rows)
                                     ? static_cast<uint32_t>(row) * static_cast<uint32_t>(n) + static_cast<uint32_t>(col0)
                                     : code_bytes;
            w[r] = buffer_load16(wrs, off);
        }
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

    };
    // The attention source's addresses depend on *pos (a scalar load): its
    // weights go first so that they do not wait for that round trip.
    if constexpr (SRC == kGemvSrcAttn) issue_weights();
    int lo = 0, hi = 0;                       // this part's slice / chunk range
    uint32_t slice_stride = 0, head_base = 0;
    int d0 = 0, rec = 0;
    __amdgpu_buffer_rsrc_t drs = buffer_rsrc(act, 0u);
    if constexpr (SRC != kGemvSrcPlain) {
        if constexpr (kAttn) {
            const int D = src.head_dim;
            const int head = kk / D;
            d0 = kk - head * D;
            const int n_keys = min(src.pos[0] + 1, src.max_seq);
            const int nc = (n_keys + src.chunk - 1) / src.chunk;
            const int per = (nc + P - 1) / P;
            lo = part * per;
            hi = min(nc, lo + per);
            rec = D + 4;
            head_base = static_cast<uint32_t>(head) * static_cast<uint32_t>(src.chunks * rec);
            drs = buffer_rsrc(act, static_cast<uint32_t>(k / D) * static_cast<uint32_t>(src.chunks * rec) * 4u);
        } else {
            slice_stride = static_cast<uint32_t>(k) * kSrcMult;
            drs = buffer_rsrc(kNorm ? src.delta : act, static_cast<uint32_t>(in_slices) * slice_stride * 4u);
            const int per = (in_slices + P - 1) / P;
            lo = part * per;
            hi = min(in_slices, lo + per);
        }
        // first batch of loads
#pragma unroll
        for (int e = 0; e < kPer; ++e) {
            const bool v = ok && lo + e < hi;
            if constexpr (kAttn) {
                const uint32_t r0 = head_base + static_cast<uint32_t>((lo + e) * rec);
                tg[e] = buffer_load16(drs, v ? (r0 + 4u + static_cast<uint32_t>(d0)) * 4u : 0xfffffff0u);
                tu[e] = buffer_load16(drs, v ? r0 * 4u : 0xfffffff0u);
            } else {
                const uint32_t base = static_cast<uint32_t>(lo + e) * slice_stride + static_cast<uint32_t>(kk);
                tg[e] = buffer_load16(drs, v ? base * 4u : 0xfffffff0u);
                if constexpr (SRC == kGemvSrcSwiglu)
                    tu[e] = buffer_load16(drs, v ? (base + static_cast<uint32_t>(k)) * 4u : 0xfffffff0u);
            }
        }
        if constexpr (kNorm) {
            if (part == 0) {
                const __amdgpu_buffer_rsrc_t hrs = buffer_rsrc(act, static_cast<uint32_t>(k) * 4u);
                const __amdgpu_buffer_rsrc_t nrs = buffer_rsrc(src.norm_w, static_cast<uint32_t>(k) * 4u);
                hres = buffer_load16(hrs, ok ? static_cast<uint32_t>(kk) * 4u : 0xfffffff0u);
                nwv = buffer_load16(nrs, ok ? static_cast<uint32_t>(kk) * 4u : 0xfffffff0u);
            }
        }
    }

    if constexpr (SRC != kGemvSrcAttn) issue_weights();

    // Activations for the lane's K range [row0 * kKPerRow, + kXLane).
    u32x4 xv[kXLane / 4];
    const int kk0 = row0 * kKPerRow;
    if constexpr (SRC == kGemvSrcPlain) {
        const __amdgpu_buffer_rsrc_t ars = buffer_rsrc(act, static_cast<uint32_t>(k) * 4u);
#pragma unroll
        for (int i = 0; i < kXLane / 4; ++i) xv[i] = buffer_load16(ars, static_cast<uint32_t>(kk0 + 4 * i) * 4u);
    } else {
        float4* pg = reinterpret_cast<float4*>(stage_g);     // [P][NQ]
        float4* pu = reinterpret_cast<float4*>(stage_u);     // [P][NQ] (SwiGLU up / attention M, L)
        float4 g = make_float4(0.f, 0.f, 0.f, 0.f), u = g;
        float M = -INFINITY, Lsum = 0.0f;
        for (int c0 = lo;; c0 += kPer) {
#pragma unroll
            for (int e = 0; e < kPer; ++e) {
                if (c0 + e < hi) {   // slices / chunks in order
                    if constexpr (kAttn) {
                        const float mc = __uint_as_float(tu[e][0]);
                        const float Mn = fmaxf(M, mc);
                        const float al = M > -INFINITY ? expf(M - Mn) : 0.0f;
                        const float be = expf(mc - Mn);
                        Lsum = fmaf(Lsum, al, __uint_as_float(tu[e][1]) * be);
                        g.x = fmaf(g.x, al, __uint_as_float(tg[e][0]) * be);
                        g.y = fmaf(g.y, al, __uint_as_float(tg[e][1]) * be);
                        g.z = fmaf(g.z, al, __uint_as_float(tg[e][2]) * be);
                        g.w = fmaf(g.w, al, __uint_as_float(tg[e][3]) * be);
                        M = Mn;
                    } else {
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
            if (c0 + kPer >= hi) break;
            // further batches (more than kPer slices or chunks per part)
#pragma unroll
            for (int e = 0; e < kPer; ++e) {
                const int c = c0 + kPer + e;
                const bool v = ok && c < hi;
                if constexpr (kAttn) {
                    const uint32_t r0 = head_base + static_cast<uint32_t>(c * rec);
                    tg[e] = buffer_load16(drs, v ? (r0 + 4u + static_cast<uint32_t>(d0)) * 4u : 0xfffffff0u);
                    tu[e] = buffer_load16(drs, v ? r0 * 4u : 0xfffffff0u);
                } else {
                    const uint32_t base = static_cast<uint32_t>(c) * slice_stride + static_cast<uint32_t>(kk);
                    tg[e] = buffer_load16(drs, v ? base * 4u : 0xfffffff0u);
                    if constexpr (SRC == kGemvSrcSwiglu)
                        tu[e] = buffer_load16(drs, v ? (base + static_cast<uint32_t>(k)) * 4u : 0xfffffff0u);
                }
            }
        }
        pg[part * NQ + q] = g;
        if constexpr (kAttn)
            pu[part * NQ + q] = make_float4(M, Lsum, 0.0f, 0.0f);
        else if constexpr (SRC == kGemvSrcSwiglu)
            pu[part * NQ + q] = u;
        __syncthreads();

        float ss_part = 0.0f;
        if (threadIdx.x < NQ) {
            g = make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (kAttn) {
                M = -INFINITY;
                Lsum = 0.0f;
                for (int pp = 0; pp < P; ++pp) {   // parts in chunk order
                    const float4 ml = pu[pp * NQ + q];
                    if (ml.y > 0.0f) {
                        const float4 o = pg[pp * NQ + q];
                        const float Mn = fmaxf(M, ml.x);
                        const float al = M > -INFINITY ? expf(M - Mn) : 0.0f;
                        const float be = expf(ml.x - Mn);
                        Lsum = fmaf(Lsum, al, ml.y * be);
                        g.x = fmaf(g.x, al, o.x * be);
                        g.y = fmaf(g.y, al, o.y * be);
                        g.z = fmaf(g.z, al, o.z * be);
                        g.w = fmaf(g.w, al, o.w * be);
                        M = Mn;
                    }
                }
                const float il = Lsum > 0.0f ? 1.0f / Lsum : 0.0f;
                g = make_float4(g.x * il, g.y * il, g.z * il, g.w * il);
            } else {
                u = g;
                if constexpr (kNorm)   // the residual first: h + (part 0) + (part 1) + ...
                    g = make_float4(__uint_as_float(hres[0]), __uint_as_float(hres[1]), __uint_as_float(hres[2]),
                                    __uint_as_float(hres[3]));
                for (int pp = 0; pp < P; ++pp) {
                    const float4 a2 = pg[pp * NQ + q];
                    g = make_float4(g.x + a2.x, g.y + a2.y, g.z + a2.z, g.w + a2.w);
                    if constexpr (SRC == kGemvSrcSwiglu) {
                        const float4 b2 = pu[pp * NQ + q];
                        u = make_float4(u.x + b2.x, u.y + b2.y, u.z + b2.z, u.w + b2.w);
                    }
                }
                if constexpr (SRC == kGemvSrcSwiglu) {
                    const float iv = inv_rms(src.ss_in, src.ss_count, src.ss_dim, src.eps);
                    g = make_float4(g.x * iv, g.y * iv, g.z * iv, g.w * iv);
                    u = make_float4(u.x * iv, u.y * iv, u.z * iv, u.w * iv);
                    g = make_float4(silu_mul(g.x, u.x), silu_mul(g.y, u.y), silu_mul(g.z, u.z), silu_mul(g.w, u.w));
                }
                if constexpr (kNorm) {
                    if (ok) {
                        if (src.h_out && tile == 0) *reinterpret_cast<float4*>(src.h_out + kk) = g;
                        ss_part = fmaf(g.x, g.x, fmaf(g.y, g.y, fmaf(g.z, g.z, g.w * g.w)));
                        g = make_float4(g.x * __uint_as_float(nwv[0]), g.y * __uint_as_float(nwv[1]),
                                        g.z * __uint_as_float(nwv[2]), g.w * __uint_as_float(nwv[3]));
                    }
                }
            }
            // K values past k stay zero (their codes are zero too).
            *reinterpret_cast<float4*>(xs + 4 * q) = ok ? g : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if constexpr (kNorm) {
            // Sum of squares of h over this split's K range (tile 0 writes it).
            for (int off = 32; off > 0; off >>= 1) ss_part += __shfl_xor(ss_part, off, 64);
            if (lane == 0) ssp[wave] = ss_part;
        }
        __syncthreads();
        if constexpr (kNorm) {
            if (src.ss_out && tile == 0 && threadIdx.x == 0) {
                float t = 0.0f;
#pragma unroll
                for (int ww = 0; ww < W; ++ww) t += ssp[ww];
                src.ss_out[split] = t;
            }
        }
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
void launch_slices(const vm_hip_gemv_src& src, const uint8_t* wq, const float* scale, float* out, int k, int n,
                   int block, int splits, hipStream_t stream) {
    const int tiles = (n + kTileCols - 1) / kTileCols;
    const int64_t rows = KIND == 2 ? (static_cast<int64_t>(k) + 1) / 2 : k;
    const int64_t nblk = KIND == 0 ? 1 : (static_cast<int64_t>(k) + block - 1) / block;
    const uint32_t code_bytes = static_cast<uint32_t>(rows * n);
    const uint32_t scale_bytes = static_cast<uint32_t>(KIND == 0 ? static_cast<int64_t>(n) * 4 : nblk * n * 4);
    hipLaunchKernelGGL((qmm_gemv_slices_kernel<KIND, R, W, SRC>), dim3(tiles, splits), dim3(W * 64), 0, stream, src,
                       wq, scale, out, k, n, block, code_bytes, scale_bytes);
}

template <int KIND, int SRC>
void dispatch_rw(const SlicesConfig& c, const vm_hip_gemv_src& src, const uint8_t* wq, const float* scale,
                 float* out, int k, int n, int block, hipStream_t stream) {
#define VM_SLICES_CASE(RR, WW)                                                                              \
    if (c.R == RR && c.W == WW)                                                                             \
        return launch_slices<KIND, RR, WW, SRC>(src, wq, scale, out, k, n, block, c.splits, stream);
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

int vm_hip_qmm_gemv_slices_src_f32(const vm_hip_gemv_src* src, const int8_t* wq, const float* scale, float* out,
                                   int64_t k, int64_t n, int quant_type, int block_size, int max_slices,
                                   void* stream) {
    int s = 0;
    VM_TRY(vm_hip_gemv_slices_count(k, n, quant_type, block_size, max_slices, &s));
    if (!src || !src->act || !wq || !scale || !out) return fail_inval("gemv_slices: null pointer");
    const int kindsrc = src->kind;
    if (kindsrc < VM_HIP_GEMV_SRC_PLAIN || kindsrc > VM_HIP_GEMV_SRC_ATTN)
        return fail_inval("gemv_slices: unknown activation source");
    const bool sliced = kindsrc == VM_HIP_GEMV_SRC_SLICES || kindsrc == VM_HIP_GEMV_SRC_SWIGLU;
    if (sliced && (src->slices < 1 || src->slices > 4096)) return fail_inval("gemv_slices: slices must be in [1, 4096]");
    if (kindsrc == VM_HIP_GEMV_SRC_NORMRES) {
        if (src->slices < 0 || src->slices > 4096 || (src->slices > 0 && !src->delta) || !src->norm_w)
            return fail_inval("gemv_slices: residual source needs norm_w and slices in [0, 4096] with delta");
        if ((src->delta && reinterpret_cast<uintptr_t>(src->delta) % 16) ||
            reinterpret_cast<uintptr_t>(src->norm_w) % 16 || (src->h_out && reinterpret_cast<uintptr_t>(src->h_out) % 16))
            return fail_inval("gemv_slices: residual operands must be 16-byte aligned");
    }
    if ((kindsrc == VM_HIP_GEMV_SRC_SWIGLU && src->ss_in) && (src->ss_count < 1 || src->ss_dim <= 0.0f))
        return fail_inval("gemv_slices: ss_in needs ss_count >= 1 and ss_dim > 0");
    if (kindsrc == VM_HIP_GEMV_SRC_ATTN) {
        if (!src->pos || src->head_dim < 4 || src->head_dim % 4 || k % src->head_dim || src->chunk < 1 ||
            src->chunks < 1 || src->max_seq < 1 || static_cast<int64_t>(src->chunks) * src->chunk < src->max_seq)
            return fail_inval("gemv_slices: attention source needs pos, head_dim | k and chunks * chunk >= max_seq");
        if ((k / src->head_dim) * src->chunks * (src->head_dim + 4) * 4 > 0x7fffffffLL)
            return fail_inval("gemv_slices: attention partials too large");
    }
    if (k % 4 != 0 || reinterpret_cast<uintptr_t>(src->act) % 16 != 0)
        return fail_inval("gemv_slices: k % 4 == 0 and a 16-byte aligned activation required");
    const int64_t rows = quant_type == VM_HIP_QUANT_INT4 ? (k + 1) / 2 : k;
    const int64_t src_floats = sliced ? src->slices * k * (kindsrc == VM_HIP_GEMV_SRC_SWIGLU ? 2 : 1)
                                      : (kindsrc == VM_HIP_GEMV_SRC_NORMRES ? std::max<int64_t>(k, src->slices * k) : k);
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
    const int ki = static_cast<int>(k), ni = static_cast<int>(n);
#define VM_SLICES_SRC(KINDV)                                                                                    \
    do {                                                                                                      \
        switch (kindsrc) {                                                                                    \
            case VM_HIP_GEMV_SRC_PLAIN: dispatch_rw<KINDV, kGemvSrcPlain>(cfg, *src, wb, scale, out, ki, ni, block, st); break; \
            case VM_HIP_GEMV_SRC_SLICES: dispatch_rw<KINDV, kGemvSrcSlices>(cfg, *src, wb, scale, out, ki, ni, block, st); break; \
            case VM_HIP_GEMV_SRC_SWIGLU: dispatch_rw<KINDV, kGemvSrcSwiglu>(cfg, *src, wb, scale, out, ki, ni, block, st); break; \
            case VM_HIP_GEMV_SRC_NORMRES: dispatch_rw<KINDV, kGemvSrcNormRes>(cfg, *src, wb, scale, out, ki, ni, block, st); break; \
            default: dispatch_rw<KINDV, kGemvSrcAttn>(cfg, *src, wb, scale, out, ki, ni, block, st); break;     \
        }                                                                                                     \
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

int vm_hip_qmm_gemv_slices_f32(const float* act, int act_kind, int64_t act_slices, const int8_t* wq,
                               const float* scale, float* out, int64_t k, int64_t n, int quant_type, int block_size,
                               int max_slices, void* stream) {
    clear_error();
    if (act_kind != VM_HIP_GEMV_SRC_PLAIN && act_kind != VM_HIP_GEMV_SRC_SLICES && act_kind != VM_HIP_GEMV_SRC_SWIGLU)
        return fail_inval("gemv_slices: unknown activation source");
    vm_hip_gemv_src src{};
    src.kind = act_kind;
    src.act = act;
    src.slices = act_kind == VM_HIP_GEMV_SRC_PLAIN ? 0 : static_cast<int>(std::min<int64_t>(act_slices, 1 << 20));
    if (act_kind != VM_HIP_GEMV_SRC_PLAIN && (act_slices < 1 || act_slices > 4096))
        return fail_inval("gemv_slices: act_slices must be in [1, 4096]");
    return vm_hip_qmm_gemv_slices_src_f32(&src, wq, scale, out, k, n, quant_type, block_size, max_slices, stream);
}

}  // extern "C"
