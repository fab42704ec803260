// Persistent decode step: one greedy LLaMA decode step (head_dim 64) as a
// single cooperative launch, one workgroup per compute unit.
//
// The reference decodes a token by building and executing a graph of ~155
// QuantizedMatMul and ~250 other operators (llama_engine.cpp:395-455,
// llama_graph.cpp:247-330).  One launch per operation costs a few
// microseconds of launch and ramp time each, more than most of these
// operations move: at decode sizes the step is latency-bound, not
// bandwidth-bound.  Here every workgroup walks the whole step:
//
//   per layer  QKV     q|k|v = (h + sum of down slices) (.) w_attn   [x Wqkv]
//              ATT     1/rms, RoPE, K/V appended at *pos, 32-key chunks
//                      of softmax(q k^T) v  ->  records {m, l, o}
//              O       ctx merged from the records                    [x Wo]
//              GU      (h + sum of O slices) (.) w_ffn               [x Wgu]
//              DOWN    silu(g/rms) * (u/rms)                          [x Wdown]
//   then       LM      (h + sum of down slices) (.) w_final          [x Wlm]
//              ARGMAX  per-workgroup candidates, reduced by workgroup 0
//
// Projections are split-K GEMVs whose partial sums ("slices") the next
// phase adds in a fixed order (deterministic), as in qmm_gemv_slices.hip.
// RMSNorm's 1/rms is a scalar, so it is applied by the consumer of the
// projection (the projection is linear); each split contributes its part of
// the sum of squares.
//
// Synchronisation without barriers.  Every value one workgroup hands to
// another (slices, residual rows, sums of squares, attention records,
// argmax candidates) is stored as a 64-bit word {tag, fp32} with an
// agent-scope store; the consumer polls the words it needs with agent-scope
// loads until each carries this step's tag for that (layer, phase).  A
// workgroup therefore waits only for the data it reads, and no phase waits
// for a device-wide barrier.  Buffers are reused by every layer: a producer
// of layer l + 1 writes a buffer only after (transitively) reading outputs
// that every reader of layer l's copy produced after reading it -- each
// phase of a dense layer reads all of the previous phase's output -- so a
// value is never overwritten before all its readers have it.  Tags are
// step * 512 + layer * 8 + phase and never 0, the zeroed workspace's value.
//
// Weights are prefetched one phase ahead into registers (two static
// buffers alternating by phase), issued right after the current phase's
// stores (the attention records, in the attention phase), so that their
// transfer overlaps the next phase's wait.  They are issued after the
// stores, not before the compute, because a compute unit's memory pipeline
// serves its requests in order: with tens of kilobytes of weights in flight
// per compute unit, stores issued behind them reach their readers
// microseconds later, and every phase waits for the slowest producer.  The
// attention phase's K/V chunk is prefetched during the QKV phase.
//
// Co-residency of all workgroups is guaranteed by the cooperative launch;
// every poll is bounded nevertheless: a poll that times out sets the status
// word and the step completes with invalid results instead of hanging.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <cstdlib>
#include <map>
#include <mutex>

#include "decode_attn.h"
#include "vm_device.h"
#include "vm_internal.h"

namespace vmhip {
namespace {

typedef unsigned long long u64;

// Phase timestamps, compiled in only with -DVM_DECODE_TRACE (build.py:
// VELOMIND_DECODE_TRACE=1): thread 0 of each of the first kTraceWgs
// workgroups stores the 100 MHz wall clock at the phase boundaries of every
// layer (slot `layer`, event `ev`; the lm_head and argmax use slot
// `layers`), read back with vm_hip_decode_trace_read.  Events per layer:
//   0 QKV stage begins      1 staged       2 computed     3 stored
//  15 reduce begins        16 reduce done (the last 40 workgroups)
//   4 attention begins     17 first item's inputs in   18 its records out
//   5 attention done        6 O staged     7 computed     8 stored
//   9 gate|up staged       10 computed    11 stored
//  12 down staged          13 computed    14 stored
// and in slot `layers`: 0 final norm begins, 1 staged, 2 lm_head done,
// 3 local argmax done, 4 workgroup 0's reduction done.
#ifdef VM_DECODE_TRACE
constexpr int kTraceWgs = 512;
constexpr int kTraceSlots = 34;
constexpr int kTraceEvents = 24;
__device__ u64 g_decode_trace[kTraceWgs * kTraceSlots * kTraceEvents];
#define VM_TRACE(slot, ev)                                                                         \
    do {                                                                                           \
        if (threadIdx.x == 0 && blockIdx.x < kTraceWgs && (slot) < kTraceSlots)                    \
            g_decode_trace[(blockIdx.x * kTraceSlots + (slot)) * kTraceEvents + (ev)] = wall_clock64(); \
    } while (0)
#else
#define VM_TRACE(slot, ev) \
    do {                   \
    } while (0)
#endif

constexpr int kT = 256;          // threads per workgroup
constexpr int kWaves = 4;
constexpr int kTile = 256;       // columns per GEMV tile (16 lanes x 16 columns)
constexpr int kChunkRows = 16;   // code byte rows per wave chunk (4 row-lanes x 4)
constexpr int kPairs = 2;        // (item, chunk) pairs per wave per phase, in registers
constexpr int kMaxItems = 2;     // items per workgroup per phase (lm_head: per round)
constexpr int kD = 64;           // head_dim
constexpr int kHalf = kD / 2;
constexpr int kD4 = kD / 4;
constexpr int kAttChunk = 32;    // keys per attention item
constexpr int kMaxG = 16;        // query heads per KV head
constexpr int kRec = kD + 4;     // attention record {m, l, 0, 0, o[64]}
constexpr int kMaxSlices = 64;
constexpr int kMaxStageK = 512;  // K values a workgroup stages per phase
constexpr unsigned kSpinLimit = 1u << 18;   // ~0.3 s of polling per site at most

enum : int { kPhQkv = 0, kPhAtt = 1, kPhO = 2, kPhGu = 3, kPhDown = 4, kPhLm = 5, kPhCand = 6, kPhRed = 7 };

struct GemvPlan {
    int splits;          // S
    int rows;            // code byte rows per split
    int chunks;          // chunks per item = ceil(rows / 16)
    int tiles;           // ceil(n / 256)
    int groups;          // workgroups per split (G / S)
    int items;           // items per workgroup (lm_head: all rounds)
};

struct DecodeArgs {
    vm_hip_decode_model m;
    GemvPlan pq, po, pg, pd, pl;
    u64 *ha, *hb, *qkv_sl, *o_sl, *gu_sl, *dn_sl, *lm_sl, *ss_attn, *ss_ffn, *ss_fin, *att, *cand;
    u64* qkv_fin;        // q (rotated, 1/rms applied), k (rotated) and v of the token, [qkv_n]
    unsigned* status;
    float* logits_out;
    uint32_t epoch;      // step * 512
    int qkv_n;
    int max_chunks;
};

__device__ __forceinline__ uint32_t tag_of(const DecodeArgs& a, int layer, int phase) {
    return a.epoch + static_cast<uint32_t>(layer * 8 + phase);
}

// ---- tagged words ----------------------------------------------------------
__device__ __forceinline__ u32x4 sc1_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off), 0, 16));
}

__device__ __forceinline__ void put1(u64* p, float v, uint32_t tag) {
    __hip_atomic_store(p, (static_cast<u64>(tag) << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Two consecutive words (two agent-scope 64-bit stores; a buffer store
// would need a wave-uniform base and per-lane offsets).
__device__ __forceinline__ void put2(u64* p, float a, float b, uint32_t tag) {
    put1(p, a, tag);
    put1(p + 1, b, tag);
}

__device__ __forceinline__ bool tags_ok(const u32x4& v, uint32_t tag) { return v[1] == tag && v[3] == tag; }

// Bounded polling: returns false (and records the failure) once the spin
// budget of this workgroup is spent; afterwards nothing waits any more.
struct Poll {
    unsigned* status;
    bool dead;
    __device__ bool again(unsigned& spins) {
        if (dead) return false;
        if (++spins > kSpinLimit) {
            dead = true;
            __hip_atomic_fetch_or(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
        __builtin_amdgcn_s_sleep(2);
        return true;
    }
};

__device__ __forceinline__ float silu_mul(float g, float u) {
    const float sig = 1.0f / (1.0f + expf(-g));
    return (sig * g) * u;
}

// ---- shared memory -----------------------------------------------------------
struct GemvSmem {
    float xs[kMaxStageK];                       // staged activations of the split
    float4 pg[kT];                              // staging parts
    float4 pu[kT];
    float red[kMaxItems][kWaves][kTile];        // per-wave partial tiles
    float ssp[kWaves];
    float scalar[4];
};

struct AttSmem {
    float sq[kMaxG * kD];
    float sk[kAttChunk * (kD + 4)];
    float sv[kAttChunk * kD];
    float knew[kD];
    float vnew[kD];
    float sp[kMaxG][kAttChunk];
    float sm[kMaxG];
    float sl[kMaxG];
    float scalar[4];
};

struct ArgSmem {
    float bv[kWaves];
    int bi[kWaves];
};

union Smem {
    GemvSmem g;
    AttSmem a;
    ArgSmem r;
};

struct Scratch {
    float ss[kMaxSlices];
};

// ---- GEMV phase ---------------------------------------------------------------
// Workgroup w < groups * splits works on split w % splits and on the tiles
// group, group + groups, ... (group = w / splits); its items' (item, chunk)
// pairs are dealt to the waves round-robin.  A lane holds 16 columns x 4
// byte rows of a chunk.
struct GemvView {
    const uint8_t* codes;
    const float* scales;
    int k;          // K (rows of the logical matrix)
    int n;
    int block;      // blockwise scale rows (INT4), 0 for INT8 per column
};

template <int KIND>
struct Gemv {
    static constexpr bool kInt4 = KIND == 2;
    static constexpr int kKpr = kInt4 ? 2 : 1;   // K values per code byte row

    // Issues this wave's weight loads for items [item0, item0 + items_here).
    // All kPairs x 5 loads are always issued (pairs without work read past
    // the buffers: zeros, no memory traffic), so that the compiler counts
    // them exactly and a later use of the other buffer waits for its own
    // loads only, not for these.
    __device__ static void issue(const GemvView& v, const GemvPlan& p, int w, int item0, u32x4 (&buf)[kPairs][5]) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int cl = lane & 15, rl = lane >> 4;
        const bool wg_ok = w < p.groups * p.splits;
        const int split = wg_ok ? w % p.splits : 0, group = wg_ok ? w / p.splits : 0;
        const int byte_rows = kInt4 ? (v.k + 1) / 2 : v.k;
        const int rs0 = split * p.rows;
        const int rs1 = min(byte_rows, rs0 + p.rows);
        const uint32_t code_bytes = static_cast<uint32_t>(byte_rows) * static_cast<uint32_t>(v.n);
        const int nblk = KIND == 0 ? 1 : (v.k + v.block - 1) / v.block;
        const uint32_t scale_bytes = static_cast<uint32_t>(nblk) * static_cast<uint32_t>(v.n) * 4u;
        const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(v.codes, code_bytes);
        const __amdgpu_buffer_rsrc_t srs = buffer_rsrc(v.scales, scale_bytes);
        const int keep = 8 * (rl & 1) + 4 * (rl >> 1);
#pragma unroll
        for (int q = 0; q < kPairs; ++q) {
            const int flat = wave + kWaves * q;
            const int item = flat / p.chunks, chunk = flat - item * p.chunks;
            const int tile = group + (item0 + item) * p.groups;
            const int crow = rs0 + chunk * kChunkRows;
            const bool pair_ok = wg_ok && item < kMaxItems && item0 + item < p.items && tile < p.tiles && crow < rs1;
            const int col0 = tile * kTile + cl * 16;
            const bool col_ok = pair_ok && col0 < v.n;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = crow + rl * 4 + r;
                buf[q][r] = buffer_load16(wrs, (col_ok && row < rs1)
                                                   ? static_cast<uint32_t>(row) * static_cast<uint32_t>(v.n) +
                                                         static_cast<uint32_t>(col0)
                                                   : code_bytes);
            }
            uint32_t soff = scale_bytes;
            if (col_ok) {
                if constexpr (KIND == 0) {
                    soff = static_cast<uint32_t>(col0 + keep) * 4u;
                } else {
                    const int blk = (crow * kKpr) / v.block;
                    soff = (static_cast<uint32_t>(blk) * static_cast<uint32_t>(v.n) + static_cast<uint32_t>(col0 + keep)) * 4u;
                }
            }
            buf[q][4] = buffer_load16(srs, soff);
        }
    }

    // Accumulates this wave's pairs into sm.red (zeroed by the caller) from
    // the staged activations sm.xs (the split's K range, K index - k0).
    __device__ static void compute(const GemvView& v, const GemvPlan& p, int w, int item0,
                                   const u32x4 (&buf)[kPairs][5], GemvSmem& sm) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int cl = lane & 15, rl = lane >> 4;
        if (w >= p.groups * p.splits) return;
        const int split = w % p.splits, group = w / p.splits;
        const int byte_rows = kInt4 ? (v.k + 1) / 2 : v.k;
        const int rs0 = split * p.rows;
        const int rs1 = min(byte_rows, rs0 + p.rows);
        const int keep = 8 * (rl & 1) + 4 * (rl >> 1);
#pragma unroll
        for (int q = 0; q < kPairs; ++q) {
            const int flat = wave + kWaves * q;
            const int item = flat / p.chunks, chunk = flat - item * p.chunks;
            const int tile = group + (item0 + item) * p.groups;
            const int crow = rs0 + chunk * kChunkRows;
            if (!(item < kMaxItems && item0 + item < p.items && tile < p.tiles && crow < rs1)) continue;
            // activations of the lane's 4 byte rows (zeros past the split are
            // multiplied by zero codes)
            const int kk = (crow - rs0 + rl * 4) * kKpr;
            float x[4 * kKpr];
#pragma unroll
            for (int i = 0; i < 4 * kKpr; ++i) x[i] = sm.xs[kk + i];
            float acc[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[j] = 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if constexpr (kInt4) {
                    const float xe = x[2 * r], xo = x[2 * r + 1];
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const uint32_t wd = buf[q][r][d];
                        const uint32_t lo8 = (wd << 4) & 0xF0F0F0F0u;
                        const uint32_t hi8 = wd & 0xF0F0F0F0u;
#pragma unroll
                        for (int b = 0; b < 4; ++b) {
                            acc[4 * d + b] = fmaf(xe, static_cast<float>(static_cast<int8_t>(lo8 >> (8 * b))), acc[4 * d + b]);
                            acc[4 * d + b] = fmaf(xo, static_cast<float>(static_cast<int8_t>(hi8 >> (8 * b))), acc[4 * d + b]);
                        }
                    }
                } else {
                    const float xr = x[r];
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        const uint32_t wd = buf[q][r][d];
#pragma unroll
                        for (int b = 0; b < 4; ++b)
                            acc[4 * d + b] =
                                fmaf(xr, static_cast<float>(static_cast<int>(wd << (24 - 8 * b)) >> 24), acc[4 * d + b]);
                    }
                }
            }
            float h[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) h[j] = swap_rows_add(acc[j], acc[j + 8]);
            float z[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) z[j] = swap_halves_add(h[j], h[j + 4]);
            const float f = kInt4 ? 0.0625f : 1.0f;   // INT4 accumulated 16 * code
            float* red = &sm.red[item][wave][cl * 16 + keep];
#pragma unroll
            for (int j = 0; j < 4; ++j) red[j] += z[j] * (__uint_as_float(buf[q][4][j]) * f);
        }
    }
};

// Writes the workgroup's tiles [item0, item0 + kMaxItems) of its split as
// tagged slices out[split][n] (after the waves' partials are in sm.red).
__device__ void gemv_store(const GemvPlan& p, int n, int w, int item0, GemvSmem& sm, u64* out, uint32_t tag) {
    if (w >= p.groups * p.splits) return;
    const int split = w % p.splits, group = w / p.splits;
#pragma unroll
    for (int item = 0; item < kMaxItems; ++item) {
        const int tile = group + (item0 + item) * p.groups;
        if (item0 + item >= p.items || tile >= p.tiles) break;
        const int col = tile * kTile + static_cast<int>(threadIdx.x);
        if (col < n) {
            float v = 0.0f;
#pragma unroll
            for (int ww = 0; ww < kWaves; ++ww) v += sm.red[item][ww][threadIdx.x];
            put1(out + static_cast<int64_t>(split) * n + col, v, tag);
        }
    }
}

__device__ void zero_red(GemvSmem& sm) {
    float* r = &sm.red[0][0][0];
    for (int i = threadIdx.x; i < kMaxItems * kWaves * kTile; i += kT) r[i] = 0.0f;
}

// ---- staging (the consumer side of the previous phase) -----------------------
// The split's K range [k0, k1) as float4 groups q = t % nq, the slices (or
// attention chunks) divided among parts = t / nq; parts are combined in
// order by threads q < nq.  Returns the number of K values staged.
struct StageRange {
    int k0, k1, nq, parts;
};

__device__ __forceinline__ StageRange stage_range(const GemvPlan& p, int kpr, int k, int w) {
    StageRange s{};
    if (w >= p.groups * p.splits) return s;
    const int split = w % p.splits;
    s.k0 = split * p.rows * kpr;
    s.k1 = min(k, s.k0 + p.rows * kpr);
    s.nq = (p.rows * kpr + 3) / 4;
    s.parts = max(1, kT / s.nq);
    return s;
}

// Sum over slices [lo, hi) of tagged words at base + s * stride + kk .. +3,
// polled until every word carries `tag`; fixed order.
__device__ float4 sum_slices(const u64* base, int stride_words, int lo, int hi, int kk, uint32_t tag, Poll& poll,
                             int total_words) {
    const __amdgpu_buffer_rsrc_t r = buffer_rsrc(base, static_cast<uint32_t>(total_words) * 8u);
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    constexpr int kB = 4;
    for (int s0 = lo; s0 < hi; s0 += kB) {
        u32x4 a[kB], b[kB];
        unsigned spins = 0;
        for (;;) {
#pragma unroll
            for (int e = 0; e < kB; ++e) {
                const bool v = s0 + e < hi;
                const uint32_t off = (static_cast<uint32_t>((s0 + e) * stride_words + kk)) * 8u;
                a[e] = sc1_load16(r, v ? off : 0xfffffff0u);
                b[e] = sc1_load16(r, v ? off + 16u : 0xfffffff0u);
            }
            bool ok = true;
#pragma unroll
            for (int e = 0; e < kB; ++e)
                if (s0 + e < hi) ok = ok && tags_ok(a[e], tag) && tags_ok(b[e], tag);
            if (ok || !poll.again(spins)) break;
        }
#pragma unroll
        for (int e = 0; e < kB; ++e)
            if (s0 + e < hi) {
                acc.x += __uint_as_float(a[e][0]);
                acc.y += __uint_as_float(a[e][2]);
                acc.z += __uint_as_float(b[e][0]);
                acc.w += __uint_as_float(b[e][2]);
            }
    }
    return acc;
}

// Four tagged words at p[kk .. kk + 3], polled.
__device__ float4 load4_tagged(const u64* p, int kk, uint32_t tag, Poll& poll, int total_words) {
    const __amdgpu_buffer_rsrc_t r = buffer_rsrc(p, static_cast<uint32_t>(total_words) * 8u);
    u32x4 a, b;
    unsigned spins = 0;
    for (;;) {
        a = sc1_load16(r, static_cast<uint32_t>(kk) * 8u);
        b = sc1_load16(r, static_cast<uint32_t>(kk) * 8u + 16u);
        if ((tags_ok(a, tag) && tags_ok(b, tag)) || !poll.again(spins)) break;
    }
    return make_float4(__uint_as_float(a[0]), __uint_as_float(a[2]), __uint_as_float(b[0]), __uint_as_float(b[2]));
}

// Sum of `count` tagged scalars (in order), polled by threads 0 .. count-1
// in parallel; 1/sqrt(sum/dim + eps).  Called by the whole workgroup.
__device__ float inv_rms_tagged(const u64* ss, int count, float dim, float eps, uint32_t tag, Poll& poll,
                                float* scratch) {
    const int t = threadIdx.x;
    if (t < count) {
        u64 v = 0;
        unsigned spins = 0;
        for (;;) {
            v = __hip_atomic_load(ss + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (static_cast<uint32_t>(v >> 32) == tag || !poll.again(spins)) break;
        }
        scratch[t] = __uint_as_float(static_cast<uint32_t>(v));
    }
    __syncthreads();
    float total = 0.0f;
    for (int i = 0; i < count; ++i) total += scratch[i];
    __syncthreads();
    return 1.0f / sqrtf(total / dim + eps);
}

// Residual + RMSNorm staged for a projection: h = h_in + sum of delta
// slices, xs = h (.) norm_w; workgroups of group 0 write h to h_out and the
// split's sum of squares to ss_out[split] (tag out_tag).  h_in is tagged
// (tag h_tag) unless embed_row is given (layer 0: the token's embedding).
__device__ void stage_normres(const DecodeArgs& a, const GemvPlan& p, int kpr, int k, int w, GemvSmem& sm, Poll& poll,
                              const float* embed_row, const u64* h_in, uint32_t h_tag, const u64* delta,
                              int delta_slices, uint32_t d_tag, const float* norm_w, u64* h_out, u64* ss_out,
                              uint32_t out_tag) {
    const StageRange s = stage_range(p, kpr, k, w);
    if (s.nq == 0) return;
    const int t = threadIdx.x, q = t % s.nq, part = t / s.nq;
    const int kk = s.k0 + 4 * q;
    const bool ok = kk < s.k1;
    float4 hres = make_float4(0.f, 0.f, 0.f, 0.f), nw = hres;
    if (part == 0 && ok) {
        nw = *reinterpret_cast<const float4*>(norm_w + kk);
        if (embed_row) hres = *reinterpret_cast<const float4*>(embed_row + kk);
    }
    if (part < s.parts) {
        // the part's delta slices and (part 0, tagged h_in) the residual,
        // polled together
        const int per = (delta_slices + s.parts - 1) / s.parts;
        const int lo = min(delta_slices, part * per), hi = min(delta_slices, lo + per);
        const bool want_h = part == 0 && ok && !embed_row;
        const __amdgpu_buffer_rsrc_t dr = buffer_rsrc(delta, static_cast<uint32_t>(delta_slices * k) * 8u);
        const __amdgpu_buffer_rsrc_t hr = buffer_rsrc(h_in, static_cast<uint32_t>(k) * 8u);
        float4 d = make_float4(0.f, 0.f, 0.f, 0.f);
        constexpr int kB = 4;
        for (int s0 = lo; ok && (s0 < hi || (s0 == lo && want_h)); s0 += kB) {
            u32x4 da[kB], db[kB], ha_, hb_;
            const bool first = s0 == lo;
            unsigned spins = 0;
            for (;;) {
#pragma unroll
                for (int e = 0; e < kB; ++e) {
                    const bool v = s0 + e < hi;
                    const uint32_t off = static_cast<uint32_t>((s0 + e) * k + kk) * 8u;
                    da[e] = sc1_load16(dr, v ? off : 0xfffffff0u);
                    db[e] = sc1_load16(dr, v ? off + 16u : 0xfffffff0u);
                }
                const bool hh = first && want_h;
                ha_ = sc1_load16(hr, hh ? static_cast<uint32_t>(kk) * 8u : 0xfffffff0u);
                hb_ = sc1_load16(hr, hh ? static_cast<uint32_t>(kk) * 8u + 16u : 0xfffffff0u);
                bool good = !hh || (tags_ok(ha_, h_tag) && tags_ok(hb_, h_tag));
#pragma unroll
                for (int e = 0; e < kB; ++e)
                    if (s0 + e < hi) good = good && tags_ok(da[e], d_tag) && tags_ok(db[e], d_tag);
                if (good || !poll.again(spins)) break;
            }
            if (first && want_h)
                hres = make_float4(__uint_as_float(ha_[0]), __uint_as_float(ha_[2]), __uint_as_float(hb_[0]),
                                   __uint_as_float(hb_[2]));
#pragma unroll
            for (int e = 0; e < kB; ++e)
                if (s0 + e < hi) {
                    d.x += __uint_as_float(da[e][0]);
                    d.y += __uint_as_float(da[e][2]);
                    d.z += __uint_as_float(db[e][0]);
                    d.w += __uint_as_float(db[e][2]);
                }
        }
        sm.pg[part * s.nq + q] = d;
    }
    __syncthreads();
    float ss_part = 0.0f;
    if (t < s.nq) {
        float4 g = hres;
        for (int pp = 0; pp < s.parts; ++pp) {
            const float4 d = sm.pg[pp * s.nq + q];
            g = make_float4(g.x + d.x, g.y + d.y, g.z + d.z, g.w + d.w);
        }
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        if (ok) {
            ss_part = fmaf(g.x, g.x, fmaf(g.y, g.y, fmaf(g.z, g.z, g.w * g.w)));
            x = make_float4(g.x * nw.x, g.y * nw.y, g.z * nw.z, g.w * nw.w);
            if (h_out && w / p.splits == 0) {
                put2(h_out + kk, g.x, g.y, out_tag);
                put2(h_out + kk + 2, g.z, g.w, out_tag);
            }
        }
        *reinterpret_cast<float4*>(sm.xs + 4 * q) = x;
    }
    if (ss_out) {
        for (int off = 32; off > 0; off >>= 1) ss_part += __shfl_xor(ss_part, off, 64);
        if ((t & 63) == 0) sm.ssp[t >> 6] = ss_part;
    }
    __syncthreads();
    if (ss_out && t == 0 && w / p.splits == 0)
        put1(ss_out + (w % p.splits), sm.ssp[0] + sm.ssp[1] + sm.ssp[2] + sm.ssp[3], out_tag);
}

// SwiGLU staged for the down projection: g and u summed from the gate|up
// slices [slices][2 * inter], scaled by the gate|up input's 1/rms (its
// per-split sums of squares polled in the same batch), then silu(g) * u
// (llama_graph.cpp:22-28).
__device__ void stage_swiglu(const DecodeArgs& a, const GemvPlan& p, int kpr, int w, GemvSmem& sm, Poll& poll,
                             const u64* gu, int gu_slices, const u64* ss, int ss_count, uint32_t tag, float* scratch) {
    const int inter = static_cast<int>(a.m.inter);
    const StageRange s = stage_range(p, kpr, inter, w);
    if (s.nq == 0) return;   // uniform: a workgroup without work in this phase
    const int t = threadIdx.x, q = t % s.nq, part = t / s.nq;
    const int kk = s.k0 + 4 * q;
    const bool ok = kk < s.k1;
    const bool want_ss = t < ss_count;
    float4 g = make_float4(0.f, 0.f, 0.f, 0.f), u = g;
    {
        const int per = part < s.parts ? (gu_slices + s.parts - 1) / s.parts : 0;
        const int lo = min(gu_slices, part * per), hi = part < s.parts ? min(gu_slices, lo + per) : lo;
        const __amdgpu_buffer_rsrc_t gr = buffer_rsrc(gu, static_cast<uint32_t>(gu_slices * 2 * inter) * 8u);
        constexpr int kB = 4;
        for (int s0 = lo; (ok && s0 < hi) || (s0 == lo && want_ss); s0 += kB) {
            u32x4 ga[kB], gb[kB], ua[kB], ub[kB];
            u64 sv = 0;
            const bool first = s0 == lo;
            unsigned spins = 0;
            for (;;) {
#pragma unroll
                for (int e = 0; e < kB; ++e) {
                    const bool v = ok && s0 + e < hi;
                    const uint32_t off = static_cast<uint32_t>((s0 + e) * 2 * inter + kk) * 8u;
                    const uint32_t offu = off + static_cast<uint32_t>(inter) * 8u;
                    ga[e] = sc1_load16(gr, v ? off : 0xfffffff0u);
                    gb[e] = sc1_load16(gr, v ? off + 16u : 0xfffffff0u);
                    ua[e] = sc1_load16(gr, v ? offu : 0xfffffff0u);
                    ub[e] = sc1_load16(gr, v ? offu + 16u : 0xfffffff0u);
                }
                if (first && want_ss) sv = __hip_atomic_load(ss + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                bool good = !(first && want_ss) || static_cast<uint32_t>(sv >> 32) == tag;
#pragma unroll
                for (int e = 0; e < kB; ++e)
                    if (ok && s0 + e < hi)
                        good = good && tags_ok(ga[e], tag) && tags_ok(gb[e], tag) && tags_ok(ua[e], tag) &&
                               tags_ok(ub[e], tag);
                if (good || !poll.again(spins)) break;
            }
            if (first && want_ss) scratch[t] = __uint_as_float(static_cast<uint32_t>(sv));
#pragma unroll
            for (int e = 0; e < kB; ++e)
                if (ok && s0 + e < hi) {
                    g.x += __uint_as_float(ga[e][0]);
                    g.y += __uint_as_float(ga[e][2]);
                    g.z += __uint_as_float(gb[e][0]);
                    g.w += __uint_as_float(gb[e][2]);
                    u.x += __uint_as_float(ua[e][0]);
                    u.y += __uint_as_float(ua[e][2]);
                    u.z += __uint_as_float(ub[e][0]);
                    u.w += __uint_as_float(ub[e][2]);
                }
            if (!(ok && s0 + kB < hi)) break;
        }
        if (part < s.parts) {
            sm.pg[part * s.nq + q] = g;
            sm.pu[part * s.nq + q] = u;
        }
    }
    __syncthreads();
    if (t < s.nq) {
        float tot = 0.0f;
        for (int i = 0; i < ss_count; ++i) tot += scratch[i];
        const float iv = 1.0f / sqrtf(tot / static_cast<float>(a.m.hidden) + a.m.eps);
        g = make_float4(0.f, 0.f, 0.f, 0.f);
        u = g;
        for (int pp = 0; pp < s.parts; ++pp) {
            const float4 a2 = sm.pg[pp * s.nq + q], b2 = sm.pu[pp * s.nq + q];
            g = make_float4(g.x + a2.x, g.y + a2.y, g.z + a2.z, g.w + a2.w);
            u = make_float4(u.x + b2.x, u.y + b2.y, u.z + b2.z, u.w + b2.w);
        }
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        if (ok)
            x = make_float4(silu_mul(g.x * iv, u.x * iv), silu_mul(g.y * iv, u.y * iv), silu_mul(g.z * iv, u.z * iv),
                            silu_mul(g.w * iv, u.w * iv));
        *reinterpret_cast<float4*>(sm.xs + 4 * q) = x;
    }
    __syncthreads();
}

// Attention output staged for the output projection: for each float4 of
// the split's K range (inside one head), the chunk records {m, l, o} of
// that head merged in chunk order (online softmax rescaling), then / l.
__device__ void stage_attn(const DecodeArgs& a, const GemvPlan& p, int kpr, int w, int nc, GemvSmem& sm, Poll& poll,
                           uint32_t tag) {
    const int hidden = static_cast<int>(a.m.hidden);
    const StageRange s = stage_range(p, kpr, hidden, w);
    if (s.nq == 0) return;
    const int t = threadIdx.x, q = t % s.nq, part = t / s.nq;
    const int kk = s.k0 + 4 * q;
    const bool ok = kk < s.k1;
    const int head = kk / kD, d0 = kk - head * kD;
    const int rec_words = static_cast<int>(a.m.heads) * a.max_chunks * kRec;
    const __amdgpu_buffer_rsrc_t rr = buffer_rsrc(a.att, static_cast<uint32_t>(rec_words) * 8u);
    if (part < s.parts) {
        const int per = (nc + s.parts - 1) / s.parts;
        const int lo = min(nc, part * per), hi = min(nc, lo + per);
        float M = -INFINITY, L = 0.0f;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int c = lo; ok && c < hi; ++c) {
            const uint32_t base = static_cast<uint32_t>((head * a.max_chunks + c) * kRec);
            u32x4 ml, o0, o1;
            unsigned spins = 0;
            for (;;) {
                ml = sc1_load16(rr, base * 8u);
                o0 = sc1_load16(rr, (base + 4u + static_cast<uint32_t>(d0)) * 8u);
                o1 = sc1_load16(rr, (base + 6u + static_cast<uint32_t>(d0)) * 8u);
                if ((tags_ok(ml, tag) && tags_ok(o0, tag) && tags_ok(o1, tag)) || !poll.again(spins)) break;
            }
            const float mc = __uint_as_float(ml[0]), lc = __uint_as_float(ml[2]);
            const float Mn = fmaxf(M, mc);
            const float al = M > -INFINITY ? expf(M - Mn) : 0.0f;
            const float be = expf(mc - Mn);
            L = fmaf(L, al, lc * be);
            o.x = fmaf(o.x, al, __uint_as_float(o0[0]) * be);
            o.y = fmaf(o.y, al, __uint_as_float(o0[2]) * be);
            o.z = fmaf(o.z, al, __uint_as_float(o1[0]) * be);
            o.w = fmaf(o.w, al, __uint_as_float(o1[2]) * be);
            M = Mn;
        }
        sm.pg[part * s.nq + q] = o;
        sm.pu[part * s.nq + q] = make_float4(M, L, 0.f, 0.f);
    }
    __syncthreads();
    if (t < s.nq) {
        float M = -INFINITY, L = 0.0f;
        float4 g = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int pp = 0; pp < s.parts; ++pp) {
            const float4 ml = sm.pu[pp * s.nq + q];
            if (ml.y > 0.0f) {
                const float4 o = sm.pg[pp * s.nq + q];
                const float Mn = fmaxf(M, ml.x);
                const float al = M > -INFINITY ? expf(M - Mn) : 0.0f;
                const float be = expf(ml.x - Mn);
                L = fmaf(L, al, ml.y * be);
                g.x = fmaf(g.x, al, o.x * be);
                g.y = fmaf(g.y, al, o.y * be);
                g.z = fmaf(g.z, al, o.z * be);
                g.w = fmaf(g.w, al, o.w * be);
                M = Mn;
            }
        }
        const float il = L > 0.0f ? 1.0f / L : 0.0f;
        *reinterpret_cast<float4*>(sm.xs + 4 * q) =
            ok ? make_float4(g.x * il, g.y * il, g.z * il, g.w * il) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    __syncthreads();
}

// ---- QKV reduction ----------------------------------------------------------------
// Head h of the q|k|v projection (q heads, then k heads, then v heads): its
// 64 columns summed over the split slices (in order), times the input's
// 1/rms, rotated with the RoPE tables at p (q and k heads,
// rotary_embedding.cpp:16-45), published as tagged words in qkv_fin; k and
// v heads also go to the cache row p, which later steps read.  One
// polling round trip: every part's slices and the sums of squares are
// loaded together.
__device__ void qkv_reduce(const DecodeArgs& a, int layer, int head, int p, GemvSmem& sm, Poll& poll,
                           float* scratch) {
    const int H = static_cast<int>(a.m.heads), Hk = static_cast<int>(a.m.kv_heads);
    const int S = a.pq.splits, width = a.qkv_n;
    const int max_seq = static_cast<int>(a.m.max_seq);
    const int t = threadIdx.x;
    constexpr int nq = kD4;
    constexpr int parts = kT / nq;
    const int q = t % nq, part = t / nq;
    const int col = head * kD + 4 * q;
    const uint32_t qtag = tag_of(a, layer, kPhQkv);
    const bool rot = head < H + Hk;
    // the rotation of this thread's output element (plain loads, issued first)
    float rc = 1.0f, rs = 0.0f;
    if (rot && t < kD) {
        rc = a.m.cos_table[static_cast<int64_t>(p) * kHalf + (t % kHalf)];
        rs = a.m.sin_table[static_cast<int64_t>(p) * kHalf + (t % kHalf)];
    }
    {
        const int per = (S + parts - 1) / parts;
        const int lo = min(S, part * per), hi = min(S, lo + per);
        const bool want_ss = t < S;
        const __amdgpu_buffer_rsrc_t r = buffer_rsrc(a.qkv_sl, static_cast<uint32_t>(S * width) * 8u);
        float4 d = make_float4(0.f, 0.f, 0.f, 0.f);
        constexpr int kB = 4;
        for (int s0 = lo; s0 < hi || (s0 == lo && want_ss); s0 += kB) {
            u32x4 da[kB], db[kB];
            u64 sv = 0;
            const bool first = s0 == lo;
            unsigned spins = 0;
            for (;;) {
#pragma unroll
                for (int e = 0; e < kB; ++e) {
                    const bool v = s0 + e < hi;
                    const uint32_t off = static_cast<uint32_t>((s0 + e) * width + col) * 8u;
                    da[e] = sc1_load16(r, v ? off : 0xfffffff0u);
                    db[e] = sc1_load16(r, v ? off + 16u : 0xfffffff0u);
                }
                if (first && want_ss) sv = __hip_atomic_load(a.ss_attn + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                bool good = !(first && want_ss) || static_cast<uint32_t>(sv >> 32) == qtag;
#pragma unroll
                for (int e = 0; e < kB; ++e)
                    if (s0 + e < hi) good = good && tags_ok(da[e], qtag) && tags_ok(db[e], qtag);
                if (good || !poll.again(spins)) break;
            }
            if (first && want_ss) scratch[t] = __uint_as_float(static_cast<uint32_t>(sv));
#pragma unroll
            for (int e = 0; e < kB; ++e)
                if (s0 + e < hi) {
                    d.x += __uint_as_float(da[e][0]);
                    d.y += __uint_as_float(da[e][2]);
                    d.z += __uint_as_float(db[e][0]);
                    d.w += __uint_as_float(db[e][2]);
                }
            if (s0 + kB >= hi) break;
        }
        sm.pg[part * nq + q] = d;
    }
    __syncthreads();
    if (t < nq) {
        float tot = 0.0f;
        for (int i = 0; i < S; ++i) tot += scratch[i];
        const float iv = 1.0f / sqrtf(tot / static_cast<float>(a.m.hidden) + a.m.eps);
        float4 g = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int pp = 0; pp < parts; ++pp) {
            const float4 d = sm.pg[pp * nq + q];
            g = make_float4(g.x + d.x, g.y + d.y, g.z + d.z, g.w + d.w);
        }
        *reinterpret_cast<float4*>(sm.xs + 4 * q) = make_float4(g.x * iv, g.y * iv, g.z * iv, g.w * iv);
    }
    __syncthreads();
    if (t < kD) {
        float v = sm.xs[t];
        if (rot) {
            const int j = t % kHalf;
            const float x0 = sm.xs[j], x1 = sm.xs[j + kHalf];
            v = t < kHalf ? x0 * rc - x1 * rs : x1 * rc + x0 * rs;
        }
        put1(a.qkv_fin + head * kD + t, v, tag_of(a, layer, kPhRed));
        if (head >= H) {
            const bool is_k = head < H + Hk;
            const int kvh = is_k ? head - H : head - H - Hk;
            float* cache = is_k ? a.m.k_cache : a.m.v_cache;
            cache[((static_cast<int64_t>(layer) * Hk + kvh) * max_seq + p) * kD + t] = v;
        }
    }
    __syncthreads();   // LDS reused
}

// ---- attention phase ------------------------------------------------------------
// Item (hk, chunk): keys chunk * 32 .. + 31 of KV head hk for its G query
// heads (attention_decode_slices_kernel's algorithm, decode_ops.hip): the
// rotated queries (and, in the chunk holding p, the new key and value) from
// qkv_fin, the cached keys and values of earlier positions (prefetched),
// scores, the chunk's softmax partial and p . V, stored as the record
// {m, l, 0, 0, o[64]}.
struct KvPrefetch {
    u32x4 k[2], v[2];
};

__device__ void att_prefetch(const DecodeArgs& a, int layer, int item, int nc, KvPrefetch& pf) {
    const int hk = item / nc, chunk = item - hk * nc;
    const int k0 = chunk * kAttChunk;
    const int max_seq = static_cast<int>(a.m.max_seq);
    const int64_t lay = static_cast<int64_t>(layer) * a.m.kv_heads * max_seq * kD;
    const int64_t off = lay + (static_cast<int64_t>(hk) * max_seq + k0) * kD;
    const uint32_t bytes = static_cast<uint32_t>(max(0, min(kAttChunk, max_seq - k0)) * kD) * 4u;
    const __amdgpu_buffer_rsrc_t krs = buffer_rsrc(a.m.k_cache + off, bytes);
    const __amdgpu_buffer_rsrc_t vrs = buffer_rsrc(a.m.v_cache + off, bytes);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        pf.k[u] = buffer_load16(krs, (threadIdx.x + u * kT) * 16u);
        pf.v[u] = buffer_load16(vrs, (threadIdx.x + u * kT) * 16u);
    }
}

// Polls the item's queries (and new key / value) and stages them with the
// prefetched cache rows in LDS.
__device__ void att_load(const DecodeArgs& a, int layer, int item, int nc, int p, const KvPrefetch& pf, AttSmem& sm,
                         Poll& poll) {
    const int H = static_cast<int>(a.m.heads), Hk = static_cast<int>(a.m.kv_heads);
    const int G = H / Hk;
    const int hk = item / nc, chunk = item - hk * nc;
    const int k0 = chunk * kAttChunk;
    const int t = threadIdx.x;
    const bool last = chunk == nc - 1;
    const uint32_t rtag = tag_of(a, layer, kPhRed);
    constexpr int kKS = kD + 4;
    // task t: q float4 t (t < G * 16), then the new key, then the new value
    const int tasks = G * kD4 + (last ? 2 * kD4 : 0);
    if (t < tasks) {
        int col;
        float* dst;
        if (t < G * kD4) {
            col = hk * G * kD + 4 * t;
            dst = sm.sq + 4 * t;
        } else if (t < G * kD4 + kD4) {
            col = (H + hk) * kD + 4 * (t - G * kD4);
            dst = sm.knew + 4 * (t - G * kD4);
        } else {
            col = (H + Hk + hk) * kD + 4 * (t - G * kD4 - kD4);
            dst = sm.vnew + 4 * (t - G * kD4 - kD4);
        }
        *reinterpret_cast<float4*>(dst) = load4_tagged(a.qkv_fin, col, rtag, poll, a.qkv_n);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int e = t + u * kT;
        const int j = e / kD4, c = e - j * kD4;
        *reinterpret_cast<u32x4*>(sm.sk + j * kKS + 4 * c) = pf.k[u];
        *reinterpret_cast<u32x4*>(sm.sv + 4 * e) = pf.v[u];
    }
    __syncthreads();
    if (last && t < kD) {   // row p of the chunk: this step's key and value
        const int jr = p - k0;
        sm.sk[jr * kKS + t] = sm.knew[t];
        sm.sv[jr * kD + t] = sm.vnew[t];
    }
    __syncthreads();
}

__device__ void att_compute(const DecodeArgs& a, int layer, int item, int nc, int p, AttSmem& sm) {
    const int H = static_cast<int>(a.m.heads), Hk = static_cast<int>(a.m.kv_heads);
    const int G = H / Hk;
    const int hk = item / nc, chunk = item - hk * nc;
    const int nk = min(kAttChunk, p + 1 - chunk * kAttChunk);
    using CA = ChunkAttention<kD>;
    static_assert(CA::kChunk == kAttChunk && CA::kMaxG == kMaxG, "decode_attn.h tile");
    // attention scale 1.0: the queries were scaled by their loaders
    CA::scores(sm.sq, sm.sk, sm.sp, sm.sm, sm.sl, G, nk, 1.0f);
    __syncthreads();
    const uint32_t atag = tag_of(a, layer, kPhAtt);
    CA::pv(sm.sv, sm.sp, G, nk, [&](int g, int c4, float4 acc) {
        u64* rec = a.att + static_cast<int64_t>((hk * G + g) * a.max_chunks + chunk) * kRec;
        put2(rec + 4 + 4 * c4, acc.x, acc.y, atag);
        put2(rec + 6 + 4 * c4, acc.z, acc.w, atag);
        if (c4 == 0) {
            put2(rec, sm.sm[g], sm.sl[g], atag);
            put2(rec + 2, 0.0f, 0.0f, atag);
        }
    });
    __syncthreads();   // LDS reused by the next item
}

// ---- argmax --------------------------------------------------------------------------
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    // first maximum, NaN skipped (sample.cpp:18-38)
    if (v != v) return false;
    if (bi < 0) return true;
    return v > bv || (v == bv && i < bi);
}

__device__ void block_argmax(float& v, int& i, ArgSmem& sm) {
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const int oi = __shfl_xor(i, off, 64);
        if (better(ov, oi, v, i)) {
            v = ov;
            i = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        sm.bv[threadIdx.x >> 6] = v;
        sm.bi[threadIdx.x >> 6] = i;
    }
    __syncthreads();
    v = sm.bv[0];
    i = sm.bi[0];
    for (int ww = 1; ww < kWaves; ++ww)
        if (better(sm.bv[ww], sm.bi[ww], v, i)) {
            v = sm.bv[ww];
            i = sm.bi[ww];
        }
    __syncthreads();
}

// ---- the step -------------------------------------------------------------------------
template <int KIND>
__global__ __launch_bounds__(kT, 2) void decode_step_kernel(DecodeArgs a) {
    __shared__ Smem smem;
    __shared__ Scratch scr;
    const int w = static_cast<int>(blockIdx.x);
    const int G = static_cast<int>(gridDim.x);
    Poll poll{a.status, false};
    const int L = static_cast<int>(a.m.layers);
    const int hidden = static_cast<int>(a.m.hidden), inter = static_cast<int>(a.m.inter);
    const int Hk = static_cast<int>(a.m.kv_heads);
    const int p = min(a.m.pos[0], static_cast<int>(a.m.max_seq) - 1);
    const int nc = (p + 1 + kAttChunk - 1) / kAttChunk;
    const int att_items = Hk * nc;
    // the token indexes the embedding: kept in range whatever the device holds
    const int token = min(max(a.m.token[0], 0), static_cast<int>(a.m.vocab) - 1);
    using K = Gemv<KIND>;
    constexpr int kpr = K::kKpr;
    const int block = KIND == 0 ? 0 : a.m.block_size;

    u32x4 wa[kPairs][5], wb[kPairs][5];
    KvPrefetch kv;

    auto view_of = [&](int layer, int which) {
        const vm_hip_decode_layer& ly = a.m.layer[layer];
        switch (which) {
            case kPhQkv: return GemvView{reinterpret_cast<const uint8_t*>(ly.qkv_codes), ly.qkv_scales, hidden, a.qkv_n, block};
            case kPhO: return GemvView{reinterpret_cast<const uint8_t*>(ly.o_codes), ly.o_scales, hidden, hidden, block};
            case kPhGu: return GemvView{reinterpret_cast<const uint8_t*>(ly.gate_up_codes), ly.gate_up_scales, hidden, 2 * inter, block};
            default: return GemvView{reinterpret_cast<const uint8_t*>(ly.down_codes), ly.down_scales, inter, hidden, block};
        }
    };
    const GemvView lm_view{reinterpret_cast<const uint8_t*>(a.m.lm_codes), a.m.lm_scales, hidden,
                           static_cast<int>(a.m.vocab), block};

    // first QKV weights
    K::issue(view_of(0, kPhQkv), a.pq, w, 0, wa);

    for (int layer = 0; layer < L; ++layer) {
        const vm_hip_decode_layer& ly = a.m.layer[layer];
        // ---- QKV: residual + RMSNorm staged, weights in wa
        VM_TRACE(layer, 0);
        {
            const GemvView v = view_of(layer, kPhQkv);
            GemvSmem& sm = smem.g;
            if (layer == 0)
                stage_normres(a, a.pq, kpr, hidden, w, sm, poll, a.m.embed + static_cast<int64_t>(token) * hidden,
                              nullptr, 0, nullptr, 0, 0, ly.attn_norm, a.hb, a.ss_attn, tag_of(a, 0, kPhQkv));
            else
                stage_normres(a, a.pq, kpr, hidden, w, sm, poll, nullptr, a.ha, tag_of(a, layer - 1, kPhGu), a.dn_sl,
                              a.pd.splits, tag_of(a, layer - 1, kPhDown), ly.attn_norm, a.hb, a.ss_attn,
                              tag_of(a, layer, kPhQkv));
            VM_TRACE(layer, 1);
            if (w < att_items) att_prefetch(a, layer, w, nc, kv);
            zero_red(sm);
            __syncthreads();
            K::compute(v, a.pq, w, 0, wa, sm);
            __syncthreads();
            VM_TRACE(layer, 2);
            gemv_store(a.pq, a.qkv_n, w, 0, sm, a.qkv_sl, tag_of(a, layer, kPhQkv));
            __syncthreads();
            VM_TRACE(layer, 3);
        }
        VM_TRACE(layer, 15);
        // ---- QKV reduction (one head per workgroup, counted from the
        // last workgroup so that they differ from the attention items')
        {
            const int head = G - 1 - w;
            if (head < a.qkv_n / kD) qkv_reduce(a, layer, head, p, smem.g, poll, scr.ss);
        }
        VM_TRACE(layer, 16);
        // ---- attention: K/V chunk prefetched; O weights issued into wb
        // after the first item's records
        VM_TRACE(layer, 4);
        {
            bool issued = false;
            for (int item = w; item < att_items; item += G) {
                if (item != w) att_prefetch(a, layer, item, nc, kv);
                att_load(a, layer, item, nc, p, kv, smem.a, poll);
                if (item == w) VM_TRACE(layer, 17);
                att_compute(a, layer, item, nc, p, smem.a);
                if (item == w) VM_TRACE(layer, 18);
                if (!issued) {
                    K::issue(view_of(layer, kPhO), a.po, w, 0, wb);
                    issued = true;
                }
            }
            if (!issued) K::issue(view_of(layer, kPhO), a.po, w, 0, wb);
        }
        VM_TRACE(layer, 5);
        // ---- O: attention records merged while staging, weights in wb;
        // gate|up weights into wa after the stores
        {
            GemvSmem& sm = smem.g;
            stage_attn(a, a.po, kpr, w, nc, sm, poll, tag_of(a, layer, kPhAtt));
            VM_TRACE(layer, 6);
            zero_red(sm);
            __syncthreads();
            K::compute(view_of(layer, kPhO), a.po, w, 0, wb, sm);
            __syncthreads();
            VM_TRACE(layer, 7);
            gemv_store(a.po, hidden, w, 0, sm, a.o_sl, tag_of(a, layer, kPhO));
            __syncthreads();
            VM_TRACE(layer, 8);
            K::issue(view_of(layer, kPhGu), a.pg, w, 0, wa);
        }
        // ---- gate|up: residual + RMSNorm staged, weights in wa; down
        // weights into wb after the stores
        {
            GemvSmem& sm = smem.g;
            stage_normres(a, a.pg, kpr, hidden, w, sm, poll, nullptr, a.hb, tag_of(a, layer, kPhQkv), a.o_sl,
                          a.po.splits, tag_of(a, layer, kPhO), ly.ffn_norm, a.ha, a.ss_ffn, tag_of(a, layer, kPhGu));
            VM_TRACE(layer, 9);
            zero_red(sm);
            __syncthreads();
            K::compute(view_of(layer, kPhGu), a.pg, w, 0, wa, sm);
            __syncthreads();
            VM_TRACE(layer, 10);
            gemv_store(a.pg, 2 * inter, w, 0, sm, a.gu_sl, tag_of(a, layer, kPhGu));
            __syncthreads();
            VM_TRACE(layer, 11);
            K::issue(view_of(layer, kPhDown), a.pd, w, 0, wb);
        }
        // ---- down: SwiGLU staged, weights in wb; the next QKV (or
        // lm_head) weights into wa after the stores
        {
            GemvSmem& sm = smem.g;
            stage_swiglu(a, a.pd, kpr, w, sm, poll, a.gu_sl, a.pg.splits, a.ss_ffn, a.pg.splits,
                         tag_of(a, layer, kPhGu), scr.ss);
            VM_TRACE(layer, 12);
            zero_red(sm);
            __syncthreads();
            K::compute(view_of(layer, kPhDown), a.pd, w, 0, wb, sm);
            __syncthreads();
            VM_TRACE(layer, 13);
            gemv_store(a.pd, hidden, w, 0, sm, a.dn_sl, tag_of(a, layer, kPhDown));
            __syncthreads();
            VM_TRACE(layer, 14);
            if (layer + 1 < L)
                K::issue(view_of(layer + 1, kPhQkv), a.pq, w, 0, wa);
            else
                K::issue(lm_view, a.pl, w, 0, wa);
        }
    }

    // ---- lm_head: final norm staged; rounds of kMaxItems items, weights
    // alternating wa / wb
    VM_TRACE(L, 0);
    {
        GemvSmem& sm = smem.g;
        const uint32_t ltag = tag_of(a, L, kPhLm);
        stage_normres(a, a.pl, kpr, hidden, w, sm, poll, nullptr, a.ha, tag_of(a, L - 1, kPhGu), a.dn_sl, a.pd.splits,
                      tag_of(a, L - 1, kPhDown), a.m.final_norm, nullptr, a.ss_fin, ltag);
        const int V = static_cast<int>(a.m.vocab);
        VM_TRACE(L, 1);
        for (int r0 = 0; r0 < a.pl.items; r0 += 2 * kMaxItems) {
            if (r0 + kMaxItems < a.pl.items) K::issue(lm_view, a.pl, w, r0 + kMaxItems, wb);
            zero_red(sm);
            __syncthreads();
            K::compute(lm_view, a.pl, w, r0, wa, sm);
            __syncthreads();
            gemv_store(a.pl, V, w, r0, sm, a.lm_sl, ltag);
            __syncthreads();
            if (r0 + kMaxItems >= a.pl.items) break;
            if (r0 + 2 * kMaxItems < a.pl.items) K::issue(lm_view, a.pl, w, r0 + 2 * kMaxItems, wa);
            zero_red(sm);
            __syncthreads();
            K::compute(lm_view, a.pl, w, r0 + kMaxItems, wb, sm);
            __syncthreads();
            gemv_store(a.pl, V, w, r0 + kMaxItems, sm, a.lm_sl, ltag);
            __syncthreads();
        }
    }

    VM_TRACE(L, 2);
    // ---- logits of this workgroup's vocabulary range (four per float4
    // group, the lm_head slices divided among parts), its argmax candidate
    {
        const int V = static_cast<int>(a.m.vocab);
        const uint32_t ltag = tag_of(a, L, kPhLm);
        const uint32_t ctag = tag_of(a, L, kPhCand);
        const float iv = inv_rms_tagged(a.ss_fin, a.pl.splits, static_cast<float>(hidden), a.m.eps, ltag, poll, scr.ss);
        const int per = ((V + G - 1) / G + 3) / 4 * 4;
        const int j0 = w * per, j1 = min(V, j0 + per);
        const int nq = per / 4;
        const int parts = max(1, kT / nq);
        const int t = threadIdx.x, q = t % nq, part = t / nq;
        GemvSmem& gs = smem.g;
        const int S = a.pl.splits;
        const int jj = j0 + 4 * q;
        if (part < parts) {
            const int sper = (S + parts - 1) / parts;
            const int lo = min(S, part * sper), hi = min(S, lo + sper);
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (jj < j1 && hi > lo) v = sum_slices(a.lm_sl, V, lo, hi, jj, ltag, poll, S * V);
            gs.pg[part * nq + q] = v;
        }
        __syncthreads();
        float bv = 0.0f;
        int bi = -1;
        if (t < nq && jj < j1) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int pp = 0; pp < parts; ++pp) {
                const float4 d = gs.pg[pp * nq + q];
                v = make_float4(v.x + d.x, v.y + d.y, v.z + d.z, v.w + d.w);
            }
            const float vals[4] = {v.x * iv, v.y * iv, v.z * iv, v.w * iv};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (jj + e >= j1) break;
                if (a.logits_out) a.logits_out[jj + e] = vals[e];
                if (better(vals[e], jj + e, bv, bi)) {
                    bv = vals[e];
                    bi = jj + e;
                }
            }
        }
        __syncthreads();
        ArgSmem& sm = smem.r;
        VM_TRACE(L, 3);
        block_argmax(bv, bi, sm);
        if (threadIdx.x == 0) {
            put1(a.cand + 2 * w, bv, ctag);
            put1(a.cand + 2 * w + 1, __int_as_float(bi), ctag);
        }
        if (w == 0 && !a.logits_out) {
            // workgroup 0 reduces the candidates in workgroup order
            float cv = 0.0f;
            int ci = -1;
            for (int c = static_cast<int>(threadIdx.x); c < G; c += kT) {
                u64 vw = 0, iw = 0;
                unsigned spins = 0;
                for (;;) {
                    vw = __hip_atomic_load(a.cand + 2 * c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    iw = __hip_atomic_load(a.cand + 2 * c + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if ((static_cast<uint32_t>(vw >> 32) == ctag && static_cast<uint32_t>(iw >> 32) == ctag) ||
                        !poll.again(spins))
                        break;
                }
                const float v = __uint_as_float(static_cast<uint32_t>(vw));
                const int i = __float_as_int(__uint_as_float(static_cast<uint32_t>(iw)));
                if (i >= 0 && better(v, i, cv, ci)) {
                    cv = v;
                    ci = i;
                }
            }
            block_argmax(cv, ci, sm);
            VM_TRACE(L, 4);
            if (threadIdx.x == 0) {
                a.m.token[0] = ci;
                const int next = p + 1;
                if (next < a.m.max_seq) a.m.tokens[next] = ci;
                a.m.pos[0] = next;
            }
        }
    }
}

// ---- host side ----------------------------------------------------------------------------
int kind_of(const vm_hip_decode_model& m) {
    if (m.quant_type == VM_HIP_QUANT_INT4 && m.block_size > 0 && m.block_size % 32 == 0) return 2;
    if (m.quant_type == VM_HIP_QUANT_INT8 && m.block_size == 0) return 0;
    return -1;
}

// The split of one projection that minimises the bytes its busiest
// workgroup moves (weights plus its share of the partial slices), within
// the register pairs per wave; lm_head (rounds) has no pair limit.
bool plan_gemv(int kind, int64_t k, int64_t n, int G, bool rounds, GemvPlan* out) {
    const int kpr = kind == 2 ? 2 : 1;
    const int64_t byte_rows = kind == 2 ? (k + 1) / 2 : k;
    const int tiles = static_cast<int>((n + kTile - 1) / kTile);
    double best = 1e300;
    bool found = false;
    const int max_s = static_cast<int>(std::min<int64_t>(rounds ? kMaxSlices : 32, byte_rows));
    for (int S = 1; S <= max_s; ++S) {
        int64_t rows = (byte_rows + S - 1) / S;
        // blockwise: a chunk of 16 byte rows lies in one scale block; INT8:
        // a split's K range is whole float4s; lm_head: one chunk per wave
        // and item (its rounds hold three items)
        rows = kind == 2 ? (rows + kChunkRows - 1) / kChunkRows * kChunkRows : (rows + 3) / 4 * 4;
        if (rounds) rows = 4 * kChunkRows;
        const int s_eff = static_cast<int>((byte_rows + rows - 1) / rows);
        if (s_eff != S) continue;
        if (rows * kpr > kMaxStageK) continue;
        const int groups = G / S;
        if (groups < 1) continue;
        const int chunks = static_cast<int>((rows + kChunkRows - 1) / kChunkRows);
        const int items = (tiles + groups - 1) / groups;
        if (!rounds) {
            if (items > kMaxItems) continue;
            const int pairs = (items * chunks + kWaves - 1) / kWaves;
            if (pairs > kPairs) continue;
        } else {
            if (chunks > kWaves) continue;
        }
        const double wbytes = static_cast<double>(items) * rows * kTile * (kind == 2 ? 1.0 : 1.0);
        const double slice_bytes = 8.0 * S * n / G;
        const double cost = wbytes + slice_bytes + (rounds ? 0.0 : 0.0);
        if (cost < best - 1e-9) {
            best = cost;
            *out = GemvPlan{S, static_cast<int>(rows), chunks, tiles, groups, items};
            found = true;
        }
    }
    return found;
}

struct Layout {
    GemvPlan pq{}, po{}, pg{}, pd{}, pl{};
    int qkv_n = 0, max_chunks = 0, G = 0;
    int64_t off_ha = 0, off_hb = 0, off_qkv = 0, off_o = 0, off_gu = 0, off_dn = 0, off_lm = 0;
    int64_t off_ss_attn = 0, off_ss_ffn = 0, off_ss_fin = 0, off_att = 0, off_cand = 0, off_qkv_fin = 0, bytes = 0;
};

int cooperative_grid(int* G) {
    static std::mutex& mu = *new std::mutex;            // never destroyed (usable during exit)
    static std::map<int, int>& cache = *new std::map<int, int>;
    int dev = 0;
    VM_TRY_HIP(hipGetDevice(&dev), "decode_step: hipGetDevice");
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(dev);
    if (it != cache.end()) {
        *G = it->second;
        return 0;
    }
    int cus = 0, coop = 0;
    VM_TRY_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "decode_step: CU count");
    VM_TRY_HIP(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev), "decode_step: attribute");
    if (!coop || cus <= 0) return VM_HIP_EUNSUPPORTED;
    int per_cu = 0, per_cu0 = 0;
    VM_TRY_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, decode_step_kernel<2>, kT, 0),
               "decode_step: occupancy");
    VM_TRY_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu0, decode_step_kernel<0>, kT, 0),
               "decode_step: occupancy");
    per_cu = std::min(per_cu, per_cu0);
    if (per_cu < 1) return VM_HIP_EUNSUPPORTED;
    // Two workgroups per compute unit when they fit: two waves per SIMD
    // hide each other's dequantisation and memory latency.
    const char* env = std::getenv("VELOMIND_DECODE_WG_PER_CU");
    int want = env ? std::atoi(env) : 2;
    want = std::max(1, std::min(want, per_cu));
    cache[dev] = cus * want;
    *G = cus * want;
    return 0;
}

int make_layout(const vm_hip_decode_model& m, Layout* lay) {
    const int kind = kind_of(m);
    if (kind < 0) return VM_HIP_EUNSUPPORTED;
    if (m.head_dim != kD || m.heads < 1 || m.kv_heads < 1 || m.heads % m.kv_heads || m.heads / m.kv_heads > kMaxG)
        return VM_HIP_EUNSUPPORTED;
    if (m.hidden != m.heads * kD || m.hidden % 4 || m.inter % 4 || m.layers < 1 || m.layers > 63 || m.vocab < 1 ||
        m.max_seq < 1)
        return VM_HIP_EUNSUPPORTED;
    // 16-byte code loads cover 16 whole columns of one row
    const int64_t qkv_n = (m.heads + 2 * m.kv_heads) * kD;
    if (qkv_n % 16 || m.hidden % 16 || (2 * m.inter) % 16 || m.vocab % 16) return VM_HIP_EUNSUPPORTED;
    int G = 0;
    VM_TRY(cooperative_grid(&G));
    lay->G = G;
    lay->qkv_n = static_cast<int>((m.heads + 2 * m.kv_heads) * kD);
    if (!plan_gemv(kind, m.hidden, lay->qkv_n, G, false, &lay->pq) ||
        !plan_gemv(kind, m.hidden, m.hidden, G, false, &lay->po) ||
        !plan_gemv(kind, m.hidden, 2 * m.inter, G, false, &lay->pg) ||
        !plan_gemv(kind, m.inter, m.hidden, G, false, &lay->pd) ||
        !plan_gemv(kind, m.hidden, m.vocab, G, true, &lay->pl))
        return VM_HIP_EUNSUPPORTED;
    lay->max_chunks = static_cast<int>((m.max_seq + kAttChunk - 1) / kAttChunk);
    int64_t off = 256;   // status word
    auto take = [&](int64_t words) {
        const int64_t at = off;
        off += (words * 8 + 255) / 256 * 256;
        return at;
    };
    lay->off_ha = take(m.hidden);
    lay->off_hb = take(m.hidden);
    lay->off_qkv = take(static_cast<int64_t>(lay->pq.splits) * lay->qkv_n);
    lay->off_o = take(static_cast<int64_t>(lay->po.splits) * m.hidden);
    lay->off_gu = take(static_cast<int64_t>(lay->pg.splits) * 2 * m.inter);
    lay->off_dn = take(static_cast<int64_t>(lay->pd.splits) * m.hidden);
    lay->off_lm = take(static_cast<int64_t>(lay->pl.splits) * m.vocab);
    lay->off_ss_attn = take(lay->pq.splits);
    lay->off_ss_ffn = take(lay->pg.splits);
    lay->off_ss_fin = take(lay->pl.splits);
    lay->off_att = take(static_cast<int64_t>(m.heads) * lay->max_chunks * kRec);
    lay->off_cand = take(2 * static_cast<int64_t>(G));
    lay->off_qkv_fin = take(lay->qkv_n);
    lay->bytes = off;
    // 32-bit buffer offsets
    if (static_cast<int64_t>(lay->pl.splits) * m.vocab * 8 >= (int64_t(1) << 31) ||
        static_cast<int64_t>(lay->pg.splits) * 2 * m.inter * 8 >= (int64_t(1) << 31) ||
        static_cast<int64_t>(m.heads) * lay->max_chunks * kRec * 8 >= (int64_t(1) << 31))
        return VM_HIP_EUNSUPPORTED;
    return 0;
}

}  // namespace
}  // namespace vmhip

using namespace vmhip;

extern "C" {

int vm_hip_decode_workspace_bytes(const vm_hip_decode_model* model, int64_t* bytes) {
    clear_error();
    if (!model || !bytes) return fail_inval("vm_hip_decode_workspace_bytes: null argument");
    Layout lay;
    const int rc = make_layout(*model, &lay);
    if (rc == VM_HIP_EUNSUPPORTED) set_error("decode_step: model outside the persistent kernel's limits");
    if (rc) return rc;
    *bytes = lay.bytes;
    return 0;
}

int vm_hip_decode_step(const vm_hip_decode_model* model, void* workspace, int64_t workspace_bytes, uint32_t step,
                       float* logits_out, void* stream) {
    clear_error();
    if (!model || !workspace) return fail_inval("vm_hip_decode_step: null argument");
    const vm_hip_decode_model& m = *model;
    if (!m.layer || !m.embed || !m.final_norm || !m.lm_codes || !m.lm_scales || !m.cos_table || !m.sin_table ||
        !m.k_cache || !m.v_cache || !m.token || !m.pos || !m.tokens)
        return fail_inval("vm_hip_decode_step: null model pointer");
    if (step == 0 || step >= (1u << 23)) return fail_inval("vm_hip_decode_step: step must be in [1, 2^23)");
    Layout lay;
    const int rc = make_layout(m, &lay);
    if (rc == VM_HIP_EUNSUPPORTED) set_error("decode_step: model outside the persistent kernel's limits");
    if (rc) return rc;
    if (workspace_bytes < lay.bytes) return fail_inval("vm_hip_decode_step: workspace too small");
    VM_TRY(injected_failure("DecodeStep", "launch"));
    char* ws = static_cast<char*>(workspace);
    DecodeArgs a{};
    a.m = m;
    a.pq = lay.pq;
    a.po = lay.po;
    a.pg = lay.pg;
    a.pd = lay.pd;
    a.pl = lay.pl;
    auto at = [&](int64_t off) { return reinterpret_cast<u64*>(ws + off); };
    a.ha = at(lay.off_ha);
    a.hb = at(lay.off_hb);
    a.qkv_sl = at(lay.off_qkv);
    a.o_sl = at(lay.off_o);
    a.gu_sl = at(lay.off_gu);
    a.dn_sl = at(lay.off_dn);
    a.lm_sl = at(lay.off_lm);
    a.ss_attn = at(lay.off_ss_attn);
    a.ss_ffn = at(lay.off_ss_ffn);
    a.ss_fin = at(lay.off_ss_fin);
    a.att = at(lay.off_att);
    a.cand = at(lay.off_cand);
    a.qkv_fin = at(lay.off_qkv_fin);
    a.status = reinterpret_cast<unsigned*>(ws);
    a.logits_out = logits_out;
    a.epoch = step * 512u;
    a.qkv_n = lay.qkv_n;
    a.max_chunks = lay.max_chunks;
    void* args[] = {&a};
    const void* fn = kind_of(m) == 2 ? reinterpret_cast<const void*>(decode_step_kernel<2>)
                                     : reinterpret_cast<const void*>(decode_step_kernel<0>);
    VM_TRY_HIP(hipLaunchCooperativeKernel(fn, dim3(lay.G), dim3(kT), args, 0, static_cast<hipStream_t>(stream)),
               "DecodeStep on HIP at launch: hipLaunchCooperativeKernel");
    return check_launch("DecodeStep", static_cast<hipStream_t>(stream));
}

int vm_hip_decode_trace_read(void* host, int64_t bytes) {
    clear_error();
#ifdef VM_DECODE_TRACE
    if (!host || bytes < 0) return fail_inval("vm_hip_decode_trace_read: bad argument");
    const int64_t all = static_cast<int64_t>(sizeof(g_decode_trace));
    VM_TRY_HIP(hipDeviceSynchronize(), "decode_trace: sync");
    VM_TRY_HIP(hipMemcpyFromSymbol(host, HIP_SYMBOL(g_decode_trace), static_cast<size_t>(std::min(bytes, all))),
               "decode_trace: copy");
    return 0;
#else
    (void)host;
    (void)bytes;
    set_error("vm_hip_decode_trace_read: libvmhip was built without VM_DECODE_TRACE (VELOMIND_DECODE_TRACE=1)");
    return VM_HIP_EUNSUPPORTED;
#endif
}

int vm_hip_decode_status(void* workspace, int* failed, void* stream) {
    clear_error();
    if (!workspace || !failed) return fail_inval("vm_hip_decode_status: null argument");
    unsigned v = 0;
    auto s = static_cast<hipStream_t>(stream);
    VM_TRY_HIP(hipMemcpyAsync(&v, workspace, sizeof v, hipMemcpyDeviceToHost, s), "decode_status: copy");
    VM_TRY_HIP(hipStreamSynchronize(s), "decode_status: sync");
    *failed = v != 0;
    if (v) {
        const unsigned zero = 0;
        VM_TRY_HIP(hipMemcpyAsync(workspace, &zero, sizeof zero, hipMemcpyHostToDevice, s), "decode_status: clear");
        VM_TRY_HIP(hipStreamSynchronize(s), "decode_status: sync");
    }
    return 0;
}

}  // extern "C"
