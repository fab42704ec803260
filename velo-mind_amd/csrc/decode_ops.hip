// Kernels of the resident LLaMA decoder (velomind::examples::llama::
// HipLlamaDecoder): the same mathematics as the reference graph
// (examples/common/llama/llama_graph.cpp:14-330) arranged for one GPU.
//
//  * The KV cache is resident, [Hkv, max_seq, D] per layer, and new keys
//    and values are written in place at their positions instead of
//    concatenated each step (Concat + RepeatKV in the reference graph copy
//    the whole cache every token).
//  * Positions live in device memory (one int32), so a decode step is a
//    fixed sequence of launches that a HIP graph replays token after token;
//    the greedy argmax also runs on the device and advances the position.
//  * Attention reads grouped KV heads directly (no RepeatKV): one
//    workgroup per (KV head, key chunk) scores all query heads of the group
//    against the chunk, and the last chunk to finish merges the chunks'
//    softmax partials (flash-decoding), with the split-K ticket protocol of
//    the GEMV.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <string>

#include "a_split.h"
#include "decode_attn.h"
#include "vm_device.h"
#include "vm_hip.h"
#include "vm_internal.h"

namespace vmhip {
namespace {

constexpr int kT = 256;

hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---- SplitMix64 (Steele, Lea & Flood 2014) as a counter-based generator and
// the Box-Muller transform: element 2j and 2j+1 come from the pair
// (mix(seed + (2j+1) * golden), mix(seed + (2j+2) * golden)).
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void fill_normal_kernel(float* __restrict__ dst, int64_t n, uint64_t seed, float mean, float stddev) {
    constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;
    const int64_t pairs = (n + 1) / 2;
    for (int64_t j = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; j < pairs;
         j += static_cast<int64_t>(gridDim.x) * kT) {
        const uint64_t h1 = mix64(seed + static_cast<uint64_t>(2 * j + 1) * kGolden);
        const uint64_t h2 = mix64(seed + static_cast<uint64_t>(2 * j + 2) * kGolden);
        const float u1 = (static_cast<float>(h1 >> 40) + 0.5f) * (1.0f / 16777216.0f);   // (0, 1)
        const float u2 = static_cast<float>(h2 >> 40) * (1.0f / 16777216.0f);             // [0, 1)
        const float r = sqrtf(-2.0f * logf(u1));
        float s, c;
        sincosf(6.283185307179586f * u2, &s, &c);
        dst[2 * j] = mean + stddev * r * c;
        if (2 * j + 1 < n) dst[2 * j + 1] = mean + stddev * r * s;
    }
}

// With `slices` > 1 the projection arrives as split-K partial slices
// [slices][rows * width] (vm_hip_qmm_gemv_slices_f32); each value read is
// their sum in slice order.
__device__ __forceinline__ float slice_sum(const float* p, int slices, int64_t stride) {
    float v = p[0];
    for (int s0 = 1; s0 < slices; s0 += 8) {
        float t[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) t[e] = s0 + e < slices ? p[(s0 + e) * stride] : 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (s0 + e < slices) v += t[e];
    }
    return v;
}

// ---- h += delta (optional), hn = rmsnorm(h) * w, one workgroup per row.
// The add is the reference's Add node (add.cpp) and the norm its RMSNorm
// (rmsnorm.cpp:17-60) on the sum.
//
// Rows of at most 1024 * NV floats (dim % 4 == 0, 16-byte aligned rows)
// stay in registers: every thread issues all of its 16-byte loads of h,
// delta and w before the first use (one memory round trip), the sum of
// squares is reduced once, and h / hn are written from registers.  Buffer
// loads past the row return zeros, which add nothing to the sum.
template <int NV>
__global__ __launch_bounds__(kT) void add_rmsnorm_vec_kernel(float* __restrict__ h, const float* __restrict__ delta,
                                                             const float* __restrict__ w, float* __restrict__ hn,
                                                             int dim, float eps) {
    __shared__ float part[kT / 64];
    const uint32_t row_bytes = static_cast<uint32_t>(dim) * 4u;
    float* hr = h + static_cast<int64_t>(blockIdx.x) * dim;
    float* nr = hn + static_cast<int64_t>(blockIdx.x) * dim;
    const __amdgpu_buffer_rsrc_t hrs = buffer_rsrc(hr, row_bytes);
    const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(w, row_bytes);
    u32x4 hv[NV], dv[NV], wv[NV];
#pragma unroll
    for (int u = 0; u < NV; ++u) {
        const uint32_t off = (threadIdx.x + u * kT) * 16u;
        hv[u] = buffer_load16(hrs, off);
        wv[u] = buffer_load16(wrs, off);
    }
    if (delta) {
        const __amdgpu_buffer_rsrc_t drs = buffer_rsrc(delta + static_cast<int64_t>(blockIdx.x) * dim, row_bytes);
#pragma unroll
        for (int u = 0; u < NV; ++u) dv[u] = buffer_load16(drs, (threadIdx.x + u * kT) * 16u);
    }
    float x[NV][4];
    float s = 0.0f;
#pragma unroll
    for (int u = 0; u < NV; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float v = __uint_as_float(hv[u][e]);
            if (delta) v = v + __uint_as_float(dv[u][e]);
            x[u][e] = v;
            s = fmaf(v, v, s);
        }
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kT / 64; ++i) tot += part[i];
    const float inv = 1.0f / sqrtf(tot / static_cast<float>(dim) + eps);
#pragma unroll
    for (int u = 0; u < NV; ++u) {
        const int i4 = threadIdx.x + u * kT;
        if (4 * i4 < dim) {
            if (delta) *reinterpret_cast<float4*>(hr + 4 * i4) = make_float4(x[u][0], x[u][1], x[u][2], x[u][3]);
            float4 y;
            y.x = x[u][0] * inv * __uint_as_float(wv[u][0]);
            y.y = x[u][1] * inv * __uint_as_float(wv[u][1]);
            y.z = x[u][2] * inv * __uint_as_float(wv[u][2]);
            y.w = x[u][3] * inv * __uint_as_float(wv[u][3]);
            *reinterpret_cast<float4*>(nr + 4 * i4) = y;
        }
    }
}

// Any row length or alignment: strided loop over the row.
__global__ __launch_bounds__(kT) void add_rmsnorm_kernel(float* __restrict__ h, const float* __restrict__ delta,
                                                         const float* __restrict__ w, float* __restrict__ hn,
                                                         int64_t dim, float eps) {
    __shared__ float part[kT / 64];
    float* hr = h + blockIdx.x * dim;
    const float* dr = delta ? delta + blockIdx.x * dim : nullptr;
    float* nr = hn + blockIdx.x * dim;
    float s = 0.0f;
    for (int64_t i = threadIdx.x; i < dim; i += kT) {
        float v = hr[i];
        if (dr) {
            v = v + dr[i];
            hr[i] = v;
        }
        s = fmaf(v, v, s);
    }
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kT / 64; ++i) tot += part[i];
    const float inv = 1.0f / sqrtf(tot / static_cast<float>(dim) + eps);
    for (int64_t i = threadIdx.x; i < dim; i += kT) nr[i] = hr[i] * inv * w[i];
}

// ---- One row: h += sum of `slices` split-K partial slices of the
// previous projection ([slices][dim], added in slice order), hn =
// rmsnorm(h) * w.  The residual Add and RMSNorm of llama_graph.cpp:118-
// 136 on the consumer side of vm_hip_qmm_gemv_slices_f32.  512 threads,
// NV float4 of the row per thread (dim <= 2048 * NV, dim % 4 == 0), every
// load of a batch of slices issued before its first use.
constexpr int kNormT = 512;

template <int NV>
__global__ __launch_bounds__(kNormT) void add_rmsnorm_slices_kernel(float* __restrict__ h,
                                                                    const float* __restrict__ delta, int slices,
                                                                    const float* __restrict__ w,
                                                                    float* __restrict__ hn, int dim, float eps) {
    __shared__ float part[kNormT / 64];
    const uint32_t row_bytes = static_cast<uint32_t>(dim) * 4u;
    const __amdgpu_buffer_rsrc_t hrs = buffer_rsrc(h, row_bytes);
    const __amdgpu_buffer_rsrc_t wrs = buffer_rsrc(w, row_bytes);
    const __amdgpu_buffer_rsrc_t drs = buffer_rsrc(delta, static_cast<uint32_t>(slices) * row_bytes);
    float x[NV][4];
    u32x4 wv[NV];
#pragma unroll
    for (int u = 0; u < NV; ++u) {
        const uint32_t off = (threadIdx.x + u * kNormT) * 16u;
        const u32x4 hv = buffer_load16(hrs, off);
        wv[u] = buffer_load16(wrs, off);
#pragma unroll
        for (int e = 0; e < 4; ++e) x[u][e] = __uint_as_float(hv[e]);
    }
    // The residual plus the slices in order: ((h + d0) + d1) + ...
    for (int s0 = 0; s0 < slices; s0 += 8) {
        u32x4 dv[8][NV];
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
            for (int u = 0; u < NV; ++u)
                // Past the row a load would reach the next slice: read zeros instead.
                dv[e][u] = buffer_load16(drs, (s0 + e < slices && 4 * static_cast<int>(threadIdx.x + u * kNormT) < dim)
                                                  ? (static_cast<uint32_t>(s0 + e) * row_bytes +
                                                     (threadIdx.x + u * kNormT) * 16u)
                                                  : 0xfffffff0u);
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (s0 + e < slices)
#pragma unroll
                for (int u = 0; u < NV; ++u)
#pragma unroll
                    for (int c = 0; c < 4; ++c) x[u][c] = x[u][c] + __uint_as_float(dv[e][u][c]);
    }
    float s = 0.0f;
#pragma unroll
    for (int u = 0; u < NV; ++u)
#pragma unroll
        for (int c = 0; c < 4; ++c) s = fmaf(x[u][c], x[u][c], s);
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormT / 64; ++i) tot += part[i];
    const float inv = 1.0f / sqrtf(tot / static_cast<float>(dim) + eps);
#pragma unroll
    for (int u = 0; u < NV; ++u) {
        const int i4 = threadIdx.x + u * kNormT;
        if (4 * i4 < dim) {
            if (slices > 0) *reinterpret_cast<float4*>(h + 4 * i4) = make_float4(x[u][0], x[u][1], x[u][2], x[u][3]);
            float4 y;
            y.x = x[u][0] * inv * __uint_as_float(wv[u][0]);
            y.y = x[u][1] * inv * __uint_as_float(wv[u][1]);
            y.z = x[u][2] * inv * __uint_as_float(wv[u][2]);
            y.w = x[u][3] * inv * __uint_as_float(wv[u][3]);
            *reinterpret_cast<float4*>(hn + 4 * i4) = y;
        }
    }
}

// ---- out[j] = sum over s of in[s * n + j], slices in order.
// With per-split sums of squares `ss` the sum is multiplied by the RMSNorm
// scale 1 / sqrt(sum(ss) / ss_dim + eps) (see VM_HIP_GEMV_SRC_NORMRES).
__global__ void slices_sum_kernel(const float* __restrict__ in, int slices, int64_t n, float* __restrict__ out,
                                  const float* __restrict__ ss, int ss_count, float ss_dim, float eps) {
    float iv = 1.0f;
    if (ss && ss_count > 0) {
        float t = 0.0f;
        for (int i = 0; i < ss_count; ++i) t += ss[i];
        iv = 1.0f / sqrtf(t / ss_dim + eps);
    }
    for (int64_t j = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; j < n; j += static_cast<int64_t>(gridDim.x) * kT)
        out[j] = slice_sum(in + j, slices, n) * iv;
}

// ---- RoPE on the fused QKV projection and in-place KV append.
// qkv rows: [S, (H + 2 Hkv) * D] = q heads, k heads, v heads.  Row r sits
// at position p = *pos + r: q is rotated into q_out [H, S, D] (the graph's
// q3t layout), k is rotated and v copied into the caches [Hkv, max_seq, D]
// at row p.  Rows at or past max_seq are dropped (the host never launches
// them; the check keeps every write in bounds).
__global__ void rope_kv_append_kernel(const float* __restrict__ qkv, const float* __restrict__ cos_t,
                                      const float* __restrict__ sin_t, const int32_t* __restrict__ pos,
                                      float* __restrict__ q_out, float* __restrict__ k_cache,
                                      float* __restrict__ v_cache, int64_t rows, int64_t heads, int64_t kv_heads,
                                      int64_t d, int64_t max_seq, int slices) {
    const int64_t half = d / 2;
    const int64_t width = (heads + 2 * kv_heads) * d;
    const int64_t p0 = pos[0];
    // Work items: per row, (heads + kv_heads) * half rotations and kv_heads * d copies.
    const int64_t rot = (heads + kv_heads) * half;
    const int64_t per_row = rot + kv_heads * d;
    const int64_t total = rows * per_row;
    for (int64_t e = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; e < total;
         e += static_cast<int64_t>(gridDim.x) * kT) {
        const int64_t r = e / per_row;
        const int64_t t = e - r * per_row;
        const int64_t p = p0 + r;
        if (p < 0 || p >= max_seq) continue;
        const float* src = qkv + r * width;
        if (t < rot) {
            const int64_t hh = t / half;
            const int64_t j = t - hh * half;
            const float* x = src + hh * d;
            const int64_t stride = rows * width;
            const float a = slice_sum(x + j, slices, stride), b = slice_sum(x + j + half, slices, stride);
            const float c = cos_t[p * half + j], s = sin_t[p * half + j];
            const float y0 = a * c - b * s;
            const float y1 = b * c + a * s;
            if (hh < heads) {
                float* q = q_out + (hh * rows + r) * d;
                q[j] = y0;
                q[j + half] = y1;
            } else {
                float* kc = k_cache + ((hh - heads) * max_seq + p) * d;
                kc[j] = y0;
                kc[j + half] = y1;
            }
        } else {
            const int64_t u = t - rot;
            const int64_t hv = u / d;
            const int64_t j = u - hv * d;
            v_cache[(hv * max_seq + p) * d + j] = slice_sum(src + (heads + kv_heads + hv) * d + j, slices, rows * width);
        }
    }
}

// ---- Decode attention over the resident cache: query rows [H, 1, D] at
// position *pos see keys 0 .. *pos (n = *pos + 1 keys).  Grid (chunks, Hkv),
// chunks = ceil(max_seq / CHUNK) so that the launch does not depend on the
// position; workgroups whose chunk starts at or past n exit at once.  A
// workgroup takes CHUNK keys of one KV head and the G = H / Hkv query heads
// that share it (no RepeatKV copy):
//   1. every thread issues its 16-byte loads of q, K and V (one memory
//      round trip) into LDS;
//   2. thread (j, g-slot) scores key j against its query heads; the CHUNK
//      (= 32) lanes of a key row reduce max and sum with DPP and a row swap
//      (decode_attn.h);
//   3. thread (g, float4 column) accumulates p . V over the chunk.
// With one chunk the result is written directly.  Otherwise each chunk
// stores (m, l, o) with agent-scope stores, takes a ticket once they are
// acknowledged, and the last chunk of the KV head merges the partials in
// chunk order (online softmax rescaling), reading them in batches of
// independent loads.  The per-stream counters are reset by the merger.
template <int D, int CHUNK>
__global__ __launch_bounds__(kT) void attention_decode_kernel(const float* __restrict__ q,
                                                              const float* __restrict__ k_cache,
                                                              const float* __restrict__ v_cache,
                                                              const int32_t* __restrict__ pos, float* __restrict__ out,
                                                              int heads, int kv_heads, int max_seq, float scale,
                                                              float* __restrict__ partials,
                                                              unsigned* __restrict__ counters) {
    constexpr int kMaxG = 16;
    constexpr int D4 = D / 4;
    constexpr int kKS = D + 4;             // padded key row in LDS (floats)
    constexpr int kPart = D + 4;           // partial record: m, l, -, -, o[0..D)
    constexpr int QV = (kMaxG * D4 + kT - 1) / kT;
    constexpr int KV = CHUNK * D4 / kT;    // 16-byte loads per thread for a K (or V) chunk
    static_assert(CHUNK == ChunkAttention<D>::kChunk && kMaxG == ChunkAttention<D>::kMaxG, "decode_attn.h tile");
    static_assert(CHUNK * D4 % kT == 0 && kT % D4 == 0, "tile shape");
    __shared__ __align__(16) float sq[kMaxG * D];
    __shared__ __align__(16) float sk[CHUNK * kKS];
    __shared__ __align__(16) float sv[CHUNK * D];
    __shared__ float sp[kMaxG][CHUNK];
    __shared__ float sm[kMaxG], sl[kMaxG];
    __shared__ unsigned ticket;

    const int chunk = blockIdx.x;
    const int hk = blockIdx.y;
    const int G = heads / kv_heads;
    const int tid = threadIdx.x;
    const int n_keys = min(pos[0] + 1, max_seq);
    const int nc = (n_keys + CHUNK - 1) / CHUNK;
    if (chunk >= nc) return;
    const int k0 = chunk * CHUNK;
    const int nk = min(CHUNK, n_keys - k0);

    {
        const __amdgpu_buffer_rsrc_t qrs = buffer_rsrc(q + static_cast<int64_t>(hk) * G * D,
                                                       static_cast<uint32_t>(G * D) * 4u);
        const uint32_t kv_bytes = static_cast<uint32_t>(nk * D) * 4u;
        const int64_t kv_off = (static_cast<int64_t>(hk) * max_seq + k0) * D;
        const __amdgpu_buffer_rsrc_t krs = buffer_rsrc(k_cache + kv_off, kv_bytes);
        const __amdgpu_buffer_rsrc_t vrs = buffer_rsrc(v_cache + kv_off, kv_bytes);
        u32x4 tq[QV], tk[KV], tv[KV];
#pragma unroll
        for (int u = 0; u < QV; ++u) tq[u] = buffer_load16(qrs, (tid + u * kT) * 16u);
#pragma unroll
        for (int u = 0; u < KV; ++u) {
            tk[u] = buffer_load16(krs, (tid + u * kT) * 16u);
            tv[u] = buffer_load16(vrs, (tid + u * kT) * 16u);
        }
#pragma unroll
        for (int u = 0; u < QV; ++u) {
            const int e = tid + u * kT;
            if (e < kMaxG * D4) *reinterpret_cast<u32x4*>(sq + 4 * e) = tq[u];
        }
#pragma unroll
        for (int u = 0; u < KV; ++u) {
            const int e = tid + u * kT;
            const int j = e / D4, c = e - j * D4;
            *reinterpret_cast<u32x4*>(sk + j * kKS + 4 * c) = tk[u];
            *reinterpret_cast<u32x4*>(sv + 4 * e) = tv[u];
        }
    }
    __syncthreads();

    // Scores, softmax partial and p . V (decode_attn.h).
    using CA = ChunkAttention<D>;
    CA::scores(sq, sk, sp, sm, sl, G, nk, scale);
    __syncthreads();
    CA::pv(sv, sp, G, nk, [&](int g, int c4, float4 acc) {
        if (nc == 1) {
            const float inv = 1.0f / sl[g];
            *reinterpret_cast<float4*>(out + (static_cast<int64_t>(hk) * G + g) * D + 4 * c4) =
                make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
        } else {
            float* part = partials + ((static_cast<int64_t>(hk) * G + g) * gridDim.x + chunk) * kPart;
            coherent_store(part + 4 + 4 * c4 + 0, acc.x);
            coherent_store(part + 4 + 4 * c4 + 1, acc.y);
            coherent_store(part + 4 + 4 * c4 + 2, acc.z);
            coherent_store(part + 4 + 4 * c4 + 3, acc.w);
            if (c4 == 0) {
                coherent_store(part, sm[g]);
                coherent_store(part + 1, sl[g]);
            }
        }
    });
    if (nc == 1) return;
    publish_partials();
    __syncthreads();
    if (tid == 0) ticket = ticket_take(&counters[hk], static_cast<unsigned>(nc));
    __syncthreads();
    if (ticket != static_cast<unsigned>(nc - 1)) return;

    // Merge in chunk order: running (M, L, O) rescaled by exp(M - M');
    // thread (c4 = tid % D4, heads tid / D4 + i * kT / D4).
    constexpr int kB = 16;
    const int c4 = tid % D4;
    for (int g = tid / D4; g < G; g += kT / D4) {
        const float* base = partials + (static_cast<int64_t>(hk) * G + g) * gridDim.x * kPart;
        float M = -INFINITY, Lsum = 0.0f;
        float4 O = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int c0 = 0; c0 < nc; c0 += kB) {
            float mc[kB], lc[kB], oc[kB][4];
#pragma unroll
            for (int u = 0; u < kB; ++u) {
                const float* rec = base + (c0 + u) * kPart;
                const bool ok = c0 + u < nc;
                mc[u] = ok ? coherent_load(rec) : -INFINITY;
                lc[u] = ok ? coherent_load(rec + 1) : 0.0f;
#pragma unroll
                for (int e = 0; e < 4; ++e) oc[u][e] = ok ? coherent_load(rec + 4 + 4 * c4 + e) : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < kB; ++u) {
                if (c0 + u < nc) {
                    const float Mn = fmaxf(M, mc[u]);
                    const float a = M > -INFINITY ? expf(M - Mn) : 0.0f;
                    const float b = expf(mc[u] - Mn);
                    Lsum = fmaf(Lsum, a, lc[u] * b);
                    O.x = fmaf(O.x, a, oc[u][0] * b);
                    O.y = fmaf(O.y, a, oc[u][1] * b);
                    O.z = fmaf(O.z, a, oc[u][2] * b);
                    O.w = fmaf(O.w, a, oc[u][3] * b);
                    M = Mn;
                }
            }
        }
        const float inv = 1.0f / Lsum;
        *reinterpret_cast<float4*>(out + (static_cast<int64_t>(hk) * G + g) * D + 4 * c4) =
            make_float4(O.x * inv, O.y * inv, O.z * inv, O.w * inv);
    }
    if (tid == 0) __hip_atomic_store(&counters[hk], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- Prefetch into the memory-side cache.  A decode step is a chain of
// latency-bound launches that leave many CUs idle; extra workgroups of one
// launch read (and discard) the weights of the launches that follow, which
// then find them in the 256 MB Infinity Cache instead of HBM.  Workgroup q
// of n reads bytes [q*slab, (q+1)*slab) of the concatenated regions with
// 16-byte loads, kBatch in flight per thread.  The loaded words feed a
// store that never happens (pf.count is never negative) so that the loads
// are kept.
__device__ void prefetch_slab(const vm_hip_prefetch& pf, int q, int n, float* sink) {
    constexpr int kBatch = 8;
    uint64_t total = 0;
    for (int r = 0; r < pf.count; ++r) total += pf.bytes[r];
    const uint64_t slab = ((total + n - 1) / n + 15) & ~uint64_t(15);
    const uint64_t lo = static_cast<uint64_t>(q) * slab, hi = min(total, lo + slab);
    uint32_t acc = 0;
    uint64_t base = 0;
    for (int r = 0; r < pf.count; ++r) {
        const uint64_t b0 = max(lo, base), b1 = min(hi, base + pf.bytes[r]);
        if (b0 < b1) {
            const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(pf.ptr[r], static_cast<uint32_t>(pf.bytes[r]));
            const uint32_t e = static_cast<uint32_t>(b1 - base);
            for (uint32_t o = static_cast<uint32_t>(b0 - base) + threadIdx.x * 16u; o < e; o += kT * 16u * kBatch) {
                u32x4 v[kBatch];
#pragma unroll
                for (int u = 0; u < kBatch; ++u) {
                    const uint32_t off = o + static_cast<uint32_t>(u) * kT * 16u;
                    v[u] = buffer_load16(rs, off < e ? off : 0xfffffff0u);
                }
#pragma unroll
                for (int u = 0; u < kBatch; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
            }
        }
        base += pf.bytes[r];
    }
    if (pf.count < 0 && acc == 0x9E3779B9u) sink[0] = 0.0f;
}

// ---- Decode attention fused with its producer's reduction and RoPE: one
// query row per head at position p = *pos, keys 0..p, the projection
// arriving as split-K partial slices [qkv_slices][(H + 2 Hkv) D] whose
// RMSNorm scale 1/rms comes from per-split sums of squares `ss` (see
// VM_HIP_GEMV_SRC_NORMRES; none: scale 1).  Grid (chunks, Hkv) as
// attention_decode_kernel.  Each workgroup
//   1. issues its K/V chunk loads from the cache and, as float4 tasks,
//      the slice sums of its G query heads (and, in the last chunk, of the
//      new key and value), scaled by 1/rms;
//   2. rotates q (and the new key) with the RoPE tables at p
//      (rotary_embedding.cpp:16-45); the last chunk writes the new key and
//      value into the caches at row p and into its own LDS tiles (no other
//      workgroup reads row p);
//   3. scores, softmax partial and p . V as attention_decode_kernel, and
//      stores the chunk's record {m, l, 0, 0, o[D]} with plain stores at
//      part[((hk * G + g) * chunks + chunk) * (D + 4)].
// The merge over chunks is left to the consumer (VM_HIP_GEMV_SRC_ATTN).
// Workgroups past chunks * kv_heads are prefetchers (see prefetch_slab).
template <int D, int CHUNK>
__global__ __launch_bounds__(kT) void attention_decode_slices_kernel(
    const float* __restrict__ qkv, int qkv_slices, const float* __restrict__ ss, int ss_count, float ss_dim,
    float eps, const float* __restrict__ cos_t, const float* __restrict__ sin_t, const int32_t* __restrict__ pos,
    float* __restrict__ k_cache, float* __restrict__ v_cache, float* __restrict__ part, int heads, int kv_heads,
    int max_seq, float scale, int chunks, vm_hip_prefetch pf, int pf_wgs) {
    if (static_cast<int>(blockIdx.x) >= chunks * kv_heads) {
        prefetch_slab(pf, static_cast<int>(blockIdx.x) - chunks * kv_heads, pf_wgs, part);
        return;
    }
    constexpr int kMaxG = 16;
    constexpr int D4 = D / 4;
    constexpr int HALF = D / 2;
    constexpr int kKS = D + 4;
    constexpr int kPart = D + 4;
    constexpr int KV = CHUNK * D4 / kT;
    constexpr int kB = 16;   // slices per batch of loads
    static_assert(CHUNK == ChunkAttention<D>::kChunk && kMaxG == ChunkAttention<D>::kMaxG, "decode_attn.h tile");
    static_assert(CHUNK * D4 % kT == 0 && kT % D4 == 0 && kT % HALF == 0, "tile shape");
    __shared__ __align__(16) float sq[kMaxG * D];
    __shared__ __align__(16) float sk[CHUNK * kKS];
    __shared__ __align__(16) float sv[CHUNK * D];
    __shared__ __align__(16) float knew[D];
    __shared__ __align__(16) float vnew[D];
    __shared__ float sp[kMaxG][CHUNK];
    __shared__ float sm[kMaxG], sl[kMaxG];

    const int chunk = static_cast<int>(blockIdx.x) % chunks;
    const int hk = static_cast<int>(blockIdx.x) / chunks;
    const int G = heads / kv_heads;
    const int tid = threadIdx.x;
    const int k0 = chunk * CHUNK;
    const int width = (heads + 2 * kv_heads) * D;

    // 1. Loads.  Those that do not depend on the position are issued before
    //    it is known (its scalar load is a memory round trip of its own):
    //    the slice sums (tasks [0, G*D4) query float4s, then D4 key and D4
    //    value float4s, used by the last chunk only) and the chunk's K/V
    //    rows from the cache, all CHUNK of them within max_seq (rows past
    //    the position are masked below; row p of the last chunk is
    //    replaced).  Small loads go first: vector memory counters retire in
    //    issue order, so waiting for the slices does not wait for K/V.
    //    Workgroups past the last chunk issue the same loads and skip all
    //    stores (no early return, which would let the loads be moved after
    //    the position test).
    const int tasks1 = G * D4 + 2 * D4;
    constexpr int kTasksMax = (kMaxG * D4 + 2 * D4 + kT - 1) / kT;
    const __amdgpu_buffer_rsrc_t qrs = buffer_rsrc(qkv, static_cast<uint32_t>(qkv_slices * width) * 4u);
    auto task_col = [&](int t, float*& dst) {
        if (t < G * D4) {
            dst = sq + 4 * t;
            return (hk * G) * D + 4 * t;
        }
        if (t < G * D4 + D4) {
            dst = knew + 4 * (t - G * D4);
            return (heads + hk) * D + 4 * (t - G * D4);
        }
        dst = vnew + 4 * (t - G * D4 - D4);
        return (heads + kv_heads + hk) * D + 4 * (t - G * D4 - D4);
    };
    u32x4 l0[kTasksMax][kB];
#pragma unroll
    for (int i = 0; i < kTasksMax; ++i) {
        const int t = tid + i * kT;
        float* dst = nullptr;
        const int col = t < tasks1 ? task_col(t, dst) : 0;
#pragma unroll
        for (int e = 0; e < kB; ++e)
            l0[i][e] = buffer_load16(qrs, (t < tasks1 && e < qkv_slices)
                                              ? static_cast<uint32_t>(e * width + col) * 4u : 0xfffffff0u);
    }
    const uint32_t kv_bytes = static_cast<uint32_t>(max(0, min(CHUNK, max_seq - k0)) * D) * 4u;
    const int64_t kv_off = (static_cast<int64_t>(hk) * max_seq + k0) * D;
    u32x4 tk[KV], tv[KV];
    {
        const __amdgpu_buffer_rsrc_t krs = buffer_rsrc(k_cache + kv_off, kv_bytes);
        const __amdgpu_buffer_rsrc_t vrs = buffer_rsrc(v_cache + kv_off, kv_bytes);
#pragma unroll
        for (int u = 0; u < KV; ++u) {
            tk[u] = buffer_load16(krs, (tid + u * kT) * 16u);
            tv[u] = buffer_load16(vrs, (tid + u * kT) * 16u);
        }
    }
    // The position: keys 0..p; chunks at or past nc are inactive.
    const int n_keys = min(pos[0] + 1, max_seq);
    const int nc = (n_keys + CHUNK - 1) / CHUNK;
    const bool active = chunk < nc;
    const int p = n_keys - 1;
    const int nk = active ? min(CHUNK, n_keys - k0) : 0;
    const bool last = chunk == nc - 1;
    const int jr_pair = tid % HALF;   // pair index of every RoPE task of this thread (kT % HALF == 0)
    const float rc = cos_t[static_cast<int64_t>(p) * HALF + jr_pair];
    const float rs = sin_t[static_cast<int64_t>(p) * HALF + jr_pair];
    {
        float iv = 1.0f;
        if (ss && ss_count > 0) {
            float t = 0.0f;
            for (int i = 0; i < ss_count; ++i) t += ss[i];
            iv = 1.0f / sqrtf(t / ss_dim + eps);
        }
#pragma unroll
        for (int i = 0; i < kTasksMax; ++i) {
            const int t = tid + i * kT;
            if (t >= tasks1) continue;
            float* dst = nullptr;
            const int col = task_col(t, dst);
            float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int e = 0; e < kB; ++e)
                if (e < qkv_slices) {   // slices in order
                    a.x += __uint_as_float(l0[i][e][0]);
                    a.y += __uint_as_float(l0[i][e][1]);
                    a.z += __uint_as_float(l0[i][e][2]);
                    a.w += __uint_as_float(l0[i][e][3]);
                }
            for (int s0 = kB; s0 < qkv_slices; s0 += kB) {   // more than kB slices
                u32x4 l[kB];
#pragma unroll
                for (int e = 0; e < kB; ++e)
                    l[e] = buffer_load16(qrs, s0 + e < qkv_slices ? static_cast<uint32_t>((s0 + e) * width + col) * 4u
                                                                 : 0xfffffff0u);
#pragma unroll
                for (int e = 0; e < kB; ++e)
                    if (s0 + e < qkv_slices) {
                        a.x += __uint_as_float(l[e][0]);
                        a.y += __uint_as_float(l[e][1]);
                        a.z += __uint_as_float(l[e][2]);
                        a.w += __uint_as_float(l[e][3]);
                    }
            }
            *reinterpret_cast<float4*>(dst) = make_float4(a.x * iv, a.y * iv, a.z * iv, a.w * iv);
        }
    }
#pragma unroll
    for (int u = 0; u < KV; ++u) {
        const int e = tid + u * kT;
        const int j = e / D4, c = e - j * D4;
        *reinterpret_cast<u32x4*>(sk + j * kKS + 4 * c) = tk[u];
        *reinterpret_cast<u32x4*>(sv + 4 * e) = tv[u];
    }
    __syncthreads();

    // 2. RoPE at p: query pairs, then (last chunk) the key pairs and value copy.
    {
        const int tasks = G * HALF + (last ? HALF + D : 0);
        const int jr = p - k0;   // the new key's row in this chunk (last chunk)
        for (int t = tid; t < tasks; t += kT) {
            if (t < G * HALF + HALF) {
                const bool is_q = t < G * HALF;
                const int g = is_q ? t / HALF : 0;
                const int j = is_q ? t - g * HALF : t - G * HALF;
                float* x = is_q ? sq + g * D : knew;
                const float c = rc, sn = rs;   // j == tid % HALF for every task of this thread
                const float a = x[j], b = x[j + HALF];
                const float y0 = a * c - b * sn;
                const float y1 = b * c + a * sn;
                if (is_q) {
                    x[j] = y0;
                    x[j + HALF] = y1;
                } else {
                    sk[jr * kKS + j] = y0;
                    sk[jr * kKS + j + HALF] = y1;
                    float* kc = k_cache + (static_cast<int64_t>(hk) * max_seq + p) * D;
                    kc[j] = y0;
                    kc[j + HALF] = y1;
                }
            } else {
                const int d = t - G * HALF - HALF;
                const float v = vnew[d];
                sv[jr * D + d] = v;
                v_cache[(static_cast<int64_t>(hk) * max_seq + p) * D + d] = v;
            }
        }
    }
    __syncthreads();

    // 3. Scores, softmax partial and p . V (decode_attn.h); the chunk's record.
    using CA = ChunkAttention<D>;
    CA::scores(sq, sk, sp, sm, sl, G, nk, scale);
    __syncthreads();
    CA::pv(sv, sp, G, nk, [&](int g, int c4, float4 acc) {
        if (active) {
            float* rec = part + ((static_cast<int64_t>(hk) * G + g) * chunks + chunk) * kPart;
            *reinterpret_cast<float4*>(rec + 4 + 4 * c4) = acc;
            if (c4 == 0) *reinterpret_cast<float4*>(rec) = make_float4(sm[g], sl[g], 0.0f, 0.0f);
        }
    });
}

// ---- Prefill attention over the resident cache with fp32 matrix cores:
// q [H, S, D] rows at positions *pos + i see keys 0 .. *pos + i (causal);
// out [S, H, D] (token-major, the layout the output projection reads).
// A workgroup of four waves takes QR = 16 RW query rows of one head: wave w
// owns rows 16 (w % RW) .. +15 and key group w / RW of KS.  The keys go by
// in steps of KS 64-key tiles staged in LDS; group g runs its online
// softmax over tile g of each step, and the groups' (max, sum, output)
// triples are merged through LDS at the end.  Splitting the keys cuts the
// longest chain of dependent MFMAs (the last query rows see every key) by
// KS; the grid is one-dimensional with the query tiles that see the most
// keys first, so the workgroups dispatched last are the short ones.
//
// v_mfma_f32_16x16x4_f32 (fp32 inputs and accumulation, so no precision is
// given up against the fp32 reference) holds A[i][k] in lane i + 16k,
// B[k][j] in lane j + 16k and D[i][j] in lane j + 16 (i / 4), element i % 4.
// Scores are computed transposed, S^T = K Q^T, so lane (row r = lane % 16,
// group g = lane / 16) holds row r's scores for keys 16b + 4g + e: exactly
// the A operand of P V once the product's reduction index is ordered as
// key(s, k) = 16 (s / 4) + 4k + s % 4 (the order of a sum's terms is free).
// Row statistics live in the lanes of row r (shared across the four
// groups); output row 4g + e fetches its factor from lane 4g + e.
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int D, int RW, int KS>
__global__ __launch_bounds__(256) void attention_prefill_kernel(const float* __restrict__ q,
                                                                const float* __restrict__ k_cache,
                                                                const float* __restrict__ v_cache,
                                                                const int32_t* __restrict__ pos,
                                                                float* __restrict__ out, int rows, int heads,
                                                                int kv_heads, int max_seq, float scale) {
    static_assert(D == 64, "one 16-dim slab per lane group");
    static_assert(RW * KS == 4, "four waves");
    constexpr int KT = 64;          // keys per tile (one key group's share of a step)
    constexpr int ST = KT * KS;     // keys per step
    constexpr int PITCH = D + 4;    // LDS row pitch in floats (conflict-free 16-byte reads)
    constexpr int QR = 16 * RW;     // query rows per workgroup
    __shared__ __align__(16) float sk[ST * PITCH];
    __shared__ __align__(16) float sv[ST * PITCH];
    const int tiles = (rows + QR - 1) / QR;
    const int h = static_cast<int>(blockIdx.x) % heads;
    const int hk = h / (heads / kv_heads);
    const int r0 = (tiles - 1 - static_cast<int>(blockIdx.x) / heads) * QR;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wr = wave % RW, kg = wave / RW;   // row block, key group
    const int lr = lane & 15, lg = lane >> 4;
    const int p0 = pos[0];
    const int n_keys = min(p0 + rows, max_seq);
    const int qrow = r0 + 16 * wr + lr;       // the query row whose Q this lane holds
    const bool row_ok = qrow < rows;
    const int my_last = p0 + qrow;            // keys <= my_last are visible to row qrow
    // keys past this are masked for every row of the wave
    const int wave_last = r0 + 16 * wr < rows ? p0 + min(r0 + 16 * wr + 15, rows - 1) : -1;

    // Q fragment: Q[qrow][16 lg + s], s = 0..15.
    float qf[16];
    {
        const float* qp = q + (static_cast<int64_t>(h) * rows + (row_ok ? qrow : 0)) * D + 16 * lg;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float4 v = row_ok ? *reinterpret_cast<const float4*>(qp + 4 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
            qf[4 * c + 0] = v.x;
            qf[4 * c + 1] = v.y;
            qf[4 * c + 2] = v.z;
            qf[4 * c + 3] = v.w;
        }
    }
    const int wg_end = min(p0 + min(r0 + QR, rows), n_keys);   // keys < wg_end reach some row of the tile
    const float* kb = k_cache + static_cast<int64_t>(hk) * max_seq * D;
    const float* vb = v_cache + static_cast<int64_t>(hk) * max_seq * D;
    f32x4 acc[4];   // O[row 4 lg + e][dim 16 db + lr]
#pragma unroll
    for (int db = 0; db < 4; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.0f;   // statistics of row lr of this wave

    // K/V steps pass through registers one step ahead: the next step's
    // loads are issued as soon as the current one is in LDS, so they are in
    // flight during its scores and p . V.
    constexpr int kU = ST * D / 4 / 256;   // float4s of K (and of V) per thread per step
    float4 nk_reg[kU], nv_reg[kU];
    auto load_step = [&](int t0) {
        const int nkt = min(ST, n_keys - t0);
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int e = tid + u * 256;
            const int j = e / (D / 4), c = e - j * (D / 4);
            nk_reg[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            nv_reg[u] = nk_reg[u];
            if (j < nkt) {
                nk_reg[u] = *reinterpret_cast<const float4*>(kb + static_cast<int64_t>(t0 + j) * D + 4 * c);
                nv_reg[u] = *reinterpret_cast<const float4*>(vb + static_cast<int64_t>(t0 + j) * D + 4 * c);
            }
        }
    };
    if (wg_end > 0) load_step(0);
    for (int s0 = 0; s0 < wg_end; s0 += ST) {
        __syncthreads();   // the previous step is consumed
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int e = tid + u * 256;
            const int j = e / (D / 4), c = e - j * (D / 4);
            *reinterpret_cast<float4*>(sk + j * PITCH + 4 * c) = nk_reg[u];
            *reinterpret_cast<float4*>(sv + j * PITCH + 4 * c) = nv_reg[u];
        }
        if (s0 + ST < wg_end) load_step(s0 + ST);
        __syncthreads();

        const int k0 = s0 + kg * KT;   // this key group's tile
        // a tile wholly past the wave's last visible key (or past the keys)
        // changes nothing
        if (k0 > wave_last || k0 >= n_keys) continue;
        const float* skt = sk + kg * KT * PITCH;
        const float* svt = sv + kg * KT * PITCH;

        // S^T = K Q^T for the four 16-key blocks.
        f32x4 st[4];
#pragma unroll
        for (int nb = 0; nb < 4; ++nb) {
            const float* krow = skt + (16 * nb + lr) * PITCH + 16 * lg;
            float ka[16];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float4 v = *reinterpret_cast<const float4*>(krow + 4 * c);
                ka[4 * c + 0] = v.x;
                ka[4 * c + 1] = v.y;
                ka[4 * c + 2] = v.z;
                ka[4 * c + 3] = v.w;
            }
            f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 16; ++s) d = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[s], qf[s], d, 0, 0, 0);
            st[nb] = d;
        }
        // Scale, causal mask, online softmax of row lr.
        float mt = -INFINITY;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int key = k0 + 16 * nb + 4 * lg + e;
                const bool vis = row_ok && key <= my_last && key < n_keys;
                const float v = vis ? st[nb][e] * scale : -INFINITY;
                st[nb][e] = v;
                mt = fmaxf(mt, v);
            }
        mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
        mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
        const float m_new = fmaxf(m_run, mt);
        float lt = 0.0f;
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float pv = st[nb][e] > -INFINITY ? expf(st[nb][e] - m_new) : 0.0f;
                st[nb][e] = pv;
                lt += pv;
            }
        lt += __shfl_xor(lt, 16, 64);
        lt += __shfl_xor(lt, 32, 64);
        const float alpha = m_run > -INFINITY ? expf(m_run - m_new) : 0.0f;
        l_run = l_run * alpha + lt;
        m_run = m_new;
        // Rescale the output rows 4 lg + e by their rows' factors.
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float ae = __shfl(alpha, 4 * lg + e, 64);
#pragma unroll
            for (int db = 0; db < 4; ++db) acc[db][e] *= ae;
        }
        // O += P V.
#pragma unroll
        for (int db = 0; db < 4; ++db) {
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const int key = 16 * (s / 4) + 4 * lg + (s % 4);
                const float bv = svt[key * PITCH + 16 * db + lr];
                acc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(st[s / 4][s % 4], bv, acc[db], 0, 0, 0);
            }
        }
    }

    // Merge the key groups' triples into group 0 (fixed order: group 0, 1,
    // ..): m = max m_g, l = sum l_g e^(m_g - m), O = sum O_g e^(m_g - m).
    if constexpr (KS > 1) {
        __syncthreads();   // every wave is past its last LDS read
        float* so = sk;                         // [KS - 1][RW][16 rows][D]
        float* sst = sv;                        // [KS - 1][RW][16 rows][2]
        if (kg > 0) {
            float* o = so + ((kg - 1) * RW + wr) * 16 * D;
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int db = 0; db < 4; ++db) o[(4 * lg + e) * D + 16 * db + lr] = acc[db][e];
            if (lg == 0) {
                float* t = sst + (((kg - 1) * RW + wr) * 16 + lr) * 2;
                t[0] = m_run;
                t[1] = l_run;
            }
        }
        __syncthreads();
        if (kg > 0) return;
        float mg[KS], lgs[KS];
        mg[0] = m_run;
        lgs[0] = l_run;
#pragma unroll
        for (int g = 1; g < KS; ++g) {
            const float* t = sst + (((g - 1) * RW + wr) * 16 + lr) * 2;
            mg[g] = t[0];
            lgs[g] = t[1];
        }
        float m = mg[0];
#pragma unroll
        for (int g = 1; g < KS; ++g) m = fmaxf(m, mg[g]);
        float fg[KS];
        float l = 0.0f;
#pragma unroll
        for (int g = 0; g < KS; ++g) {
            fg[g] = mg[g] > -INFINITY ? expf(mg[g] - m) : 0.0f;
            l += lgs[g] * fg[g];
        }
        l_run = l;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float f0 = __shfl(fg[0], 4 * lg + e, 64);
#pragma unroll
            for (int db = 0; db < 4; ++db) acc[db][e] *= f0;
#pragma unroll
            for (int g = 1; g < KS; ++g) {
                const float fe = __shfl(fg[g], 4 * lg + e, 64);
                const float* o = so + ((g - 1) * RW + wr) * 16 * D;
#pragma unroll
                for (int db = 0; db < 4; ++db) acc[db][e] += o[(4 * lg + e) * D + 16 * db + lr] * fe;
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float le = __shfl(l_run, 4 * lg + e, 64);
        const float inv = le > 0.0f ? 1.0f / le : 0.0f;
        const int row = r0 + 16 * wr + 4 * lg + e;
        if (row < rows) {
            float* o = out + (static_cast<int64_t>(row) * heads + h) * D + lr;
#pragma unroll
            for (int db = 0; db < 4; ++db) o[16 * db] = acc[db][e] * inv;
        }
    }
}

// ---- SwiGLU on the fused gate|up projection (llama_graph.cpp:22-28):
// out = (sigmoid(g) * g) * u with g = x[r, j], u = x[r, inter + j].
__global__ void silu_mul_kernel(const float* __restrict__ gu, float* __restrict__ out, int64_t rows, int64_t inter) {
    const int64_t total = rows * inter;
    for (int64_t e = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; e < total;
         e += static_cast<int64_t>(gridDim.x) * kT) {
        const int64_t r = e / inter, j = e - r * inter;
        const float g = gu[r * 2 * inter + j];
        const float u = gu[r * 2 * inter + inter + j];
        const float sig = 1.0f / (1.0f + expf(-g));
        out[e] = (sig * g) * u;
    }
}

// Four elements per thread (inter % 4 == 0, 16-byte aligned operands); the
// same arithmetic as silu_mul_kernel.
__global__ void silu_mul_vec_kernel(const float4* __restrict__ gu, float4* __restrict__ out, int rows, int inter4) {
    const int e = blockIdx.x * kT + threadIdx.x;
    if (e >= rows * inter4) return;
    const int r = e / inter4, j = e - r * inter4;
    const float4 g = gu[r * 2 * inter4 + j];
    const float4 u = gu[r * 2 * inter4 + inter4 + j];
    float4 y;
    y.x = ((1.0f / (1.0f + expf(-g.x))) * g.x) * u.x;
    y.y = ((1.0f / (1.0f + expf(-g.y))) * g.y) * u.y;
    y.z = ((1.0f / (1.0f + expf(-g.z))) * g.z) * u.z;
    y.w = ((1.0f / (1.0f + expf(-g.w))) * g.w) * u.w;
    out[e] = y;
}

// ---- Greedy sampling: first index of the maximum, NaN skipped
// (examples/tinyllama/sample.cpp:18-38).  One workgroup of 1024 threads;
// each pass issues all of a thread's loads (kArgVec 16-byte loads, 32768
// elements per pass for the workgroup) before comparing, so a 32000-entry
// vocabulary costs one memory round trip.  Elements are visited in
// increasing index order per thread and ties resolve to the lower index,
// so the result is the first maximum whatever the schedule.  With `pos`,
// the token is also stored at tokens[*pos + 1] (the sequence buffer) and
// *pos advances by one.
constexpr int kArgT = 1024;
constexpr int kArgVec = 8;

__device__ __forceinline__ bool argmax_better(float v1, int i1, float v2, int i2) {
    if (i2 < 0) return false;
    if (i1 < 0) return true;
    return v2 > v1 || (v2 == v1 && i2 < i1);
}

__global__ __launch_bounds__(kArgT) void argmax_kernel(const float* __restrict__ x, int64_t n,
                                                       int32_t* __restrict__ token_out, int32_t* __restrict__ pos,
                                                       int32_t* __restrict__ tokens, int64_t max_seq, int vec,
                                                       int slices) {
    __shared__ float bv[kArgT / 64];
    __shared__ int bi[kArgT / 64];
    float best = -INFINITY;
    int idx = -1;
    if (vec) {
        // 16-byte aligned x: element 4q + c of pass p is x[p * 32768 + 4 * (tid + u * 1024) + c].
        // Slices (split-K partial logits [slices][n]) are added in slice
        // order before the comparison.
        const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(x, static_cast<uint32_t>(n * slices) * 4u);
        constexpr int kPass = kArgT * kArgVec * 4;
        for (int64_t p0 = 0; p0 < n; p0 += kPass) {
            float t[kArgVec][4];
            {
                u32x4 l[kArgVec];
#pragma unroll
                for (int u = 0; u < kArgVec; ++u)
                    l[u] = buffer_load16(rs, static_cast<uint32_t>(p0 + 4 * (threadIdx.x + u * kArgT)) * 4u);
#pragma unroll
                for (int u = 0; u < kArgVec; ++u)
#pragma unroll
                    for (int c = 0; c < 4; ++c) t[u][c] = __uint_as_float(l[u][c]);
            }
            for (int sl = 1; sl < slices; ++sl) {
                u32x4 l[kArgVec];
#pragma unroll
                for (int u = 0; u < kArgVec; ++u)
                    l[u] = buffer_load16(rs, static_cast<uint32_t>(sl * n + p0 + 4 * (threadIdx.x + u * kArgT)) * 4u);
#pragma unroll
                for (int u = 0; u < kArgVec; ++u)
#pragma unroll
                    for (int c = 0; c < 4; ++c) t[u][c] += __uint_as_float(l[u][c]);
            }
#pragma unroll
            for (int u = 0; u < kArgVec; ++u)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int64_t i = p0 + 4 * (threadIdx.x + u * kArgT) + c;
                    const float v = t[u][c];
                    if (i < n && v == v && (idx < 0 || v > best)) {
                        best = v;
                        idx = static_cast<int>(i);
                    }
                }
        }
    } else {
        for (int64_t i = threadIdx.x; i < n; i += kArgT) {
            float v = x[i];
            for (int sl = 1; sl < slices; ++sl) v += x[sl * n + i];
            if (v != v) continue;
            if (idx < 0 || v > best) {
                best = v;
                idx = static_cast<int>(i);
            }
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(best, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        if (argmax_better(best, idx, ov, oi)) {
            best = ov;
            idx = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        bv[threadIdx.x >> 6] = best;
        bi[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = bv[0];
        int bidx = bi[0];
        for (int w = 1; w < kArgT / 64; ++w)
            if (argmax_better(b, bidx, bv[w], bi[w])) {
                b = bv[w];
                bidx = bi[w];
            }
        token_out[0] = bidx;
        if (pos) {
            const int next = pos[0] + 1;
            if (tokens && next >= 0 && next < max_seq) tokens[next] = bidx;
            pos[0] = next;
        }
    }
}

// ---- Greedy argmax over the sum of split-K slices, across workgroups.
// The single-workgroup argmax_kernel reads every slice of the vocabulary
// through one CU; here workgroup w takes elements [1024 w, 1024 (w + 1))
// (a float4 per thread), issues the loads of up to kAmSl slices at once,
// adds them in slice order, and leaves its first maximum (NaN skipped) in
// the workspace; the last workgroup to finish (atomic ticket; the partials
// are stored with agent-scope stores and acknowledged before it) reduces
// the candidates with the same rule -- maximum, lowest index on ties, so
// the result does not depend on which workgroup finishes last -- writes
// the token, advances *pos and resets the ticket for the next call.
constexpr int kAmT = 256;
constexpr int kAmPer = 4 * kAmT;
constexpr int kAmSl = 8;

__global__ __launch_bounds__(kAmT) void argmax_slices_multi_kernel(
    const float* __restrict__ x, int n, int slices, int32_t* __restrict__ token_out, int32_t* __restrict__ pos,
    int32_t* __restrict__ tokens, int64_t max_seq, float* __restrict__ part_v, int* __restrict__ part_i,
    unsigned* __restrict__ counter) {
    __shared__ float bv[kAmT / 64];
    __shared__ int bi[kAmT / 64];
    __shared__ unsigned ticket;
    const int tid = threadIdx.x;
    const int base = static_cast<int>(blockIdx.x) * kAmPer + 4 * tid;
    const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(x, static_cast<uint32_t>(n) * static_cast<uint32_t>(slices) * 4u);
    float t[4] = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < slices; s0 += kAmSl) {
        u32x4 l[kAmSl];
#pragma unroll
        for (int u = 0; u < kAmSl; ++u)
            l[u] = buffer_load16(rs, (s0 + u < slices && base < n)
                                         ? (static_cast<uint32_t>(s0 + u) * static_cast<uint32_t>(n) + base) * 4u
                                         : 0xfffffff0u);
#pragma unroll
        for (int u = 0; u < kAmSl; ++u)
            if (s0 + u < slices) {   // slices in order; slice 0 is taken as is
#pragma unroll
                for (int c = 0; c < 4; ++c) t[c] = s0 + u == 0 ? __uint_as_float(l[u][c]) : t[c] + __uint_as_float(l[u][c]);
            }
    }
    float best = -INFINITY;
    int idx = -1;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const float v = t[c];
        if (base + c < n && v == v && (idx < 0 || v > best)) {
            best = v;
            idx = base + c;
        }
    }
    auto reduce = [&]() {
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(best, off, 64);
            const int oi = __shfl_xor(idx, off, 64);
            if (argmax_better(best, idx, ov, oi)) {
                best = ov;
                idx = oi;
            }
        }
        if ((tid & 63) == 0) {
            bv[tid >> 6] = best;
            bi[tid >> 6] = idx;
        }
        __syncthreads();
        if (tid == 0)
            for (int w = 1; w < kAmT / 64; ++w)
                if (argmax_better(best, idx, bv[w], bi[w])) {
                    best = bv[w];
                    idx = bi[w];
                }
    };
    reduce();
    if (tid == 0) {
        coherent_store(part_v + blockIdx.x, best);
        __hip_atomic_store(part_i + blockIdx.x, idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        publish_partials();
        ticket = ticket_take(counter, gridDim.x);
    }
    __syncthreads();
    if (ticket != gridDim.x - 1) return;
    best = -INFINITY;
    idx = -1;
    for (int w = tid; w < static_cast<int>(gridDim.x); w += kAmT) {
        const float v = coherent_load(part_v + w);
        const int i = __hip_atomic_load(part_i + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (argmax_better(best, idx, v, i)) {
            best = v;
            idx = i;
        }
    }
    __syncthreads();   // bv / bi are reused
    reduce();
    if (tid == 0) {
        token_out[0] = idx;
        if (pos) {
            const int next = pos[0] + 1;
            if (tokens && next >= 0 && next < max_seq) tokens[next] = idx;
            pos[0] = next;
        }
        __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

int grid_for(int64_t work) {
    const int64_t b = (work + kT - 1) / kT;
    return static_cast<int>(b < 1 ? 1 : (b > 65536 ? 65536 : b));
}

// Validates a prefetch list and sizes its workgroups: about 96 KB each
// (two dozen 16-byte loads per thread), at most 256.
int prefetch_plan(const vm_hip_prefetch* in, vm_hip_prefetch* out, int* wgs) {
    *out = vm_hip_prefetch{};
    *wgs = 0;
    if (!in || in->count == 0) return 0;
    if (in->count < 0 || in->count > VM_HIP_PREFETCH_MAX) return fail_inval("prefetch: count must be in [0, 4]");
    uint64_t total = 0;
    for (int r = 0; r < in->count; ++r) {
        if (in->bytes[r] >= (uint64_t{1} << 31) || (in->bytes[r] > 0 && !in->ptr[r]))
            return fail_inval("prefetch: each region must be non-null and below 2 GiB");
        total += in->bytes[r];
    }
    *out = *in;
    constexpr uint64_t kSlab = 96 * 1024;
    *wgs = static_cast<int>(std::min<uint64_t>(256, (total + kSlab - 1) / kSlab));
    return 0;
}

// ---- Producers that stage the prefill GEMM's activations (a_split.h) in
// the same pass: add + RMSNorm (the GEMM input of q|k|v and gate|up) and
// SiLU(g) * u (the down projection's input).  A workgroup takes R rows;
// thread t holds the 8-groups t + 256 u (u < GT) of each row in registers,
// so a row's largest magnitude is known before its parts are written.  In
// operand order R consecutive rows are R consecutive 16-byte pieces of a
// thread's stores.  `out_f32` (optional) also receives the fp32 rows.
template <int R>
__device__ __forceinline__ void block_reduce_rows(float (&v)[R], float (*part)[kT / 64], bool is_max) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        for (int off = 32; off > 0; off >>= 1) {
            const float o = __shfl_xor(v[r], off, 64);
            v[r] = is_max ? fmaxf(v[r], o) : v[r] + o;
        }
        if ((threadIdx.x & 63) == 0) part[r][threadIdx.x >> 6] = v[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float t = part[r][0];
#pragma unroll
        for (int i = 1; i < kT / 64; ++i) t = is_max ? fmaxf(t, part[r][i]) : t + part[r][i];
        v[r] = t;
    }
    __syncthreads();
}

template <int GT, int R, bool PIECES>
__device__ __forceinline__ void stage_rows(float4 (&y)[R][GT][2], int row0, int m, int k, _Float16* ah,
                                           int* row_exp, int64_t half_elems, float* out_f32,
                                           float (*part)[kT / 64]) {
    const int groups = k / 8;
    float mx[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        mx[r] = 0.0f;
        bool special = false;
#pragma unroll
        for (int u = 0; u < GT; ++u) {
            a_scan4(y[r][u][0], mx[r], special);
            a_scan4(y[r][u][1], mx[r], special);
        }
        // an infinity or NaN anywhere in the row disables the scaling
        if (special) mx[r] = __builtin_inff();
    }
    block_reduce_rows<R>(mx, part, true);
    half8_t* hi = reinterpret_cast<half8_t*>(ah);
    half8_t* lo = reinterpret_cast<half8_t*>(ah + half_elems);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = row0 + r;
        if (row >= m) break;
        const int x = a_row_exponent(mx[r]);
        if (threadIdx.x == 0) row_exp[row] = x;
#pragma unroll
        for (int u = 0; u < GT; ++u) {
            const int g = static_cast<int>(threadIdx.x) + u * kT;
            if (g >= groups) break;
            half8_t h, l;
            a_split8<PIECES>(y[r][u][0], y[r][u][1], x, h, l);
            const int64_t pc = a_piece<PIECES>(row, g, k);
            hi[pc] = h;
            lo[pc] = l;
            if (out_f32) {
                float4* o = reinterpret_cast<float4*>(out_f32 + static_cast<int64_t>(row) * k + 8 * g);
                o[0] = y[r][u][0];
                o[1] = y[r][u][1];
            }
        }
    }
}

template <int GT, int R, bool PIECES>
__global__ __launch_bounds__(kT) void add_rmsnorm_stage_kernel(float* __restrict__ h, const float* __restrict__ delta,
                                                               const float* __restrict__ w, _Float16* __restrict__ ah,
                                                               int* __restrict__ row_exp, int64_t half_elems,
                                                               float* __restrict__ out_f32, int m, int dim, float eps) {
    __shared__ float part[R][kT / 64];
    const int row0 = a_stage_wg(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x)) * R;
    const int groups = dim / 8;
    float4 wv[GT][2];
    float4 y[R][GT][2];
#pragma unroll
    for (int u = 0; u < GT; ++u) {
        const int g = static_cast<int>(threadIdx.x) + u * kT;
        const bool ok = g < groups;
        wv[u][0] = ok ? reinterpret_cast<const float4*>(w)[2 * g] : make_float4(0.f, 0.f, 0.f, 0.f);
        wv[u][1] = ok ? reinterpret_cast<const float4*>(w)[2 * g + 1] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const bool in = ok && row0 + r < m;
            const int64_t base = static_cast<int64_t>(row0 + r) * dim + 8 * g;
            float4 a0 = in ? *reinterpret_cast<const float4*>(h + base) : make_float4(0.f, 0.f, 0.f, 0.f);
            float4 a1 = in ? *reinterpret_cast<const float4*>(h + base + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
            if (delta && in) {
                const float4 d0 = *reinterpret_cast<const float4*>(delta + base);
                const float4 d1 = *reinterpret_cast<const float4*>(delta + base + 4);
                a0 = make_float4(a0.x + d0.x, a0.y + d0.y, a0.z + d0.z, a0.w + d0.w);
                a1 = make_float4(a1.x + d1.x, a1.y + d1.y, a1.z + d1.z, a1.w + d1.w);
            }
            y[r][u][0] = a0;
            y[r][u][1] = a1;
        }
    }
    float ss[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        ss[r] = 0.0f;
#pragma unroll
        for (int u = 0; u < GT; ++u)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const float4 v = y[r][u][q];
                ss[r] = fmaf(v.x, v.x, fmaf(v.y, v.y, fmaf(v.z, v.z, fmaf(v.w, v.w, ss[r]))));
            }
    }
    block_reduce_rows<R>(ss, part, false);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float inv = 1.0f / sqrtf(ss[r] / static_cast<float>(dim) + eps);
        const bool in = row0 + r < m;
#pragma unroll
        for (int u = 0; u < GT; ++u) {
            const int g = static_cast<int>(threadIdx.x) + u * kT;
            if (delta && in && g < groups) {
                float4* hr = reinterpret_cast<float4*>(h + static_cast<int64_t>(row0 + r) * dim + 8 * g);
                hr[0] = y[r][u][0];
                hr[1] = y[r][u][1];
            }
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const float4 v = y[r][u][q], wq = wv[u][q];
                y[r][u][q] = make_float4(v.x * inv * wq.x, v.y * inv * wq.y, v.z * inv * wq.z, v.w * inv * wq.w);
            }
        }
    }
    stage_rows<GT, R, PIECES>(y, row0, m, dim, ah, row_exp, half_elems, out_f32, part);
}

template <int GT, int R, bool PIECES>
__global__ __launch_bounds__(kT) void silu_mul_stage_kernel(const float* __restrict__ gu, _Float16* __restrict__ ah,
                                                            int* __restrict__ row_exp, int64_t half_elems,
                                                            float* __restrict__ out_f32, int m, int inter) {
    __shared__ float part[R][kT / 64];
    const int row0 = a_stage_wg(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x)) * R;
    const int groups = inter / 8;
    float4 y[R][GT][2];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int u = 0; u < GT; ++u) {
            const int g = static_cast<int>(threadIdx.x) + u * kT;
            const bool in = g < groups && row0 + r < m;
            const float* gr = gu + static_cast<int64_t>(row0 + r) * 2 * inter + 8 * g;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const float4 gv = in ? *reinterpret_cast<const float4*>(gr + 4 * q) : make_float4(0.f, 0.f, 0.f, 0.f);
                const float4 uv =
                    in ? *reinterpret_cast<const float4*>(gr + inter + 4 * q) : make_float4(0.f, 0.f, 0.f, 0.f);
                // silu_mul_vec_kernel's arithmetic
                y[r][u][q] = make_float4(((1.0f / (1.0f + expf(-gv.x))) * gv.x) * uv.x,
                                         ((1.0f / (1.0f + expf(-gv.y))) * gv.y) * uv.y,
                                         ((1.0f / (1.0f + expf(-gv.z))) * gv.z) * uv.z,
                                         ((1.0f / (1.0f + expf(-gv.w))) * gv.w) * uv.w);
            }
        }
    stage_rows<GT, R, PIECES>(y, row0, m, inter, ah, row_exp, half_elems, out_f32, part);
}

// Rows per workgroup: as many as the registers allow (4 / GT, at least
// 1, at most 2 for GT = 3) while leaving at least 512 workgroups (two per
// CU, so that one workgroup's loads overlap the other's arithmetic: 512
// rows, SiLU staging for K = 5632 11.9 -> 10.1 us, RMSNorm staging for K =
// 2048 6.6 -> 5.5 us against at least 256); one row when the parts are
// row-major (a row's stores are contiguous already).
// VELOMIND_STAGE_MIN_WGS overrides the minimum (sweeps).
int stage_rows_per_wg(int64_t rows, int gt, bool pieces) {
    if (!pieces) return 1;
    static const int min_wgs = [] {
        const char* e = std::getenv("VELOMIND_STAGE_MIN_WGS");
        return e ? std::max(1, std::atoi(e)) : 512;
    }();
    int r = gt == 1 ? 4 : 2;
    while (r > 1 && (rows + r - 1) / r < min_wgs) r /= 2;
    return r;
}

int check_stage(const void* a_staged, int layout, int64_t rows, int64_t k, const char* who) {
    if (layout != VM_HIP_A_ROWS && layout != VM_HIP_A_PIECES)
        return fail_inval(std::string(who) + ": layout must be VM_HIP_A_ROWS or VM_HIP_A_PIECES");
    if (!a_staged) return fail_inval(std::string(who) + ": null staged buffer");
    static_assert(3 * 8 * kT == kStageMaxK, "staging row limit");
    if (k % 32 != 0 || k > kStageMaxK) return fail_inval(std::string(who) + ": the row length must be a multiple of 32, at most 6144");
    if (rows > 0x7fffffff / 2) return fail_inval(std::string(who) + ": too many rows");
    if (!aligned16(a_staged)) return fail_inval(std::string(who) + ": the staged buffer must be 16-byte aligned");
    return 0;
}

}  // namespace
}  // namespace vmhip

using namespace vmhip;

extern "C" {

int vm_hip_fill_normal_f32(float* dst, int64_t n, uint64_t seed, float mean, float stddev, void* stream) {
    clear_error();
    if (n < 0) return fail_inval("fill_normal: negative size");
    if (n == 0) return 0;
    if (!dst) return fail_inval("fill_normal: null pointer");
    hipLaunchKernelGGL(fill_normal_kernel, dim3(grid_for((n + 1) / 2)), dim3(kT), 0, S(stream), dst, n, seed, mean,
                       stddev);
    return check_launch("fill_normal", S(stream));
}

int vm_hip_add_rmsnorm_f32(float* h, const float* delta, const float* w, float* hn, int64_t rows, int64_t dim,
                           float eps, void* stream) {
    clear_error();
    if (rows < 0 || dim < 0) return fail_inval("add_rmsnorm: negative size");
    if (rows == 0 || dim == 0) return 0;
    if (!h || !w || !hn) return fail_inval("add_rmsnorm: null pointer");
    if (rows > 0x7fffffff) return fail_inval("add_rmsnorm: too many rows");
    const dim3 grid(static_cast<unsigned>(rows));
    const bool vec = dim % 4 == 0 && dim <= 8 * 4 * kT && aligned16(h) && aligned16(w) && aligned16(hn) &&
                     (!delta || aligned16(delta));
    if (vec) {
        const int d = static_cast<int>(dim);
        if (dim <= 4 * kT)
            hipLaunchKernelGGL(add_rmsnorm_vec_kernel<1>, grid, dim3(kT), 0, S(stream), h, delta, w, hn, d, eps);
        else if (dim <= 2 * 4 * kT)
            hipLaunchKernelGGL(add_rmsnorm_vec_kernel<2>, grid, dim3(kT), 0, S(stream), h, delta, w, hn, d, eps);
        else if (dim <= 4 * 4 * kT)
            hipLaunchKernelGGL(add_rmsnorm_vec_kernel<4>, grid, dim3(kT), 0, S(stream), h, delta, w, hn, d, eps);
        else
            hipLaunchKernelGGL(add_rmsnorm_vec_kernel<8>, grid, dim3(kT), 0, S(stream), h, delta, w, hn, d, eps);
    } else {
        hipLaunchKernelGGL(add_rmsnorm_kernel, grid, dim3(kT), 0, S(stream), h, delta, w, hn, dim, eps);
    }
    return check_launch("add_rmsnorm", S(stream));
}

int vm_hip_rope_kv_append_f32(const float* qkv, int64_t rows, const float* cos_table, const float* sin_table,
                              const int32_t* pos, float* q_out, float* k_cache, float* v_cache, int64_t heads,
                              int64_t kv_heads, int64_t head_dim, int64_t max_seq, void* stream) {
    clear_error();
    if (rows < 0 || heads < 1 || kv_heads < 1 || head_dim < 2 || head_dim % 2 || max_seq < 1 || heads % kv_heads)
        return fail_inval("rope_kv_append: bad shape");
    if (rows == 0) return 0;
    if (!qkv || !cos_table || !sin_table || !pos || !q_out || !k_cache || !v_cache)
        return fail_inval("rope_kv_append: null pointer");
    const int64_t work = rows * ((heads + kv_heads) * (head_dim / 2) + kv_heads * head_dim);
    hipLaunchKernelGGL(rope_kv_append_kernel, dim3(grid_for(work)), dim3(kT), 0, S(stream), qkv, cos_table, sin_table,
                       pos, q_out, k_cache, v_cache, rows, heads, kv_heads, head_dim, max_seq, 1);
    return check_launch("rope_kv_append", S(stream));
}

int vm_hip_attention_decode_f32(const float* q, const float* k_cache, const float* v_cache, const int32_t* pos,
                                float* out, int64_t heads, int64_t kv_heads, int64_t head_dim, int64_t max_seq,
                                float scale, void* stream) {
    clear_error();
    if (heads < 1 || kv_heads < 1 || heads % kv_heads || max_seq < 1) return fail_inval("attention_decode: bad shape");
    if (heads / kv_heads > 16) return fail_inval("attention_decode: more than 16 query heads per KV head");
    if (head_dim != 64 && head_dim != 128) {
        set_error("attention_decode: head_dim must be 64 or 128");
        return VM_HIP_EUNSUPPORTED;
    }
    if (!q || !k_cache || !v_cache || !pos || !out) return fail_inval("attention_decode: null pointer");
    if (max_seq > (1 << 24) || heads > 65535) return fail_inval("attention_decode: too large");
    const int chunk = 32;
    const int64_t chunks = (max_seq + chunk - 1) / chunk;
    if (chunks > 65535) return fail_inval("attention_decode: max_seq too large");
    Workspace ws;
    if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out))
        return fail_inval("attention_decode: operands must be 16-byte aligned");
    if (max_seq * head_dim > (int64_t{1} << 28)) return fail_inval("attention_decode: cache too large");
    int st = get_workspace(S(stream), static_cast<std::size_t>(heads * chunks * (head_dim + 4)),
                           static_cast<std::size_t>(kv_heads), &ws);
    if (st) return st;
    const float sc = scale > 0.0f ? scale : 1.0f / sqrtf(static_cast<float>(head_dim));
    const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(kv_heads));
    if (head_dim == 64)
        hipLaunchKernelGGL((attention_decode_kernel<64, 32>), grid, dim3(kT), 0, S(stream), q, k_cache, v_cache, pos,
                           out, static_cast<int>(heads), static_cast<int>(kv_heads), static_cast<int>(max_seq), sc,
                           ws.partials, ws.counters);
    else
        hipLaunchKernelGGL((attention_decode_kernel<128, 32>), grid, dim3(kT), 0, S(stream), q, k_cache, v_cache,
                           pos, out, static_cast<int>(heads), static_cast<int>(kv_heads), static_cast<int>(max_seq),
                           sc, ws.partials, ws.counters);
    return check_launch("attention_decode", S(stream));
}

// Key groups per prefill-attention workgroup (64 / split query rows each).
// Two when one-group workgroups would number at most 512 (512 rows x 32
// heads: 25.3 us vs 33.7 with one group; 128 rows x 15 heads: 7.2 vs 10.0),
// one for longer prompts, whose grid already spreads (2048 x 32: 219.5 us
// vs 225.0 with two); four groups (139 KB of LDS, one workgroup per CU) were
// slower everywhere.  VELOMIND_ATTN_SPLIT = 1 or 2 overrides (sweeps).
static int attention_prefill_split(int64_t rows, int64_t heads) {
    static const int forced = [] {
        const char* e = std::getenv("VELOMIND_ATTN_SPLIT");
        const int v = e ? std::atoi(e) : 0;
        return (v == 1 || v == 2) ? v : 0;
    }();
    if (forced) return forced;
    return (rows + 63) / 64 * heads <= 512 ? 2 : 1;
}

int vm_hip_attention_prefill_f32(const float* q, const float* k_cache, const float* v_cache, const int32_t* pos,
                                 float* out, int64_t rows, int64_t heads, int64_t kv_heads, int64_t head_dim,
                                 int64_t max_seq, float scale, void* stream) {
    clear_error();
    if (rows < 0 || heads < 1 || kv_heads < 1 || heads % kv_heads || max_seq < 1)
        return fail_inval("attention_prefill: bad shape");
    if (head_dim != 64) {
        set_error("attention_prefill: head_dim must be 64");
        return VM_HIP_EUNSUPPORTED;
    }
    if (rows == 0) return 0;
    if (!q || !k_cache || !v_cache || !pos || !out) return fail_inval("attention_prefill: null pointer");
    if (rows > max_seq || heads > 65535 || max_seq > (1 << 24) || (rows + 15) / 16 * heads > INT32_MAX)
        return fail_inval("attention_prefill: too large");
    const float sc = scale > 0.0f ? scale : 1.0f / sqrtf(static_cast<float>(head_dim));
    const int split = attention_prefill_split(rows, heads);
    const int r = static_cast<int>(rows), hd = static_cast<int>(heads), kvh = static_cast<int>(kv_heads),
              ms = static_cast<int>(max_seq);
    const int qr = 64 / split;   // query rows per workgroup
    const dim3 grid(static_cast<unsigned>(((rows + qr - 1) / qr) * heads));
    if (split == 1)
        hipLaunchKernelGGL((attention_prefill_kernel<64, 4, 1>), grid, dim3(256), 0, S(stream), q, k_cache, v_cache,
                           pos, out, r, hd, kvh, ms, sc);
    else
        hipLaunchKernelGGL((attention_prefill_kernel<64, 2, 2>), grid, dim3(256), 0, S(stream), q, k_cache, v_cache,
                           pos, out, r, hd, kvh, ms, sc);
    return check_launch("attention_prefill", S(stream));
}

int vm_hip_silu_mul_f32(const float* gate_up, float* out, int64_t rows, int64_t inter, void* stream) {
    clear_error();
    if (rows < 0 || inter < 0) return fail_inval("silu_mul: negative size");
    if (rows == 0 || inter == 0) return 0;
    if (!gate_up || !out) return fail_inval("silu_mul: null pointer");
    if (inter % 4 == 0 && rows * inter <= 0x7fffffff && aligned16(gate_up) && aligned16(out)) {
        const int total4 = static_cast<int>(rows * inter / 4);
        hipLaunchKernelGGL(silu_mul_vec_kernel, dim3((total4 + kT - 1) / kT), dim3(kT), 0, S(stream),
                           reinterpret_cast<const float4*>(gate_up), reinterpret_cast<float4*>(out),
                           static_cast<int>(rows), static_cast<int>(inter / 4));
    } else {
        hipLaunchKernelGGL(silu_mul_kernel, dim3(grid_for(rows * inter)), dim3(kT), 0, S(stream), gate_up, out, rows,
                           inter);
    }
    return check_launch("silu_mul", S(stream));
}

int vm_hip_add_rmsnorm_stage_f32(float* h, const float* delta, const float* w, void* a_staged, int layout,
                                 float* hn_out, int64_t rows, int64_t dim, float eps, void* stream) {
    clear_error();
    if (rows < 0 || dim < 0) return fail_inval("add_rmsnorm_stage: negative size");
    if (rows == 0 || dim == 0) return 0;
    if (!h || !w) return fail_inval("add_rmsnorm_stage: null pointer");
    VM_TRY(check_stage(a_staged, layout, rows, dim, "add_rmsnorm_stage"));
    if (!aligned16(h) || !aligned16(w) || (delta && !aligned16(delta)) || (hn_out && !aligned16(hn_out)))
        return fail_inval("add_rmsnorm_stage: operands must be 16-byte aligned");
    const bool pieces = layout == VM_HIP_A_PIECES;
    const int gt = static_cast<int>((dim / 8 + kT - 1) / kT);
    const int r = stage_rows_per_wg(rows, gt, pieces);
    const int64_t half_elems = static_cast<int64_t>(a_stage_rows(rows, pieces)) * dim;
    auto* ah = static_cast<_Float16*>(a_staged);
    auto* rexp = reinterpret_cast<int*>(static_cast<char*>(a_staged) + a_stage_half_bytes(rows, dim, pieces));
    const dim3 grid(static_cast<unsigned>((rows + r - 1) / r));
    const int m = static_cast<int>(rows), d = static_cast<int>(dim);
#define VM_STAGE(GX, RX, PX)                                                                                     \
    if (gt == GX && r == RX && pieces == PX)                                                                     \
        hipLaunchKernelGGL((add_rmsnorm_stage_kernel<GX, RX, PX>), grid, dim3(kT), 0, S(stream), h, delta, w, ah, \
                           rexp, half_elems, hn_out, m, d, eps);                                                 \
    else
    VM_STAGE(1, 1, false) VM_STAGE(2, 1, false) VM_STAGE(3, 1, false) VM_STAGE(1, 1, true) VM_STAGE(1, 2, true)
    VM_STAGE(1, 4, true) VM_STAGE(2, 1, true) VM_STAGE(2, 2, true) VM_STAGE(3, 1, true) VM_STAGE(3, 2, true)
#undef VM_STAGE
    return fail_inval("add_rmsnorm_stage: internal error: no kernel for this row length");
    return check_launch("add_rmsnorm_stage", S(stream));
}

int vm_hip_silu_mul_stage_f32(const float* gate_up, void* a_staged, int layout, float* out_f32, int64_t rows,
                              int64_t inter, void* stream) {
    clear_error();
    if (rows < 0 || inter < 0) return fail_inval("silu_mul_stage: negative size");
    if (rows == 0 || inter == 0) return 0;
    if (!gate_up) return fail_inval("silu_mul_stage: null pointer");
    VM_TRY(check_stage(a_staged, layout, rows, inter, "silu_mul_stage"));
    if (!aligned16(gate_up) || (out_f32 && !aligned16(out_f32)))
        return fail_inval("silu_mul_stage: operands must be 16-byte aligned");
    const bool pieces = layout == VM_HIP_A_PIECES;
    const int gt = static_cast<int>((inter / 8 + kT - 1) / kT);
    const int r = stage_rows_per_wg(rows, gt, pieces);
    const int64_t half_elems = static_cast<int64_t>(a_stage_rows(rows, pieces)) * inter;
    auto* ah = static_cast<_Float16*>(a_staged);
    auto* rexp = reinterpret_cast<int*>(static_cast<char*>(a_staged) + a_stage_half_bytes(rows, inter, pieces));
    const dim3 grid(static_cast<unsigned>((rows + r - 1) / r));
    const int m = static_cast<int>(rows), d = static_cast<int>(inter);
#define VM_STAGE(GX, RX, PX)                                                                                     \
    if (gt == GX && r == RX && pieces == PX)                                                                     \
        hipLaunchKernelGGL((silu_mul_stage_kernel<GX, RX, PX>), grid, dim3(kT), 0, S(stream), gate_up, ah, rexp,  \
                           half_elems, out_f32, m, d);                                                           \
    else
    VM_STAGE(1, 1, false) VM_STAGE(2, 1, false) VM_STAGE(3, 1, false) VM_STAGE(1, 1, true) VM_STAGE(1, 2, true)
    VM_STAGE(1, 4, true) VM_STAGE(2, 1, true) VM_STAGE(2, 2, true) VM_STAGE(3, 1, true) VM_STAGE(3, 2, true)
#undef VM_STAGE
    return fail_inval("silu_mul_stage: internal error: no kernel for this row length");
    return check_launch("silu_mul_stage", S(stream));
}

int vm_hip_argmax_f32(const float* x, int64_t n, int32_t* token_out, int32_t* pos, int32_t* tokens, int64_t max_seq,
                      void* stream) {
    clear_error();
    if (n < 1 || n > 0x7fffffff) return fail_inval("argmax: n must be in [1, 2^31)");
    if (!x || !token_out) return fail_inval("argmax: null pointer");
    const int vec = aligned16(x) && n < (int64_t{1} << 29) ? 1 : 0;
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kArgT), 0, S(stream), x, n, token_out, pos, tokens, max_seq, vec,
                       1);
    return check_launch("argmax", S(stream));
}

int vm_hip_add_rmsnorm_slices_f32(float* h, const float* delta, int64_t delta_slices, const float* w, float* hn,
                                  int64_t dim, float eps, void* stream) {
    clear_error();
    if (dim < 4 || dim % 4 != 0 || dim > 4 * 2048) return fail_inval("add_rmsnorm_slices: dim must be a multiple of 4 in [4, 8192]");
    if (delta_slices < 0 || delta_slices > 4096) return fail_inval("add_rmsnorm_slices: delta_slices must be in [0, 4096]");
    if (!h || !w || !hn || (delta_slices > 0 && !delta)) return fail_inval("add_rmsnorm_slices: null pointer");
    if (!aligned16(h) || !aligned16(w) || !aligned16(hn) || (delta && !aligned16(delta)))
        return fail_inval("add_rmsnorm_slices: operands must be 16-byte aligned");
    if (delta_slices * dim * 4 > 0x7fffffffLL) return fail_inval("add_rmsnorm_slices: slices too large");
    const int d = static_cast<int>(dim), sl = static_cast<int>(delta_slices);
    const float* dp = delta ? delta : w;
    if (dim <= 4 * kNormT)
        hipLaunchKernelGGL(add_rmsnorm_slices_kernel<1>, dim3(1), dim3(kNormT), 0, S(stream), h, dp, sl, w, hn, d, eps);
    else if (dim <= 2 * 4 * kNormT)
        hipLaunchKernelGGL(add_rmsnorm_slices_kernel<2>, dim3(1), dim3(kNormT), 0, S(stream), h, dp, sl, w, hn, d, eps);
    else
        hipLaunchKernelGGL(add_rmsnorm_slices_kernel<4>, dim3(1), dim3(kNormT), 0, S(stream), h, dp, sl, w, hn, d, eps);
    return check_launch("add_rmsnorm_slices", S(stream));
}

int vm_hip_rope_kv_append_slices_f32(const float* qkv, int64_t qkv_slices, const float* cos_table,
                                     const float* sin_table, const int32_t* pos, float* q_out, float* k_cache,
                                     float* v_cache, int64_t heads, int64_t kv_heads, int64_t head_dim,
                                     int64_t max_seq, void* stream) {
    clear_error();
    if (heads < 1 || kv_heads < 1 || head_dim < 2 || head_dim % 2 || max_seq < 1 || heads % kv_heads)
        return fail_inval("rope_kv_append_slices: bad shape");
    if (qkv_slices < 1 || qkv_slices > 4096) return fail_inval("rope_kv_append_slices: qkv_slices must be in [1, 4096]");
    if (!qkv || !cos_table || !sin_table || !pos || !q_out || !k_cache || !v_cache)
        return fail_inval("rope_kv_append_slices: null pointer");
    const int64_t work = (heads + kv_heads) * (head_dim / 2) + kv_heads * head_dim;
    hipLaunchKernelGGL(rope_kv_append_kernel, dim3(grid_for(work)), dim3(kT), 0, S(stream), qkv, cos_table, sin_table,
                       pos, q_out, k_cache, v_cache, int64_t{1}, heads, kv_heads, head_dim, max_seq,
                       static_cast<int>(qkv_slices));
    return check_launch("rope_kv_append_slices", S(stream));
}

int vm_hip_argmax_slices_f32(const float* x, int64_t slices, int64_t n, int32_t* token_out, int32_t* pos,
                             int32_t* tokens, int64_t max_seq, void* stream) {
    clear_error();
    if (n < 1 || n > 0x7fffffff) return fail_inval("argmax_slices: n must be in [1, 2^31)");
    if (slices < 1 || slices > 4096) return fail_inval("argmax_slices: slices must be in [1, 4096]");
    if (!x || !token_out) return fail_inval("argmax_slices: null pointer");
    const int vec = aligned16(x) && n % 4 == 0 && n * slices < (int64_t{1} << 29) ? 1 : 0;
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kArgT), 0, S(stream), x, n, token_out, pos, tokens, max_seq, vec,
                       static_cast<int>(slices));
    return check_launch("argmax_slices", S(stream));
}

int64_t vm_hip_argmax_workspace_bytes(int64_t n) {
    if (n < 1) return 0;
    const int64_t wgs = (n + kAmPer - 1) / kAmPer;
    return 256 + wgs * 8;   // ticket, then per-workgroup value and index
}

int vm_hip_argmax_slices_ws_f32(const float* x, int64_t slices, int64_t n, int32_t* token_out, int32_t* pos,
                                int32_t* tokens, int64_t max_seq, void* workspace, int64_t workspace_bytes,
                                void* stream) {
    clear_error();
    if (n < 1 || n > 0x7fffffff) return fail_inval("argmax_slices: n must be in [1, 2^31)");
    if (slices < 1 || slices > 4096) return fail_inval("argmax_slices: slices must be in [1, 4096]");
    if (!x || !token_out || !workspace) return fail_inval("argmax_slices: null pointer");
    if (workspace_bytes < vm_hip_argmax_workspace_bytes(n) || !aligned16(workspace))
        return fail_inval("argmax_slices: workspace smaller than vm_hip_argmax_workspace_bytes(n) or unaligned");
    // 16-byte loads need aligned rows; buffer offsets are 32-bit
    if (!aligned16(x) || n % 4 != 0 || n * slices >= (int64_t{1} << 29))
        return vm_hip_argmax_slices_f32(x, slices, n, token_out, pos, tokens, max_seq, stream);
    const int64_t wgs = (n + kAmPer - 1) / kAmPer;
    auto* ws = static_cast<unsigned char*>(workspace);
    hipLaunchKernelGGL(argmax_slices_multi_kernel, dim3(static_cast<unsigned>(wgs)), dim3(kAmT), 0, S(stream), x,
                       static_cast<int>(n), static_cast<int>(slices), token_out, pos, tokens, max_seq,
                       reinterpret_cast<float*>(ws + 256), reinterpret_cast<int*>(ws + 256 + 4 * wgs),
                       reinterpret_cast<unsigned*>(ws));
    return check_launch("argmax_slices", S(stream));
}

int vm_hip_slices_sum_f32(const float* in, int64_t slices, int64_t n, float* out, void* stream) {
    clear_error();
    if (n < 0 || slices < 1 || slices > 4096) return fail_inval("slices_sum: bad size");
    if (n == 0) return 0;
    if (!in || !out) return fail_inval("slices_sum: null pointer");
    hipLaunchKernelGGL(slices_sum_kernel, dim3(grid_for(n)), dim3(kT), 0, S(stream), in, static_cast<int>(slices), n,
                       out, static_cast<const float*>(nullptr), 0, 1.0f, 0.0f);
    return check_launch("slices_sum", S(stream));
}

int vm_hip_attention_decode_chunks(int64_t head_dim, int64_t max_seq, int* chunk, int* chunks) {
    clear_error();
    if (!chunk || !chunks) return fail_inval("attention_decode_chunks: null pointer");
    if (head_dim != 64 && head_dim != 128) {
        set_error("attention_decode: head_dim must be 64 or 128");
        return VM_HIP_EUNSUPPORTED;
    }
    if (max_seq < 1 || max_seq > (1 << 24)) return fail_inval("attention_decode_chunks: bad max_seq");
    // 32 keys per workgroup: twice the workgroups of 64-key chunks for the
    // same cache, which shortens each workgroup's serial score / p.V phases
    // (measured faster at TinyLlama decode lengths).
    *chunk = 32;
    *chunks = static_cast<int>((max_seq + *chunk - 1) / *chunk);
    return 0;
}

int vm_hip_attention_decode_slices_f32(const float* qkv, int64_t qkv_slices, const float* ss, int64_t ss_count,
                                       float ss_dim, float eps, const float* cos_table, const float* sin_table,
                                       const int32_t* pos, float* k_cache, float* v_cache, float* partials,
                                       int64_t heads, int64_t kv_heads, int64_t head_dim, int64_t max_seq,
                                       float scale, void* stream) {
    return vm_hip_attention_decode_slices_prefetch_f32(qkv, qkv_slices, ss, ss_count, ss_dim, eps, cos_table,
                                                       sin_table, pos, k_cache, v_cache, partials, heads, kv_heads,
                                                       head_dim, max_seq, scale, nullptr, stream);
}

int vm_hip_attention_decode_slices_prefetch_f32(const float* qkv, int64_t qkv_slices, const float* ss,
                                                int64_t ss_count, float ss_dim, float eps, const float* cos_table,
                                                const float* sin_table, const int32_t* pos, float* k_cache,
                                                float* v_cache, float* partials, int64_t heads, int64_t kv_heads,
                                                int64_t head_dim, int64_t max_seq, float scale,
                                                const vm_hip_prefetch* prefetch, void* stream) {
    clear_error();
    int chunk = 0, chunks = 0;
    VM_TRY(vm_hip_attention_decode_chunks(head_dim, max_seq, &chunk, &chunks));
    if (heads < 1 || kv_heads < 1 || heads % kv_heads) return fail_inval("attention_decode_slices: bad shape");
    if (heads / kv_heads > 16) return fail_inval("attention_decode_slices: more than 16 query heads per KV head");
    if (qkv_slices < 1 || qkv_slices > 4096) return fail_inval("attention_decode_slices: qkv_slices must be in [1, 4096]");
    if (ss_count < 0 || (ss_count > 0 && (!ss || ss_dim <= 0.0f)))
        return fail_inval("attention_decode_slices: ss needs ss_count >= 1 and ss_dim > 0");
    if (!qkv || !cos_table || !sin_table || !pos || !k_cache || !v_cache || !partials)
        return fail_inval("attention_decode_slices: null pointer");
    if (!aligned16(qkv) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(partials))
        return fail_inval("attention_decode_slices: operands must be 16-byte aligned");
    if (max_seq * head_dim > (int64_t{1} << 28) || qkv_slices * (heads + 2 * kv_heads) * head_dim * 4 > 0x7fffffffLL ||
        heads > 65535 || kv_heads > 65535)
        return fail_inval("attention_decode_slices: too large");
    vm_hip_prefetch pf{};
    int pf_wgs = 0;
    VM_TRY(prefetch_plan(prefetch, &pf, &pf_wgs));
    const float sc = scale > 0.0f ? scale : 1.0f / sqrtf(static_cast<float>(head_dim));
    const int64_t wgs = static_cast<int64_t>(chunks) * kv_heads + pf_wgs;
    if (wgs > 0x7fffffff) return fail_inval("attention_decode_slices: too large");
    const dim3 grid(static_cast<unsigned>(wgs));
    const int sl = static_cast<int>(qkv_slices), sc_n = static_cast<int>(ss_count);
    if (head_dim == 64)
        hipLaunchKernelGGL((attention_decode_slices_kernel<64, 32>), grid, dim3(kT), 0, S(stream), qkv, sl, ss, sc_n,
                           ss_dim, eps, cos_table, sin_table, pos, k_cache, v_cache, partials,
                           static_cast<int>(heads), static_cast<int>(kv_heads), static_cast<int>(max_seq), sc, chunks,
                           pf, pf_wgs);
    else
        hipLaunchKernelGGL((attention_decode_slices_kernel<128, 32>), grid, dim3(kT), 0, S(stream), qkv, sl, ss, sc_n,
                           ss_dim, eps, cos_table, sin_table, pos, k_cache, v_cache, partials,
                           static_cast<int>(heads), static_cast<int>(kv_heads), static_cast<int>(max_seq), sc, chunks,
                           pf, pf_wgs);
    return check_launch("attention_decode_slices", S(stream));
}

int vm_hip_slices_sum_scaled_f32(const float* in, int64_t slices, int64_t n, const float* ss, int64_t ss_count,
                                 float ss_dim, float eps, float* out, void* stream) {
    clear_error();
    if (n < 0 || slices < 1 || slices > 4096 || ss_count < 0) return fail_inval("slices_sum: bad size");
    if (n == 0) return 0;
    if (!in || !out || (ss_count > 0 && (!ss || ss_dim <= 0.0f))) return fail_inval("slices_sum: null pointer");
    hipLaunchKernelGGL(slices_sum_kernel, dim3(grid_for(n)), dim3(kT), 0, S(stream), in, static_cast<int>(slices), n,
                       out, ss, static_cast<int>(ss_count), ss_dim, eps);
    return check_launch("slices_sum", S(stream));
}

}  // extern "C"
