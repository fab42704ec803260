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

#include <cmath>
#include <cstdint>

#include "vm_device.h"
#include "vm_hip.h"
#include "vm_internal.h"

namespace vmhip {
namespace {

constexpr int kT = 256;

hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }

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

// ---- h += delta (optional), hn = rmsnorm(h) * w, one workgroup per row.
// The add is the reference's Add node (add.cpp) and the norm its RMSNorm
// (rmsnorm.cpp:17-60) on the sum.
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
                                      int64_t d, int64_t max_seq) {
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
            const float a = x[j], b = x[j + half];
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
            v_cache[(hv * max_seq + p) * d + j] = src[(heads + kv_heads + hv) * d + j];
        }
    }
}

// ---- Decode attention over the resident cache: query rows [H, 1, D] at
// position *pos see keys 0..*pos.  Grid (chunks, Hkv): each workgroup takes
// CHUNK keys and the G = H / Hkv query heads of its KV head.
template <int D, int CHUNK>
__global__ __launch_bounds__(kT) void attention_decode_kernel(const float* __restrict__ q,
                                                              const float* __restrict__ k_cache,
                                                              const float* __restrict__ v_cache,
                                                              const int32_t* __restrict__ pos, float* __restrict__ out,
                                                              int heads, int kv_heads, int max_seq, float scale,
                                                              float* __restrict__ partials,
                                                              unsigned* __restrict__ counters) {
    constexpr int kMaxG = 16;
    __shared__ float sq[kMaxG][D];
    __shared__ float sk[CHUNK][D + 1];
    __shared__ float sv[CHUNK][D];
    __shared__ float sp[kMaxG][CHUNK];
    __shared__ float sm[kMaxG], sl[kMaxG];
    __shared__ unsigned ticket;

    const int chunk = blockIdx.x;
    const int chunks = gridDim.x;
    const int hk = blockIdx.y;
    const int g_n = heads / kv_heads;
    const int tid = threadIdx.x;
    const int n_keys = min(pos[0] + 1, max_seq);
    const int k0 = chunk * CHUNK;
    const int nk = max(0, min(CHUNK, n_keys - k0));
    constexpr int kPart = D + 2;

    if (nk > 0) {
        for (int e = tid; e < g_n * D; e += kT) sq[e / D][e % D] = q[(hk * g_n + e / D) * D + e % D];
        const float* kb = k_cache + (static_cast<int64_t>(hk) * max_seq + k0) * D;
        const float* vb = v_cache + (static_cast<int64_t>(hk) * max_seq + k0) * D;
        for (int e = tid; e < nk * D; e += kT) {
            sk[e / D][e % D] = kb[e];
            sv[e / D][e % D] = vb[e];
        }
        __syncthreads();
        for (int e = tid; e < g_n * CHUNK; e += kT) {
            const int g = e / CHUNK, j = e % CHUNK;
            float s = -INFINITY;
            if (j < nk) {
                float dot = 0.0f;
#pragma unroll 16
                for (int t = 0; t < D; ++t) dot = fmaf(sq[g][t], sk[j][t], dot);
                s = dot * scale;
            }
            sp[g][j] = s;
        }
        __syncthreads();
        // Softmax partials per query head: one wave per head, lanes over keys.
        const int wave = tid >> 6, lane = tid & 63;
        for (int g = wave; g < g_n; g += kT / 64) {
            float mx = -INFINITY;
            for (int j = lane; j < CHUNK; j += 64) mx = fmaxf(mx, sp[g][j]);
            for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
            float sum = 0.0f;
            for (int j = lane; j < CHUNK; j += 64) {
                const float pv = j < nk ? expf(sp[g][j] - mx) : 0.0f;
                sp[g][j] = pv;
                sum += pv;
            }
            for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
            if (lane == 0) {
                sm[g] = mx;
                sl[g] = sum;
            }
        }
        __syncthreads();
        for (int e = tid; e < g_n * D; e += kT) {
            const int g = e / D, t = e % D;
            float acc = 0.0f;
            for (int j = 0; j < nk; ++j) acc = fmaf(sp[g][j], sv[j][t], acc);
            float* part = partials + (static_cast<int64_t>(hk * g_n + g) * chunks + chunk) * kPart;
            coherent_store(part + 2 + t, acc);
            if (t == 0) {
                coherent_store(part, sm[g]);
                coherent_store(part + 1, sl[g]);
            }
        }
    } else {
        for (int g = tid; g < g_n; g += kT) {
            float* part = partials + (static_cast<int64_t>(hk * g_n + g) * chunks + chunk) * kPart;
            coherent_store(part, -INFINITY);
            coherent_store(part + 1, 0.0f);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // partial stores acknowledged before the ticket
    __syncthreads();
    if (tid == 0) ticket = __hip_atomic_fetch_add(&counters[hk], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (ticket != static_cast<unsigned>(chunks - 1)) return;

    // Merge: O = sum_c o_c exp(m_c - M) / sum_c l_c exp(m_c - M), chunks in order.
    for (int g = tid; g < g_n; g += kT) {
        const float* base = partials + static_cast<int64_t>(hk * g_n + g) * chunks * kPart;
        float mx = -INFINITY;
        for (int c = 0; c < chunks; ++c) mx = fmaxf(mx, coherent_load(base + c * kPart));
        float l = 0.0f;
        for (int c = 0; c < chunks; ++c) {
            const float mc = coherent_load(base + c * kPart);
            if (mc > -INFINITY) l += coherent_load(base + c * kPart + 1) * expf(mc - mx);
        }
        sm[g] = mx;
        sl[g] = l > 0.0f ? 1.0f / l : 0.0f;
    }
    __syncthreads();
    for (int e = tid; e < g_n * D; e += kT) {
        const int g = e / D, t = e % D;
        const float* base = partials + static_cast<int64_t>(hk * g_n + g) * chunks * kPart;
        float acc = 0.0f;
        for (int c = 0; c < chunks; ++c) {
            const float mc = coherent_load(base + c * kPart);
            if (mc > -INFINITY) acc += coherent_load(base + c * kPart + 2 + t) * expf(mc - sm[g]);
        }
        out[(hk * g_n + g) * D + t] = acc * sl[g];
    }
    if (tid == 0) __hip_atomic_store(&counters[hk], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- Prefill attention over the resident cache: q [H, S, D] rows at
// positions *pos + i, causal over keys 0 .. *pos + i; output [S, H, D]
// (token-major, the layout the output projection reads).  Grid
// (ceil(S/64), H): 64 query rows per workgroup, four threads per row, key
// tiles of 64 through LDS with an online softmax.
template <int D>
__global__ __launch_bounds__(kT) void attention_prefill_kernel(const float* __restrict__ q,
                                                               const float* __restrict__ k_cache,
                                                               const float* __restrict__ v_cache,
                                                               const int32_t* __restrict__ pos,
                                                               float* __restrict__ out, int rows, int heads,
                                                               int kv_heads, int max_seq, float scale) {
    constexpr int kRows = 64, kKeys = 64, kDq = D / 4;
    __shared__ float sq[kRows][D + 1];
    __shared__ float sk[kKeys][D + 1];
    __shared__ float sv[kKeys][D];
    __shared__ float sp[kRows][kKeys + 1];
    const int h = blockIdx.y;
    const int hk = h / (heads / kv_heads);
    const int r0 = blockIdx.x * kRows;
    const int tid = threadIdx.x;
    const int row = tid >> 2, sub = tid & 3;
    const int p0 = pos[0];
    const int n_keys = min(p0 + rows, max_seq);
    const int last_key = min(p0 + min(r0 + kRows, rows), n_keys);  // keys visible to the tile's last row

    for (int e = tid; e < kRows * D; e += kT) {
        const int rr = e / D, t = e % D;
        sq[rr][t] = (r0 + rr < rows) ? q[(static_cast<int64_t>(h) * rows + r0 + rr) * D + t] : 0.0f;
    }
    const int my_pos = p0 + r0 + row;  // absolute position of this thread's query row
    float m = -INFINITY, l = 0.0f;
    float acc[kDq];
#pragma unroll
    for (int i = 0; i < kDq; ++i) acc[i] = 0.0f;
    const float* kb = k_cache + static_cast<int64_t>(hk) * max_seq * D;
    const float* vb = v_cache + static_cast<int64_t>(hk) * max_seq * D;

    for (int k0 = 0; k0 < last_key; k0 += kKeys) {
        __syncthreads();
        const int nk = min(kKeys, last_key - k0);
        for (int e = tid; e < kKeys * D; e += kT) {
            const int j = e / D, t = e % D;
            const bool ok = j < nk;
            sk[j][t] = ok ? kb[static_cast<int64_t>(k0 + j) * D + t] : 0.0f;
            sv[j][t] = ok ? vb[static_cast<int64_t>(k0 + j) * D + t] : 0.0f;
        }
        __syncthreads();
        float tile_max = -INFINITY;
        float s_loc[kKeys / 4];
#pragma unroll
        for (int u = 0; u < kKeys / 4; ++u) {
            const int j = sub + 4 * u;
            float dot = 0.0f;
#pragma unroll 16
            for (int t = 0; t < D; ++t) dot = fmaf(sq[row][t], sk[j][t], dot);
            const bool vis = (j < nk) && (k0 + j <= my_pos);
            s_loc[u] = vis ? dot * scale : -INFINITY;
            tile_max = fmaxf(tile_max, s_loc[u]);
        }
        tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 1, 64));
        tile_max = fmaxf(tile_max, __shfl_xor(tile_max, 2, 64));
        const float m_new = fmaxf(m, tile_max);
        float psum = 0.0f;
#pragma unroll
        for (int u = 0; u < kKeys / 4; ++u) {
            const float pv = s_loc[u] > -INFINITY ? expf(s_loc[u] - m_new) : 0.0f;
            sp[row][sub + 4 * u] = pv;
            psum += pv;
        }
        psum += __shfl_xor(psum, 1, 64);
        psum += __shfl_xor(psum, 2, 64);
        const float alpha = m > -INFINITY ? expf(m - m_new) : 0.0f;
        l = l * alpha + psum;
        m = m_new;
#pragma unroll
        for (int i = 0; i < kDq; ++i) acc[i] *= alpha;
        __syncthreads();
        for (int j = 0; j < nk; ++j) {
            const float pv = sp[row][j];
#pragma unroll
            for (int i = 0; i < kDq; ++i) acc[i] = fmaf(pv, sv[j][sub + 4 * i], acc[i]);
        }
    }
    const int r = r0 + row;
    if (r < rows) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        float* o = out + (static_cast<int64_t>(r) * heads + h) * D;
#pragma unroll
        for (int i = 0; i < kDq; ++i) o[sub + 4 * i] = acc[i] * inv;
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

// ---- Greedy sampling: first index of the maximum, NaN skipped
// (examples/tinyllama/sample.cpp:18-38).  One workgroup of 1024 threads.
// With `pos`, the token is also stored at tokens[*pos + 1] (the sequence
// buffer) and *pos advances by one.
__global__ __launch_bounds__(1024) void argmax_kernel(const float* __restrict__ x, int64_t n,
                                                      int32_t* __restrict__ token_out, int32_t* __restrict__ pos,
                                                      int32_t* __restrict__ tokens, int64_t max_seq) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    float best = -INFINITY;
    int idx = -1;
    for (int64_t i = threadIdx.x; i < n; i += 1024) {
        const float v = x[i];
        if (v != v) continue;
        if (idx < 0 || v > best) {
            best = v;
            idx = static_cast<int>(i);
        }
    }
    auto better = [](float v1, int i1, float v2, int i2) {
        if (i2 < 0) return false;
        if (i1 < 0) return true;
        return v2 > v1 || (v2 == v1 && i2 < i1);
    };
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(best, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        if (better(best, idx, ov, oi)) {
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
        for (int w = 1; w < 16; ++w)
            if (better(b, bidx, bv[w], bi[w])) {
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

int grid_for(int64_t work) {
    const int64_t b = (work + kT - 1) / kT;
    return static_cast<int>(b < 1 ? 1 : (b > 65536 ? 65536 : b));
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
    hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(static_cast<unsigned>(rows)), dim3(kT), 0, S(stream), h, delta, w,
                       hn, dim, eps);
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
                       pos, q_out, k_cache, v_cache, rows, heads, kv_heads, head_dim, max_seq);
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
    const int chunk = head_dim == 64 ? 64 : 32;
    const int64_t chunks = (max_seq + chunk - 1) / chunk;
    if (chunks > 65535) return fail_inval("attention_decode: max_seq too large");
    Workspace ws;
    int st = get_workspace(S(stream), static_cast<std::size_t>(heads * chunks * (head_dim + 2)),
                           static_cast<std::size_t>(kv_heads), &ws);
    if (st) return st;
    const float sc = scale > 0.0f ? scale : 1.0f / sqrtf(static_cast<float>(head_dim));
    const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(kv_heads));
    if (head_dim == 64)
        hipLaunchKernelGGL((attention_decode_kernel<64, 64>), grid, dim3(kT), 0, S(stream), q, k_cache, v_cache, pos,
                           out, static_cast<int>(heads), static_cast<int>(kv_heads), static_cast<int>(max_seq), sc,
                           ws.partials, ws.counters);
    else
        hipLaunchKernelGGL((attention_decode_kernel<128, 32>), grid, dim3(kT), 0, S(stream), q, k_cache, v_cache,
                           pos, out, static_cast<int>(heads), static_cast<int>(kv_heads), static_cast<int>(max_seq),
                           sc, ws.partials, ws.counters);
    return check_launch("attention_decode", S(stream));
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
    if (rows > max_seq || heads > 65535 || max_seq > (1 << 24)) return fail_inval("attention_prefill: too large");
    const float sc = scale > 0.0f ? scale : 1.0f / sqrtf(static_cast<float>(head_dim));
    const dim3 grid(static_cast<unsigned>((rows + 63) / 64), static_cast<unsigned>(heads));
    hipLaunchKernelGGL(attention_prefill_kernel<64>, grid, dim3(kT), 0, S(stream), q, k_cache, v_cache, pos, out,
                       static_cast<int>(rows), static_cast<int>(heads), static_cast<int>(kv_heads),
                       static_cast<int>(max_seq), sc);
    return check_launch("attention_prefill", S(stream));
}

int vm_hip_silu_mul_f32(const float* gate_up, float* out, int64_t rows, int64_t inter, void* stream) {
    clear_error();
    if (rows < 0 || inter < 0) return fail_inval("silu_mul: negative size");
    if (rows == 0 || inter == 0) return 0;
    if (!gate_up || !out) return fail_inval("silu_mul: null pointer");
    hipLaunchKernelGGL(silu_mul_kernel, dim3(grid_for(rows * inter)), dim3(kT), 0, S(stream), gate_up, out, rows,
                       inter);
    return check_launch("silu_mul", S(stream));
}

int vm_hip_argmax_f32(const float* x, int64_t n, int32_t* token_out, int32_t* pos, int32_t* tokens, int64_t max_seq,
                      void* stream) {
    clear_error();
    if (n < 1 || n > 0x7fffffff) return fail_inval("argmax: n must be in [1, 2^31)");
    if (!x || !token_out) return fail_inval("argmax: null pointer");
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, S(stream), x, n, token_out, pos, tokens, max_seq);
    return check_launch("argmax", S(stream));
}

}  // extern "C"
