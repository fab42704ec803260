// The LLaMA graph's other operators on gfx950 (fp32, contiguous tensors):
// everything the reference's decode/prefill graph
// (examples/common/llama/llama_graph.cpp:14-304) runs besides
// QuantizedMatMul.  Semantics follow the reference's CPU kernels
// (src/cpu/ops/*.cpp, cited per entry point in include/vm_hip.h).
//
// All of these move a few KB to a few MB per call, so they are simple
// grid-stride kernels with 16-byte accesses where the shapes allow; the
// exception is attention, which keeps each query row's scores in LDS.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "vm_device.h"
#include "vm_hip.h"
#include "vm_internal.h"

namespace vmhip {
namespace {

constexpr int kT = 256;

int grid_for(int64_t work) {
    const int64_t b = (work + kT - 1) / kT;
    return static_cast<int>(b < 1 ? 1 : (b > 65536 ? 65536 : b));
}

// ---- Embedding: out[i, :] = table[idx[i], :] (embedding.cpp:17-33).
// Rows of out-of-range indices are zero; the executor rejects such indices
// before launching (executable.cpp:54-66).
__global__ void embedding_kernel(const float* __restrict__ table, int64_t vocab, int64_t hidden,
                                 const int32_t* __restrict__ idx, int64_t count, float* __restrict__ out) {
    const int64_t total = count * hidden;
    for (int64_t e = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; e < total;
         e += static_cast<int64_t>(gridDim.x) * kT) {
        const int64_t i = e / hidden;
        const int64_t j = e - i * hidden;
        const int64_t t = idx[i];
        out[e] = (t >= 0 && t < vocab) ? table[t * hidden + j] : 0.0f;
    }
}

// ---- RMSNorm over the last axis: y = x / sqrt(mean(x^2) + eps) * w
// (rmsnorm.cpp:17-60), one workgroup per row.
__global__ __launch_bounds__(kT) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                     float* __restrict__ y, int64_t dim, float eps) {
    __shared__ float part[kT / 64];
    const float* xr = x + blockIdx.x * dim;
    float* yr = y + blockIdx.x * dim;
    float s = 0.0f;
    for (int64_t i = threadIdx.x; i < dim; i += kT) s = fmaf(xr[i], xr[i], s);
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kT / 64; ++i) tot += part[i];
    const float inv = 1.0f / sqrtf(tot / static_cast<float>(dim) + eps);
    for (int64_t i = threadIdx.x; i < dim; i += kT) yr[i] = xr[i] * inv * w[i];
}

// ---- Rotary embedding on rows of head_dim (rotary_embedding.cpp:17-45):
// the first and second halves rotate by (cos, sin) of position
// row % cos_rows.  One rotation, shared by every kernel that applies it so
// that they round alike.
__device__ __forceinline__ void rope_rotate(float a, float b, float c, float s, float* y0, float* y1) {
    *y0 = a * c - b * s;
    *y1 = b * c + a * s;
}

__global__ void rope_kernel(const float* __restrict__ x, const float* __restrict__ cs, const float* __restrict__ sn,
                            float* __restrict__ y, int64_t rows, int64_t head_dim, int64_t cos_rows) {
    const int64_t half = head_dim / 2;
    const int64_t total = rows * half;
    for (int64_t e = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; e < total;
         e += static_cast<int64_t>(gridDim.x) * kT) {
        const int64_t r = e / half;
        const int64_t j = e - r * half;
        const int64_t pos = cos_rows > 1 ? r % cos_rows : 0;
        const float a = x[r * head_dim + j];
        const float b = x[r * head_dim + j + half];
        const float c = cs[pos * half + j];
        const float s = sn[pos * half + j];
        rope_rotate(a, b, c, s, y + r * head_dim + j, y + r * head_dim + j + half);
    }
}

// ---- One decode position's attention inputs in one launch: RoPE on the
// query [hq, 1, d] and on the new key [hkv, 1, d], each appended to its
// cache as Concat(past, new) on the sequence axis (llama_graph.cpp:79-84,
// :296-305), and the new value appended to its cache: q_out [hq, 1, d],
// k_out [hkv, s + 1, d], v_out [hkv, s + 1, dv].  cos/sin hold one row
// (the position).  Elements equal the RoPE and Concat kernels' bit for bit.
__global__ void rope_append_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                   const float* __restrict__ v, const float* __restrict__ pk,
                                   const float* __restrict__ pv, const float* __restrict__ cs,
                                   const float* __restrict__ sn, float* __restrict__ q_out, float* __restrict__ k_out,
                                   float* __restrict__ v_out, int64_t hq, int64_t hkv, int64_t s, int64_t d,
                                   int64_t dv) {
    const int64_t half = d / 2;
    const int64_t n_q = hq * half;               // rotated pairs of the query
    const int64_t n_kn = hkv * half;             // rotated pairs of the new key
    const int64_t n_kp = hkv * s * d;            // cached key elements
    const int64_t n_v = hkv * (s + 1) * dv;      // value cache with the new row
    const int64_t total = n_q + n_kn + n_kp + n_v;
    for (int64_t e = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; e < total;
         e += static_cast<int64_t>(gridDim.x) * kT) {
        if (e < n_q + n_kn) {
            const bool is_q = e < n_q;
            const int64_t p = is_q ? e : e - n_q;
            const int64_t r = p / half, j = p - r * half;
            const float* x = is_q ? q + r * d : k + r * d;
            float* y = is_q ? q_out + r * d : k_out + (r * (s + 1) + s) * d;
            rope_rotate(x[j], x[j + half], cs[j], sn[j], y + j, y + j + half);
        } else if (e < n_q + n_kn + n_kp) {
            const int64_t p = e - n_q - n_kn;
            const int64_t h = p / (s * d), t = p - h * s * d;
            k_out[h * (s + 1) * d + t] = pk[p];
        } else {
            const int64_t p = e - n_q - n_kn - n_kp;
            const int64_t h = p / ((s + 1) * dv), t = p - h * (s + 1) * dv;
            v_out[p] = t < s * dv ? pv[h * s * dv + t] : v[h * dv + (t - s * dv)];
        }
    }
}

// ---- Up to rank-6 index arithmetic for transpose and slice.
struct Dims {
    int rank;
    int64_t out_shape[6];
    int64_t in_step[6];   // input offset per unit step of each OUTPUT axis
    int64_t in_base;
};

__global__ void gather_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t total, Dims d) {
    for (int64_t e = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; e < total;
         e += static_cast<int64_t>(gridDim.x) * kT) {
        int64_t rem = e;
        int64_t off = d.in_base;
        for (int ax = d.rank - 1; ax >= 0; --ax) {
            const int64_t c = rem % d.out_shape[ax];
            rem /= d.out_shape[ax];
            off += c * d.in_step[ax];
        }
        y[e] = x[off];
    }
}

// ---- Concat of two tensors along an axis (concat.cpp:17-60): per outer
// index, a's block then b's block.
__global__ void concat_kernel(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ y,
                              int64_t outer, int64_t a_block, int64_t b_block) {
    const int64_t o_block = a_block + b_block;
    const int64_t total = outer * o_block;
    for (int64_t e = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; e < total;
         e += static_cast<int64_t>(gridDim.x) * kT) {
        const int64_t o = e / o_block;
        const int64_t r = e - o * o_block;
        y[e] = r < a_block ? a[o * a_block + r] : b[o * b_block + (r - a_block)];
    }
}

// ---- RepeatKV (repeat_kv.cpp:17-56): head h of the output copies input
// head h / repeats.
__global__ void repeat_kv_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t outer, int64_t kv_heads,
                                 int64_t repeats, int64_t inner) {
    const int64_t q_heads = kv_heads * repeats;
    const int64_t total = outer * q_heads * inner;
    for (int64_t e = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; e < total;
         e += static_cast<int64_t>(gridDim.x) * kT) {
        const int64_t t = e % inner;
        const int64_t h = (e / inner) % q_heads;
        const int64_t o = e / (inner * q_heads);
        y[e] = x[(o * kv_heads + h / repeats) * inner + t];
    }
}

// ---- Elementwise Add / Mul / Sigmoid (add.cpp, mul.cpp, sigmoid.cpp), and
// the SwiGLU chain Mul(Mul(Sigmoid(a), a), b) in one pass with the same
// three roundings in the same order (the graph compiler's fused step).
__global__ void elementwise_kernel(int op, const float* __restrict__ a, const float* __restrict__ b,
                                   float* __restrict__ y, int64_t n) {
    for (int64_t e = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; e < n;
         e += static_cast<int64_t>(gridDim.x) * kT) {
        const float x = a[e];
        float r;
        if (op == VM_HIP_EW_ADD) r = x + b[e];
        else if (op == VM_HIP_EW_MUL) r = x * b[e];
        else if (op == VM_HIP_EW_SILU_MUL) r = silu_mul_f32(x, b[e]);
        else r = sigmoid_f32(x);
        y[e] = r;
    }
}

// ---- Softmax along an axis of [outer, cols, inner] (softmax.cpp:18-48).
// inner == 1: one wave per row, lanes over the columns.  Otherwise one
// thread per (outer, inner) row walks its strided column.
__global__ __launch_bounds__(kT) void softmax_rows_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                          int64_t rows, int64_t cols) {
    const int lane = threadIdx.x & 63;
    const int64_t r = blockIdx.x * static_cast<int64_t>(kT / 64) + (threadIdx.x >> 6);
    if (r >= rows) return;
    const float* xr = x + r * cols;
    float* yr = y + r * cols;
    float mx = -INFINITY;
    for (int64_t j = lane; j < cols; j += 64) mx = fmaxf(mx, xr[j]);
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    float sum = 0.0f;
    for (int64_t j = lane; j < cols; j += 64) sum += expf(xr[j] - mx);
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    for (int64_t j = lane; j < cols; j += 64) yr[j] = expf(xr[j] - mx) / sum;
}

__global__ void softmax_strided_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t outer,
                                       int64_t cols, int64_t inner) {
    const int64_t rows = outer * inner;
    for (int64_t r = blockIdx.x * static_cast<int64_t>(kT) + threadIdx.x; r < rows;
         r += static_cast<int64_t>(gridDim.x) * kT) {
        const int64_t base = (r / inner) * cols * inner + r % inner;
        float mx = x[base];
        for (int64_t j = 1; j < cols; ++j) mx = fmaxf(mx, x[base + j * inner]);
        float sum = 0.0f;
        for (int64_t j = 0; j < cols; ++j) sum += expf(x[base + j * inner] - mx);
        for (int64_t j = 0; j < cols; ++j) y[base + j * inner] = expf(x[base + j * inner] - mx) / sum;
    }
}

// ---- Batched fp32 matrix product C[b] = A[b] B[b] (matmul.cpp, fp32 path).
// 64x64 output tile per workgroup, 4x4 per thread, K in steps of 16 through
// LDS.  fp32 FMA keeps the result within rounding of the reference's fp32
// dot products.
constexpr int kMmTile = 64;
constexpr int kMmK = 16;

__global__ __launch_bounds__(kT) void matmul_f32_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                        float* __restrict__ c, int64_t m, int64_t k, int64_t n) {
    __shared__ float sA[kMmK][kMmTile + 4];
    __shared__ float sB[kMmK][kMmTile + 4];
    const int64_t bat = blockIdx.z;
    const int64_t row0 = static_cast<int64_t>(blockIdx.y) * kMmTile;
    const int64_t col0 = static_cast<int64_t>(blockIdx.x) * kMmTile;
    const float* ab = a + bat * m * k;
    const float* bb = b + bat * k * n;
    float* cb = c + bat * m * n;
    const int tx = threadIdx.x & 15;   // column group
    const int ty = threadIdx.x >> 4;   // row group
    float acc[4][4] = {};
    for (int64_t k0 = 0; k0 < k; k0 += kMmK) {
        // A tile: 64 rows x 16 k, stored transposed (k-major) in LDS.
        for (int e = threadIdx.x; e < kMmTile * kMmK; e += kT) {
            const int r = e / kMmK, kk = e % kMmK;
            const int64_t gr = row0 + r, gk = k0 + kk;
            sA[kk][r] = (gr < m && gk < k) ? ab[gr * k + gk] : 0.0f;
        }
        for (int e = threadIdx.x; e < kMmTile * kMmK; e += kT) {
            const int kk = e / kMmTile, cc = e % kMmTile;
            const int64_t gk = k0 + kk, gc = col0 + cc;
            sB[kk][cc] = (gk < k && gc < n) ? bb[gk * n + gc] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kMmK; ++kk) {
            float av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) av[i] = sA[kk][ty * 4 + i];
#pragma unroll
            for (int j = 0; j < 4; ++j) bv[j] = sB[kk][tx * 4 + j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t gr = row0 + ty * 4 + i;
        if (gr >= m) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t gc = col0 + tx * 4 + j;
            if (gc < n) cb[gr * n + gc] = acc[i][j];
        }
    }
}

// ---- Attention with grouped KV heads (fused_attention.cpp:20-139): one
// wave per query row.  Scores of the row's visible keys go to LDS (lanes
// over keys), softmax with the row maximum, then lanes over the value
// dimension accumulate p_j * v_j.  Query head h reads KV head h / (Hq / Hk);
// causal rows see keys 0 .. Sk - Sq + i.
__global__ __launch_bounds__(64) void attention_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                       const float* __restrict__ v, float* __restrict__ o,
                                                       int64_t hq, int64_t hk, int64_t sq, int64_t sk, int64_t d,
                                                       int64_t dv, float scale, int causal) {
    extern __shared__ float sh[];
    float* qs = sh;          // [d]
    float* sc = sh + d;      // [sk]
    const int lane = threadIdx.x;
    const int64_t row = blockIdx.x;              // (batch, head, query row)
    const int64_t i = row % sq;
    const int64_t bh = row / sq;
    const int64_t h = bh % hq;
    const int64_t bidx = bh / hq;
    const int64_t g = hq / hk;
    const int64_t hkv = h / g;
    const float* qr = q + row * d;
    const float* kb = k + (bidx * hk + hkv) * sk * d;
    const float* vb = v + (bidx * hk + hkv) * sk * dv;
    float* orow = o + row * dv;

    int64_t valid = sk;
    if (causal) {
        valid = sk - sq + i + 1;
        valid = valid < 0 ? 0 : (valid > sk ? sk : valid);
    }
    for (int64_t t = lane; t < d; t += 64) qs[t] = qr[t];
    __syncthreads();
    if (valid == 0) {
        for (int64_t t = lane; t < dv; t += 64) orow[t] = 0.0f;
        return;
    }
    float mx = -INFINITY;
    for (int64_t j = lane; j < valid; j += 64) {
        const float* kr = kb + j * d;
        float dot = 0.0f;
        for (int64_t t = 0; t < d; ++t) dot = fmaf(qs[t], kr[t], dot);
        const float s = dot * scale;
        sc[j] = s;
        mx = fmaxf(mx, s);
    }
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    float sum = 0.0f;
    for (int64_t j = lane; j < valid; j += 64) {
        const float p = expf(sc[j] - mx);
        sc[j] = p;
        sum += p;
    }
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
    __syncthreads();
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    for (int64_t t = lane; t < dv; t += 64) {
        float acc = 0.0f;
        for (int64_t j = 0; j < valid; ++j) acc = fmaf(sc[j], vb[j * dv + t], acc);
        orow[t] = acc * inv;
    }
}

// ---- The same attention for one query row per (batch, head) (decode,
// Sq = 1), one 256-thread workgroup per row: the scores' fma chains run on
// all four waves (each in attention_kernel's order, its float4 loads
// batched), wave 0 reduces max and sum over the same lane-strided partials
// and butterflies as attention_kernel, and the value chain runs as there.
// Every value equals attention_kernel's bit for bit.  VLDS: the head's V is
// copied into LDS by direct global-to-LDS loads issued at entry, so the
// copy overlaps the scores.  Layout [V: sk * dv][q: d][scores: sk][max, sum].
template <bool VLDS>
__global__ __launch_bounds__(kT) void attention_row_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                           const float* __restrict__ v, float* __restrict__ o,
                                                           int64_t hq, int64_t hk, int64_t sk, int64_t d, int64_t dv,
                                                           float scale) {
    extern __shared__ float sh[];   // no static LDS: V's copy lands 16-byte aligned
    float* vs = sh;
    float* qs = VLDS ? sh + sk * dv : sh;
    float* sc = qs + d;
    float* stat = sc + sk;
    const int64_t row = blockIdx.x;   // (batch, head)
    const int64_t h = row % hq;
    const int64_t bidx = row / hq;
    const int64_t hkv = h / (hq / hk);
    const float* kb = k + (bidx * hk + hkv) * sk * d;
    const float* vb = v + (bidx * hk + hkv) * sk * dv;
    if constexpr (VLDS) {
        const int n4 = static_cast<int>(sk * dv / 4);   // dv % 4 == 0, v 16-byte aligned
        const int lane = threadIdx.x & 63;
        for (int blk = threadIdx.x >> 6; blk * 64 < n4; blk += kT / 64)
            if (blk * 64 + lane < n4)
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(vb + 4 * (blk * 64 + lane)),
                                                 (__attribute__((address_space(3))) void*)(vs + 256 * blk), 16, 0, 0);
    }
    for (int64_t t = threadIdx.x; t < d; t += kT) qs[t] = q[row * d + t];
    __syncthreads();
    const bool vec = d % 4 == 0 && reinterpret_cast<uintptr_t>(kb) % 16 == 0;
    for (int64_t j = threadIdx.x; j < sk; j += kT) {
        const float* kr = kb + j * d;
        float dot = 0.0f;
        int64_t t = 0;
        if (vec)
            for (; t + 64 <= d; t += 64) {
                float4 r[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) r[u] = *reinterpret_cast<const float4*>(kr + t + 4 * u);
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    dot = fmaf(qs[t + 4 * u], r[u].x, dot);
                    dot = fmaf(qs[t + 4 * u + 1], r[u].y, dot);
                    dot = fmaf(qs[t + 4 * u + 2], r[u].z, dot);
                    dot = fmaf(qs[t + 4 * u + 3], r[u].w, dot);
                }
            }
        for (; t < d; ++t) dot = fmaf(qs[t], kr[t], dot);
        sc[j] = dot * scale;
    }
    if constexpr (VLDS) __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        float mx = -INFINITY;
        for (int64_t j = lane; j < sk; j += 64) mx = fmaxf(mx, sc[j]);
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        if (lane == 0) stat[0] = mx;
    }
    __syncthreads();
    const float mx = stat[0];
    for (int64_t j = threadIdx.x; j < sk; j += kT) sc[j] = expf(sc[j] - mx);
    __syncthreads();
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        float sum = 0.0f;
        for (int64_t j = lane; j < sk; j += 64) sum += sc[j];
        for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
        if (lane == 0) stat[1] = sum;
    }
    __syncthreads();
    const float sum = stat[1];
    const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
    for (int64_t t = threadIdx.x; t < dv; t += kT) {
        float acc = 0.0f;
        int64_t j = 0;
        if constexpr (VLDS) {
            for (; j + 16 <= sk; j += 16) {
                float vv[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) vv[u] = vs[(j + u) * dv + t];
#pragma unroll
                for (int u = 0; u < 16; ++u) acc = fmaf(sc[j + u], vv[u], acc);
            }
            for (; j < sk; ++j) acc = fmaf(sc[j], vs[j * dv + t], acc);
        } else {
            for (; j + 32 <= sk; j += 32) {
                float vv[32];
#pragma unroll
                for (int u = 0; u < 32; ++u) vv[u] = vb[(j + u) * dv + t];
#pragma unroll
                for (int u = 0; u < 32; ++u) acc = fmaf(sc[j + u], vv[u], acc);
            }
            for (; j < sk; ++j) acc = fmaf(sc[j], vb[j * dv + t], acc);
        }
        o[row * dv + t] = acc * inv;
    }
}

// ---- Decode attention as the reference graph's unfused chain computes it
// (llama_graph.cpp:95-107: RepeatKV on K and V, Transpose of K, MatMul,
// Softmax, MatMul) for one query row per head, in one launch: one
// workgroup per query head h reads kv head h / (hq / hkv) directly.  Every
// value follows the fp32 operations of the kernels the chain launches, in
// their order: a score is matmul_f32_kernel's FMA chain over d from 0 (its
// zero padding of K to a multiple of 16 included), the softmax is
// softmax_rows_kernel's (64 lane-strided partial max and sum, xor
// butterflies, exp(x - max) / sum), the context is matmul_f32_kernel's FMA
// chain over the positions (padding included).  The result equals the
// chain's bit for bit, without the repeated K/V, the transposed K and the
// score rows in memory.
//
// VLDS (the head's V fits in LDS beside the scores): V is copied into LDS
// by direct global-to-LDS loads issued at entry, before the scores -- its
// rows are independent of them -- so the copy overlaps the score phase and
// the context chain reads LDS instead of waiting on global loads one batch
// at a time.  Layout [V: s * dv][q: d][scores: s][max, sum].
template <bool VLDS>
__global__ __launch_bounds__(kT) void attention_decode_chain_kernel(
    const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v, float* __restrict__ o,
    int64_t hq, int64_t hkv, int64_t s, int64_t d, int64_t dv) {
    // No static LDS: the dynamic block starts at LDS address 0, so V's copy
    // (16 bytes per lane) lands 16-byte aligned.
    extern __shared__ float sh[];
    float* vs = sh;                       // [s * dv] (VLDS)
    float* qs = VLDS ? sh + s * dv : sh;  // [d]
    float* sc = qs + d;                   // [s]: scores, then probabilities
    float* stat = sc + s;                 // [2]: max, sum
    const int64_t h = blockIdx.x;
    const int64_t kvh = h / (hq / hkv);
    const float* kb = k + kvh * s * d;
    const float* vb = v + kvh * s * dv;
    if constexpr (VLDS) {
        // Wave w copies 1 KiB blocks w, w + 4, ...: lane l moves float4
        // 64 * block + l (16 bytes to LDS at the block's base + 16 l).
        const int n4 = static_cast<int>(s * dv / 4);   // dv % 4 == 0, v 16-byte aligned
        const int lane = threadIdx.x & 63;
        for (int blk = threadIdx.x >> 6; blk * 64 < n4; blk += kT / 64)
            if (blk * 64 + lane < n4)
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(vb + 4 * (blk * 64 + lane)),
                                                 (__attribute__((address_space(3))) void*)(vs + 256 * blk), 16, 0, 0);
    }
    for (int64_t t = threadIdx.x; t < d; t += kT) qs[t] = q[h * d + t];
    __syncthreads();
    const int64_t dpad = (d + 15) / 16 * 16;
    // Each score's fma chain runs in order over d; the K row is loaded ahead
    // in batches of 16 float4 (16-byte aligned rows) so the chain does not
    // wait on one load per step.
    const bool vec = d % 4 == 0 && reinterpret_cast<uintptr_t>(kb) % 16 == 0;
    for (int64_t j = threadIdx.x; j < s; j += kT) {
        const float* kr = kb + j * d;
        float acc = 0.0f;
        int64_t t = 0;
        if (vec)
            for (; t + 64 <= d; t += 64) {
                float4 r[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) r[u] = *reinterpret_cast<const float4*>(kr + t + 4 * u);
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    acc = fmaf(qs[t + 4 * u], r[u].x, acc);
                    acc = fmaf(qs[t + 4 * u + 1], r[u].y, acc);
                    acc = fmaf(qs[t + 4 * u + 2], r[u].z, acc);
                    acc = fmaf(qs[t + 4 * u + 3], r[u].w, acc);
                }
            }
        for (; t < d; ++t) acc = fmaf(qs[t], kr[t], acc);
        for (t = d; t < dpad; ++t) acc = fmaf(0.0f, 0.0f, acc);
        sc[j] = acc;
    }
    // VLDS: the LDS copy of V is complete once this wave's loads are, and
    // visible to every wave after the barrier.
    if constexpr (VLDS) __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        float mx = -INFINITY;
        for (int64_t j = lane; j < s; j += 64) mx = fmaxf(mx, sc[j]);
        for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        float sum = 0.0f;
        for (int64_t j = lane; j < s; j += 64) sum += expf(sc[j] - mx);
        for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 64);
        if (lane == 0) {
            stat[0] = mx;
            stat[1] = sum;
        }
    }
    __syncthreads();
    const float mx = stat[0], sum = stat[1];
    for (int64_t j = threadIdx.x; j < s; j += kT) sc[j] = expf(sc[j] - mx) / sum;
    __syncthreads();
    const int64_t spad = (s + 15) / 16 * 16;
    for (int64_t t = threadIdx.x; t < dv; t += kT) {
        float acc = 0.0f;
        int64_t j = 0;
        if constexpr (VLDS) {
            for (; j + 16 <= s; j += 16) {   // LDS reads of 16 V rows ahead of the in-order chain
                float vv[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) vv[u] = vs[(j + u) * dv + t];
#pragma unroll
                for (int u = 0; u < 16; ++u) acc = fmaf(sc[j + u], vv[u], acc);
            }
            for (; j < s; ++j) acc = fmaf(sc[j], vs[j * dv + t], acc);
        } else {
            for (; j + 32 <= s; j += 32) {   // 32 V rows' loads ahead of the in-order chain
                float vv[32];
#pragma unroll
                for (int u = 0; u < 32; ++u) vv[u] = vb[(j + u) * dv + t];
#pragma unroll
                for (int u = 0; u < 32; ++u) acc = fmaf(sc[j + u], vv[u], acc);
            }
            for (; j < s; ++j) acc = fmaf(sc[j], vb[j * dv + t], acc);
        }
        for (j = s; j < spad; ++j) acc = fmaf(0.0f, 0.0f, acc);
        o[h * dv + t] = acc;
    }
}

}  // namespace
}  // namespace vmhip

using namespace vmhip;

namespace {

hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }

constexpr size_t kChainMaxLds = 160 * 1024;   // dynamic LDS of the V-staging attention kernels (no static LDS)

// Raises both kernels' dynamic LDS limit to kChainMaxLds; false (the error
// cleared) when the runtime refuses, which keeps launches on their
// global-memory forms.
bool raise_lds_limit(const void* a, const void* b) {
    hipError_t e = hipFuncSetAttribute(a, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kChainMaxLds));
    if (e == hipSuccess)
        e = hipFuncSetAttribute(b, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kChainMaxLds));
    if (e != hipSuccess) (void)hipGetLastError();
    return e == hipSuccess;
}

}  // namespace

extern "C" {

int vm_hip_embedding_f32(const float* table, int64_t vocab, int64_t hidden, const int32_t* idx, int64_t count,
                         float* out, void* stream) {
    clear_error();
    if (vocab < 0 || hidden < 0 || count < 0) return fail_inval("Embedding: negative size");
    if (count == 0 || hidden == 0) return 0;
    if (!table || !idx || !out) return fail_inval("Embedding: null pointer");
    hipLaunchKernelGGL(embedding_kernel, dim3(grid_for(count * hidden)), dim3(kT), 0, S(stream), table, vocab, hidden,
                       idx, count, out);
    return check_launch("Embedding", S(stream));
}

int vm_hip_rmsnorm_f32(const float* x, const float* w, float* y, int64_t rows, int64_t dim, float eps, void* stream) {
    clear_error();
    if (rows < 0 || dim < 0) return fail_inval("RMSNorm: negative size");
    if (rows == 0 || dim == 0) return 0;
    if (!x || !w || !y) return fail_inval("RMSNorm: null pointer");
    if (rows > 0x7fffffff) return fail_inval("RMSNorm: too many rows");
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(static_cast<unsigned>(rows)), dim3(kT), 0, S(stream), x, w, y, dim, eps);
    return check_launch("RMSNorm", S(stream));
}

int vm_hip_rope_f32(const float* x, const float* cos_table, const float* sin_table, float* y, int64_t rows,
                    int64_t head_dim, int64_t cos_rows, void* stream) {
    clear_error();
    if (rows < 0 || head_dim < 0 || cos_rows < 1 || head_dim % 2 != 0) return fail_inval("RotaryEmbedding: bad shape");
    if (rows == 0 || head_dim == 0) return 0;
    if (!x || !cos_table || !sin_table || !y) return fail_inval("RotaryEmbedding: null pointer");
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(rows * head_dim / 2)), dim3(kT), 0, S(stream), x, cos_table,
                       sin_table, y, rows, head_dim, cos_rows);
    return check_launch("RotaryEmbedding", S(stream));
}

int vm_hip_rope_append_f32(const float* q, const float* k, const float* v, const float* k_past, const float* v_past,
                           const float* cos_table, const float* sin_table, float* q_out, float* k_out, float* v_out,
                           int64_t hq, int64_t hkv, int64_t s_past, int64_t d, int64_t dv, void* stream) {
    clear_error();
    if (hq < 1 || hkv < 1 || s_past < 0 || d < 2 || d % 2 != 0 || dv < 1) return fail_inval("RopeAppend: bad shape");
    if (!q || !k || !v || !cos_table || !sin_table || !q_out || !k_out || !v_out || (s_past > 0 && (!k_past || !v_past)))
        return fail_inval("RopeAppend: null pointer");
    const int64_t total = hq * (d / 2) + hkv * (d / 2) + hkv * s_past * d + hkv * (s_past + 1) * dv;
    hipLaunchKernelGGL(rope_append_kernel, dim3(grid_for(total)), dim3(kT), 0, S(stream), q, k, v, k_past, v_past,
                       cos_table, sin_table, q_out, k_out, v_out, hq, hkv, s_past, d, dv);
    return check_launch("RopeAppend", S(stream));
}

int vm_hip_transpose_f32(const float* x, float* y, int rank, const int64_t* in_shape, const int* perm, void* stream) {
    clear_error();
    if (rank < 1 || rank > 6 || !in_shape) return fail_inval("Transpose: rank must be 1..6");
    Dims d{};
    d.rank = rank;
    int64_t in_stride[6];
    int64_t total = 1;
    int64_t stride = 1;
    for (int ax = rank - 1; ax >= 0; --ax) {
        if (in_shape[ax] < 0) return fail_inval("Transpose: negative dimension");
        in_stride[ax] = stride;
        stride *= in_shape[ax] > 0 ? in_shape[ax] : 1;
    }
    bool seen[6] = {false, false, false, false, false, false};
    for (int ax = 0; ax < rank; ++ax) {
        const int p = perm ? perm[ax] : rank - 1 - ax;
        if (p < 0 || p >= rank || seen[p]) return fail_inval("Transpose: invalid permutation");
        seen[p] = true;
        d.out_shape[ax] = in_shape[p];
        d.in_step[ax] = in_stride[p];
        total *= in_shape[p];
    }
    if (total == 0) return 0;
    if (!x || !y) return fail_inval("Transpose: null pointer");
    hipLaunchKernelGGL(gather_kernel, dim3(grid_for(total)), dim3(kT), 0, S(stream), x, y, total, d);
    return check_launch("Transpose", S(stream));
}

int vm_hip_slice_f32(const float* x, float* y, int rank, const int64_t* in_shape, const int64_t* begins,
                     const int64_t* steps, const int64_t* out_shape, void* stream) {
    clear_error();
    if (rank < 1 || rank > 6 || !in_shape || !begins || !steps || !out_shape)
        return fail_inval("Slice: rank must be 1..6");
    Dims d{};
    d.rank = rank;
    int64_t stride = 1, total = 1;
    for (int ax = rank - 1; ax >= 0; --ax) {
        if (out_shape[ax] < 0 || steps[ax] < 1 || begins[ax] < 0) return fail_inval("Slice: bad bounds");
        if (out_shape[ax] > 0 && begins[ax] + (out_shape[ax] - 1) * steps[ax] >= in_shape[ax])
            return fail_inval("Slice: out of range");
        d.out_shape[ax] = out_shape[ax];
        d.in_step[ax] = steps[ax] * stride;
        d.in_base += begins[ax] * stride;
        stride *= in_shape[ax];
        total *= out_shape[ax];
    }
    if (total == 0) return 0;
    if (!x || !y) return fail_inval("Slice: null pointer");
    hipLaunchKernelGGL(gather_kernel, dim3(grid_for(total)), dim3(kT), 0, S(stream), x, y, total, d);
    return check_launch("Slice", S(stream));
}

int vm_hip_concat_f32(const float* a, const float* b, float* y, int64_t outer, int64_t a_block, int64_t b_block,
                      void* stream) {
    clear_error();
    if (outer < 0 || a_block < 0 || b_block < 0) return fail_inval("Concat: negative size");
    if (outer == 0 || a_block + b_block == 0) return 0;
    if ((a_block && !a) || (b_block && !b) || !y) return fail_inval("Concat: null pointer");
    hipLaunchKernelGGL(concat_kernel, dim3(grid_for(outer * (a_block + b_block))), dim3(kT), 0, S(stream), a, b, y,
                       outer, a_block, b_block);
    return check_launch("Concat", S(stream));
}

int vm_hip_repeat_kv_f32(const float* x, float* y, int64_t outer, int64_t kv_heads, int64_t repeats, int64_t inner,
                         void* stream) {
    clear_error();
    if (outer < 0 || kv_heads < 0 || repeats < 1 || inner < 0) return fail_inval("RepeatKV: bad shape");
    if (outer == 0 || kv_heads == 0 || inner == 0) return 0;
    if (!x || !y) return fail_inval("RepeatKV: null pointer");
    hipLaunchKernelGGL(repeat_kv_kernel, dim3(grid_for(outer * kv_heads * repeats * inner)), dim3(kT), 0, S(stream),
                       x, y, outer, kv_heads, repeats, inner);
    return check_launch("RepeatKV", S(stream));
}

int vm_hip_elementwise_f32(int op, const float* a, const float* b, float* y, int64_t n, void* stream) {
    clear_error();
    if (op != VM_HIP_EW_ADD && op != VM_HIP_EW_MUL && op != VM_HIP_EW_SIGMOID && op != VM_HIP_EW_SILU_MUL)
        return fail_inval("elementwise: bad op");
    if (n < 0) return fail_inval("elementwise: negative size");
    if (n == 0) return 0;
    if (!a || !y || (op != VM_HIP_EW_SIGMOID && !b)) return fail_inval("elementwise: null pointer");
    hipLaunchKernelGGL(elementwise_kernel, dim3(grid_for(n)), dim3(kT), 0, S(stream), op, a, b, y, n);
    return check_launch(op == VM_HIP_EW_ADD   ? "Add"
                        : op == VM_HIP_EW_MUL ? "Mul"
                        : op == VM_HIP_EW_SIGMOID ? "Sigmoid"
                                                  : "SiluMul",
                        S(stream));
}

int vm_hip_softmax_f32(const float* x, float* y, int64_t outer, int64_t cols, int64_t inner, void* stream) {
    clear_error();
    if (outer < 0 || cols < 0 || inner < 0) return fail_inval("Softmax: negative size");
    if (outer == 0 || cols == 0 || inner == 0) return 0;
    if (!x || !y) return fail_inval("Softmax: null pointer");
    if (inner == 1) {
        const int64_t blocks = (outer + kT / 64 - 1) / (kT / 64);
        if (blocks > 0x7fffffff) return fail_inval("Softmax: too many rows");
        hipLaunchKernelGGL(softmax_rows_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kT), 0, S(stream), x, y,
                           outer, cols);
    } else {
        hipLaunchKernelGGL(softmax_strided_kernel, dim3(grid_for(outer * inner)), dim3(kT), 0, S(stream), x, y, outer,
                           cols, inner);
    }
    return check_launch("Softmax", S(stream));
}

int vm_hip_matmul_f32(const float* a, const float* b, float* c, int64_t batch, int64_t m, int64_t k, int64_t n,
                      void* stream) {
    clear_error();
    if (batch < 0 || m < 0 || k < 0 || n < 0) return fail_inval("MatMul: negative size");
    if (batch == 0 || m == 0 || n == 0) return 0;
    if (!a || !b || !c) return fail_inval("MatMul: null pointer");
    const int64_t gx = (n + kMmTile - 1) / kMmTile, gy = (m + kMmTile - 1) / kMmTile;
    if (gx > 0x7fffffff || gy > 65535 || batch > 65535) return fail_inval("MatMul: grid too large");
    hipLaunchKernelGGL(matmul_f32_kernel, dim3(static_cast<unsigned>(gx), static_cast<unsigned>(gy),
                                               static_cast<unsigned>(batch)),
                       dim3(kT), 0, S(stream), a, b, c, m, k, n);
    return check_launch("MatMul", S(stream));
}

int vm_hip_attention_decode_chain_f32(const float* q, const float* k, const float* v, float* o, int64_t hq,
                                      int64_t hkv, int64_t s, int64_t d, int64_t dv, void* stream) {
    clear_error();
    if (hq < 1 || hkv < 1 || hq % hkv != 0 || s < 1 || d < 1 || dv < 1)
        return fail_inval("AttentionDecodeChain: bad shape");
    if (s + d > 16384) return fail_inval("AttentionDecodeChain: S + D exceeds 16384 on this kernel");
    if (hq > 0x7fffffff) return fail_inval("AttentionDecodeChain: too many heads");
    if (!q || !k || !v || !o) return fail_inval("AttentionDecodeChain: null pointer");
    // V staged in LDS when it fits (gfx950: 160 KiB per workgroup) and
    // loads as float4.
    const size_t lds = static_cast<size_t>(d + s + 2) * sizeof(float);
    const size_t lds_v = lds + static_cast<size_t>(s * dv) * sizeof(float);
    // The dynamic LDS limit is raised once per process (a refusal, cleared
    // here, keeps every launch on the global-memory form).
    static const bool big_lds = raise_lds_limit(reinterpret_cast<const void*>(&attention_decode_chain_kernel<true>),
                                                reinterpret_cast<const void*>(&attention_decode_chain_kernel<false>));
    const bool vlds = big_lds && dv % 4 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0 && lds_v <= kChainMaxLds;
    if (vlds) {
        hipLaunchKernelGGL(attention_decode_chain_kernel<true>, dim3(static_cast<unsigned>(hq)), dim3(kT), lds_v,
                           S(stream), q, k, v, o, hq, hkv, s, d, dv);
    } else {
        hipLaunchKernelGGL(attention_decode_chain_kernel<false>, dim3(static_cast<unsigned>(hq)), dim3(kT), lds,
                           S(stream), q, k, v, o, hq, hkv, s, d, dv);
    }
    return check_launch("AttentionDecodeChain", S(stream));
}

int vm_hip_attention_f32(const float* q, const float* k, const float* v, float* o, int64_t batch, int64_t hq,
                         int64_t hk, int64_t sq, int64_t sk, int64_t d, int64_t dv, float scale, int causal,
                         void* stream) {
    clear_error();
    if (batch < 0 || hq < 0 || hk < 1 || sq < 0 || sk < 0 || d < 1 || dv < 1 || hq % hk != 0)
        return fail_inval("FusedAttention: bad shape");
    if (causal && sk < sq) return fail_inval("FusedAttention: causal attention requires Sk >= Sq");
    const int64_t rows = batch * hq * sq;
    if (rows == 0) return 0;
    if (!q || !o || (sk > 0 && (!k || !v))) return fail_inval("FusedAttention: null pointer");
    const int64_t lds = (d + sk) * static_cast<int64_t>(sizeof(float));
    if (lds > 64 * 1024) return fail_inval("FusedAttention: Sk + D exceeds 16384 on this kernel");
    if (rows > 0x7fffffff) return fail_inval("FusedAttention: too many rows");
    const float sc = scale > 0.0f ? scale : 1.0f / sqrtf(static_cast<float>(d));
    if (sq == 1 && sk > 0) {
        // One query row per head: four waves per row, V in LDS when it fits.
        static const bool big_lds = raise_lds_limit(reinterpret_cast<const void*>(&attention_row_kernel<true>),
                                                    reinterpret_cast<const void*>(&attention_row_kernel<false>));
        const size_t row_lds = static_cast<size_t>(d + sk + 2) * sizeof(float);
        const size_t row_lds_v = row_lds + static_cast<size_t>(sk * dv) * sizeof(float);
        if (big_lds && dv % 4 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0 && row_lds_v <= kChainMaxLds)
            hipLaunchKernelGGL(attention_row_kernel<true>, dim3(static_cast<unsigned>(rows)), dim3(kT), row_lds_v,
                               S(stream), q, k, v, o, hq, hk, sk, d, dv, sc);
        else
            hipLaunchKernelGGL(attention_row_kernel<false>, dim3(static_cast<unsigned>(rows)), dim3(kT), row_lds,
                               S(stream), q, k, v, o, hq, hk, sk, d, dv, sc);
        return check_launch("FusedAttention", S(stream));
    }
    hipLaunchKernelGGL(attention_kernel, dim3(static_cast<unsigned>(rows)), dim3(64), static_cast<size_t>(lds),
                       S(stream), q, k, v, o, hq, hk, sq, sk, d, dv, sc, causal ? 1 : 0);
    return check_launch("FusedAttention", S(stream));
}

}  // extern "C"
