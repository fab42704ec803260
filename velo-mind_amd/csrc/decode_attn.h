// Decode attention over one chunk of 32 cached keys for the G <= 16 query
// heads of one KV head, from LDS (256 threads).  Shared by the
// launch-per-projection step (attention_decode_slices_kernel) and the
// one-launch step (decode_persistent.hip).
//
// LDS operands: sq [16][D] the rotated queries, sk [32][D + 4] the keys
// (rows padded by 4 floats), sv [32][D] the values; keys 0 .. nk - 1 are
// valid.  scores() leaves the chunk's softmax partial, sp[g][j] =
// exp(s_gj - m_g) (0 for j >= nk), sm[g] = m_g and sl[g] = sum_j sp[g][j],
// with s_gj = scale * q_g . k_j; pv() then hands every (head, float4 of
// dims) its sum over the chunk's keys of sp[g][j] * v_j.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>

namespace vmhip {

// Reductions over the 32 lanes of each half of a wave without LDS: DPP
// within rows of 16 lanes (quad swaps, then the half-row and row mirrors,
// each leaving the running result uniform over twice as many lanes), then
// v_permlane16_swap exchanges the two rows of each half.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

template <class Op>
__device__ __forceinline__ float reduce_half_wave(float v, Op op) {
    v = op(v, dpp_mov<0xB1>(v));    // quad_perm [1, 0, 3, 2]
    v = op(v, dpp_mov<0x4E>(v));    // quad_perm [2, 3, 0, 1]
    v = op(v, dpp_mov<0x141>(v));   // row_half_mirror
    v = op(v, dpp_mov<0x140>(v));   // row_mirror
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    unsigned q[2];
    __builtin_memcpy(q, &p, sizeof q);
    return op(__uint_as_float(q[0]), __uint_as_float(q[1]));
}

template <int D>
struct ChunkAttention {
    static constexpr int kChunk = 32;
    static constexpr int kMaxG = 16;
    static constexpr int D4 = D / 4;
    static constexpr int kKS = D + 4;   // sk row stride (floats)
    static constexpr int kPiece = 16;   // float4s of a key row held in registers at a time
    static_assert(D4 % kPiece == 0, "head_dim a multiple of 64");

    // Thread t scores key j = t % 32 against heads t / 32 and t / 32 + 8:
    // the key row is read into registers a piece at a time and every
    // query float4 is a broadcast read, so each piece costs one LDS round
    // trip; four partial sums per head shorten the FMA chains.
    __device__ static void scores(const float* sq, const float* sk, float (*sp)[kChunk], float* sm, float* sl, int G,
                                  int nk, float scale) {
        const int t = static_cast<int>(threadIdx.x), j = t & 31, slot = t >> 5;
        float acc[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int c0 = 0; c0 < D4; c0 += kPiece) {
            float4 kr[kPiece];
#pragma unroll
            for (int c = 0; c < kPiece; ++c) kr[c] = *reinterpret_cast<const float4*>(sk + j * kKS + 4 * (c0 + c));
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int g = slot + 8 * i;
                if (g >= G) continue;   // uniform over each half wave
#pragma unroll
                for (int c = 0; c < kPiece; ++c) {
                    const float4 q = *reinterpret_cast<const float4*>(sq + g * D + 4 * (c0 + c));
                    acc[i][0] = fmaf(q.x, kr[c].x, acc[i][0]);
                    acc[i][1] = fmaf(q.y, kr[c].y, acc[i][1]);
                    acc[i][2] = fmaf(q.z, kr[c].z, acc[i][2]);
                    acc[i][3] = fmaf(q.w, kr[c].w, acc[i][3]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int g = slot + 8 * i;
            if (g >= G) continue;
            const float s = ((acc[i][0] + acc[i][1]) + (acc[i][2] + acc[i][3])) * scale;
            const float sv = j < nk ? s : -INFINITY;
            const float m = reduce_half_wave(sv, [](float a, float b) { return fmaxf(a, b); });
            const float pr = j < nk ? expf(sv - m) : 0.0f;
            const float l = reduce_half_wave(pr, [](float a, float b) { return a + b; });
            sp[g][j] = pr;
            if (j == 0) {
                sm[g] = m;
                sl[g] = l;
            }
        }
    }

    // Thread (c4 = t % D4, head t / D4 + k * 256 / D4): the chunk's p . V for
    // dims 4 c4 .. 4 c4 + 3, over keys 0 .. nk - 1 (rows past nk are never
    // read: they may hold anything), even and odd keys summed apart.
    template <class Emit>
    __device__ static void pv(const float* sv, const float (*sp)[kChunk], int G, int nk, Emit emit) {
        const int t = static_cast<int>(threadIdx.x), c4 = t % D4;
        for (int g = t / D4; g < G; g += 256 / D4) {
            float4 a0 = make_float4(0.f, 0.f, 0.f, 0.f), a1 = a0;
            int jj = 0;
            for (; jj + 8 <= nk; jj += 8) {
                float pr[8];
                float4 v[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    pr[u] = sp[g][jj + u];
                    v[u] = *reinterpret_cast<const float4*>(sv + (jj + u) * D + 4 * c4);
                }
#pragma unroll
                for (int u = 0; u < 8; u += 2) {
                    a0.x = fmaf(pr[u], v[u].x, a0.x);
                    a0.y = fmaf(pr[u], v[u].y, a0.y);
                    a0.z = fmaf(pr[u], v[u].z, a0.z);
                    a0.w = fmaf(pr[u], v[u].w, a0.w);
                    a1.x = fmaf(pr[u + 1], v[u + 1].x, a1.x);
                    a1.y = fmaf(pr[u + 1], v[u + 1].y, a1.y);
                    a1.z = fmaf(pr[u + 1], v[u + 1].z, a1.z);
                    a1.w = fmaf(pr[u + 1], v[u + 1].w, a1.w);
                }
            }
            for (; jj < nk; ++jj) {
                const float pr = sp[g][jj];
                const float4 v = *reinterpret_cast<const float4*>(sv + jj * D + 4 * c4);
                a0.x = fmaf(pr, v.x, a0.x);
                a0.y = fmaf(pr, v.y, a0.y);
                a0.z = fmaf(pr, v.z, a0.z);
                a0.w = fmaf(pr, v.w, a0.w);
            }
            emit(g, c4, make_float4(a0.x + a1.x, a0.y + a1.y, a0.z + a1.z, a0.w + a1.w));
        }
    }
};

}  // namespace vmhip
