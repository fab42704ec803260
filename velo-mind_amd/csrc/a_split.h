// Staging of the prefill GEMM's activations (qmm_gemm.hip), shared with
// the kernels that produce them (decode_ops.hip).
//
// Row r of A is scaled by 2^x_r, the power of two that puts its largest
// magnitude in [2^14, 2^15) (x_r = 0 when the row holds an infinity or NaN
// or is all zeros), and written as two fp16 parts, hi = fp16(a 2^x_r) and
// lo = fp16(a 2^x_r - hi): 22 significant bits of any finite fp32 row.  The
// parts are stored per 8-group of consecutive k either row-major (the
// small-tile kernel) or in the wide kernel's operand order, where a 1 KB
// piece holds 32 rows x 16 k and position i of an 8-group holds
// k = i / 2 + 4 (i % 2).  The staged buffer is [hi: mp x k][lo: mp x k]
// halves, then the m row exponents (int32) at a 256-byte boundary; mp is m
// rounded up to 32 rows in operand order, m otherwise.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstddef>
#include <cstdint>

namespace vmhip {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));

// Longest row the staging producers write (three 8-groups per thread of a
// 256-thread workgroup holding the whole row).
constexpr int64_t kStageMaxK = 6144;

// Rows padded for the layout, and the staged buffer's parts.
inline int64_t a_stage_rows(int64_t m, bool pieces) { return pieces ? (m + 31) / 32 * 32 : m; }
inline std::size_t a_stage_half_bytes(int64_t m, int64_t k, bool pieces) {
    return (static_cast<std::size_t>(a_stage_rows(m, pieces)) * static_cast<std::size_t>(k) * 4 + 255) &
           ~std::size_t(255);
}
inline std::size_t a_stage_bytes(int64_t m, int64_t k, bool pieces) {
    return a_stage_half_bytes(m, k, pieces) + ((static_cast<std::size_t>(m) * 4 + 255) & ~std::size_t(255));
}

__device__ __forceinline__ int a_row_exponent(float mx) {
    int x = 0;
    if (mx > 0.0f && mx <= 3.4028235e38f) {
        int e = 0;
        (void)frexpf(mx, &e);   // mx = f * 2^e, f in [0.5, 1)
        x = 15 - e;
    }
    return x;
}

// Largest magnitude of four values, and whether one is an infinity or NaN.
__device__ __forceinline__ void a_scan4(const float4& v, float& mx, bool& special) {
    mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    special = special || !(fabsf(v.x) <= 3.4028235e38f) || !(fabsf(v.y) <= 3.4028235e38f) ||
              !(fabsf(v.z) <= 3.4028235e38f) || !(fabsf(v.w) <= 3.4028235e38f);
}

// hi / lo of one 8-group; an infinite part (|a| beyond fp16 in an unscaled
// row) leaves lo at 0.
template <bool PIECES>
__device__ __forceinline__ void a_split8(const float4& p, const float4& q, int x, half8_t& h, half8_t& l) {
    const float s[8] = {ldexpf(p.x, x), ldexpf(p.y, x), ldexpf(p.z, x), ldexpf(p.w, x),
                        ldexpf(q.x, x), ldexpf(q.y, x), ldexpf(q.z, x), ldexpf(q.w, x)};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int kk = PIECES ? (i >> 1) + 4 * (i & 1) : i;
        const _Float16 hh = static_cast<_Float16>(s[kk]);
        const float d = s[kk] - static_cast<float>(hh);
        h[i] = hh;
        l[i] = static_cast<_Float16>(d == d && fabsf(d) <= 65504.0f ? d : 0.0f);
    }
}

// Workgroup b of a staging grid as a linear index whose runs of grid / 8
// are dispatched to one XCD (workgroups go to the 8 XCDs round-robin by id):
// the rows of a 128-byte line of operand-order pieces (8 rows x 16 bytes)
// are then written by workgroups of one XCD, whose L2 merges the partial
// lines, instead of being written back in pieces from several XCDs.
__device__ __forceinline__ int a_stage_wg(int b, int grid) {
    const int full = grid & ~7;
    return b < full ? (b & 7) * (full >> 3) + (b >> 3) : b;
}

// 16-byte piece index of (row, 8-group g) in a buffer of k columns.
template <bool PIECES>
__device__ __forceinline__ int64_t a_piece(int64_t row, int g, int k) {
    if constexpr (PIECES) return ((row / 32) * (k / 16) + g / 2) * 64 + row % 32 + 32 * (g % 2);
    return row * (k / 8) + g;
}

}  // namespace vmhip
