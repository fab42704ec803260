// Half-precision value types and conversions.  Rounding follows the
// reference (include/velomind/dtype.h:21-107): fp32 -> fp16/bf16 round to
// nearest even, overflow to infinity, NaN kept quiet.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <span>

#include "velomind/types.h"
#include "velomind_core_export.h"

namespace velomind {

inline float bits_to_float(std::uint32_t u) noexcept {
    float f;
    std::memcpy(&f, &u, sizeof f);
    return f;
}

inline std::uint32_t float_to_bits(float f) noexcept {
    std::uint32_t u;
    std::memcpy(&u, &f, sizeof u);
    return u;
}

inline float float16_to_float(std::uint16_t h) noexcept {
    const std::uint32_t sign = static_cast<std::uint32_t>(h & 0x8000u) << 16;
    const std::uint32_t e = (h >> 10) & 0x1Fu;
    std::uint32_t m = h & 0x3FFu;
    if (e == 0) {
        if (m == 0) return bits_to_float(sign);
        int exp = -14;  // subnormal: normalise the mantissa
        while (!(m & 0x400u)) {
            m <<= 1;
            --exp;
        }
        return bits_to_float(sign | (static_cast<std::uint32_t>(exp + 127) << 23) | ((m & 0x3FFu) << 13));
    }
    if (e == 0x1F) return bits_to_float(sign | 0x7F800000u | (m << 13) | (m ? 0x400000u : 0u));
    return bits_to_float(sign | ((e + 112u) << 23) | (m << 13));
}

inline std::uint16_t float_to_float16(float f) noexcept {
    const std::uint32_t x = float_to_bits(f);
    const std::uint32_t sign = (x >> 16) & 0x8000u;
    const std::uint32_t raw_e = (x >> 23) & 0xFFu;
    const std::uint32_t mant = x & 0x7FFFFFu;
    if (raw_e == 0xFF) return static_cast<std::uint16_t>(sign | (mant ? 0x7E00u : 0x7C00u));
    int e = static_cast<int>(raw_e) - 112;
    if (e <= 0) {
        if (e < -10) return static_cast<std::uint16_t>(sign);
        std::uint32_t m = (mant | 0x800000u) >> (1 - e);
        if ((m & 0x1000u) && (m & 0x2FFFu)) m += 0x2000u;
        return static_cast<std::uint16_t>(sign | (m >> 13));
    }
    if (e >= 31) return static_cast<std::uint16_t>(sign | 0x7C00u);
    std::uint32_t m = mant;
    if ((m & 0x1000u) && (m & 0x2FFFu)) {
        m += 0x2000u;
        if (m & 0x800000u) {
            m = 0;
            if (++e >= 31) return static_cast<std::uint16_t>(sign | 0x7C00u);
        }
    }
    return static_cast<std::uint16_t>(sign | (static_cast<std::uint32_t>(e) << 10) | (m >> 13));
}

inline float bfloat16_to_float(std::uint16_t b) noexcept { return bits_to_float(static_cast<std::uint32_t>(b) << 16); }

inline std::uint16_t float_to_bfloat16(float f) noexcept {
    std::uint32_t x = float_to_bits(f);
    if ((x & 0x7F800000u) == 0x7F800000u && (x & 0x7FFFFFu)) return static_cast<std::uint16_t>((x >> 16) | 0x40u);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return static_cast<std::uint16_t>(x >> 16);
}

// IEEE binary16 value (1 sign, 5 exponent, 10 mantissa bits).
struct float16_t {
    std::uint16_t bits = 0;
    constexpr float16_t() noexcept = default;
    constexpr explicit float16_t(std::uint16_t raw, bool) noexcept : bits(raw) {}
    float16_t(float f) noexcept : bits(float_to_float16(f)) {}
    static constexpr float16_t from_bits(std::uint16_t b) noexcept { return float16_t(b, true); }
    constexpr std::uint16_t to_bits() const noexcept { return bits; }
    operator float() const noexcept { return float16_to_float(bits); }
    friend constexpr bool operator==(float16_t a, float16_t b) noexcept { return a.bits == b.bits; }
};

// bfloat16 value (1 sign, 8 exponent, 7 mantissa bits).
struct bfloat16_t {
    std::uint16_t bits = 0;
    constexpr bfloat16_t() noexcept = default;
    constexpr explicit bfloat16_t(std::uint16_t raw, bool) noexcept : bits(raw) {}
    bfloat16_t(float f) noexcept : bits(float_to_bfloat16(f)) {}
    static constexpr bfloat16_t from_bits(std::uint16_t b) noexcept { return bfloat16_t(b, true); }
    constexpr std::uint16_t to_bits() const noexcept { return bits; }
    operator float() const noexcept { return bfloat16_to_float(bits); }
    friend constexpr bool operator==(bfloat16_t a, bfloat16_t b) noexcept { return a.bits == b.bits; }
};

enum class Op : std::uint16_t;

// Whether `device` has a storage allocator and `dtype` is a valid element type.
VELOMIND_CORE_EXPORT auto is_dtype_supported(DeviceType device, DataType dtype) noexcept -> bool;

// Whether a kernel is registered for (device, op, input dtypes, output dtype).
VELOMIND_CORE_EXPORT auto is_op_dtype_supported(DeviceType device, Op op,
                                                std::span<const DataType> input_dtypes,
                                                DataType output_dtype) noexcept -> bool;

// Element-wise conversion between host buffers of two dtypes
// (src/dtype.cpp:74-95 in the reference).
VELOMIND_CORE_EXPORT auto convert_dtype(const void* src, DataType src_dtype, void* dst, DataType dst_dtype,
                                        std::size_t numel) -> void;

}  // namespace velomind
