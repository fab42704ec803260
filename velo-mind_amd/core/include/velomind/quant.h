// Weight quantization API (the reference's include/velomind/quant.h:15-93).
//
// Layouts, byte for byte as the reference's quant.cpp:
//   INT8: codes int8 [rows, cols], one fp32 scale per column [cols];
//         scale = max|col| / 127 (1.0 for an all-zero column), code =
//         clamp(roundf(x * (1 / scale)), -127, 127).
//   INT4: codes packed [(rows + 1) / 2, cols]: rows 2r and 2r+1 share byte
//         row r, the even row in the low nibble; one fp32 scale per
//         (block of rows, column) [ceil(rows / block), cols]; scale =
//         max|block| / 7.
//
// In this build the packers run on the GPU (libvmhip); the host-pointer
// entry points stage through device memory and require a HIP device.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <utility>

#include "velomind/dtype.h"
#include "velomind/tensor_storage.h"
#include "velomind/types.h"
#include "velomind_core_export.h"

namespace velomind {

enum class QuantType : std::uint8_t {
    None = 0,
    Int8 = 1,
    Int4 = 2,
};

constexpr const char* quant_type_name(QuantType type) noexcept {
    switch (type) {
        case QuantType::None: return "None";
        case QuantType::Int8: return "Int8";
        case QuantType::Int4: return "Int4";
    }
    return "Unknown";
}

struct QuantizationMetrics {
    float max_diff = 0.0f;
    float rmse = 0.0f;
    float snr_db = 0.0f;
    float cosine_sim = 1.0f;
};

// Error metrics between an original and a reconstructed buffer (double
// accumulation; SNR 100 dB for identical data; quant.cpp:26-72).
VELOMIND_CORE_EXPORT auto compute_quantization_metrics(const float* original, const float* reconstructed,
                                                       std::size_t count) -> QuantizationMetrics;

VELOMIND_CORE_EXPORT void quantize_weights_int8_per_channel(const float* src, std::int8_t* dst_q, float* dst_scale,
                                                            std::size_t rows, std::size_t cols);
VELOMIND_CORE_EXPORT void dequantize_weights_int8_per_channel(const std::int8_t* src_q, const float* scale,
                                                              float* dst, std::size_t rows, std::size_t cols);
VELOMIND_CORE_EXPORT void quantize_weights_int4_block(const float* src, std::uint8_t* dst_packed, float* dst_scale,
                                                      std::size_t rows, std::size_t cols,
                                                      std::size_t block_size = 32);
VELOMIND_CORE_EXPORT void dequantize_weights_int4_block(const std::uint8_t* src_packed, const float* scale,
                                                        float* dst, std::size_t rows, std::size_t cols,
                                                        std::size_t block_size = 32);

// Quantizes a 2-D fp32/fp16/bf16 storage (host or HIP) and returns
// (codes, scales) storages allocated on `device`.
VELOMIND_CORE_EXPORT auto quantize_storage_int8(const TensorStorage& src_storage, DeviceType device = DeviceType::CPU)
    -> std::pair<std::shared_ptr<TensorStorage>, std::shared_ptr<TensorStorage>>;
VELOMIND_CORE_EXPORT auto quantize_storage_int4(const TensorStorage& src_storage, std::size_t block_size = 32,
                                                DeviceType device = DeviceType::CPU)
    -> std::pair<std::shared_ptr<TensorStorage>, std::shared_ptr<TensorStorage>>;

}  // namespace velomind
