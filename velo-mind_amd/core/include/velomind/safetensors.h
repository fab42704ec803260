// safetensors files: the reference's reader interface
// (include/velomind/safetensors.h, src/safetensors.cpp) plus a writer, so
// that pre-packed quantized weights (I8 codes + F32 scales) can be stored
// and loaded like any other checkpoint.
//
// Format: an 8-byte little-endian header length, a JSON object mapping
// tensor names to {"dtype", "shape", "data_offsets": [begin, end]} (offsets
// relative to the data area that follows the header) and an optional
// "__metadata__" object of string values, then the tensor bytes.
#pragma once

#include <cstddef>
#include <filesystem>
#include <memory>
#include <optional>
#include <span>
#include <string>
#include <unordered_map>
#include <vector>

#include "velomind/tensor_storage.h"
#include "velomind/types.h"
#include "velomind/velomind_core_export.h"

namespace velomind {

// Offsets are relative to the data area, not to the start of the file.
struct SafetensorsHeaderEntry {
    DataType dtype = DataType::Float32;
    shape_t shape;
    std::size_t begin = 0;
    std::size_t end = 0;
};

struct SafetensorsHeader {
    std::unordered_map<std::string, SafetensorsHeaderEntry> tensors;
    // "__metadata__" (string values; the reference reader skips it).
    std::unordered_map<std::string, std::string> metadata;
};

// Parses the JSON header bytes: dtypes F32/F16/BF16/I32/I8/BOOL, byte
// counts consistent with dtype and shape, non-overlapping ranges.  nullopt
// on any violation (src/safetensors.cpp:222-400).
VELOMIND_CORE_EXPORT auto parse_safetensors_header(std::span<const std::byte> header_bytes)
    -> std::optional<SafetensorsHeader>;

// A loaded file: every tensor in its own host (DeviceType::CPU) storage.
struct SafetensorsFile {
    std::unordered_map<std::string, std::shared_ptr<TensorStorage>> tensors;
    std::unordered_map<std::string, std::string> metadata;
};

VELOMIND_CORE_EXPORT auto load_safetensors(const std::filesystem::path& path) -> std::optional<SafetensorsFile>;

// One tensor to write: `bytes` must hold shape's element count times the
// dtype's width (row-major).
struct SafetensorsTensorView {
    std::string name;
    DataType dtype = DataType::Float32;
    shape_t shape;
    std::span<const std::byte> bytes;
};

// Writes a safetensors file: tensors back to back in the given order (the
// format allows no holes in the data area), the header padded with spaces
// to a multiple of 8 bytes.  Throws std::invalid_argument on inconsistent
// views or duplicate names and std::runtime_error on I/O errors.
VELOMIND_CORE_EXPORT void save_safetensors(const std::filesystem::path& path,
                                           std::span<const SafetensorsTensorView> tensors,
                                           const std::unordered_map<std::string, std::string>& metadata = {});

}  // namespace velomind
