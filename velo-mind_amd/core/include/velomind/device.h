// Device handle: type + index, availability and capability queries
// (the reference's include/velomind/device.h:130-179, with "hip").
#pragma once

#include <compare>
#include <cstddef>
#include <functional>
#include <optional>
#include <span>
#include <string>
#include <string_view>
#include <vector>

#include "velomind/types.h"
#include "velomind_core_export.h"

namespace velomind {

enum class Op : std::uint16_t;

struct DeviceMemoryInfo {
    std::size_t total_bytes = 0;
    std::size_t used_bytes = 0;
    std::size_t free_bytes = 0;
};

class VELOMIND_CORE_EXPORT Device {
public:
    constexpr Device() noexcept = default;
    constexpr Device(DeviceType type, int index = 0) noexcept : _type(type), _index(index) {}

    static constexpr auto cpu() noexcept -> Device { return Device(DeviceType::CPU, 0); }
    static constexpr auto ispc() noexcept -> Device { return Device(DeviceType::ISPC, 0); }
    static constexpr auto cuda(int index = 0) noexcept -> Device { return Device(DeviceType::CUDA, index); }
    static constexpr auto hip(int index = 0) noexcept -> Device { return Device(DeviceType::HIP, index); }

    // "cpu", "cuda[:n]", "ispc", "hip[:n]" (case-insensitive).
    static auto from_string(std::string_view str) -> std::optional<Device>;
    static auto available_devices() -> std::vector<Device>;
    static auto default_device() -> Device;

    [[nodiscard]] constexpr auto type() const noexcept -> DeviceType { return _type; }
    [[nodiscard]] constexpr auto index() const noexcept -> int { return _index; }
    [[nodiscard]] auto is_available() const noexcept -> bool;
    [[nodiscard]] auto name() const -> std::string;
    [[nodiscard]] auto description() const -> std::string;
    [[nodiscard]] auto supports(DataType dtype) const noexcept -> bool;
    [[nodiscard]] auto supports(Op op, DataType dtype) const noexcept -> bool;
    [[nodiscard]] auto supports(Op op, std::span<const DataType> input_dtypes, DataType output_dtype) const noexcept
        -> bool;
    [[nodiscard]] auto memory_info() const -> std::optional<DeviceMemoryInfo>;

    constexpr operator DeviceType() const noexcept { return _type; }
    auto operator==(const Device& other) const noexcept -> bool = default;
    auto operator<=>(const Device& other) const noexcept = default;

private:
    DeviceType _type{DeviceType::CPU};
    int _index{0};
};

VELOMIND_CORE_EXPORT auto to_string(const Device& device) -> std::string;
VELOMIND_CORE_EXPORT auto operator<<(std::ostream& os, const Device& device) -> std::ostream&;

}  // namespace velomind

template <>
struct std::hash<velomind::Device> {
    auto operator()(const velomind::Device& d) const noexcept -> std::size_t {
        return (static_cast<std::size_t>(d.type()) << 16) ^ static_cast<std::size_t>(d.index());
    }
};
