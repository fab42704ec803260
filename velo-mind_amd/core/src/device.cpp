// Device parsing, enumeration and capability queries.
#include "velomind/device.h"

#include <cctype>
#include <ostream>
#include <string>

#include "internal/registry/kernel.h"
#include "internal/registry/storage.h"
#include "velomind/dtype.h"
#include "vm_hip.h"

namespace velomind {

auto Device::from_string(std::string_view str) -> std::optional<Device> {
    if (str.empty()) return std::nullopt;
    const auto colon = str.find(':');
    std::string base;
    for (char c : str.substr(0, colon)) base.push_back(static_cast<char>(std::tolower(static_cast<unsigned char>(c))));
    int index = 0;
    if (colon != std::string_view::npos) {
        const std::string idx(str.substr(colon + 1));
        if (idx.empty()) return std::nullopt;
        for (char c : idx)
            if (!std::isdigit(static_cast<unsigned char>(c))) return std::nullopt;
        try {
            index = std::stoi(idx);
        } catch (...) {
            return std::nullopt;
        }
    }
    if (base == "cpu") return Device(DeviceType::CPU, index);
    if (base == "ispc") return Device(DeviceType::ISPC, index);
    if (base == "cuda") return Device(DeviceType::CUDA, index);
    if (base == "hip") return Device(DeviceType::HIP, index);
    return std::nullopt;
}

auto Device::available_devices() -> std::vector<Device> {
    std::vector<Device> out;
    for (auto t : {DeviceType::CPU, DeviceType::ISPC, DeviceType::CUDA})
        if (Device(t).is_available()) out.push_back(Device(t));
    if (Device::hip().is_available()) {
        int n = 0;
        if (vm_hip_device_count(&n) == 0)
            for (int i = 0; i < n; ++i) out.push_back(Device::hip(i));
    }
    return out;
}

auto Device::default_device() -> Device { return Device::hip().is_available() ? Device::hip() : Device::cpu(); }

auto Device::is_available() const noexcept -> bool {
    if (!internal::is_device_available(_type)) return false;
    if (_type == DeviceType::HIP) {
        int n = 0;
        return vm_hip_device_count(&n) == 0 && _index >= 0 && _index < n;
    }
    return _index == 0;
}

auto Device::name() const -> std::string {
    std::string n = device_type_name(_type);
    for (auto& c : n) c = static_cast<char>(std::tolower(static_cast<unsigned char>(c)));
    return (_type == DeviceType::CUDA || _type == DeviceType::HIP) ? n + ":" + std::to_string(_index) : n;
}

auto Device::description() const -> std::string {
    if (_type == DeviceType::HIP) return "AMD Instinct gfx950 (HIP) device " + std::to_string(_index);
    return std::string(device_type_name(_type)) + " device";
}

auto Device::supports(DataType dtype) const noexcept -> bool { return is_dtype_supported(_type, dtype); }

auto Device::supports(Op op, DataType dtype) const noexcept -> bool {
    try {
        for (const auto& e : internal::op_kernels(_type)[static_cast<std::size_t>(op)])
            for (std::size_t i = 0; i < e.key.num_inputs; ++i)
                if (e.key.input_dtypes[i] == dtype || e.key.output_dtype == dtype) return true;
    } catch (...) {
    }
    return false;
}

auto Device::supports(Op op, std::span<const DataType> input_dtypes, DataType output_dtype) const noexcept -> bool {
    return is_op_dtype_supported(_type, op, input_dtypes, output_dtype);
}

auto Device::memory_info() const -> std::optional<DeviceMemoryInfo> { return std::nullopt; }

auto to_string(const Device& d) -> std::string { return d.name(); }
auto operator<<(std::ostream& os, const Device& d) -> std::ostream& { return os << d.name(); }

}  // namespace velomind
