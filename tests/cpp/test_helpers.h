// Shared helpers for the C++ tests.  The oracle (oracle/qmm_oracle.c) is
// linked into the test binary only, as the checker: test_helpers.cpp
// registers it as the DeviceType::CPU QuantizedMatMul kernel so that tests
// can build the same graph on CPU (oracle) and on HIP and compare, the
// pattern of the reference's tests/test_coverage_matrix.cpp:601-688.
#pragma once

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <random>
#include <span>
#include <string>
#include <vector>

#include "vm_test.h"
#include "velomind/velomind.h"
#include "vm_hip.h"

extern "C" {
#include "qmm_oracle.h"
}

namespace vmtest {

template <typename T>
std::span<const std::byte> as_bytes(const std::vector<T>& v) {
    return std::as_bytes(std::span<const T>(v));
}

template <typename T>
std::span<std::byte> as_writeable_bytes(std::vector<T>& v) {
    return std::as_writable_bytes(std::span<T>(v));
}

// tests/test_quantization.cpp:37-45 of the reference: mt19937(1337), U(lo, hi).
inline std::vector<float> generate_random_weights(std::size_t rows, std::size_t cols, float lo = -1.0f, float hi = 1.0f) {
    std::vector<float> v(rows * cols);
    std::mt19937 rng(1337);
    std::uniform_real_distribution<float> dist(lo, hi);
    for (auto& x : v) x = dist(rng);
    return v;
}

// tests/test_quantization.cpp:47-53 of the reference.
inline std::vector<float> generate_activations(std::size_t m, std::size_t k) {
    std::vector<float> v(m * k);
    for (std::size_t i = 0; i < v.size(); ++i) v[i] = 0.05f * static_cast<float>(static_cast<int>(i % 23) - 11);
    return v;
}

inline std::vector<float> normal(std::size_t n, std::uint32_t seed, float std = 1.0f) {
    std::mt19937 rng(seed);
    std::normal_distribution<float> d(0.0f, std);
    std::vector<float> v(n);
    for (auto& x : v) x = d(rng);
    return v;
}

inline void require_all_finite(const std::vector<float>& v) {
    for (float x : v) REQUIRE(std::isfinite(x));
}

inline float max_abs(const std::vector<float>& v) {
    float m = 0.0f;
    for (float x : v) m = std::max(m, std::abs(x));
    return m;
}

inline float max_abs_diff(const std::vector<float>& a, const std::vector<float>& b) {
    float m = 0.0f;
    for (std::size_t i = 0; i < a.size(); ++i) m = std::max(m, std::abs(a[i] - b[i]));
    return m;
}

inline bool hip_available() { return velomind::Device::hip().is_available(); }

#define REQUIRE_HIP()                                         \
    do {                                                      \
        if (!::vmtest::hip_available()) SKIP("HIP device not available"); \
    } while (0)

// Scoped environment variable.
struct ScopedEnv {
    std::string name;
    ScopedEnv(const char* n, const char* v) : name(n) { setenv(n, v, 1); }
    ~ScopedEnv() { unsetenv(name.c_str()); }
};

}  // namespace vmtest
