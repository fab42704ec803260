// safetensors reader/writer (velomind/safetensors.h), host only.  The
// parser cases mirror the reference's tests/io/test_safetensors.cpp:127-253
// (single and multiple tensors, malformed JSON, unknown dtype, byte-count
// mismatch, overflow, overlap, duplicate keys, deep nesting) and the load
// cases :255-377 (round trips, missing / truncated files, huge header length
// and offsets).  The writer is pinned by exact expected bytes written out by
// hand from the format, and the reader by the toy_llama fixture, which was
// written by the Hugging Face safetensors library.
#include <array>
#include <cstdint>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <limits>
#include <string>
#include <unistd.h>
#include <vector>

#include "test_helpers.h"
#include "velomind/safetensors.h"

using namespace velomind;

namespace {

std::span<const std::byte> as_bytes(const std::string& s) { return std::as_bytes(std::span(s.data(), s.size())); }

std::filesystem::path tmp_path(const char* name) {
    return std::filesystem::temp_directory_path() / (std::string("vm_st_") + std::to_string(::getpid()) + "_" + name);
}

std::string read_all(const std::filesystem::path& p) {
    std::ifstream f(p, std::ios::binary);
    return std::string(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
}

void write_raw(const std::filesystem::path& p, std::uint64_t hlen, const std::string& body) {
    std::ofstream f(p, std::ios::binary | std::ios::trunc);
    unsigned char le[8];
    for (int i = 0; i < 8; ++i) le[i] = static_cast<unsigned char>(hlen >> (8 * i));
    f.write(reinterpret_cast<const char*>(le), 8);
    f.write(body.data(), static_cast<std::streamsize>(body.size()));
}

std::filesystem::path fixture_dir() {
    // the test binary sits in tests/cpp; fixtures in tests/golden
    std::error_code ec;
    auto exe = std::filesystem::read_symlink("/proc/self/exe", ec);
    return exe.parent_path().parent_path() / "golden";
}

template <class T>
std::vector<T> values(const TensorStorage& s) {
    std::vector<T> v(s.size_bytes / sizeof(T));
    std::memcpy(v.data(), s.data, s.size_bytes);
    return v;
}

}  // namespace

TEST_CASE("safetensors header: single F32 tensor", "[safetensors]") {
    const std::string j = R"({"w":{"dtype":"F32","shape":[2,3],"data_offsets":[0,24]}})";
    auto h = parse_safetensors_header(as_bytes(j));
    REQUIRE(h.has_value());
    REQUIRE(h->tensors.size() == 1);
    const auto& e = h->tensors.at("w");
    REQUIRE(e.dtype == DataType::Float32);
    REQUIRE(e.shape == shape_t({2, 3}));
    REQUIRE(e.begin == 0);
    REQUIRE(e.end == 24);
    REQUIRE(h->metadata.empty());
}

TEST_CASE("safetensors header: several tensors, metadata and whitespace", "[safetensors]") {
    const std::string j = " { \"__metadata__\" : {\"format\":\"pt\", \"note\":\"a\\\"b\\u00e9\"},\n"
                          "\"a\":{\"dtype\":\"F16\",\"shape\":[4],\"data_offsets\":[0,8]},"
                          "\"b\":{\"dtype\":\"I32\",\"shape\":[2],\"data_offsets\":[8,16]},"
                          "\"c\":{\"dtype\":\"BF16\",\"shape\":[],\"data_offsets\":[16,18]},"
                          "\"d\":{\"dtype\":\"I8\",\"shape\":[0,5],\"data_offsets\":[18,18]},"
                          "\"e\":{\"dtype\":\"BOOL\",\"shape\":[3],\"data_offsets\":[18,21]}} ";
    auto h = parse_safetensors_header(as_bytes(j));
    REQUIRE(h.has_value());
    REQUIRE(h->tensors.size() == 5);
    REQUIRE(h->tensors.at("a").dtype == DataType::Float16);
    REQUIRE(h->tensors.at("b").dtype == DataType::Int32);
    REQUIRE(h->tensors.at("b").begin == 8);
    REQUIRE(h->tensors.at("c").dtype == DataType::BFloat16);
    REQUIRE(h->tensors.at("c").shape.empty());   // scalar: one element
    REQUIRE(h->tensors.at("d").end == 18);       // empty tensor
    REQUIRE(h->tensors.at("e").dtype == DataType::Bool);
    REQUIRE(h->metadata.at("format") == "pt");
    REQUIRE(h->metadata.at("note") == "a\"b\xc3\xa9");   // escapes decoded, U+00E9 as UTF-8
}

TEST_CASE("safetensors header: invalid headers are rejected", "[safetensors]") {
    const std::vector<std::string> bad{
        // malformed JSON
        R"({"w":{"dtype":"F32","shape":[2,3],"data_offsets":[0,24]})",
        R"({"w":{"dtype":"F32","shape":[2,3],"data_offsets":[0,24]}} x)",
        R"(["w"])",
        // unknown dtype, byte count that does not match the shape
        R"({"w":{"dtype":"F64","shape":[1],"data_offsets":[0,8]}})",
        R"({"w":{"dtype":"F32","shape":[2,3],"data_offsets":[0,20]}})",
        R"({"w":{"dtype":"F32","shape":[-1],"data_offsets":[0,4]}})",
        R"({"w":{"dtype":"F32","shape":[1],"data_offsets":[4,0]}})",
        R"({"w":{"dtype":"F32","shape":[1]}})",
        // element counts that overflow, overlapping ranges
        R"({"x":{"dtype":"F32","shape":[9223372036854775807,9223372036854775807],"data_offsets":[0,4]}})",
        R"({"x":{"dtype":"F32","shape":[9223372036854775807],"data_offsets":[0,4]}})",
        R"({"x":{"dtype":"F32","shape":[1],"data_offsets":[0,99999999999999999999]}})",
        R"({"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},"b":{"dtype":"F32","shape":[1],"data_offsets":[2,6]}})",
        // duplicate keys, inside an entry and at the top level
        R"({"x":{"dtype":"F32","dtype":"I32","shape":[1],"data_offsets":[0,4]}})",
        R"({"x":{"dtype":"F32","shape":[1],"data_offsets":[0,4]},"x":{"dtype":"F32","shape":[1],"data_offsets":[4,8]}})",
        // metadata must be an object of strings
        R"({"__metadata__":{"k":1}})",
        R"({"__metadata__":"k"})",
        "",
    };
    for (const auto& j : bad) {
        if (parse_safetensors_header(as_bytes(j)).has_value())
            throw vmtest::Failure("accepted invalid header: " + j);
    }
    const std::string deep = std::string("{\"__metadata__\":") + std::string(70, '[') + "0" + std::string(70, ']') + "}";
    REQUIRE(!parse_safetensors_header(as_bytes(deep)).has_value());
}

TEST_CASE("safetensors writer: exact bytes of a small file", "[safetensors]") {
    // Header JSON, padded with spaces to a multiple of 8, then the data.
    const std::array<float, 2> x{1.0f, -2.0f};
    const std::array<std::int8_t, 3> c{-8, 0, 7};
    const std::vector<SafetensorsTensorView> views{
        {"x", DataType::Float32, {2}, std::as_bytes(std::span(x))},
        {"c", DataType::Int8, {1, 3}, std::as_bytes(std::span(c))},
    };
    const auto p = tmp_path("exact.safetensors");
    save_safetensors(p, views, {{"k", "v"}});
    std::string hdr = R"({"__metadata__":{"k":"v"},"x":{"dtype":"F32","shape":[2],"data_offsets":[0,8]},)"
                      R"("c":{"dtype":"I8","shape":[1,3],"data_offsets":[8,11]}})";
    while (hdr.size() % 8) hdr += ' ';
    std::string expect(8, '\0');
    for (int i = 0; i < 8; ++i) expect[i] = static_cast<char>((hdr.size() >> (8 * i)) & 0xFF);
    expect += hdr;
    // 1.0f = 0x3F800000, -2.0f = 0xC0000000 (little endian)
    expect += std::string("\x00\x00\x80\x3f\x00\x00\x00\xc0", 8);
    expect += std::string("\xf8\x00\x07", 3);
    const std::string got = read_all(p);
    std::filesystem::remove(p);
    REQUIRE(got == expect);
}

TEST_CASE("safetensors writer/reader round trip for every dtype", "[safetensors]") {
    const std::vector<float> f32{1.5f, -0.25f, 3.0f, 1e-30f, -7.0f, 0.0f};
    const std::vector<std::uint16_t> f16{0x3C00, 0xC000, 0x7BFF, 0x0001};
    const std::vector<std::uint16_t> bf16{0x3F80, 0xBF80, 0x7F7F};
    const std::vector<std::int32_t> i32{-2147483647 - 1, 0, 2147483647};
    const std::vector<std::int8_t> i8{-128, -1, 0, 1, 127};
    const std::vector<std::uint8_t> b{1, 0, 1, 1};
    const std::vector<SafetensorsTensorView> views{
        {"f32", DataType::Float32, {2, 3}, std::as_bytes(std::span(f32))},
        {"f16", DataType::Float16, {4}, std::as_bytes(std::span(f16))},
        {"bf16", DataType::BFloat16, {3, 1}, std::as_bytes(std::span(bf16))},
        {"i32", DataType::Int32, {3}, std::as_bytes(std::span(i32))},
        {"i8", DataType::Int8, {5}, std::as_bytes(std::span(i8))},
        {"bool", DataType::Bool, {2, 2}, std::as_bytes(std::span(b))},
        {"empty", DataType::Float32, {0, 4}, {}},
        {"name with \"quote\"", DataType::Int8, {1}, std::as_bytes(std::span(i8).subspan(0, 1))},
    };
    const auto p = tmp_path("rt.safetensors");
    save_safetensors(p, views, {{"velomind.format", "x"}, {"b", "line\nbreak"}});
    auto f = load_safetensors(p);
    std::filesystem::remove(p);
    REQUIRE(f.has_value());
    REQUIRE(f->tensors.size() == views.size());
    REQUIRE(f->metadata.at("velomind.format") == "x");
    REQUIRE(f->metadata.at("b") == "line\nbreak");
    for (const auto& v : views) {
        const auto& s = *f->tensors.at(v.name);
        REQUIRE(s.dtype == v.dtype);
        REQUIRE(s.shape == v.shape);
        REQUIRE(s.size_bytes == v.bytes.size());
        REQUIRE(s.device == DeviceType::CPU);
        if (!v.bytes.empty()) REQUIRE(std::memcmp(s.data, v.bytes.data(), v.bytes.size()) == 0);
    }
    REQUIRE(values<float>(*f->tensors.at("f32")) == f32);
}

TEST_CASE("safetensors writer rejects inconsistent views", "[safetensors]") {
    const std::vector<float> x{1.0f, 2.0f};
    const auto p = tmp_path("bad.safetensors");
    const std::vector<SafetensorsTensorView> short_bytes{{"x", DataType::Float32, {3}, std::as_bytes(std::span(x))}};
    REQUIRE_THROWS_AS(save_safetensors(p, short_bytes), std::invalid_argument);
    const std::vector<SafetensorsTensorView> dup{{"x", DataType::Float32, {1}, std::as_bytes(std::span(x).subspan(0, 1))},
                                                 {"x", DataType::Float32, {1}, std::as_bytes(std::span(x).subspan(1, 1))}};
    REQUIRE_THROWS_AS(save_safetensors(p, dup), std::invalid_argument);
    const std::vector<SafetensorsTensorView> reserved{{"__metadata__", DataType::Float32, {2}, std::as_bytes(std::span(x))}};
    REQUIRE_THROWS_AS(save_safetensors(p, reserved), std::invalid_argument);
    REQUIRE_THROWS_AS(save_safetensors("/nonexistent_dir_vm/x.safetensors", std::span<const SafetensorsTensorView>{}),
                      std::runtime_error);
    std::filesystem::remove(p);
}

TEST_CASE("safetensors reader: missing, truncated and oversized files", "[safetensors]") {
    REQUIRE(!load_safetensors("/nonexistent_dir_vm/none.safetensors").has_value());
    const auto p = tmp_path("trunc.safetensors");
    const std::string j = R"({"x":{"dtype":"F32","shape":[4],"data_offsets":[0,16]}})";
    write_raw(p, j.size(), j + std::string(8, '\0'));   // 8 of 16 data bytes
    REQUIRE(!load_safetensors(p).has_value());
    write_raw(p, j.size(), j + std::string(16, '\0'));
    REQUIRE(load_safetensors(p).has_value());
    write_raw(p, j.size() + 100, j);                     // header longer than the file
    REQUIRE(!load_safetensors(p).has_value());
    write_raw(p, std::numeric_limits<std::uint64_t>::max(), "");
    REQUIRE(!load_safetensors(p).has_value());
    const std::string far = R"({"x":{"dtype":"F32","shape":[1],"data_offsets":[9223372036854775800,9223372036854775804]}})";
    write_raw(p, far.size(), far);
    REQUIRE(!load_safetensors(p).has_value());
    {
        std::ofstream f(p, std::ios::binary | std::ios::trunc);
        f.write("\x01\x00\x00", 3);                      // shorter than the length field
    }
    REQUIRE(!load_safetensors(p).has_value());
    std::filesystem::remove(p);
}

TEST_CASE("safetensors reader: the toy_llama fixture", "[safetensors]") {
    const auto path = fixture_dir() / "toy_llama" / "model.safetensors";
    if (!std::filesystem::exists(path)) throw vmtest::Skip("fixture missing: " + path.string());
    auto f = load_safetensors(path);
    REQUIRE(f.has_value());
    // 2 layers x 9 tensors + embed, final norm, lm_head (config.json)
    REQUIRE(f->tensors.size() == 21);
    const auto& emb = *f->tensors.at("model.embed_tokens.weight");
    REQUIRE(emb.dtype == DataType::Float32);
    REQUIRE(emb.shape == shape_t({256, 64}));
    const auto& gate = *f->tensors.at("model.layers.1.mlp.gate_proj.weight");
    REQUIRE(gate.shape == shape_t({128, 64}));
    const auto& norm = *f->tensors.at("model.norm.weight");
    REQUIRE(norm.shape == shape_t({64}));
    for (const auto& [name, s] : f->tensors)
        vmtest::require_all_finite(values<float>(*s));
}
