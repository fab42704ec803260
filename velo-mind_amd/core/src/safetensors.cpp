// safetensors reader and writer (include/velomind/safetensors.h).
//
// The header is parsed by a small recursive-descent JSON reader that
// handles exactly what the format uses (objects, arrays, strings with
// escapes, non-negative integers); the checks follow the reference reader
// (src/safetensors.cpp:222-400): known dtypes only, byte spans equal to
// numel * width, ranges that do not overlap and lie inside the file.
#include "velomind/safetensors.h"

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <limits>
#include <map>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace velomind {

namespace {

constexpr std::size_t kMaxHeader = 100u << 20;
constexpr int kMaxDepth = 64;

struct Json {
    enum Kind { Obj, Arr, Str, Int } kind = Obj;
    std::string s;
    std::int64_t i = 0;
    std::vector<std::pair<std::string, Json>> obj;   // insertion order
    std::vector<Json> arr;
};

class Reader {
public:
    explicit Reader(std::span<const std::byte> b) : b_(b) {}

    Json value(int depth) {
        if (depth > kMaxDepth) throw std::runtime_error("nesting too deep");
        ws();
        const char c = peek();
        if (c == '{') return object(depth);
        if (c == '[') return array(depth);
        if (c == '"') {
            Json j;
            j.kind = Json::Str;
            j.s = string();
            return j;
        }
        if (c == '-' || (c >= '0' && c <= '9')) return integer();
        throw std::runtime_error(std::string("unexpected character '") + c + "'");
    }
    bool done() {
        ws();
        return p_ >= b_.size();
    }

private:
    char peek() const {
        if (p_ >= b_.size()) throw std::runtime_error("unexpected end");
        return static_cast<char>(b_[p_]);
    }
    char get() {
        const char c = peek();
        ++p_;
        return c;
    }
    void expect(char c) {
        if (get() != c) throw std::runtime_error(std::string("expected '") + c + "'");
    }
    void ws() {
        while (p_ < b_.size()) {
            const char c = static_cast<char>(b_[p_]);
            if (c != ' ' && c != '\t' && c != '\n' && c != '\r') break;
            ++p_;
        }
    }
    static void utf8(std::string& out, std::uint32_t cp) {
        if (cp < 0x80) {
            out += static_cast<char>(cp);
        } else if (cp < 0x800) {
            out += static_cast<char>(0xC0 | (cp >> 6));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            out += static_cast<char>(0xE0 | (cp >> 12));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        } else {
            out += static_cast<char>(0xF0 | (cp >> 18));
            out += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
            out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
            out += static_cast<char>(0x80 | (cp & 0x3F));
        }
    }
    std::uint32_t hex4() {
        std::uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = get();
            v <<= 4;
            if (c >= '0' && c <= '9') v |= static_cast<std::uint32_t>(c - '0');
            else if (c >= 'a' && c <= 'f') v |= static_cast<std::uint32_t>(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= static_cast<std::uint32_t>(c - 'A' + 10);
            else throw std::runtime_error("bad \\u escape");
        }
        return v;
    }
    std::string string() {
        expect('"');
        std::string out;
        for (;;) {
            const char c = get();
            if (c == '"') return out;
            if (static_cast<unsigned char>(c) < 0x20) throw std::runtime_error("control character in string");
            if (c != '\\') {
                out += c;
                continue;
            }
            const char e = get();
            switch (e) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    std::uint32_t cp = hex4();
                    if (cp >= 0xD800 && cp < 0xDC00) {   // surrogate pair
                        expect('\\');
                        expect('u');
                        const std::uint32_t lo = hex4();
                        if (lo < 0xDC00 || lo >= 0xE000) throw std::runtime_error("bad surrogate pair");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    utf8(out, cp);
                    break;
                }
                default: throw std::runtime_error("bad escape");
            }
        }
    }
    Json integer() {
        Json j;
        j.kind = Json::Int;
        bool neg = false;
        if (peek() == '-') {
            neg = true;
            ++p_;
        }
        if (p_ >= b_.size() || peek() < '0' || peek() > '9') throw std::runtime_error("bad number");
        std::uint64_t v = 0;
        while (p_ < b_.size() && peek() >= '0' && peek() <= '9') {
            const auto d = static_cast<std::uint64_t>(get() - '0');
            if (v > (static_cast<std::uint64_t>(std::numeric_limits<std::int64_t>::max()) - d) / 10)
                throw std::runtime_error("integer overflow");
            v = v * 10 + d;
        }
        if (p_ < b_.size() && (peek() == '.' || peek() == 'e' || peek() == 'E'))
            throw std::runtime_error("non-integer number");
        j.i = neg ? -static_cast<std::int64_t>(v) : static_cast<std::int64_t>(v);
        return j;
    }
    Json array(int depth) {
        Json j;
        j.kind = Json::Arr;
        expect('[');
        ws();
        if (peek() == ']') {
            ++p_;
            return j;
        }
        for (;;) {
            j.arr.push_back(value(depth + 1));
            ws();
            const char c = get();
            if (c == ']') return j;
            if (c != ',') throw std::runtime_error("expected ',' or ']'");
        }
    }
    Json object(int depth) {
        Json j;
        j.kind = Json::Obj;
        expect('{');
        ws();
        if (peek() == '}') {
            ++p_;
            return j;
        }
        for (;;) {
            ws();
            std::string key = string();
            ws();
            expect(':');
            for (const auto& kv : j.obj)
                if (kv.first == key) throw std::runtime_error("duplicate key");
            j.obj.emplace_back(std::move(key), value(depth + 1));
            ws();
            const char c = get();
            if (c == '}') return j;
            if (c != ',') throw std::runtime_error("expected ',' or '}'");
        }
    }

    std::span<const std::byte> b_;
    std::size_t p_ = 0;
};

struct DtypeInfo {
    const char* name;
    DataType dtype;
    std::size_t width;
};
constexpr DtypeInfo kDtypes[] = {
    {"F32", DataType::Float32, 4}, {"F16", DataType::Float16, 2}, {"BF16", DataType::BFloat16, 2},
    {"I32", DataType::Int32, 4},   {"I8", DataType::Int8, 1},     {"BOOL", DataType::Bool, 1},
};

const DtypeInfo* dtype_by_name(const std::string& s) {
    for (const auto& d : kDtypes)
        if (s == d.name) return &d;
    return nullptr;
}

const DtypeInfo* dtype_by_type(DataType t) {
    for (const auto& d : kDtypes)
        if (d.dtype == t) return &d;
    return nullptr;
}

const Json* field(const Json& o, const char* key) {
    for (const auto& [k, v] : o.obj)
        if (k == key) return &v;
    return nullptr;
}

std::optional<SafetensorsHeaderEntry> parse_entry(const Json& v) {
    if (v.kind != Json::Obj) return std::nullopt;
    const Json* dt = field(v, "dtype");
    const Json* sh = field(v, "shape");
    const Json* of = field(v, "data_offsets");
    if (!dt || !sh || !of || dt->kind != Json::Str || sh->kind != Json::Arr || of->kind != Json::Arr)
        return std::nullopt;
    const DtypeInfo* info = dtype_by_name(dt->s);
    if (!info) return std::nullopt;
    SafetensorsHeaderEntry e;
    e.dtype = info->dtype;
    std::size_t numel = 1;
    bool empty = false;
    for (const Json& d : sh->arr) {
        if (d.kind != Json::Int || d.i < 0) return std::nullopt;
        e.shape.push_back(static_cast<dim_t>(d.i));
        if (d.i == 0) empty = true;
    }
    if (!empty) {
        for (dim_t d : e.shape) {
            const auto w = static_cast<std::size_t>(d);
            if (numel > std::numeric_limits<std::size_t>::max() / w) return std::nullopt;
            numel *= w;
        }
    } else {
        numel = 0;
    }
    if (of->arr.size() != 2 || of->arr[0].kind != Json::Int || of->arr[1].kind != Json::Int) return std::nullopt;
    const std::int64_t b = of->arr[0].i, en = of->arr[1].i;
    if (b < 0 || en < b) return std::nullopt;
    if (numel > std::numeric_limits<std::size_t>::max() / info->width) return std::nullopt;
    if (static_cast<std::size_t>(en - b) != numel * info->width) return std::nullopt;
    e.begin = static_cast<std::size_t>(b);
    e.end = static_cast<std::size_t>(en);
    return e;
}

std::string json_escape(const std::string& s) {
    std::string out;
    out.reserve(s.size() + 2);
    for (const char c : s) {
        switch (c) {
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            case '\n': out += "\\n"; break;
            case '\r': out += "\\r"; break;
            case '\t': out += "\\t"; break;
            default:
                if (static_cast<unsigned char>(c) < 0x20) {
                    static const char* hex = "0123456789abcdef";
                    out += "\\u00";
                    out += hex[(c >> 4) & 0xF];
                    out += hex[c & 0xF];
                } else {
                    out += c;
                }
        }
    }
    return out;
}

}  // namespace

auto parse_safetensors_header(std::span<const std::byte> header_bytes) -> std::optional<SafetensorsHeader> {
    if (header_bytes.empty() || header_bytes.size() > kMaxHeader) return std::nullopt;
    Json root;
    try {
        Reader r(header_bytes);
        root = r.value(0);
        if (!r.done()) return std::nullopt;
    } catch (const std::exception&) {
        return std::nullopt;
    }
    if (root.kind != Json::Obj) return std::nullopt;
    SafetensorsHeader out;
    for (const auto& [name, v] : root.obj) {
        if (name == "__metadata__") {
            if (v.kind != Json::Obj) return std::nullopt;
            for (const auto& [k, mv] : v.obj) {
                if (mv.kind != Json::Str) return std::nullopt;
                out.metadata[k] = mv.s;
            }
            continue;
        }
        auto e = parse_entry(v);
        if (!e || !out.tensors.emplace(name, std::move(*e)).second) return std::nullopt;
    }
    std::vector<std::pair<std::size_t, std::size_t>> ranges;
    for (const auto& [_, e] : out.tensors) ranges.emplace_back(e.begin, e.end);
    std::sort(ranges.begin(), ranges.end());
    std::size_t prev = 0;
    for (const auto& [b, e] : ranges) {
        if (b < prev) return std::nullopt;   // overlap
        prev = std::max(prev, e);
    }
    return out;
}

auto load_safetensors(const std::filesystem::path& path) -> std::optional<SafetensorsFile> {
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) return std::nullopt;
    const std::streamoff total = f.tellg();
    if (total < 8) return std::nullopt;
    f.seekg(0);
    unsigned char len_le[8];
    if (!f.read(reinterpret_cast<char*>(len_le), 8)) return std::nullopt;
    std::uint64_t hlen = 0;
    for (int i = 0; i < 8; ++i) hlen |= static_cast<std::uint64_t>(len_le[i]) << (8 * i);
    if (hlen == 0 || hlen > kMaxHeader || hlen > static_cast<std::uint64_t>(total) - 8) return std::nullopt;
    std::vector<std::byte> hdr(static_cast<std::size_t>(hlen));
    if (!f.read(reinterpret_cast<char*>(hdr.data()), static_cast<std::streamsize>(hlen))) return std::nullopt;
    auto header = parse_safetensors_header(hdr);
    if (!header) return std::nullopt;
    const std::size_t data_bytes = static_cast<std::size_t>(total) - 8 - static_cast<std::size_t>(hlen);
    SafetensorsFile out;
    out.metadata = header->metadata;
    for (const auto& [name, e] : header->tensors) {
        if (e.end > data_bytes) return std::nullopt;
        const std::size_t bytes = e.end - e.begin;
        auto s = TensorStorage::allocate(bytes, DeviceType::CPU);
        if (!s) return std::nullopt;
        s->shape = e.shape;
        s->dtype = e.dtype;
        s->size_bytes = bytes;
        if (bytes) {
            f.seekg(static_cast<std::streamoff>(8 + hlen + e.begin));
            if (!f.read(static_cast<char*>(s->data), static_cast<std::streamsize>(bytes))) return std::nullopt;
        }
        out.tensors.emplace(name, std::move(s));
    }
    return out;
}

void save_safetensors(const std::filesystem::path& path, std::span<const SafetensorsTensorView> tensors,
                      const std::unordered_map<std::string, std::string>& metadata) {
    std::string hdr = "{";
    bool first = true;
    if (!metadata.empty()) {
        // sorted keys: the same metadata always writes the same bytes
        std::map<std::string, std::string> sorted(metadata.begin(), metadata.end());
        hdr += "\"__metadata__\":{";
        bool mfirst = true;
        for (const auto& [k, v] : sorted) {
            if (!mfirst) hdr += ",";
            mfirst = false;
            hdr += "\"" + json_escape(k) + "\":\"" + json_escape(v) + "\"";
        }
        hdr += "}";
        first = false;
    }
    std::size_t offset = 0;
    std::unordered_map<std::string, int> seen;
    for (const auto& t : tensors) {
        if (t.name.empty() || t.name == "__metadata__" || !seen.emplace(t.name, 1).second)
            throw std::invalid_argument("save_safetensors: empty, reserved or duplicate tensor name '" + t.name + "'");
        const DtypeInfo* info = dtype_by_type(t.dtype);
        if (!info) throw std::invalid_argument("save_safetensors: unsupported dtype for '" + t.name + "'");
        std::size_t numel = 1;
        for (dim_t d : t.shape) {
            if (d < 0) throw std::invalid_argument("save_safetensors: negative dimension in '" + t.name + "'");
            numel *= static_cast<std::size_t>(d);
        }
        if (numel * info->width != t.bytes.size())
            throw std::invalid_argument("save_safetensors: byte count of '" + t.name + "' does not match its shape");
        if (!first) hdr += ",";
        first = false;
        hdr += "\"" + json_escape(t.name) + "\":{\"dtype\":\"" + info->name + "\",\"shape\":[";
        for (std::size_t i = 0; i < t.shape.size(); ++i) {
            if (i) hdr += ",";
            hdr += std::to_string(t.shape[i]);
        }
        hdr += "],\"data_offsets\":[" + std::to_string(offset) + "," + std::to_string(offset + t.bytes.size()) + "]}";
        offset += t.bytes.size();
    }
    hdr += "}";
    while (hdr.size() % 8) hdr += ' ';
    std::ofstream f(path, std::ios::binary | std::ios::trunc);
    if (!f) throw std::runtime_error("save_safetensors: cannot open '" + path.string() + "' for writing");
    unsigned char len_le[8];
    const std::uint64_t hlen = hdr.size();
    for (int i = 0; i < 8; ++i) len_le[i] = static_cast<unsigned char>(hlen >> (8 * i));
    f.write(reinterpret_cast<const char*>(len_le), 8);
    f.write(hdr.data(), static_cast<std::streamsize>(hdr.size()));
    for (const auto& t : tensors)
        if (!t.bytes.empty()) f.write(reinterpret_cast<const char*>(t.bytes.data()), static_cast<std::streamsize>(t.bytes.size()));
    if (!f) throw std::runtime_error("save_safetensors: write to '" + path.string() + "' failed");
}

}  // namespace velomind
