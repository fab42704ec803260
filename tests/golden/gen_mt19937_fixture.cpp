// Writes the first values of std::mt19937(1337) fed through libstdc++'s
// std::uniform_real_distribution<float> for the ranges the reference's
// quantization tests use (tests/test_quantization.cpp:37-45), as JSON.
// The fixture pins tests/golden/ref_inputs.py, which regenerates the same
// stream in numpy at any size.
#include <cstdio>
#include <cstring>
#include <cstdint>
#include <random>

static void dump(const char* name, float lo, float hi, int count, bool last) {
    std::mt19937 rng(1337);
    std::uniform_real_distribution<float> dist(lo, hi);
    std::printf("  \"%s\": [", name);
    for (int i = 0; i < count; ++i) {
        float v = dist(rng);
        std::uint32_t bits;
        std::memcpy(&bits, &v, 4);
        std::printf("%s%u", i ? ", " : "", bits);
    }
    std::printf("]%s\n", last ? "" : ",");
}

int main() {
    std::printf("{\n");
    std::mt19937 raw(1337);
    std::printf("  \"raw_u32\": [");
    for (int i = 0; i < 16; ++i) std::printf("%s%u", i ? ", " : "", (unsigned)raw());
    std::printf("],\n");
    dump("u_m1_p1_bits", -1.0f, 1.0f, 1024, false);
    dump("u_m1p5_p1p5_bits", -1.5f, 1.5f, 1024, true);
    std::printf("}\n");
    return 0;
}
