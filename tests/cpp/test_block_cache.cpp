// The HIP storage creator's block cache (core/src/backend_hip/block_cache.h)
// on a fake device: size classes, reuse only after a device
// synchronization, and the release-and-retry path when the device
// allocator fails while blocks sit idle in the cache.
#include <cstdlib>
#include <set>

#include "backend_hip/block_cache.h"
#include "vm_test.h"

using namespace velomind::backend::hip;

namespace {

// A device with `capacity` bytes: every block is a host allocation, and
// the fake records outstanding bytes, synchronizations and frees.
struct FakeDevice {
    std::size_t capacity = 0, used = 0;
    int syncs = 0, frees = 0, mallocs = 0;
    std::set<void*> live;
    std::map<void*, std::size_t> size;
};
FakeDevice* g_dev = nullptr;

int fake_malloc(void** p, std::size_t n) {
    ++g_dev->mallocs;
    if (g_dev->used + n > g_dev->capacity) return -1;
    *p = std::malloc(n);
    g_dev->used += n;
    g_dev->live.insert(*p);
    g_dev->size[*p] = n;
    return 0;
}

int fake_free(void* p) {
    ++g_dev->frees;
    g_dev->used -= g_dev->size.at(p);
    g_dev->size.erase(p);
    g_dev->live.erase(p);
    std::free(p);
    return 0;
}

int fake_sync() {
    ++g_dev->syncs;
    return 0;
}

BlockOps fake_ops() { return BlockOps{fake_malloc, fake_free, fake_sync}; }

}  // namespace

TEST_CASE("block size classes: 256-byte steps, then eight per power of two", "[core][memory]") {
    CHECK(block_size_class(1) == 256);
    CHECK(block_size_class(256) == 256);
    CHECK(block_size_class(257) == 512);
    CHECK(block_size_class(2048) == 2048);
    CHECK(block_size_class(2049) == 2304);            // 2048 + 2048/8
    CHECK(block_size_class(4096) == 4096);
    CHECK(block_size_class(4097) == 4608);
    CHECK(block_size_class((1u << 20) + 1) == (1u << 20) + (1u << 17));
    // a K/V cache grown by one 256-float row keeps its class
    const std::size_t kv = std::size_t(32) * 5 * 200 * 64 * 4;
    CHECK(block_size_class(kv) == block_size_class(kv + 64 * 4));
    for (std::size_t b = 1; b < (1u << 22); b = b * 3 + 7) {
        const std::size_t c = block_size_class(b);
        CHECK(c >= b);
        CHECK(c - b <= std::max<std::size_t>(255, b / 8));
    }
}

TEST_CASE("block cache reuses a freed block only after a device synchronization", "[core][memory]") {
    FakeDevice dev;
    dev.capacity = 1 << 20;
    g_dev = &dev;
    BlockCache cache(fake_ops(), 1 << 20);
    void* a = cache.allocate(0, 4096);
    REQUIRE(a);
    REQUIRE(cache.park(0, 4096, a));
    CHECK(dev.syncs == 0);
    void* b = cache.allocate(0, 4096);   // only a parked block of the class: synchronize, then reuse
    CHECK(b == a);
    CHECK(dev.syncs == 1);
    CHECK(dev.mallocs == 1);
    void* c = cache.allocate(0, 8192);   // other class: new block
    CHECK(c != a);
    CHECK(dev.mallocs == 2);
    REQUIRE(cache.park(0, 4096, b));
    REQUIRE(cache.park(1, 8192, c));     // another device's blocks stay apart
    void* d = cache.allocate(0, 8192);
    CHECK(d != c);
    CHECK(cache.cached_bytes() == 4096 + 8192);
    REQUIRE(cache.park(0, 8192, d));
    cache.release_device(0);
    cache.release_device(1);
    CHECK(cache.cached_bytes() == 0);
}

TEST_CASE("block cache reclaim makes parked blocks reusable with one synchronization", "[core][memory]") {
    FakeDevice dev;
    dev.capacity = 1 << 20;
    g_dev = &dev;
    BlockCache cache(fake_ops(), 1 << 20);
    cache.reclaim(0);                    // nothing parked: no synchronization
    CHECK(dev.syncs == 0);
    void* a = cache.allocate(0, 4096);
    void* b = cache.allocate(0, 8192);
    REQUIRE(cache.park(0, 4096, a));
    REQUIRE(cache.park(0, 8192, b));
    cache.reclaim(0);
    CHECK(dev.syncs == 1);
    CHECK(cache.allocate(0, 8192) == b);  // both classes reusable without another synchronization
    CHECK(cache.allocate(0, 4096) == a);
    CHECK(dev.syncs == 1);
    CHECK(dev.mallocs == 2);
    REQUIRE(cache.park(0, 4096, a));
    REQUIRE(cache.park(0, 8192, b));
    cache.release_device(0);
    CHECK(dev.live.empty());
}

TEST_CASE("block cache gives idle blocks back when the device allocator fails", "[core][memory]") {
    FakeDevice dev;
    dev.capacity = 64 << 10;
    g_dev = &dev;
    BlockCache cache(fake_ops(), 1 << 30);
    // fill the device with idle blocks of a small class
    std::vector<void*> small;
    for (int i = 0; i < 16; ++i) small.push_back(cache.allocate(0, 4096));
    for (void* p : small) REQUIRE(p);
    for (void* p : small) REQUIRE(cache.park(0, 4096, p));
    CHECK(dev.used == 64u << 10);
    // a larger class fails at first, then succeeds after the cache is released
    const int syncs = dev.syncs;
    void* big = cache.allocate(0, 32 << 10);
    REQUIRE(big);
    CHECK(dev.syncs == syncs + 1);      // parked blocks are freed only after the device drained
    CHECK(cache.cached_bytes() == 0);
    CHECK(dev.used == 32u << 10);
    // nothing left to release: a request beyond the device fails cleanly
    CHECK(cache.allocate(0, 64 << 10) == nullptr);
    REQUIRE(cache.park(0, 32 << 10, big));
    CHECK(cache.release_device(0) == (32u << 10));
    CHECK(dev.live.empty());
}

TEST_CASE("block cache frees blocks beyond its limit at once", "[core][memory]") {
    FakeDevice dev;
    dev.capacity = 1 << 20;
    g_dev = &dev;
    BlockCache cache(fake_ops(), 8192);
    void* a = cache.allocate(0, 8192);
    void* b = cache.allocate(0, 4096);
    REQUIRE(cache.park(0, 8192, a));
    CHECK(!cache.park(0, 4096, b));     // over the limit: freed, not cached
    CHECK(dev.frees == 1);
    CHECK(cache.cached_bytes() == 8192);
    cache.release_device(0);
    CHECK(dev.live.empty());
}
