// Per-device cache of device blocks in size classes, behind the HIP storage
// creator (hip_backend.cpp).  The device calls (allocate, free, device-wide
// synchronize) come in through BlockOps, so the cache logic runs on the CPU
// in tests with a fake device.
//
// A freed block is parked, and becomes reusable only after a device-wide
// synchronization that began after it was freed (the guarantee hipFree
// gives).  take() performs that synchronization itself when a request finds
// only parked blocks of its class.  allocate() falls back to the device
// allocator, and when that fails, releases every cached block of the device
// (after a synchronization) and tries once more, so idle cached memory never
// causes an out-of-memory error.  No device call runs under the cache's lock.
#pragma once

#include <cstddef>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

namespace velomind::backend::hip {

// Size class of a request: 256-byte multiples up to 2 KiB, then eight
// classes per power of two (a K/V cache grown by one row usually keeps its
// class).
inline std::size_t block_size_class(std::size_t bytes) {
    constexpr std::size_t kMin = 256;
    if (bytes <= 8 * kMin) return (bytes + kMin - 1) / kMin * kMin;
    std::size_t p = 1;
    while (p * 2 <= bytes) p *= 2;   // p <= bytes < 2p
    const std::size_t step = p / 8;
    return (bytes + step - 1) / step * step;
}

struct BlockOps {
    // 0 on success, like the vm_hip_* entry points.
    int (*malloc)(void** p, std::size_t bytes) = nullptr;
    int (*free)(void* p) = nullptr;
    int (*synchronize)() = nullptr;   // device-wide, on the current device
};

class BlockCache {
public:
    BlockCache(BlockOps ops, std::size_t max_cached_bytes) : _ops(ops), _max(max_cached_bytes) {}

    // A block of class `cls` (block_size_class of the request) on device d,
    // or nullptr when the device allocator fails even after the cache is
    // released.
    void* allocate(int d, std::size_t cls) {
        if (void* p = take(d, cls)) return p;
        void* p = nullptr;
        if (_ops.malloc(&p, cls) == 0 && p) return p;
        release_device(d);
        p = nullptr;
        if (_ops.malloc(&p, cls) == 0 && p) return p;
        return nullptr;
    }

    // Parks a freed block; false when the cache is full (the block is then
    // freed here).
    bool park(int d, std::size_t cls, void* p) {
        {
            std::lock_guard<std::mutex> lock(_mu);
            if (_cached + cls <= _max) {
                _dev[d].parked[cls].push_back(p);
                _cached += cls;
                return true;
            }
        }
        (void)_ops.free(p);
        return false;
    }

    // Frees every cached block of device d (parked ones after a device
    // synchronization).  Returns the bytes given back.
    std::size_t release_device(int d) {
        Lists ready, parked;
        {
            std::lock_guard<std::mutex> lock(_mu);
            auto it = _dev.find(d);
            if (it == _dev.end()) return 0;
            ready.swap(it->second.ready);
            parked.swap(it->second.parked);
            _cached -= bytes_of(ready) + bytes_of(parked);
        }
        if (!parked.empty()) (void)_ops.synchronize();
        std::size_t freed = 0;
        for (Lists* l : {&ready, &parked})
            for (auto& [cls, v] : *l)
                for (void* p : v) {
                    (void)_ops.free(p);
                    freed += cls;
                }
        return freed;
    }

    // Makes every block parked on device d reusable, after one device-wide
    // synchronization (none when nothing is parked).  Called where the device
    // is idle anyway, it spares a later take() that synchronization while
    // other work runs.
    void reclaim(int d) {
        Lists parked;
        {
            std::lock_guard<std::mutex> lock(_mu);
            auto it = _dev.find(d);
            if (it == _dev.end() || it->second.parked.empty()) return;
            parked.swap(it->second.parked);
        }
        const bool drained = _ops.synchronize() == 0;
        std::lock_guard<std::mutex> lock(_mu);
        PerDevice& pd = _dev[d];
        Lists& dst = drained ? pd.ready : pd.parked;
        for (auto& [c, v] : parked) {
            auto& r = dst[c];
            r.insert(r.end(), v.begin(), v.end());
        }
    }
    std::size_t cached_bytes() {
        std::lock_guard<std::mutex> lock(_mu);
        return _cached;
    }

private:
    using Lists = std::map<std::size_t, std::vector<void*>>;
    struct PerDevice {
        Lists ready;    // idle: reusable now
        Lists parked;   // freed since the last device synchronization
    };

    static std::size_t bytes_of(const Lists& l) {
        std::size_t b = 0;
        for (const auto& [cls, v] : l) b += cls * v.size();
        return b;
    }

    static void* pop(Lists& l, std::size_t cls) {
        auto it = l.find(cls);
        if (it == l.end() || it->second.empty()) return nullptr;
        void* p = it->second.back();
        it->second.pop_back();
        return p;
    }

    void* take(int d, std::size_t cls) {
        Lists parked;
        {
            std::lock_guard<std::mutex> lock(_mu);
            PerDevice& pd = _dev[d];
            if (void* p = pop(pd.ready, cls)) {
                _cached -= cls;
                return p;
            }
            auto pk = pd.parked.find(cls);
            if (pk == pd.parked.end() || pk->second.empty()) return nullptr;
            // Every block parked so far becomes idle once the device has
            // drained; blocks parked while it drains stay parked.
            parked.swap(pd.parked);
        }
        const bool drained = _ops.synchronize() == 0;
        std::lock_guard<std::mutex> lock(_mu);
        PerDevice& pd = _dev[d];
        Lists& dst = drained ? pd.ready : pd.parked;
        for (auto& [c, v] : parked) {
            auto& r = dst[c];
            r.insert(r.end(), v.begin(), v.end());
        }
        if (!drained) return nullptr;
        void* p = pop(pd.ready, cls);
        if (p) _cached -= cls;
        return p;
    }

    BlockOps _ops;
    std::size_t _max;
    std::mutex _mu;
    std::map<int, PerDevice> _dev;
    std::size_t _cached = 0;
};

}  // namespace velomind::backend::hip
