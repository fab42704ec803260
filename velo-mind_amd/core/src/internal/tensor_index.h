// Tensor storage -> index into a graph's tensor list, for the graph's own
// passes (validation order, compilation).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <vector>

#include "velomind/tensor_storage.h"

namespace velomind::internal {

// A flat open-addressing table over a graph's storages (a LLaMA decode
// graph holds ~1600; a node-based hash map of them cost more than the rest
// of a build).
class TensorIndex {
public:
    static constexpr std::size_t npos = SIZE_MAX;
    explicit TensorIndex(const std::vector<std::shared_ptr<TensorStorage>>& tensors) {
        while (_cap < 2 * tensors.size()) _cap <<= 1;
        _keys.assign(_cap, nullptr);
        _vals.assign(_cap, 0);
        for (std::size_t i = 0; i < tensors.size(); ++i) {
            std::size_t h = slot(tensors[i].get());
            while (_keys[h] && _keys[h] != tensors[i].get()) h = (h + 1) & (_cap - 1);
            _keys[h] = tensors[i].get();
            _vals[h] = i;
        }
    }
    std::size_t find(pConstTensorStorage t) const {
        for (std::size_t h = slot(t);; h = (h + 1) & (_cap - 1)) {
            if (_keys[h] == t) return _vals[h];
            if (!_keys[h]) return npos;
        }
    }
    std::size_t at(pConstTensorStorage t) const {
        const std::size_t i = find(t);
        if (i == npos) throw std::out_of_range("velomind: node operand is not a tensor of its graph");
        return i;
    }

private:
    std::size_t slot(pConstTensorStorage t) const {
        auto x = static_cast<std::uint64_t>(reinterpret_cast<std::uintptr_t>(t));
        x ^= x >> 29;
        x *= 0x9E3779B97F4A7C15ull;
        return static_cast<std::size_t>(x >> 32) & (_cap - 1);
    }
    std::size_t _cap = 16;
    std::vector<pConstTensorStorage> _keys;
    std::vector<std::size_t> _vals;
};

}  // namespace velomind::internal
