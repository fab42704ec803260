// InlineList: a short list kept in place up to N elements (on the heap
// beyond).  Node operands and compiled steps use it: a graph build makes
// thousands of such lists, nearly all of one to eight elements.
#pragma once

#include <array>
#include <cstddef>
#include <span>
#include <utility>
#include <vector>

namespace velomind {

template <typename T, std::size_t N>
class InlineList {
public:
    InlineList() = default;
    InlineList(const InlineList& o) { *this = o; }
    InlineList& operator=(const InlineList& o) {
        if (this != &o) {
            clear();
            reserve(o.size());
            for (const T& v : o) push_back(v);
        }
        return *this;
    }
    InlineList(InlineList&& o) noexcept : _in(o._in), _heap(std::move(o._heap)), _n(o._n), _on_heap(o._on_heap) {
        o.clear();
    }
    InlineList& operator=(InlineList&& o) noexcept {
        _in = o._in;
        _heap = std::move(o._heap);
        _n = o._n;
        _on_heap = o._on_heap;
        o.clear();
        return *this;
    }
    void reserve(std::size_t n) {
        if (_on_heap) {
            _heap.reserve(n);
        } else if (n > N) {
            _heap.reserve(n);
            _heap.assign(_in.begin(), _in.begin() + static_cast<std::ptrdiff_t>(_n));
            _on_heap = true;
        }
    }
    void push_back(const T& v) {
        if (!_on_heap) {
            if (_n < N) {
                _in[_n++] = v;
                return;
            }
            reserve(2 * N);
        }
        _heap.push_back(v);
        _n = _heap.size();
    }
    void clear() noexcept {
        _heap.clear();
        _n = 0;
        _on_heap = false;
    }
    std::size_t size() const noexcept { return _n; }
    bool empty() const noexcept { return _n == 0; }
    T* data() noexcept { return _on_heap ? _heap.data() : _in.data(); }
    const T* data() const noexcept { return _on_heap ? _heap.data() : _in.data(); }
    T* begin() noexcept { return data(); }
    T* end() noexcept { return data() + _n; }
    const T* begin() const noexcept { return data(); }
    const T* end() const noexcept { return data() + _n; }
    T& operator[](std::size_t i) noexcept { return data()[i]; }
    const T& operator[](std::size_t i) const noexcept { return data()[i]; }

private:
    std::array<T, N> _in{};
    std::vector<T> _heap;
    std::size_t _n = 0;
    bool _on_heap = false;
};

}  // namespace velomind
