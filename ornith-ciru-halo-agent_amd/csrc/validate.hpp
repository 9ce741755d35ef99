// Host-side argument checks shared by the C entry points: alignment, byte
// ranges that must not wrap, and the no-alias rule for mutable buffers.
#pragma once
#include <cstddef>
#include <cstdint>
#include <limits>

namespace ornith {

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

struct Range { uintptr_t lo, hi; };

inline bool to_range(const void* p, size_t n, Range& r) {
    const uintptr_t lo = reinterpret_cast<uintptr_t>(p);
    if (!p || n > std::numeric_limits<uintptr_t>::max() - lo) return false;
    r = {lo, lo + n};
    return true;
}

// One buffer argument of an entry point.  `optional` buffers may be null
// (then they are skipped); every other buffer must be non-null, aligned and
// not wrap the address space.
struct Buffer {
    const void* ptr;
    size_t bytes;
    size_t align;
    bool mutable_;
    bool optional;
};

// True when every present buffer is valid and no mutable buffer overlaps any
// other present buffer (inputs may overlap each other).
template <size_t N>
bool check_buffers(const Buffer (&b)[N]) {
    Range r[N]{};
    bool present[N]{};
    for (size_t i = 0; i < N; ++i) {
        if (!b[i].ptr && b[i].optional) continue;
        if (!aligned(b[i].ptr, b[i].align) || !to_range(b[i].ptr, b[i].bytes, r[i])) return false;
        present[i] = true;
    }
    for (size_t i = 0; i < N; ++i) {
        if (!present[i] || !b[i].mutable_) continue;
        for (size_t j = 0; j < N; ++j)
            if (j != i && present[j] && r[i].lo < r[j].hi && r[j].lo < r[i].hi) return false;
    }
    return true;
}

}  // namespace ornith
