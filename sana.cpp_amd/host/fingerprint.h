// Identity of a host weight object for the device-residency caches of the
// drop-in API: FNV-1a over each tensor's storage address, shape and values
// (all of them up to 4096, else 64 spread samples plus the last), so a
// reallocated or refilled weights object is uploaded again.
#pragma once

#include <cstdint>
#include <cstring>

#include "tensor.h"

namespace sana_fp {

constexpr uint64_t kSeed = 14695981039346656037ULL;

inline void mix(uint64_t & h, uint64_t v) {
    h ^= v;
    h *= 1099511628211ULL;
}

inline void tensor(uint64_t & h, const Tensor & t) {
    const std::vector<float> & d = t.data();
    mix(h, static_cast<uint64_t>(reinterpret_cast<uintptr_t>(d.data())));
    mix(h, t.rank());
    for (size_t s : t.shape()) mix(h, s);
    const size_t n = d.size(), step = n <= 4096 ? 1 : n / 64;
    for (size_t i = 0; i < n; i += step) {
        uint32_t b;
        std::memcpy(&b, &d[i], 4);
        mix(h, b);
    }
    if (n) {
        uint32_t b;
        std::memcpy(&b, &d[n - 1], 4);
        mix(h, b);
    }
}

}  // namespace sana_fp
