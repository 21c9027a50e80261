// torch.randn on the CPU generator, as published in ATen, filling a float
// buffer: one mt19937 draw per element mapped to a 24-bit uniform in [0, 1),
// then the Box-Muller transform over blocks of 16 (u1 = 1 - d[j], u2 = d[j + 8],
// j < 8; radius sqrt(-2 ln u1), angle 2 pi u2 evaluated in double then
// rounded), with a ragged tail recomputed from 16 fresh uniforms at the end of
// the buffer.  Same steps as the reference's src/torch_rng.cpp:14-68, so seeded
// latents (and the seeded synthetic weights the benchmarks use) match it.
// Host code only; shared by the drop-in's randn_torch_cpu and the C ABI.
#pragma once

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <random>

namespace sana_host {

inline float randn_uniform24(std::mt19937 & gen) {
    return static_cast<float>(static_cast<uint32_t>(gen()) & 0xffffffu) * (1.0f / 16777216.0f);
}

inline void randn_box_muller16(float * d) {
    for (int j = 0; j < 8; ++j) {
        const float u1 = 1.0f - d[j], u2 = d[j + 8];
        const float r = std::sqrt(-2.0f * std::log(u1));
        const float a = static_cast<float>(2.0 * 3.14159265358979323846 * static_cast<double>(u2));
        d[j] = r * std::cos(a);
        d[j + 8] = r * std::sin(a);
    }
}

// n >= 16 (torch's own requirement for this path).
inline void randn_torch_fill(float * d, size_t n, uint64_t seed) {
    std::mt19937 gen(static_cast<std::mt19937::result_type>(seed & 0xffffffffULL));
    for (size_t i = 0; i < n; ++i) d[i] = randn_uniform24(gen);
    size_t i = 0;
    for (; i + 16 <= n; i += 16) randn_box_muller16(d + i);
    if (n % 16) {
        float * tail = d + n - 16;
        for (int j = 0; j < 16; ++j) tail[j] = randn_uniform24(gen);
        randn_box_muller16(tail);
    }
}

}  // namespace sana_host
