// torch.randn on the CPU generator, as published in ATen: one mt19937 draw per
// element mapped to a 24-bit uniform in [0, 1), then the Box-Muller transform
// over blocks of 16 (u1 = 1 - d[j], u2 = d[j + 8], j < 8; radius
// sqrt(-2 ln u1), angle 2 pi u2 evaluated in double then rounded), with a
// ragged tail recomputed from 16 fresh uniforms at the end of the buffer.
// Same steps as the reference's src/torch_rng.cpp:14-68, so the seeded
// latents of a caller match.
#include "torch_rng.h"

#include <cmath>
#include <random>
#include <stdexcept>

namespace {

float uniform24(std::mt19937 & gen) {
    return static_cast<float>(static_cast<uint32_t>(gen()) & 0xffffffu) * (1.0f / 16777216.0f);
}

void box_muller16(float * d) {
    for (int j = 0; j < 8; ++j) {
        const float u1 = 1.0f - d[j], u2 = d[j + 8];
        const float r = std::sqrt(-2.0f * std::log(u1));
        const float a = static_cast<float>(2.0 * 3.14159265358979323846 * static_cast<double>(u2));
        d[j] = r * std::cos(a);
        d[j + 8] = r * std::sin(a);
    }
}

}  // namespace

Tensor randn_torch_cpu(const std::vector<size_t> & shape, uint64_t seed) {
    Tensor t(shape);
    std::vector<float> & d = t.data();
    if (d.size() < 16) throw std::invalid_argument("randn_torch_cpu requires at least 16 elements");
    std::mt19937 gen(static_cast<std::mt19937::result_type>(seed & 0xffffffffULL));
    for (float & v : d) v = uniform24(gen);
    size_t i = 0;
    for (; i + 16 <= d.size(); i += 16) box_muller16(d.data() + i);
    if (d.size() % 16) {
        float * tail = d.data() + d.size() - 16;
        for (int j = 0; j < 16; ++j) tail[j] = uniform24(gen);
        box_muller16(tail);
    }
    return t;
}
