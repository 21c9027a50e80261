// torch.randn on the CPU generator (the steps are in csrc/torch_randn.h,
// shared with the C ABI's sana_randn_torch_cpu): the same steps as the
// reference's src/torch_rng.cpp:14-68, so the seeded latents of a caller match.
#include "torch_rng.h"

#include <stdexcept>

#include "../csrc/torch_randn.h"

Tensor randn_torch_cpu(const std::vector<size_t> & shape, uint64_t seed) {
    Tensor t(shape);
    std::vector<float> & d = t.data();
    if (d.size() < 16) throw std::invalid_argument("randn_torch_cpu requires at least 16 elements");
    sana_host::randn_torch_fill(d.data(), d.size(), seed);
    return t;
}
