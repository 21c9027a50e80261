// Seeded normal draws with torch.randn's CPU semantics (the interface of the
// reference's src/torch_rng.h:14): used by callers for the initial latent.
#pragma once

#include <cstdint>
#include <vector>

#include "tensor.h"

Tensor randn_torch_cpu(const std::vector<size_t> & shape, uint64_t seed);
