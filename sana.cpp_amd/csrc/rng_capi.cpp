// C ABI of the seeded torch.randn CPU generator (include/sana_dit.h).
#include <string>

#include "../../include/sana_dit.h"
#include "torch_randn.h"

namespace sana {
void set_last_error(const std::string & m);
}

extern "C" int sana_randn_torch_cpu(float * out, int64_t n, uint64_t seed) {
    if (!out) {
        sana::set_last_error("null argument");
        return SANA_ERR_INVALID_ARGUMENT;
    }
    if (n < 16) {
        sana::set_last_error("randn_torch_cpu requires at least 16 elements");
        return SANA_ERR_INVALID_ARGUMENT;
    }
    sana_host::randn_torch_fill(out, (size_t)n, seed);
    return SANA_OK;
}
