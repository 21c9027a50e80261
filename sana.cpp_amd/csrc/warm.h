// Cache warm-up carried by a kernel launch: extra workgroups that stream
// device ranges (weights a later kernel reads) into the last-level cache and
// discard the data.  Included by the .hip files whose kernels carry one.
#pragma once

#include "hip_common.h"
#include "kernels.h"

namespace sana {

struct WarmDev {
    const f32x4 * p[CacheWarm::kMax];
    int64_t n16[CacheWarm::kMax];
};

// Host: the device view of `warm` and its workgroup count (0 without one);
// hipErrorInvalidValue for ranges that are not 16-byte multiples at 16-byte
// aligned addresses.
inline hipError_t make_warm(const CacheWarm * warm, WarmDev & wd, int & wwg) {
    wd = WarmDev{};
    wwg = 0;
    if (!warm || warm->workgroups <= 0) return hipSuccess;
    if (warm->n < 0 || warm->n > CacheWarm::kMax || warm->workgroups > 4096) return hipErrorInvalidValue;
    for (int k = 0; k < warm->n; ++k) {
        if (warm->bytes[k] < 0 || warm->bytes[k] % 16 || (reinterpret_cast<uintptr_t>(warm->p[k]) & 15) ||
            (warm->bytes[k] && !warm->p[k]))
            return hipErrorInvalidValue;
        wd.p[k] = static_cast<const f32x4 *>(warm->p[k]);
        wd.n16[k] = warm->bytes[k] / 16;
    }
    wwg = warm->workgroups;
    return hipSuccess;
}

// Device: workgroup wg of nwg streams its share of the ranges (four 16-byte
// loads in flight per thread).  The sum only keeps the loads alive: the empty
// asm consumes it, so nothing is stored.
__device__ __forceinline__ void warm_ranges(const WarmDev & w, int wg, int nwg) {
    const int64_t T = (int64_t)nwg * blockDim.x;
    const int64_t g = (int64_t)wg * blockDim.x + threadIdx.x;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < CacheWarm::kMax; ++k) {
        const f32x4 * p = w.p[k];
        const int64_t n = w.n16[k];
        int64_t i = g;
        for (; i + 3 * T < n; i += 4 * T) {
            const f32x4 v0 = p[i], v1 = p[i + T], v2 = p[i + 2 * T], v3 = p[i + 3 * T];
            acc += (v0 + v1) + (v2 + v3);
        }
        for (; i < n; i += T) acc += p[i];
    }
    const float s = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    asm volatile("" ::"v"(s));
}

}  // namespace sana
