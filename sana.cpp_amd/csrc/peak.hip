// Measured ceilings for roofline reporting: the dense fp16 MFMA rate this part
// reaches with no memory traffic (independent v_mfma_f32_32x32x16_f16 chains).
// The HBM ceiling is measured by the caller with a device-to-device copy.
#include "hip_common.h"
#include "kernels.h"

namespace sana {
namespace {

constexpr int kPeakChains = 8;  // independent accumulators per wave

__global__ __launch_bounds__(256) void mfma_peak_kernel(float * __restrict__ sink, int iters) {
    const int lane = threadIdx.x & 63;
    f16x8 a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[e] = (f16)(0.001f * (float)(lane + e));
        b[e] = (f16)(0.001f * (float)(lane - e));
    }
    f32x16 acc[kPeakChains];
#pragma unroll
    for (int c = 0; c < kPeakChains; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[c][r] = 0.0f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int c = 0; c < kPeakChains; ++c) acc[c] = mfma_32x32x16(a, b, acc[c]);
    }
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < kPeakChains; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[c][r];
    sink[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

}  // namespace

hipError_t mfma_peak(int workgroups, int iters, float * sink, hipStream_t s) {
    if (workgroups <= 0 || workgroups > 65536 || iters <= 0 || !sink) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mfma_peak_kernel, dim3((unsigned)workgroups), dim3(256), 0, s, sink, iters);
    return hipGetLastError();
}

double mfma_peak_flops(int workgroups, int iters) {
    // 4 waves x chains x iters MFMAs of 32x32x16 (2 * 32 * 32 * 16 flops) per workgroup
    return (double)workgroups * 4.0 * kPeakChains * (double)iters * 32768.0;
}

}  // namespace sana
