// Measured ceilings for roofline reporting (no counterpart in the reference):
//   * the dense fp16 MFMA rate: workgroups of 4 waves, each wave 8 independent
//     v_mfma_f32_32x32x16_f16 accumulators (4 A x 2 B register fragments, the
//     operand reuse of a 128 x 64 wave tile) and no memory traffic.  The rate
//     depends on the operand values (the part is power limited): uniformly
//     spread fp16 values in [-1, 1), as random weights are, or all zeros;
//   * the HBM rate: grid-stride streaming of 16-byte loads (read only, one
//     partial sum per thread) or of 16-byte loads + stores (copy), 8
//     workgroups of 256 threads per CU, over a buffer far larger than the
//     256 MB last-level cache.
// The caller times the launches (e.g. with events on `stream`).
#include "hip_common.h"
#include "kernels.h"

namespace sana {
namespace {

constexpr int kPeakA = 4, kPeakB = 2;  // A and B fragments per wave: 8 accumulators

// A spread value in [-1, 1) from a multiplicative hash of (lane, element, fragment).
__device__ __forceinline__ float spread_value(unsigned key) {
    const unsigned h = key * 2654435761u;
    return (float)((int)(h >> 16) - 32768) * (1.0f / 32768.0f);
}

__global__ __launch_bounds__(256) void mfma_peak_kernel(float * __restrict__ sink, int iters, int zero_operands) {
    const int lane = threadIdx.x & 63;
    const float on = zero_operands ? 0.0f : 1.0f;
    f16x8 a[kPeakA], b[kPeakB];
#pragma unroll
    for (int i = 0; i < kPeakA; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) a[i][e] = (f16)(on * spread_value(lane * 8 + e + 97 * i));
#pragma unroll
    for (int j = 0; j < kPeakB; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) b[j][e] = (f16)(on * spread_value(lane * 8 + e + 131 * j + 7 + 4096));
    f32x16 acc[kPeakA][kPeakB];
#pragma unroll
    for (int i = 0; i < kPeakA; ++i)
#pragma unroll
        for (int j = 0; j < kPeakB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    // four k-steps per iteration with their own fragment registers, as a GEMM
    // main loop holds them
    f16x8 a2[kPeakA], b2[kPeakB];
#pragma unroll
    for (int i = 0; i < kPeakA; ++i) a2[i] = a[i] * (f16)0.5f;
#pragma unroll
    for (int j = 0; j < kPeakB; ++j) b2[j] = b[j] * (f16)0.5f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < kPeakA; ++i)
#pragma unroll
                for (int j = 0; j < kPeakB; ++j)
                    acc[i][j] = mfma_32x32x16((s & 1) ? a2[i] : a[i], (s & 2) ? b2[j] : b[j], acc[i][j]);
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kPeakA; ++i)
#pragma unroll
        for (int j = 0; j < kPeakB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) s += acc[i][j][r];
    sink[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

// n16: 16-byte elements.  Each thread handles elements g, g + T, g + 2T, ...
// four at a time, so four loads are in flight per thread.
__global__ __launch_bounds__(256) void hbm_read_kernel(const f32x4 * __restrict__ src, int64_t n16,
                                                       float * __restrict__ sink) {
    const int64_t T = (int64_t)gridDim.x * 256;
    const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
    f32x4 s0 = {0.0f, 0.0f, 0.0f, 0.0f}, s1 = s0, s2 = s0, s3 = s0;
    int64_t i = g;
    for (; i + 3 * T < n16; i += 4 * T) {
        const f32x4 v0 = src[i], v1 = src[i + T], v2 = src[i + 2 * T], v3 = src[i + 3 * T];
        s0 += v0;
        s1 += v1;
        s2 += v2;
        s3 += v3;
    }
    for (; i < n16; i += T) s0 += src[i];
    const f32x4 s = (s0 + s1) + (s2 + s3);
    sink[g] = s[0] + s[1] + s[2] + s[3];
}

__global__ __launch_bounds__(256) void hbm_copy_kernel(const f32x4 * __restrict__ src, f32x4 * __restrict__ dst,
                                                       int64_t n16) {
    const int64_t T = (int64_t)gridDim.x * 256;
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    for (; i + 3 * T < n16; i += 4 * T) {
        const f32x4 v0 = src[i], v1 = src[i + T], v2 = src[i + 2 * T], v3 = src[i + 3 * T];
        dst[i] = v0;
        dst[i + T] = v1;
        dst[i + 2 * T] = v2;
        dst[i + 3 * T] = v3;
    }
    for (; i < n16; i += T) dst[i] = src[i];
}

}  // namespace

hipError_t mfma_peak(int workgroups, int iters, bool zero_operands, float * sink, hipStream_t s) {
    if (workgroups <= 0 || workgroups > 65536 || iters <= 0 || !sink) return hipErrorInvalidValue;
    hipLaunchKernelGGL(mfma_peak_kernel, dim3((unsigned)workgroups), dim3(256), 0, s, sink, iters,
                       zero_operands ? 1 : 0);
    return hipGetLastError();
}

double mfma_peak_flops(int workgroups, int iters) {
    // 4 waves x 4 k-steps x 8 accumulators x iters MFMAs of 32x32x16 (2 * 32 * 32 * 16 flops) per workgroup
    return (double)workgroups * 4.0 * 4.0 * kPeakA * kPeakB * (double)iters * 32768.0;
}

int hbm_peak_workgroups() { return 256 * 8; }

hipError_t hbm_peak(const void * src, void * dst, int64_t bytes, float * sink, hipStream_t s) {
    if (!src || bytes < 16 || bytes % 16 || (reinterpret_cast<uintptr_t>(src) & 15) ||
        (dst && (reinterpret_cast<uintptr_t>(dst) & 15)) || (!dst && !sink))
        return hipErrorInvalidValue;
    const int wg = hbm_peak_workgroups();
    const int64_t n16 = bytes / 16;
    if (dst)
        hipLaunchKernelGGL(hbm_copy_kernel, dim3(wg), dim3(256), 0, s, static_cast<const f32x4 *>(src),
                           static_cast<f32x4 *>(dst), n16);
    else
        hipLaunchKernelGGL(hbm_read_kernel, dim3(wg), dim3(256), 0, s, static_cast<const f32x4 *>(src), n16, sink);
    return hipGetLastError();
}

}  // namespace sana
