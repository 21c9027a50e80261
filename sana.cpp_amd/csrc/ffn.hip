// K5: Mix-FFN depthwise 3x3 conv + GLU gate, fused, on a token-major grid.
//
// Replaces, in glumb_conv (src/common_ops.cpp:733-761): depthwise_conv2d_3x3
// (zero padding, taps summed in (ky, kx) order, then + bias; :483-505),
// split_channels_4d (src/tensor.cpp:465-493), SiLU of the gate half and the
// data * gate product.  The SiLU after the inverted 1x1 conv is fused into the
// producing GEMM's epilogue, so the input here is already silu(inv(x) + b).
//
// Layout: channels are contiguous per token, so 8 channels of one token are
// one 16-byte load; a thread owns 8 data channels and the matching 8 gate
// channels of one output token and reads the 3x3 neighbourhood (halo rows come
// from L2).  Depthwise weights are stored tap-major [9][E] so the 8 weights of
// a tap are two float4 loads.
#include "hip_common.h"
#include "kernels.h"

namespace sana {
namespace {

__global__ __launch_bounds__(256) void dwglu_vec_kernel(const f16 * __restrict__ x, int64_t ldx,
                                                        const float * __restrict__ wt, const float * __restrict__ bias,
                                                        f16 * __restrict__ out, int64_t ldo, int B, int Hh, int Ww,
                                                        int F) {
    const int groups = F / 8;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t total = (int64_t)B * Hh * Ww * groups;
    if (gid >= total) return;
    const int g = (int)(gid % groups);
    const int64_t m = gid / groups;
    const int xx = (int)(m % Ww);
    const int64_t r = m / Ww;
    const int y = (int)(r % Hh);
    const int b = (int)(r / Hh);
    const int c0 = g * 8;
    const int E = 2 * F;
    float ad[8], ag[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) ad[e] = ag[e] = 0.0f;
#pragma unroll
    for (int ky = 0; ky < 3; ++ky) {
        const int iy = y + ky - 1;
        if (iy < 0 || iy >= Hh) continue;
#pragma unroll
        for (int kx = 0; kx < 3; ++kx) {
            const int ix = xx + kx - 1;
            if (ix < 0 || ix >= Ww) continue;
            const f16 * px = x + (((int64_t)b * Hh + iy) * Ww + ix) * ldx + c0;
            const f16x8 vd = *reinterpret_cast<const f16x8 *>(px);
            const f16x8 vg = *reinterpret_cast<const f16x8 *>(px + F);
            const float * wp = wt + (int64_t)(ky * 3 + kx) * E + c0;
            const float4 wd0 = *reinterpret_cast<const float4 *>(wp);
            const float4 wd1 = *reinterpret_cast<const float4 *>(wp + 4);
            const float4 wg0 = *reinterpret_cast<const float4 *>(wp + F);
            const float4 wg1 = *reinterpret_cast<const float4 *>(wp + F + 4);
            const float wd[8] = {wd0.x, wd0.y, wd0.z, wd0.w, wd1.x, wd1.y, wd1.z, wd1.w};
            const float wg[8] = {wg0.x, wg0.y, wg0.z, wg0.w, wg1.x, wg1.y, wg1.z, wg1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                ad[e] += (float)vd[e] * wd[e];
                ag[e] += (float)vg[e] * wg[e];
            }
        }
    }
    f16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float d = ad[e] + bias[c0 + e];
        const float gt = ag[e] + bias[F + c0 + e];
        o[e] = (f16)(d * silu_f(gt));
    }
    *reinterpret_cast<f16x8 *>(out + m * ldo + c0) = o;
}

// Scalar variant for channel counts that are not a multiple of 8.
__global__ __launch_bounds__(256) void dwglu_scalar_kernel(const f16 * __restrict__ x, int64_t ldx,
                                                           const float * __restrict__ wt,
                                                           const float * __restrict__ bias, f16 * __restrict__ out,
                                                           int64_t ldo, int B, int Hh, int Ww, int F) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t total = (int64_t)B * Hh * Ww * F;
    if (gid >= total) return;
    const int c = (int)(gid % F);
    const int64_t m = gid / F;
    const int xx = (int)(m % Ww);
    const int64_t r = m / Ww;
    const int y = (int)(r % Hh);
    const int b = (int)(r / Hh);
    const int E = 2 * F;
    float ad = 0.0f, ag = 0.0f;
    for (int ky = 0; ky < 3; ++ky) {
        const int iy = y + ky - 1;
        if (iy < 0 || iy >= Hh) continue;
        for (int kx = 0; kx < 3; ++kx) {
            const int ix = xx + kx - 1;
            if (ix < 0 || ix >= Ww) continue;
            const f16 * px = x + (((int64_t)b * Hh + iy) * Ww + ix) * ldx;
            ad += (float)px[c] * wt[(ky * 3 + kx) * E + c];
            ag += (float)px[F + c] * wt[(ky * 3 + kx) * E + F + c];
        }
    }
    const float d = ad + bias[c], g = ag + bias[F + c];
    out[m * ldo + c] = (f16)(d * silu_f(g));
}

}  // namespace

hipError_t dwconv_glu(const half_t * x, int64_t ldx, const float * wt, const float * bias, half_t * out, int64_t ldo,
                      int B, int Hh, int Ww, int F, hipStream_t s) {
    if (B <= 0 || Hh <= 0 || Ww <= 0 || F <= 0 || ldx < 2 * (int64_t)F || ldo < F || !bias || !wt)
        return hipErrorInvalidValue;
    const bool vec = F % 8 == 0 && ldx % 8 == 0 && ldo % 8 == 0 &&
                     ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                       reinterpret_cast<uintptr_t>(wt)) & 15) == 0;
    const f16 * xx = reinterpret_cast<const f16 *>(x);
    f16 * oo = reinterpret_cast<f16 *>(out);
    if (vec) {
        const int64_t total = (int64_t)B * Hh * Ww * (F / 8);
        hipLaunchKernelGGL(dwglu_vec_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, xx, ldx, wt, bias,
                           oo, ldo, B, Hh, Ww, F);
    } else {
        const int64_t total = (int64_t)B * Hh * Ww * F;
        hipLaunchKernelGGL(dwglu_scalar_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, xx, ldx, wt,
                           bias, oo, ldo, B, Hh, Ww, F);
    }
    return hipGetLastError();
}

}  // namespace sana
