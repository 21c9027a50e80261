// Bandwidth-bound row kernels of the DiT path: fused LayerNorm + adaLN
// modulate (K2), caption RMSNorm (K7), the final adaLN + proj_out layer, the
// time-embedding MLP (K6) and the patch embed.  One 64-lane wave per row; the
// row stays in registers between the statistics and the normalised write.
#include <cmath>

#include "hip_common.h"
#include "kernels.h"

namespace sana {
namespace {

constexpr int kMaxPerLane = 32;  // rows up to 64 * 32 = 2048 channels

// LayerNorm as src/tensor.cpp:235-268 (mean, then mean of squared deviations,
// 1/sqrt(var + eps), optional gamma/beta) followed by modulate_3d_lastdim
// (src/tensor.cpp:364-372) with the block modulation table add of
// compute_sana_block_modulation (src/transformer.cpp:521-531) done on load.
__global__ __launch_bounds__(256) void ln_modulate_kernel(const float * __restrict__ x, int64_t ldx,
                                                          f16 * __restrict__ out, int64_t ldo, int M, int C, int rpb,
                                                          float eps, const float * __restrict__ gamma,
                                                          const float * __restrict__ beta,
                                                          const float * __restrict__ mod_a,
                                                          const float * __restrict__ mod_t, int64_t mod_stride,
                                                          int64_t shift_off, int64_t scale_off) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    const float * xr = x + (int64_t)row * ldx;
    float v[kMaxPerLane];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
        const int c = lane + 64 * i;
        v[i] = c < C ? xr[c] : 0.0f;
        s += v[i];
    }
    const float mean = wave_sum(s) / (float)C;
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
        const int c = lane + 64 * i;
        if (c < C) {
            const float d = v[i] - mean;
            q += d * d;
        }
    }
    const float var = wave_sum(q) / (float)C;
    const float inv = 1.0f / sqrtf(var + eps);
    const int b = row / rpb;
    const float * ma = mod_a + (int64_t)b * mod_stride;
    f16 * orow = out + (int64_t)row * ldo;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
        const int c = lane + 64 * i;
        if (c < C) {
            float y = (v[i] - mean) * inv;
            if (gamma) y *= gamma[c];
            if (beta) y += beta[c];
            float sh = ma[shift_off + c], sc = ma[scale_off + c];
            if (mod_t) {
                sh += mod_t[shift_off + c];
                sc += mod_t[scale_off + c];
            }
            orow[c] = (f16)(y * (1.0f + sc) + sh);
        }
    }
}

// RMSNorm as src/tensor.cpp:276-316 (eps, weight), fp16 out.
__global__ __launch_bounds__(256) void rms_norm_kernel(const float * __restrict__ x, int64_t ldx,
                                                       const float * __restrict__ w, f16 * __restrict__ out,
                                                       int64_t ldo, float * __restrict__ out32, int M, int C,
                                                       float eps) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    const float * xr = x + (int64_t)row * ldx;
    float v[kMaxPerLane];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
        const int c = lane + 64 * i;
        v[i] = c < C ? xr[c] : 0.0f;
        s += v[i] * v[i];
    }
    const float inv = 1.0f / sqrtf(wave_sum(s) / (float)C + eps);
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
        const int c = lane + 64 * i;
        if (c < C) {
            float y = v[i] * inv;
            if (w) y *= w[c];
            out[(int64_t)row * ldo + c] = (f16)y;
            if (out32) out32[(int64_t)row * C + c] = y;
        }
    }
}

__global__ void to_f16_kernel(const float * __restrict__ x, int M, int C, f16 * __restrict__ out, int64_t ldo) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)M * ldo) return;
    const int64_t m = i / ldo;
    const int c = (int)(i - m * ldo);
    out[i] = c < C ? (f16)x[m * C + c] : (f16)0.0f;
}

// src/transformer.cpp:96-115: [cos(t * f_i), sin(t * f_i)], f_i precomputed on the host.
__global__ void sinusoid_kernel(const float * __restrict__ t, const float * __restrict__ freq, int B, int half,
                                float * __restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= B * half) return;
    const int b = i / half, j = i - b * half;
    const float v = t[b] * freq[j];
    out[b * 2 * half + j] = cosf(v);
    out[b * 2 * half + half + j] = sinf(v);
}

// out[b, n] = bias[n] + sum_k act(in[b, k]) * W[n, k]; one wave per output n,
// up to 8 batch rows per pass (linear_2d, src/common_ops.cpp:114-143).
__global__ __launch_bounds__(256) void gemv_kernel(const float * __restrict__ in, const float * __restrict__ W,
                                                   const float * __restrict__ bias, float * __restrict__ out, int B,
                                                   int K, int N, int act_in) {
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (n >= N) return;
    const float * wr = W + (int64_t)n * K;
    for (int b0 = 0; b0 < B; b0 += 8) {
        float acc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
        for (int k = lane; k < K; k += 64) {
            const float w = wr[k];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (b0 + j < B) {
                    float a = in[(int64_t)(b0 + j) * K + k];
                    if (act_in == 1) a = silu_f(a);
                    acc[j] += a * w;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float r = wave_sum(acc[j]);
            if (lane == 0 && b0 + j < B) out[(int64_t)(b0 + j) * N + n] = r + (bias ? bias[n] : 0.0f);
        }
    }
}

// conv2d_1x1 patch embed (src/common_ops.cpp:322-405) writing token-major
// [B, S, C]; weight transposed to [Cl, C] on upload so reads coalesce.
__global__ __launch_bounds__(256) void patch_embed_kernel(const float * __restrict__ latent, int Bl, int Cl, int S,
                                                          const float * __restrict__ Wt,
                                                          const float * __restrict__ bias, float * __restrict__ out,
                                                          int C) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    const int s = blockIdx.y;
    const int b = blockIdx.z;
    if (c >= C) return;
    const float * lat = latent + (int64_t)(b % Bl) * Cl * S + s;
    float acc = bias ? bias[c] : 0.0f;
    for (int ic = 0; ic < Cl; ++ic) acc += lat[(int64_t)ic * S] * Wt[(int64_t)ic * C + c];
    out[((int64_t)b * S + s) * C + c] = acc;
}

// Final layer (src/transformer.cpp:668-681): LN(eps, no affine), modulate with
// shift = emb + T[0], scale = emb + T[1] (compute_final_modulation, :126-163),
// proj_out C -> Cl (+bias), stored NCHW [B, Cl, S] (tokens_to_grid_4d).
__global__ __launch_bounds__(256) void final_layer_kernel(const float * __restrict__ x, const float * __restrict__ emb,
                                                          const float * __restrict__ T, const float * __restrict__ W,
                                                          const float * __restrict__ bias, float * __restrict__ out,
                                                          int B, int S, int C, int Cl, float eps) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= B * S) return;
    const int b = row / S, s = row - b * S;
    const float * xr = x + (int64_t)row * C;
    float v[kMaxPerLane];
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
        const int c = lane + 64 * i;
        v[i] = c < C ? xr[c] : 0.0f;
        sum += v[i];
    }
    const float mean = wave_sum(sum) / (float)C;
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
        const int c = lane + 64 * i;
        if (c < C) {
            const float d = v[i] - mean;
            q += d * d;
        }
    }
    const float inv = 1.0f / sqrtf(wave_sum(q) / (float)C + eps);
    const float * e = emb + (int64_t)b * C;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
        const int c = lane + 64 * i;
        if (c < C) {
            const float sh = e[c] + T[c], sc = e[c] + T[C + c];
            v[i] = ((v[i] - mean) * inv) * (1.0f + sc) + sh;
        }
    }
    for (int o = 0; o < Cl; ++o) {
        const float * wr = W + (int64_t)o * C;
        float p = 0.0f;
#pragma unroll
        for (int i = 0; i < kMaxPerLane; ++i) {
            const int c = lane + 64 * i;
            if (c < C) p += v[i] * wr[c];
        }
        p = wave_sum(p);
        if (lane == 0) out[((int64_t)b * Cl + o) * S + s] = p + (bias ? bias[o] : 0.0f);
    }
}

}  // namespace

hipError_t ln_modulate(const float * x, int64_t ldx, half_t * out, int64_t ldo, int M, int C, int rpb, float eps,
                       const float * gamma, const float * beta, const float * mod_a, const float * mod_t,
                       int64_t mod_stride, int64_t shift_off, int64_t scale_off, hipStream_t s) {
    if (M <= 0 || C <= 0 || C > 64 * kMaxPerLane || ldx < C || ldo < C || rpb <= 0 || !mod_a)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(ln_modulate_kernel, dim3((M + 3) / 4), dim3(256), 0, s, x, ldx,
                       reinterpret_cast<f16 *>(out), ldo, M, C, rpb, eps, gamma, beta, mod_a, mod_t, mod_stride,
                       shift_off, scale_off);
    return hipGetLastError();
}

hipError_t rms_norm_f16(const float * x, int64_t ldx, const float * w, half_t * out, int64_t ldo, float * out32,
                        int M, int C, float eps, hipStream_t s) {
    if (M <= 0 || C <= 0 || C > 64 * kMaxPerLane || ldx < C || ldo < C) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rms_norm_kernel, dim3((M + 3) / 4), dim3(256), 0, s, x, ldx, w, reinterpret_cast<f16 *>(out),
                       ldo, out32, M, C, eps);
    return hipGetLastError();
}

hipError_t to_f16_padded(const float * x, int M, int C, half_t * out, int64_t ldo, hipStream_t s) {
    if (M <= 0 || C <= 0 || ldo < C) return hipErrorInvalidValue;
    const int64_t n = (int64_t)M * ldo;
    hipLaunchKernelGGL(to_f16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, M, C,
                       reinterpret_cast<f16 *>(out), ldo);
    return hipGetLastError();
}

hipError_t timestep_sinusoid(const float * t, const float * freq, int B, int half, float * out, hipStream_t s) {
    if (B <= 0 || half <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(sinusoid_kernel, dim3((B * half + 255) / 256), dim3(256), 0, s, t, freq, B, half, out);
    return hipGetLastError();
}

hipError_t gemv_f32(const float * in, const float * W, const float * bias, float * out, int B, int K, int N,
                    int act_in, hipStream_t s) {
    if (B <= 0 || K <= 0 || N <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(gemv_kernel, dim3((N + 3) / 4), dim3(256), 0, s, in, W, bias, out, B, K, N, act_in);
    return hipGetLastError();
}

hipError_t patch_embed(const float * latent, int Bl, int B, int Cl, int S, const float * Wt, const float * bias,
                       float * out, int C, hipStream_t s) {
    if (Bl <= 0 || B <= 0 || Cl <= 0 || S <= 0 || C <= 0 || S > 65535 || B > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL(patch_embed_kernel, dim3((C + 255) / 256, S, B), dim3(256), 0, s, latent, Bl, Cl, S, Wt, bias,
                       out, C);
    return hipGetLastError();
}

hipError_t final_layer(const float * x, const float * emb, const float * table, const float * W, const float * bias,
                       float * out, int B, int S, int C, int Cl, float eps, hipStream_t s) {
    if (B <= 0 || S <= 0 || C <= 0 || C > 64 * kMaxPerLane || Cl <= 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL(final_layer_kernel, dim3((B * S + 3) / 4), dim3(256), 0, s, x, emb, table, W, bias, out, B, S,
                       C, Cl, eps);
    return hipGetLastError();
}

}  // namespace sana
