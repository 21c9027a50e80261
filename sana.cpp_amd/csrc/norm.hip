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

// Same as ln_modulate_kernel for rows whose width and strides are multiples of
// 4: float4 loads of x and of the modulation rows, 8-byte fp16x4 stores.
__global__ __launch_bounds__(256) void ln_modulate_vec_kernel(const float * __restrict__ x, int64_t ldx,
                                                              f16 * __restrict__ out, int64_t ldo, int M, int C,
                                                              int rpb, float eps, const float * __restrict__ gamma,
                                                              const float * __restrict__ beta,
                                                              const float * __restrict__ mod_a,
                                                              const float * __restrict__ mod_t, int64_t mod_stride,
                                                              int64_t shift_off, int64_t scale_off) {
    constexpr int kMax4 = kMaxPerLane / 4;  // float4 chunks per lane
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    const int n4 = C >> 2;
    const float4 * xr = reinterpret_cast<const float4 *>(x + (int64_t)row * ldx);
    float4 v[kMax4];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kMax4; ++i) {
        const int c4 = lane + 64 * i;
        v[i] = c4 < n4 ? xr[c4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    }
    const float mean = wave_sum(s) / (float)C;
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < kMax4; ++i) {
        if (lane + 64 * i < n4) {
            const float a = v[i].x - mean, b = v[i].y - mean, c = v[i].z - mean, d = v[i].w - mean;
            q += (a * a + b * b) + (c * c + d * d);
        }
    }
    const float inv = 1.0f / sqrtf(wave_sum(q) / (float)C + eps);
    const int b = row / rpb;
    const float4 * sh4 = reinterpret_cast<const float4 *>(mod_a + (int64_t)b * mod_stride + shift_off);
    const float4 * sc4 = reinterpret_cast<const float4 *>(mod_a + (int64_t)b * mod_stride + scale_off);
    const float4 * tsh4 = mod_t ? reinterpret_cast<const float4 *>(mod_t + shift_off) : nullptr;
    const float4 * tsc4 = mod_t ? reinterpret_cast<const float4 *>(mod_t + scale_off) : nullptr;
    f16x4 * orow = reinterpret_cast<f16x4 *>(out + (int64_t)row * ldo);
#pragma unroll
    for (int i = 0; i < kMax4; ++i) {
        const int c4 = lane + 64 * i;
        if (c4 < n4) {
            float y[4] = {(v[i].x - mean) * inv, (v[i].y - mean) * inv, (v[i].z - mean) * inv, (v[i].w - mean) * inv};
            if (gamma) {
                const float4 g = reinterpret_cast<const float4 *>(gamma)[c4];
                y[0] *= g.x; y[1] *= g.y; y[2] *= g.z; y[3] *= g.w;
            }
            if (beta) {
                const float4 bb = reinterpret_cast<const float4 *>(beta)[c4];
                y[0] += bb.x; y[1] += bb.y; y[2] += bb.z; y[3] += bb.w;
            }
            float4 sh = sh4[c4], sc = sc4[c4];
            if (tsh4) {
                const float4 a = tsh4[c4], d = tsc4[c4];
                sh.x += a.x; sh.y += a.y; sh.z += a.z; sh.w += a.w;
                sc.x += d.x; sc.y += d.y; sc.z += d.z; sc.w += d.w;
            }
            f16x4 o;
            o[0] = (f16)(y[0] * (1.0f + sc.x) + sh.x);
            o[1] = (f16)(y[1] * (1.0f + sc.y) + sh.y);
            o[2] = (f16)(y[2] * (1.0f + sc.z) + sh.z);
            o[3] = (f16)(y[3] * (1.0f + sc.w) + sh.w);
            orow[c4] = o;
        }
    }
}

// comb[blk][b][i] = t_mod[b][i] + table[blk][i] for every block at once: the
// per-block modulation of compute_sana_block_modulation (src/transformer.cpp:521-531);
// t_mod is shared by all blocks of a forward.
__global__ void mod_combine_kernel(const float * __restrict__ tmod, const float * __restrict__ tables, int L, int B,
                                   int W, float * __restrict__ comb) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t n = (int64_t)L * B * W;
    if (i >= n) return;
    const int w = (int)(i % W);
    const int64_t lb = i / W;
    const int b = (int)(lb % B);
    const int l = (int)(lb / B);
    comb[i] = tmod[(int64_t)b * W + w] + tables[(int64_t)l * W + w];
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

// out[b, n] = bias[n] + sum_k act(in[b, k]) * W[n, k] (linear_2d,
// src/common_ops.cpp:114-143); one wave per output n, float4 loads along k,
// up to 8 batch rows per pass.  K % 4 == 0.
__global__ __launch_bounds__(256) void gemv_kernel(const float * __restrict__ in, const float * __restrict__ W,
                                                   const float * __restrict__ bias, float * __restrict__ out, int B,
                                                   int K, int N, int act_in) {
    const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (n >= N) return;
    const float4 * wr = reinterpret_cast<const float4 *>(W + (int64_t)n * K);
    const int k4n = K >> 2;
    for (int b0 = 0; b0 < B; b0 += 8) {
        float acc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
        for (int k4 = lane; k4 < k4n; k4 += 64) {
            const float4 w = wr[k4];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (b0 + j < B) {
                    float4 a = reinterpret_cast<const float4 *>(in + (int64_t)(b0 + j) * K)[k4];
                    if (act_in == 1) {
                        a.x = silu_f(a.x); a.y = silu_f(a.y); a.z = silu_f(a.z); a.w = silu_f(a.w);
                    }
                    acc[j] += (a.x * w.x + a.y * w.y) + (a.z * w.z + a.w * w.w);
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
// [B, S, C]; weight transposed to [Cl, C] on upload so reads coalesce.  A
// block handles 8 tokens: their Cl input channels are staged in LDS and each
// thread produces output channels c = tid, tid + 256, ... for the 8 tokens
// (bias first, then input channels in order, as the reference accumulates).
constexpr int kPatchTok = 8;
__global__ __launch_bounds__(256) void patch_embed_kernel(const float * __restrict__ latent, int Bl, int Cl, int S,
                                                          const float * __restrict__ Wt,
                                                          const float * __restrict__ bias, float * __restrict__ out,
                                                          int C) {
    extern __shared__ float lat_s[];  // [Cl][kPatchTok]
    const int s0 = blockIdx.x * kPatchTok;
    const int b = blockIdx.y;
    const float * lat = latent + (int64_t)(b % Bl) * Cl * S;
    for (int i = threadIdx.x; i < Cl * kPatchTok; i += blockDim.x) {
        const int ic = i / kPatchTok, t = i - ic * kPatchTok;
        lat_s[i] = (s0 + t < S) ? lat[(int64_t)ic * S + s0 + t] : 0.0f;
    }
    __syncthreads();
    for (int c = threadIdx.x; c < C; c += blockDim.x) {
        float acc[kPatchTok];
        const float bv = bias ? bias[c] : 0.0f;
#pragma unroll
        for (int t = 0; t < kPatchTok; ++t) acc[t] = bv;
#pragma unroll 8
        for (int ic = 0; ic < Cl; ++ic) {
            const float w = Wt[(int64_t)ic * C + c];
#pragma unroll
            for (int t = 0; t < kPatchTok; ++t) acc[t] += lat_s[ic * kPatchTok + t] * w;
        }
#pragma unroll
        for (int t = 0; t < kPatchTok; ++t)
            if (s0 + t < S) out[((int64_t)b * S + s0 + t) * C + c] = acc[t];
    }
}

// Final layer (src/transformer.cpp:668-681): LN(eps, no affine), modulate with
// shift = emb + T[0], scale = emb + T[1] (compute_final_modulation, :126-163),
// proj_out C -> Cl (+bias), stored NCHW [B, Cl, S] (tokens_to_grid_4d).  A
// block handles kFinalRows rows: each wave normalises rows into LDS, then
// thread (row, o) reduces over C with Wt [C, Cl] (o contiguous).
constexpr int kFinalRows = 8;
__global__ __launch_bounds__(256) void final_layer_kernel(const float * __restrict__ x, const float * __restrict__ emb,
                                                          const float * __restrict__ T, const float * __restrict__ Wt,
                                                          const float * __restrict__ bias, float * __restrict__ out,
                                                          int B, int S, int C, int Cl, float eps) {
    extern __shared__ float xs[];  // [kFinalRows][C]
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int r0 = blockIdx.x * kFinalRows;
    for (int rr = w; rr < kFinalRows; rr += 4) {
        const int row = r0 + rr;
        float * dst = xs + rr * C;
        if (row >= B * S) {
            for (int c = lane; c < C; c += 64) dst[c] = 0.0f;
            continue;
        }
        const int b = row / S;
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
                dst[c] = ((v[i] - mean) * inv) * (1.0f + sc) + sh;
            }
        }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < kFinalRows * Cl; idx += blockDim.x) {
        const int rr = idx / Cl, o = idx - rr * Cl;
        const int row = r0 + rr;
        if (row >= B * S) continue;
        const float * xv = xs + rr * C;
        // 8 independent partial sums so the Wt loads of 8 channels are in flight together
        float pp[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        int c = 0;
        for (; c + 8 <= C; c += 8) {
#pragma unroll
            for (int u = 0; u < 8; ++u) pp[u] += xv[c + u] * Wt[(int64_t)(c + u) * Cl + o];
        }
        for (; c < C; ++c) pp[0] += xv[c] * Wt[(int64_t)c * Cl + o];
        const float p = ((pp[0] + pp[1]) + (pp[2] + pp[3])) + ((pp[4] + pp[5]) + (pp[6] + pp[7]));
        const int b = row / S, sidx = row - b * S;
        out[((int64_t)b * Cl + o) * S + sidx] = p + (bias ? bias[o] : 0.0f);
    }
}

}  // namespace

hipError_t ln_modulate(const float * x, int64_t ldx, half_t * out, int64_t ldo, int M, int C, int rpb, float eps,
                       const float * gamma, const float * beta, const float * mod_a, const float * mod_t,
                       int64_t mod_stride, int64_t shift_off, int64_t scale_off, hipStream_t s) {
    if (M <= 0 || C <= 0 || C > 64 * kMaxPerLane || ldx < C || ldo < C || rpb <= 0 || !mod_a)
        return hipErrorInvalidValue;
    const bool vec = C % 4 == 0 && ldx % 4 == 0 && ldo % 4 == 0 && mod_stride % 4 == 0 && shift_off % 4 == 0 &&
                     scale_off % 4 == 0 &&
                     ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                       reinterpret_cast<uintptr_t>(mod_a) | reinterpret_cast<uintptr_t>(mod_t) |
                       reinterpret_cast<uintptr_t>(gamma) | reinterpret_cast<uintptr_t>(beta)) & 15) == 0;
    if (vec)
        hipLaunchKernelGGL(ln_modulate_vec_kernel, dim3((M + 3) / 4), dim3(256), 0, s, x, ldx,
                           reinterpret_cast<f16 *>(out), ldo, M, C, rpb, eps, gamma, beta, mod_a, mod_t, mod_stride,
                           shift_off, scale_off);
    else
        hipLaunchKernelGGL(ln_modulate_kernel, dim3((M + 3) / 4), dim3(256), 0, s, x, ldx,
                           reinterpret_cast<f16 *>(out), ldo, M, C, rpb, eps, gamma, beta, mod_a, mod_t, mod_stride,
                           shift_off, scale_off);
    return hipGetLastError();
}

hipError_t mod_combine(const float * tmod, const float * tables, int L, int B, int W, float * comb, hipStream_t s) {
    if (L <= 0 || B <= 0 || W <= 0) return hipErrorInvalidValue;
    const int64_t n = (int64_t)L * B * W;
    hipLaunchKernelGGL(mod_combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, tmod, tables, L, B, W,
                       comb);
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
    if (B <= 0 || K <= 0 || N <= 0 || K % 4 ||
        ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(W)) & 15))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(gemv_kernel, dim3((N + 3) / 4), dim3(256), 0, s, in, W, bias, out, B, K, N, act_in);
    return hipGetLastError();
}

hipError_t patch_embed(const float * latent, int Bl, int B, int Cl, int S, const float * Wt, const float * bias,
                       float * out, int C, hipStream_t s) {
    if (Bl <= 0 || B <= 0 || Cl <= 0 || Cl > 1024 || S <= 0 || C <= 0 || B > 65535) return hipErrorInvalidValue;
    hipLaunchKernelGGL(patch_embed_kernel, dim3((S + kPatchTok - 1) / kPatchTok, B), dim3(256),
                       sizeof(float) * Cl * kPatchTok, s, latent, Bl, Cl, S, Wt, bias, out, C);
    return hipGetLastError();
}

hipError_t final_layer(const float * x, const float * emb, const float * table, const float * Wt, const float * bias,
                       float * out, int B, int S, int C, int Cl, float eps, hipStream_t s) {
    if (B <= 0 || S <= 0 || C <= 0 || C > 64 * kMaxPerLane || Cl <= 0) return hipErrorInvalidValue;
    const int rows = B * S;
    hipLaunchKernelGGL(final_layer_kernel, dim3((rows + kFinalRows - 1) / kFinalRows), dim3(256),
                       sizeof(float) * kFinalRows * C, s, x, emb, table, Wt, bias, out, B, S, C, Cl, eps);
    return hipGetLastError();
}

}  // namespace sana
