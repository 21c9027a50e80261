// Bandwidth-bound row kernels of the DiT path: fused LayerNorm + adaLN
// modulate (K2), caption RMSNorm (K7), the final adaLN + proj_out layer, the
// time-embedding MLP (K6) and the patch embed.  One 64-lane wave per row; the
// row stays in registers between the statistics and the normalised write.
#include <cmath>

#include "hip_common.h"
#include "kernels.h"
#include "warm.h"

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
// kMax4 = float4 chunks per lane (C <= 256 * kMax4), so the row and its shift /
// scale vectors stay in registers.
template <int kMax4>
__global__ __launch_bounds__(256) void ln_modulate_vec_kernel(const float * __restrict__ x, int64_t ldx,
                                                              f16 * __restrict__ out, int64_t ldo, int M, int C,
                                                              int rpb, float eps, const float * __restrict__ gamma,
                                                              const float * __restrict__ beta,
                                                              const float * __restrict__ mod_a,
                                                              const float * __restrict__ mod_t, int64_t mod_stride,
                                                              int64_t shift_off, int64_t scale_off, WarmDev warm,
                                                              int warm_blocks) {
    // the first warm_blocks workgroups carry the cache warm-up (dispatched
    // first, so they run beside the rows instead of after them)
    if ((int)blockIdx.x < warm_blocks) {
        warm_ranges(warm, (int)blockIdx.x, warm_blocks);
        return;
    }
    const int row = (blockIdx.x - warm_blocks) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;
    const int n4 = C >> 2;
    const float4 * xr = reinterpret_cast<const float4 *>(x + (int64_t)row * ldx);
    const int b = row / rpb;
    const float4 * sh4 = reinterpret_cast<const float4 *>(mod_a + (int64_t)b * mod_stride + shift_off);
    const float4 * sc4 = reinterpret_cast<const float4 *>(mod_a + (int64_t)b * mod_stride + scale_off);
    // the row and its shift / scale vectors are all requested before the
    // reductions, so their latencies overlap
    float4 v[kMax4], shv[kMax4], scv[kMax4];
#pragma unroll
    for (int i = 0; i < kMax4; ++i) {
        const int c4 = lane + 64 * i;
        if (c4 < n4) {
            v[i] = xr[c4];
            shv[i] = sh4[c4];
            scv[i] = sc4[c4];
        } else {
            v[i] = shv[i] = scv[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kMax4; ++i) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
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
            float4 sh = shv[i], sc = scv[i];
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

// out[b, n] = bias[n] + sum_k act(in[b, k]) * W[n, k] (linear_2d,
// src/common_ops.cpp:114-143); one wave per output n, float4 loads along k,
// up to 8 batch rows per pass.  K % 4 == 0.
// SIN: in[b] is the timestep t_b and the row multiplied is its sinusoid
// [cos(t_b f_j), sin(t_b f_j)] (K = 2 half; src/transformer.cpp:96-115), computed
// in place.  COMB: the epilogue also writes comb[(l B + b) N + n] = out[b, n] +
// tables[l N + n] for the L tables (mod_combine_kernel's sums), lane l storing
// table l.
template <bool SIN = false, bool COMB = false>
__global__ __launch_bounds__(256) void gemv_kernel(const float * __restrict__ in, const float * __restrict__ W,
                                                   const float * __restrict__ bias, float * __restrict__ out, int B,
                                                   int K, int N, int act_in, const float * __restrict__ freq = nullptr,
                                                   const float * __restrict__ tables = nullptr, int L = 0,
                                                   float * __restrict__ comb = nullptr) {
    constexpr int kRows = 4;  // outputs per wave: their weight rows are streamed together
    const int n0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * kRows;
    const int lane = threadIdx.x & 63;
    if (n0 >= N) return;
    const int k4n = K >> 2;
    for (int b0 = 0; b0 < B; b0 += 2) {
        float acc[kRows][2];
#pragma unroll
        for (int r = 0; r < kRows; ++r) acc[r][0] = acc[r][1] = 0.0f;
        // unrolled so the weight loads of several k steps are in flight at
        // once (the weights come from HBM on every forward)
#pragma unroll 6
        for (int k4 = lane; k4 < k4n; k4 += 64) {
            float4 a[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                if constexpr (SIN) {
                    // in = t: element k of the sinusoid is cos (k < half) or sin of t_b * freq[k mod half]
                    const int half = K >> 1, k0 = 4 * k4;
                    const bool second = k0 >= half;
                    const int f0 = second ? k0 - half : k0;
                    const float tb = b0 + j < B ? in[b0 + j] : 0.0f;
                    float e4[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float v = tb * freq[f0 + e];
                        e4[e] = second ? sinf(v) : cosf(v);
                    }
                    a[j] = b0 + j < B ? make_float4(e4[0], e4[1], e4[2], e4[3]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                } else {
                    a[j] = b0 + j < B ? reinterpret_cast<const float4 *>(in + (int64_t)(b0 + j) * K)[k4]
                                      : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                }
                if (act_in == 1) {
                    a[j].x = silu_f(a[j].x); a[j].y = silu_f(a[j].y); a[j].z = silu_f(a[j].z); a[j].w = silu_f(a[j].w);
                }
            }
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                if (n0 + r < N) {
                    const float4 w = reinterpret_cast<const float4 *>(W + (int64_t)(n0 + r) * K)[k4];
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[r][j] += (a[j].x * w.x + a[j].y * w.y) + (a[j].z * w.z + a[j].w * w.w);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < kRows; ++r)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float v = wave_sum(acc[r][j]);
                const float o = v + (bias ? bias[n0 + r] : 0.0f);
                if (lane == 0 && n0 + r < N && b0 + j < B) out[(int64_t)(b0 + j) * N + n0 + r] = o;
                if constexpr (COMB) {
                    if (n0 + r < N && b0 + j < B)
                        for (int l = lane; l < L; l += 64)
                            comb[((int64_t)l * B + b0 + j) * N + n0 + r] = o + tables[(int64_t)l * N + n0 + r];
                }
            }
    }
}

// conv2d_1x1 patch embed (src/common_ops.cpp:322-405) writing token-major
// [B, S, C] with v_mfma_f32_32x32x2_f32 (fp32 products, fp32 accumulation):
// out[s][c] = bias[c] + sum_ic lat[ic][s] * Wt[ic][c], weight transposed to
// [Cl, C] on upload.  One wave per 32 tokens x 32 channels; the A operand
// (lane: token l%32, channel pair l/32) and the B operand (lane: channel
// pair l/32, output l%32) are both contiguous across lanes.
__global__ __launch_bounds__(256) void patch_embed_kernel(const float * __restrict__ latent, int Bl, int Cl, int S,
                                                          const float * __restrict__ Wt,
                                                          const float * __restrict__ bias, float * __restrict__ out,
                                                          int C) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int c0 = (blockIdx.x * 4 + w) * 32;
    const int s0 = blockIdx.y * 32;
    const int b = blockIdx.z;
    if (c0 >= C) return;
    const float * lat = latent + (int64_t)(b % Bl) * Cl * S;
    const int s = s0 + (lane & 31), c = c0 + (lane & 31), kh = lane >> 5;
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    for (int ic = 0; ic < Cl; ic += 2) {
        const int k = ic + kh;
        const float a = (k < Cl && s < S) ? lat[(int64_t)k * S + s] : 0.0f;
        const float bw = (k < Cl && c < C) ? Wt[(int64_t)k * C + c] : 0.0f;
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, bw, acc, 0, 0, 0);
    }
    if (c >= C) return;
    const float bv = bias ? bias[c] : 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int row = s0 + 8 * (i >> 2) + 4 * kh + (i & 3);
        if (row < S) out[((int64_t)b * S + row) * C + c] = acc[i] + bv;
    }
}

// Final layer (src/transformer.cpp:668-681), first half: LN(eps, no affine)
// and modulate with shift = emb + T[0], scale = emb + T[1]
// (compute_final_modulation, :126-163), fp32 rows out.  One wave per row.
__global__ __launch_bounds__(256) void final_norm_kernel(const float * __restrict__ x, const float * __restrict__ emb,
                                                         const float * __restrict__ T, float * __restrict__ y, int B,
                                                         int S, int C, float eps) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= B * S) return;
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
    float * yr = y + (int64_t)row * C;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
        const int c = lane + 64 * i;
        if (c < C) {
            const float sh = e[c] + T[c], sc = e[c] + T[C + c];
            yr[c] = ((v[i] - mean) * inv) * (1.0f + sc) + sh;
        }
    }
}

// Final layer, second half: proj_out C -> Cl (+bias), stored NCHW [B, Cl, S]
// (tokens_to_grid_4d), on v_mfma_f32_32x32x2_f32 (fp32 products and sums).
// A workgroup covers 32 rows; its 4 waves split C into quarters and their
// 32x32 partial tiles are summed in LDS in fixed order.  Lane (row l%32,
// half h = l/32) loads 4 consecutive channels c0 + 4h .. c0 + 4h + 3 of its row
// with one 16-byte load and feeds them to 4 MFMAs; the B operand supplies the
// same channel order (the reduction order over C is permuted, not its terms).
__global__ __launch_bounds__(256) void proj_out_kernel(const float * __restrict__ y, const float * __restrict__ Wt,
                                                       const float * __restrict__ bias, float * __restrict__ out,
                                                       int B, int S, int C, int Cl) {
    __shared__ float part[4][32][33];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int r0 = blockIdx.x * 32;
    const int rows = B * S;
    const int rr = min(r0 + (lane & 31), rows - 1);
    const int h = lane >> 5, n = lane & 31;
    const int q = C / 4;  // channels per wave (C % 128 == 0)
    const float * yr = y + (int64_t)rr * C;
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    // 32 channels per iteration: all loads of the iteration are issued before its 16 MFMAs
    for (int c0 = w * q; c0 < (w + 1) * q; c0 += 32) {
        float av[4][4], bw[4][4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const float4 a = *reinterpret_cast<const float4 *>(yr + c0 + 8 * u + 4 * h);
            av[u][0] = a.x; av[u][1] = a.y; av[u][2] = a.z; av[u][3] = a.w;
#pragma unroll
            for (int e = 0; e < 4; ++e) bw[u][e] = n < Cl ? Wt[(int64_t)(c0 + 8 * u + 4 * h + e) * Cl + n] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u][e], bw[u][e], acc, 0, 0, 0);
    }
    // lane holds output column n, rows 8*(i/4) + 4*h + i%4
#pragma unroll
    for (int i = 0; i < 16; ++i) part[w][8 * (i >> 2) + 4 * h + (i & 3)][n] = acc[i];
    __syncthreads();
    for (int idx = threadIdx.x; idx < 32 * 32; idx += 256) {
        const int r = idx >> 5, o = idx & 31;
        const int row = r0 + r;
        if (row >= rows || o >= Cl) continue;
        const float v = ((part[0][r][o] + part[1][r][o]) + (part[2][r][o] + part[3][r][o])) + (bias ? bias[o] : 0.0f);
        const int b = row / S, sidx = row - b * S;
        out[((int64_t)b * Cl + o) * S + sidx] = v;
    }
}

// The final layer in one pass (C % 384 == 0, S % 32 == 0, Cl <= 32): a
// workgroup of NW waves takes 32 rows of one image, computes their LayerNorm
// statistics as final_norm_kernel does (one wave per row, the same order of
// sums) and the image's shift / scale per channel into LDS, then feeds the
// modulated rows ((x - mean) * inv) * (1 + scale) + shift to
// v_mfma_f32_32x32x2_f32 as proj_out_kernel does, without the fp32 round trip
// of the normalized rows.  Wave w takes C / NW channels in 32-channel blocks,
// the next block's loads issued before the current block's MFMAs; the NW
// partial tiles are summed in LDS in fixed order.
template <int NW>
__global__ __launch_bounds__(64 * NW) void final_proj_kernel(const float * __restrict__ x,
                                                              const float * __restrict__ emb,
                                                              const float * __restrict__ T,
                                                              const float * __restrict__ Wt,
                                                              const float * __restrict__ bias,
                                                              float * __restrict__ out, int B, int S, int C, int Cl,
                                                              float eps) {
    __shared__ float part[NW][32][33];
    __shared__ float stat[32][2];
    __shared__ __attribute__((aligned(16))) float mods[2][kMaxPerLane * 64];  // shift, scale per channel
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int r0 = blockIdx.x * 32;
    const int rows = B * S;
    {
        const float * e = emb + (int64_t)(r0 / S) * C;
        for (int c = threadIdx.x; c < C; c += 64 * NW) {
            mods[0][c] = e[c] + T[c];
            mods[1][c] = e[c] + T[C + c];
        }
    }
    // 1. statistics (two-pass mean and variance, as final_norm_kernel).  Wave w
    // takes rows w, w + NW, ...: all of them are requested before the first
    // reduction, so the row loads overlap instead of following one another.
    constexpr int RW = (32 + NW - 1) / NW;  // rows per wave
    constexpr int PL = kMaxPerLane;
    float v[RW][PL];
#pragma unroll
    for (int k = 0; k < RW; ++k) {
        const int r = w + k * NW;
        const float * xr = x + (int64_t)min(r0 + min(r, 31), rows - 1) * C;
#pragma unroll
        for (int i = 0; i < PL; ++i) {
            const int c = lane + 64 * i;
            v[k][i] = (r < 32 && c < C) ? xr[c] : 0.0f;
        }
    }
#pragma unroll
    for (int k = 0; k < RW; ++k) {
        const int r = w + k * NW;
        if (r >= 32) continue;
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < PL; ++i) sum += v[k][i];
        const float mean = wave_sum(sum) / (float)C;
        float q = 0.0f;
#pragma unroll
        for (int i = 0; i < PL; ++i) {
            const int c = lane + 64 * i;
            if (c < C) {
                const float d = v[k][i] - mean;
                q += d * d;
            }
        }
        const float inv = 1.0f / sqrtf(wave_sum(q) / (float)C + eps);
        if (lane == 0) {
            stat[r][0] = mean;
            stat[r][1] = inv;
        }
    }
    __syncthreads();
    // 2. projection: lane (row l % 32, half h = l / 32) feeds channels c + 4 h .. c + 4 h + 3
    const int rr = min(r0 + (lane & 31), rows - 1);
    const int h = lane >> 5, n = lane & 31;
    const float mean = stat[lane & 31][0], inv = stat[lane & 31][1];
    const float * xr = x + (int64_t)rr * C;
    const int q = C / NW;  // channels per wave, a multiple of 32
    const int cb = w * q;
    float4 xa[2][4];
    float bw[2][4][4];
    int cbuf[2] = {0, 0};
    auto load = [&](int buf, int c0) {
        cbuf[buf] = c0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int c = c0 + 8 * u + 4 * h;
            xa[buf][u] = *reinterpret_cast<const float4 *>(xr + c);
#pragma unroll
            for (int k = 0; k < 4; ++k) bw[buf][u][k] = n < Cl ? Wt[(int64_t)(c + k) * Cl + n] : 0.0f;
        }
    };
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    auto step = [&](int buf) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int c = cbuf[buf] + 8 * u + 4 * h;
            const float xv[4] = {xa[buf][u].x, xa[buf][u].y, xa[buf][u].z, xa[buf][u].w};
            const float4 sh4 = *reinterpret_cast<const float4 *>(&mods[0][c]);
            const float4 sc4 = *reinterpret_cast<const float4 *>(&mods[1][c]);
            const float sv[4] = {sh4.x, sh4.y, sh4.z, sh4.w}, cv[4] = {sc4.x, sc4.y, sc4.z, sc4.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float sh = sv[k], sc = cv[k];
                const float yv = ((xv[k] - mean) * inv) * (1.0f + sc) + sh;
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(yv, bw[buf][u][k], acc, 0, 0, 0);
            }
        }
    };
    load(0, cb);
    for (int c0 = cb; c0 < cb + q; c0 += 64) {
        const bool second = c0 + 32 < cb + q;
        if (second) load(1, c0 + 32);
        step(0);
        if (second) {
            if (c0 + 64 < cb + q) load(0, c0 + 64);
            step(1);
        }
    }
    // lane holds output column n, rows 8*(i/4) + 4*h + i%4
#pragma unroll
    for (int i = 0; i < 16; ++i) part[w][8 * (i >> 2) + 4 * h + (i & 3)][n] = acc[i];
    __syncthreads();
    for (int idx = threadIdx.x; idx < 32 * 32; idx += 64 * NW) {
        const int r = idx >> 5, o = idx & 31;
        const int row = r0 + r;
        if (row >= rows || o >= Cl) continue;
        float v = 0.0f;
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) v += part[ww][r][o];
        v += bias ? bias[o] : 0.0f;
        const int b = row / S, sidx = row - b * S;
        out[((int64_t)b * Cl + o) * S + sidx] = v;
    }
}

// Plain fp32 proj_out for hidden sizes that are not a multiple of 32.
__global__ __launch_bounds__(256) void proj_out_scalar_kernel(const float * __restrict__ y,
                                                              const float * __restrict__ Wt,
                                                              const float * __restrict__ bias,
                                                              float * __restrict__ out, int B, int S, int C, int Cl) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= B * S * Cl) return;
    const int row = idx / Cl, o = idx - row * Cl;
    float p = 0.0f;
    for (int c = 0; c < C; ++c) p += y[(int64_t)row * C + c] * Wt[(int64_t)c * Cl + o];
    const int b = row / S, sidx = row - b * S;
    out[((int64_t)b * Cl + o) * S + sidx] = p + (bias ? bias[o] : 0.0f);
}

}  // namespace

hipError_t ln_modulate(const float * x, int64_t ldx, half_t * out, int64_t ldo, int M, int C, int rpb, float eps,
                       const float * gamma, const float * beta, const float * mod_a, const float * mod_t,
                       int64_t mod_stride, int64_t shift_off, int64_t scale_off, hipStream_t s,
                       const CacheWarm * warm) {
    if (M <= 0 || C <= 0 || C > 64 * kMaxPerLane || ldx < C || ldo < C || rpb <= 0 || !mod_a)
        return hipErrorInvalidValue;
    WarmDev wd;
    int wwg;
    if (make_warm(warm, wd, wwg) != hipSuccess) return hipErrorInvalidValue;
    const bool vec = C % 4 == 0 && ldx % 4 == 0 && ldo % 4 == 0 && mod_stride % 4 == 0 && shift_off % 4 == 0 &&
                     scale_off % 4 == 0 &&
                     ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                       reinterpret_cast<uintptr_t>(mod_a) | reinterpret_cast<uintptr_t>(mod_t) |
                       reinterpret_cast<uintptr_t>(gamma) | reinterpret_cast<uintptr_t>(beta)) & 15) == 0;
    if (vec) {
#define SANA_LN_VEC(n4)                                                                                           \
    do {                                                                                                          \
        note_kernel("ln_modulate_vec_kernel<" #n4 ">");                                                            \
        hipLaunchKernelGGL((ln_modulate_vec_kernel<n4>), dim3((M + 3) / 4 + wwg), dim3(256), 0, s, x, ldx,         \
                           reinterpret_cast<f16 *>(out), ldo, M, C, rpb, eps, gamma, beta, mod_a, mod_t,          \
                           mod_stride, shift_off, scale_off, wd, wwg);                                            \
    } while (0)
        const int per = (C / 4 + 63) / 64;  // float4 chunks per lane
        if (per <= 2) SANA_LN_VEC(2);
        else if (per <= 3) SANA_LN_VEC(3);
        else if (per <= 5) SANA_LN_VEC(5);
        else SANA_LN_VEC(kMaxPerLane / 4);
#undef SANA_LN_VEC
    } else {
        note_kernel("ln_modulate_kernel");
        hipLaunchKernelGGL(ln_modulate_kernel, dim3((M + 3) / 4), dim3(256), 0, s, x, ldx,
                           reinterpret_cast<f16 *>(out), ldo, M, C, rpb, eps, gamma, beta, mod_a, mod_t, mod_stride,
                           shift_off, scale_off);
    }
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

hipError_t gemv_f32(const float * in, const float * W, const float * bias, float * out, int B, int K, int N,
                    int act_in, hipStream_t s) {
    if (B <= 0 || K <= 0 || N <= 0 || K % 4 ||
        ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(W)) & 15))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL((gemv_kernel<false, false>), dim3((N + 15) / 16), dim3(256), 0, s, in, W, bias, out, B, K, N,
                       act_in, nullptr, nullptr, 0, nullptr);
    return hipGetLastError();
}

hipError_t gemv_sinusoid_f32(const float * t, const float * freq, const float * W, const float * bias, float * out,
                             int B, int K, int N, hipStream_t s) {
    if (B <= 0 || K <= 0 || N <= 0 || K % 8 || (reinterpret_cast<uintptr_t>(W) & 15)) return hipErrorInvalidValue;
    hipLaunchKernelGGL((gemv_kernel<true, false>), dim3((N + 15) / 16), dim3(256), 0, s, t, W, bias, out, B, K, N, 0,
                       freq, nullptr, 0, nullptr);
    return hipGetLastError();
}

hipError_t gemv_comb_f32(const float * in, const float * W, const float * bias, float * out, const float * tables,
                         int L, float * comb, int B, int K, int N, int act_in, hipStream_t s) {
    if (B <= 0 || K <= 0 || N <= 0 || K % 4 || L <= 0 || !tables || !comb ||
        ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(W)) & 15))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL((gemv_kernel<false, true>), dim3((N + 15) / 16), dim3(256), 0, s, in, W, bias, out, B, K, N,
                       act_in, nullptr, tables, L, comb);
    return hipGetLastError();
}

hipError_t patch_embed(const float * latent, int Bl, int B, int Cl, int S, const float * Wt, const float * bias,
                       float * out, int C, hipStream_t s) {
    if (Bl <= 0 || B <= 0 || Cl <= 0 || S <= 0 || C <= 0 || B > 65535 || (S + 31) / 32 > 65535)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(patch_embed_kernel, dim3((C + 127) / 128, (S + 31) / 32, B), dim3(256), 0, s, latent, Bl, Cl, S,
                       Wt, bias, out, C);
    return hipGetLastError();
}

hipError_t final_layer(const float * x, const float * emb, const float * table, const float * Wt, const float * bias,
                       float * y, float * out, int B, int S, int C, int Cl, float eps, hipStream_t s) {
    if (B <= 0 || S <= 0 || C <= 0 || C > 64 * kMaxPerLane || Cl <= 0 || Cl > 32 || !y ||
        (reinterpret_cast<uintptr_t>(y) & 15))
        return hipErrorInvalidValue;
    const int rows = B * S;
    if (C % 384 == 0 && S % 32 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0) {
        // one pass: y is not written
        hipLaunchKernelGGL(final_proj_kernel<12>, dim3((rows + 31) / 32), dim3(64 * 12), 0, s, x, emb, table, Wt,
                           bias, out, B, S, C, Cl, eps);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(final_norm_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, x, emb, table, y, B, S, C, eps);
    if (C % 128 == 0)
        hipLaunchKernelGGL(proj_out_kernel, dim3((rows + 31) / 32), dim3(256), 0, s, y, Wt, bias, out, B, S, C, Cl);
    else
        hipLaunchKernelGGL(proj_out_scalar_kernel, dim3((rows * Cl + 255) / 256), dim3(256), 0, s, y, Wt, bias, out, B,
                           S, C, Cl);
    return hipGetLastError();
}

}  // namespace sana
