// K3 ReLU linear attention and K4 softmax cross-attention.
#include <cmath>

#include "hip_common.h"
#include "kernels.h"

namespace sana {
namespace {

// ---------------------------------------------------------------------------
// K3: linear attention (src/transformer_ops.cpp:496-537).  Per (b, h) the
// state is the (D+1) x D matrix S[r][d] = sum_t v[t][r] relu(k[t][d]) with the
// extra row r = D holding ksum[d] = sum_t relu(k[t][d]) (the "padded
// denominator column").  The token reduction is split over chunks (one
// workgroup each), the chunk partials are summed in fixed order by a second
// kernel (deterministic, no atomics), and a third kernel applies
// out[t][r] = sum_d S[r][d] relu(q[t][d]) / (sum_d S[D][d] relu(q[t][d]) + 1e-15).

constexpr int kLaTok = 32;      // tokens per LDS sub-tile
constexpr int kLaChunk = 256;   // tokens per partial-state workgroup
constexpr int kLaApplyTok = 32; // tokens per apply workgroup

template <int EPT>
__global__ __launch_bounds__(256) void la_state_kernel(const f16 * __restrict__ k, const f16 * __restrict__ v,
                                                       int64_t ld, int N, int H, int D, int nch,
                                                       float * __restrict__ part) {
    __shared__ float Ks[kLaTok][128];
    __shared__ float Vs[kLaTok][129];
    const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x;
    const int E = (D + 1) * D;
    const int t0 = c * kLaChunk, t1 = min(N, t0 + kLaChunk);
    float acc[EPT];
    int er[EPT], ed[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        acc[e] = 0.0f;
        const int g = tid + 256 * e;
        // entries past E read row D / column 0 (in bounds) and are never stored
        er[e] = g < E ? g / D : D;
        ed[e] = g < E ? g - er[e] * D : 0;
    }
    for (int ts = t0; ts < t1; ts += kLaTok) {
        for (int idx = tid; idx < kLaTok * D; idx += 256) {
            const int t = idx / D, d = idx - t * D;
            const int gt = ts + t;
            float kv = 0.0f, vv = 0.0f;
            if (gt < t1) {
                const int64_t off = ((int64_t)b * N + gt) * ld + (int64_t)h * D + d;
                kv = fmaxf(0.0f, (float)k[off]);
                vv = (float)v[off];
            }
            Ks[t][d] = kv;
            Vs[t][d] = vv;
        }
        if (tid < kLaTok) Vs[tid][D] = 1.0f;
        __syncthreads();
#pragma unroll 4
        for (int t = 0; t < kLaTok; ++t) {
#pragma unroll
            for (int e = 0; e < EPT; ++e) acc[e] += Vs[t][er[e]] * Ks[t][ed[e]];
        }
        __syncthreads();
    }
    float * out = part + (((int64_t)b * H + h) * nch + c) * E;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int g = tid + 256 * e;
        if (g < E) out[g] = acc[e];
    }
}

__global__ __launch_bounds__(256) void la_reduce_kernel(const float * __restrict__ part, int nch, int E,
                                                        float * __restrict__ state) {
    const int bh = blockIdx.x;
    for (int e = threadIdx.x; e < E; e += 256) {
        float s = 0.0f;
        for (int c = 0; c < nch; ++c) s += part[((int64_t)bh * nch + c) * E + e];
        state[(int64_t)bh * E + e] = s;
    }
}

__global__ __launch_bounds__(256) void la_apply_kernel(const f16 * __restrict__ q, int64_t ld,
                                                       const float * __restrict__ state, f16 * __restrict__ out,
                                                       int64_t ldo, int N, int H, int D) {
    extern __shared__ float smem[];
    // St[d][r] (r = 0..D, transposed so consecutive r are contiguous), Qs[t][d], den[t].
    float * St = smem;                          // D * (D + 1)
    float * Qs = St + D * (D + 1);              // kLaApplyTok * D
    float * den = Qs + kLaApplyTok * D;         // kLaApplyTok
    const int tb = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x;
    const int E = (D + 1) * D;
    const float * S = state + ((int64_t)b * H + h) * E;
    for (int e = tid; e < E; e += 256) {
        const int r = e / D, d = e - r * D;
        St[d * (D + 1) + r] = S[e];
    }
    const int t0 = tb * kLaApplyTok;
    for (int idx = tid; idx < kLaApplyTok * D; idx += 256) {
        const int t = idx / D, d = idx - t * D;
        const int gt = t0 + t;
        Qs[idx] = gt < N ? fmaxf(0.0f, (float)q[((int64_t)b * N + gt) * ld + (int64_t)h * D + d]) : 0.0f;
    }
    __syncthreads();
    if (tid < kLaApplyTok) {
        float s = 0.0f;
        for (int d = 0; d < D; ++d) s += St[d * (D + 1) + D] * Qs[tid * D + d];
        den[tid] = s + 1e-15f;
    }
    __syncthreads();
    for (int idx = tid; idx < kLaApplyTok * D; idx += 256) {
        const int t = idx / D, r = idx - t * D;
        const int gt = t0 + t;
        if (gt >= N) continue;
        float s = 0.0f;
        for (int d = 0; d < D; ++d) s += St[d * (D + 1) + r] * Qs[t * D + d];
        out[((int64_t)b * N + gt) * ldo + (int64_t)h * D + r] = (f16)(s / den[t]);
    }
}

// ---------------------------------------------------------------------------
// K4: softmax cross-attention (attention_4d, src/transformer_ops.cpp:348-392:
// scores * 1/sqrt(D), + bias, softmax over keys, . V) fused per
// (b, h, 64-query tile).  4 waves x 16 queries; v_mfma_f32_16x16x32_f16 for
// Q.K^T (contraction over head dims, padded to 32 with zeros) and for P.V
// (contraction over keys).  K is read as [key][dim] rows and V pre-transposed
// as [dim][key], so every MFMA operand is one 16-byte read.  Keys past L get
// probability exactly 0.

template <int LT>
__global__ __launch_bounds__(256) void xattn_kernel(const f16 * __restrict__ q, int64_t ldq,
                                                    const f16 * __restrict__ k, int64_t ldk,
                                                    const f16 * __restrict__ vt, int64_t ldvt,
                                                    const float * __restrict__ bias, f16 * __restrict__ out,
                                                    int64_t ldo, int N, int L, int H, int D, float scale, int vec) {
    constexpr int LP = ((LT * 16 + 31) / 32) * 32;  // keys padded to the P.V step
    __shared__ __attribute__((aligned(16))) f16 Ps[4][16][LP + 8];
    const int h = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int q0 = blockIdx.x * 64 + w * 16;
    const int lr = lane & 15, lg = lane >> 4;  // row/col within 16, k-group 0..3
    const int Dp = (D + 31) / 32 * 32;

    // S = Q K^T
    f32x4 S[LT];
#pragma unroll
    for (int t = 0; t < LT; ++t) S[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int qrow = q0 + lr;
    const f16 * qp = q + ((int64_t)b * N + min(qrow, N - 1)) * ldq + (int64_t)h * D;
    const f16 * kb = k + (int64_t)b * L * ldk + (int64_t)h * D;
    for (int kk = 0; kk < Dp; kk += 32) {
        const int d0 = kk + 8 * lg;
        f16x8 qf;
        if (vec && d0 + 8 <= D) {
            qf = *reinterpret_cast<const f16x8 *>(qp + d0);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) qf[e] = (d0 + e < D) ? qp[d0 + e] : (f16)0.0f;
        }
#pragma unroll
        for (int t = 0; t < LT; ++t) {
            const int key = t * 16 + lr;
            f16x8 kf;
            if (key < L) {
                const f16 * kp = kb + (int64_t)key * ldk;
                if (vec && d0 + 8 <= D) {
                    kf = *reinterpret_cast<const f16x8 *>(kp + d0);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) kf[e] = (d0 + e < D) ? kp[d0 + e] : (f16)0.0f;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) kf[e] = (f16)0.0f;
            }
            S[t] = mfma_16x16x32(qf, kf, S[t]);
        }
    }
    // scale, bias, mask; rows 4*lg + i, key column t*16 + lr
    float mx[4], sm[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) mx[i] = -INFINITY;
#pragma unroll
    for (int t = 0; t < LT; ++t) {
        const int key = t * 16 + lr;
        const float bv = (bias && key < L) ? bias[(int64_t)b * L + key] : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float s = key < L ? S[t][i] * scale + bv : -INFINITY;
            S[t][i] = s;
            mx[i] = fmaxf(mx[i], s);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) mx[i] = fmaxf(mx[i], __shfl_xor(mx[i], o, 64));
        sm[i] = 0.0f;
    }
#pragma unroll
    for (int t = 0; t < LT; ++t) {
        const int key = t * 16 + lr;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float e = key < L ? expf(S[t][i] - mx[i]) : 0.0f;
            sm[i] += e;
            Ps[w][4 * lg + i][key] = (f16)e;
        }
    }
    // zero the P columns between LT*16 and LP
    for (int c = LT * 16 + lane; c < LP; c += 64)
#pragma unroll
        for (int r = 0; r < 16; ++r) Ps[w][r][c] = (f16)0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) sm[i] += __shfl_xor(sm[i], o, 64);
    __syncthreads();

    // O = P V over key steps of 32; head dims in tiles of 16.
    const int DT = (D + 15) / 16;
    const f16 * vb = vt + ((int64_t)b * H * D + (int64_t)h * D) * ldvt;
    for (int dt = 0; dt < DT; ++dt) {
        f32x4 o = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        const int dim = dt * 16 + lr;
        const f16 * vp = vb + (int64_t)min(dim, D - 1) * ldvt;
        for (int kc = 0; kc < LP; kc += 32) {
            const int k0 = kc + 8 * lg;
            const f16x8 pf = *reinterpret_cast<const f16x8 *>(&Ps[w][lr][k0]);
            f16x8 vf;
            if (dim < D && vec && k0 + 8 <= L) {
                vf = *reinterpret_cast<const f16x8 *>(vp + k0);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) vf[e] = (dim < D && k0 + e < L) ? vp[k0 + e] : (f16)0.0f;
            }
            o = mfma_16x16x32(pf, vf, o);
        }
        // o[i] = O[row 4*lg + i][dim]; row sums live in sm[i] of the same lanes.
        if (dim < D) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = q0 + 4 * lg + i;
                if (row < N) out[((int64_t)b * N + row) * ldo + (int64_t)h * D + dim] = (f16)(o[i] / sm[i]);
            }
        }
    }
}

template <int LT>
hipError_t launch_xattn(const f16 * q, int64_t ldq, const f16 * k, int64_t ldk, const f16 * vt, int64_t ldvt,
                        const float * bias, f16 * out, int64_t ldo, int B, int N, int L, int H, int D, float scale,
                        int vec, hipStream_t s) {
    hipLaunchKernelGGL((xattn_kernel<LT>), dim3((N + 63) / 64, H, B), dim3(256), 0, s, q, ldq, k, ldk, vt, ldvt, bias,
                       out, ldo, N, L, H, D, scale, vec);
    return hipGetLastError();
}

}  // namespace

size_t linattn_workspace_floats(int B, int N, int H, int D) {
    const size_t nch = (size_t)(N + kLaChunk - 1) / kLaChunk;
    const size_t E = (size_t)(D + 1) * D;
    return (size_t)B * H * E * (nch + 1);
}

hipError_t linear_attention(const half_t * q, const half_t * k, const half_t * v, int64_t ld, half_t * out,
                            int64_t ldo, int B, int N, int H, int D, float * ws, hipStream_t s) {
    if (B <= 0 || N <= 0 || H <= 0 || D <= 0 || D > 100 || ld < (int64_t)H * D || ldo < (int64_t)H * D || !ws)
        return hipErrorInvalidValue;
    const int nch = (N + kLaChunk - 1) / kLaChunk;
    const int E = (D + 1) * D;
    float * part = ws;
    float * state = ws + (size_t)B * H * E * nch;
    const f16 * kq = reinterpret_cast<const f16 *>(k);
    const f16 * vq = reinterpret_cast<const f16 *>(v);
    const dim3 g1(nch, H, B);
    if (E <= 256 * 8)
        hipLaunchKernelGGL((la_state_kernel<8>), g1, dim3(256), 0, s, kq, vq, ld, N, H, D, nch, part);
    else if (E <= 256 * 24)
        hipLaunchKernelGGL((la_state_kernel<24>), g1, dim3(256), 0, s, kq, vq, ld, N, H, D, nch, part);
    else
        hipLaunchKernelGGL((la_state_kernel<40>), g1, dim3(256), 0, s, kq, vq, ld, N, H, D, nch, part);
    hipLaunchKernelGGL(la_reduce_kernel, dim3(B * H), dim3(256), 0, s, part, nch, E, state);
    const size_t lds = sizeof(float) * ((size_t)D * (D + 1) + (size_t)kLaApplyTok * D + kLaApplyTok);
    hipLaunchKernelGGL(la_apply_kernel, dim3((N + kLaApplyTok - 1) / kLaApplyTok, H, B), dim3(256), lds, s,
                       reinterpret_cast<const f16 *>(q), ld, state, reinterpret_cast<f16 *>(out), ldo, N, H, D);
    return hipGetLastError();
}

hipError_t cross_attention(const half_t * q, int64_t ldq, const half_t * k, int64_t ldk, const half_t * vt,
                           int64_t ldvt, const float * bias, half_t * out, int64_t ldo, int B, int N, int L, int H,
                           int D, hipStream_t s) {
    if (B <= 0 || N <= 0 || L <= 0 || L > 512 || H <= 0 || D <= 0 || D > 256 || ldq < (int64_t)H * D ||
        ldk < (int64_t)H * D || ldvt < L || ldo < (int64_t)H * D || H > 65535 || B > 65535)
        return hipErrorInvalidValue;
    // 16-byte operand reads need 8-element alignment of every row and head offset.
    const int vec = (D % 8 == 0 && ldq % 8 == 0 && ldk % 8 == 0 && ldvt % 8 == 0 &&
                     ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                       reinterpret_cast<uintptr_t>(vt)) & 15) == 0) ? 1 : 0;
    const float scale = static_cast<float>(1.0f / std::sqrt(static_cast<double>(D)));
    const f16 * qq = reinterpret_cast<const f16 *>(q);
    const f16 * kk = reinterpret_cast<const f16 *>(k);
    const f16 * vv = reinterpret_cast<const f16 *>(vt);
    f16 * oo = reinterpret_cast<f16 *>(out);
    const int lt = (L + 15) / 16;
    if (lt <= 2) return launch_xattn<2>(qq, ldq, kk, ldk, vv, ldvt, bias, oo, ldo, B, N, L, H, D, scale, vec, s);
    if (lt <= 8) return launch_xattn<8>(qq, ldq, kk, ldk, vv, ldvt, bias, oo, ldo, B, N, L, H, D, scale, vec, s);
    if (lt <= 20) return launch_xattn<20>(qq, ldq, kk, ldk, vv, ldvt, bias, oo, ldo, B, N, L, H, D, scale, vec, s);
    return launch_xattn<32>(qq, ldq, kk, ldk, vv, ldvt, bias, oo, ldo, B, N, L, H, D, scale, vec, s);
}

}  // namespace sana
