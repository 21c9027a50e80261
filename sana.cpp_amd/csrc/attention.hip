// K3 ReLU linear attention and K4 softmax cross-attention.
#include <algorithm>
#include <cmath>
#include <string>

#include "hip_common.h"
#include "kernels.h"

namespace sana {
namespace {

// ---------------------------------------------------------------------------
// K3: linear attention (src/transformer_ops.cpp:496-537).  Per (b, h) the
// state is the (D+1) x D matrix S[r][d] = sum_t v[t][r] relu(k[t][d]) with the
// extra row r = D holding ksum[d] = sum_t relu(k[t][d]) (the "padded
// denominator column"); then
//   out[t][r] = sum_d S[r][d] relu(q[t][d]) / (sum_d S[D][d] relu(q[t][d]) + 1e-15).
//
// la_state_kernel: one workgroup of 4 waves per (token chunk, h, b).  Sub-chunks
//   of 64 tokens of relu(K) and V are staged in LDS transposed (token-contiguous
//   rows) by all four waves, so S^T = relu(K)^T . V is a chain of
//   v_mfma_f32_32x32x16_f16 over tokens with 16-byte operand reads; fp32
//   accumulation of exact fp16 products.  The waves split the 32x32 tiles of
//   the state, or for D <= 32 (one tile) the 16-token steps, added in LDS in
//   wave order.  ksum is summed on the VALU from the same LDS rows.  Each chunk
//   writes its partial (D+1) x D state.
// la_reduce_kernel: sums the chunk partials in fixed chunk order (no atomics,
//   bit-reproducible) into an fp16 hi/lo pair of the state, scaled by 2^k.
// la_apply_kernel: relu(Q) . [S | ksum]^T on MFMA (hi and lo halves), one wave
//   per 32 tokens, then the division by the denominator column.
//
// Range of the fp16 state.  S and ksum grow with the token count (|S| reaches
// ~7e3 at 1024 tokens of the 0.6B model, so ~1e5 at 16384 tokens, past fp16's
// 65504).  Each (b, h) state is therefore scaled by a power of two 2^k chosen
// from an upper bound m of its largest |entry|: m 2^k lies in [2^13, 2^14).
// Scaling by 2^k is exact in fp32 and cancels in
// (S . q) / (ksum . q + 1e-15) once the 1e-15 is scaled by 2^k as well.

// Exponent k of the state scale 2^k for an upper bound m of max |S|; a zero,
// NaN or infinite bound leaves the state unscaled.
SANA_DEV int la_state_exponent(float m) {
    if (!(m > 0.0f) || !(m <= 3.402823466e38f)) return 0;
    int ex;
    (void)frexpf(m, &ex);  // m = f 2^ex, f in [0.5, 1)
    return min(60, max(-60, 14 - ex));
}

// Upper bound of max |S| over the nch chunk partials of one (b, h): the sum of
// their maxima, in chunk order (every kernel computes the same k from it).
SANA_DEV float la_bound(const float * __restrict__ pmax, int nch) {
    float m = 0.0f;
    int c = 0;
    // eight loads in flight, summed in chunk order
    for (; c + 8 <= nch; c += 8) {
        float x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = pmax[c + u];
#pragma unroll
        for (int u = 0; u < 8; ++u) m += x[u];
    }
    for (; c < nch; ++c) m += pmax[c];
    return m;
}

constexpr int kLaSub = 64;                 // tokens per LDS sub-chunk
constexpr int kLaChunks = 16;              // partial states per (b, h)
constexpr int kLaRow = kLaSub + 8;         // halves per transposed LDS row (144 B: conflict-free reads)

constexpr int kLsWaves = 4;                // waves per la_state_kernel workgroup

template <int TD>  // ceil(D / 32): 32x32 MFMA tiles per side of the state
__global__ __launch_bounds__(64 * kLsWaves) void la_state_kernel(const f16 * __restrict__ k,
                                                                 const f16 * __restrict__ v, int64_t ld, int N,
                                                                 int H, int D, int T, int nch, int vec,
                                                                 float * __restrict__ part,
                                                                 float * __restrict__ pmax) {
    constexpr int DP = TD * 32;
    constexpr int NTILE = TD * TD;
    // one tile (D <= 32): the waves split each sub-chunk's four 16-token steps
    // and their partials are added in LDS; more tiles: the waves split the tiles
    constexpr bool kSplitSteps = TD == 1;
    constexpr int MYT = kSplitSteps ? 1 : (NTILE + kLsWaves - 1) / kLsWaves;
    __shared__ __attribute__((aligned(16))) f16 Kt[DP][kLaRow];
    __shared__ __attribute__((aligned(16))) f16 Vt[DP][kLaRow];
    __shared__ float red[kSplitSteps ? kLsWaves : 1][kSplitSteps ? 32 : 1][33];
    __shared__ float wmax[kLsWaves];
    const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    for (int i = tid; i < DP * kLaRow; i += 64 * kLsWaves) {
        (&Kt[0][0])[i] = (f16)0.0f;
        (&Vt[0][0])[i] = (f16)0.0f;
    }
    f32x16 acc[MYT];
#pragma unroll
    for (int u = 0; u < MYT; ++u)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[u][r] = 0.0f;
    float ks = 0.0f;  // ksum[tid] for tid < D

    const int t_begin = c * T, t_end = min(N, t_begin + T);
    const f16 * kb = k + (int64_t)b * N * ld + (int64_t)h * D;
    const f16 * vb = v + (int64_t)b * N * ld + (int64_t)h * D;
    const int G = D / 8;
    // vec: one item per thread = 8 head dims (group g) of 4 consecutive tokens,
    // loaded for the next sub-chunk while the MFMAs of this one run, written to
    // LDS as 8-byte runs of 4 tokens (D <= 112: at most 64 x 14 / 4 = 224 items)
    const int item_t = tid / max(G, 1), item_g = tid - item_t * max(G, 1);
    const bool has_item = vec && tid < (kLaSub / 4) * G;
    f16x8 kreg[4], vreg[4];
    auto load_item = [&](int t0) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int gt = t0 + 4 * item_t + u;
            if (gt < t_end) {
                kreg[u] = *reinterpret_cast<const f16x8 *>(kb + (int64_t)gt * ld + item_g * 8);
                vreg[u] = *reinterpret_cast<const f16x8 *>(vb + (int64_t)gt * ld + item_g * 8);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) kreg[u][e] = vreg[u][e] = (f16)0.0f;
            }
        }
    };
    if (has_item && t_begin < t_end) load_item(t_begin);
    for (int t0 = t_begin; t0 < t_end; t0 += kLaSub) {
        __syncthreads();
        if (vec) {
            if (has_item) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    f16x4 k4, v4;
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        k4[u] = kreg[u][e] > (f16)0.0f ? kreg[u][e] : (f16)0.0f;
                        v4[u] = vreg[u][e];
                    }
                    *reinterpret_cast<f16x4 *>(&Kt[item_g * 8 + e][4 * item_t]) = k4;
                    *reinterpret_cast<f16x4 *>(&Vt[item_g * 8 + e][4 * item_t]) = v4;
                }
            }
        } else {
            for (int idx = tid; idx < kLaSub * D; idx += 64 * kLsWaves) {
                const int t = idx / D, d = idx - t * D;
                const int gt = t0 + t;
                f16 kv = (f16)0.0f, vv = (f16)0.0f;
                if (gt < t_end) {
                    kv = kb[(int64_t)gt * ld + d];
                    vv = vb[(int64_t)gt * ld + d];
                }
                Kt[d][t] = kv > (f16)0.0f ? kv : (f16)0.0f;
                Vt[d][t] = vv;
            }
        }
        __syncthreads();
        if (has_item && t0 + kLaSub < t_end) load_item(t0 + kLaSub);
        if (tid < D) {
            float sum = 0.0f;
            for (int t = 0; t < kLaSub; t += 8) {
                const f16x8 x = *reinterpret_cast<const f16x8 *>(&Kt[tid][t]);
#pragma unroll
                for (int e = 0; e < 8; ++e) sum += (float)x[e];
            }
            ks += sum;
        }
        if constexpr (kSplitSteps) {
            const int col = 16 * w + 8 * (lane >> 5);
            const f16x8 af = *reinterpret_cast<const f16x8 *>(&Kt[lane & 31][col]);
            const f16x8 bf = *reinterpret_cast<const f16x8 *>(&Vt[lane & 31][col]);
            acc[0] = mfma_32x32x16(af, bf, acc[0]);
        } else {
#pragma unroll
            for (int kk = 0; kk < kLaSub; kk += 16) {
                const int col = kk + 8 * (lane >> 5);
#pragma unroll
                for (int u = 0; u < MYT; ++u) {
                    const int tile = w + u * kLsWaves;
                    if (tile < NTILE) {
                        const int i = tile / TD, j = tile - (tile / TD) * TD;
                        const f16x8 af = *reinterpret_cast<const f16x8 *>(&Kt[i * 32 + (lane & 31)][col]);
                        const f16x8 bf = *reinterpret_cast<const f16x8 *>(&Vt[j * 32 + (lane & 31)][col]);
                        acc[u] = mfma_32x32x16(af, bf, acc[u]);
                    }
                }
            }
        }
    }
    // acc tile (i, j): lane holds r = j*32 + (lane & 31) and d = i*32 + 8*(q/4) + 4*(lane/32) + q%4.
    const int E = (D + 1) * D;
    float * out = part + (((int64_t)b * H + h) * nch + c) * E;
    float m = 0.0f;
    if constexpr (kSplitSteps) {
#pragma unroll
        for (int q = 0; q < 16; ++q) red[w][8 * (q >> 2) + 4 * (lane >> 5) + (q & 3)][lane & 31] = acc[0][q];
        __syncthreads();
        for (int e = tid; e < 32 * 32; e += 64 * kLsWaves) {
            const int r = e >> 5, d = e & 31;
            float a = 0.0f;
#pragma unroll
            for (int ww = 0; ww < kLsWaves; ++ww) a += red[ww][d][r];
            if (r < D && d < D) {
                out[r * D + d] = a;
                m = fmaxf(m, fabsf(a));
            }
        }
    } else {
#pragma unroll
        for (int u = 0; u < MYT; ++u) {
            const int tile = w + u * kLsWaves;
            if (tile >= NTILE) continue;
            const int i = tile / TD, j = tile - (tile / TD) * TD;
            const int r = j * 32 + (lane & 31);
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int d = i * 32 + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
                if (r < D && d < D) {
                    out[r * D + d] = acc[u][q];
                    m = fmaxf(m, fabsf(acc[u][q]));
                }
            }
        }
    }
    if (tid < D) {
        out[D * D + tid] = ks;
        m = fmaxf(m, ks);
    }
    // max |entry| of this partial
    m = wave_max(m);
    if (lane == 0) wmax[w] = m;
    __syncthreads();
    if (tid == 0) {
        float mm = 0.0f;
#pragma unroll
        for (int ww = 0; ww < kLsWaves; ++ww) mm = fmaxf(mm, wmax[ww]);
        pmax[((int64_t)b * H + h) * nch + c] = mm;
    }
}

// Sums the chunk partials in fixed order and writes the state 2^k S, transposed
// to the apply kernel's MFMA operand layout, as an fp16 hi/lo pair:
// 2^k S[r][d] = hi[r][d] + lo[r][d] with hi = f16(2^k S), lo = f16(2^k S - hi),
// so the fp16 products of the apply step carry the fp32 state to ~2^-22
// relative error.  Layout [NP][KP] (r rows incl. the ksum row r = D, d
// contiguous), zero padded.
__global__ __launch_bounds__(256) void la_reduce_kernel(const float * __restrict__ part,
                                                        const float * __restrict__ pmax, int nch, int D, int NP,
                                                        int KP, f16 * __restrict__ hi, f16 * __restrict__ lo) {
    const int e = blockIdx.x * 256 + threadIdx.x;
    const int bh = blockIdx.y;
    if (e >= NP * KP) return;
    const float scale = ldexpf(1.0f, la_state_exponent(la_bound(pmax + (int64_t)bh * nch, nch)));
    const int r = e / KP, d = e - r * KP;
    float s = 0.0f;
    if (r <= D && d < D) {
        const int E = (D + 1) * D;
        const float * p = part + (int64_t)bh * nch * E + r * D + d;
        int c = 0;
        // eight loads in flight, summed in chunk order
        for (; c + 8 <= nch; c += 8) {
            float x[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) x[u] = p[(int64_t)(c + u) * E];
#pragma unroll
            for (int u = 0; u < 8; ++u) s += x[u];
        }
        for (; c < nch; ++c) s += p[(int64_t)c * E];
    }
    s *= scale;
    const f16 h = (f16)s;
    hi[(int64_t)bh * NP * KP + e] = h;
    lo[(int64_t)bh * NP * KP + e] = (f16)(s - (float)h);
}

// out[t][r] = (relu(q) . S^T)[t][r] / ((relu(q) . S^T)[t][D] + 1e-15) (both
// terms of the ratio scaled by the state's 2^k) on
// v_mfma_f32_32x32x16_f16: one wave per 32 tokens of one (b, h).  The A
// operand (8 consecutive head dims of one token) comes straight from the
// token-major q rows; columns past D are masked to zero.
template <int NT, int KS>  // NT: 32-wide column tiles of [S | ksum]; KS: 16-deep steps over d
__global__ __launch_bounds__(256) void la_apply_kernel(const f16 * __restrict__ q, int64_t ld,
                                                       const f16 * __restrict__ shi, const f16 * __restrict__ slo,
                                                       const float * __restrict__ pmax, int nch,
                                                       f16 * __restrict__ out, int64_t ldo, int N, int H, int D,
                                                       int vec) {
    constexpr int NP = NT * 32, KP = KS * 16;
    const int h = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int t0 = (blockIdx.x * 4 + w) * 32;
    if (t0 >= N) return;
    const int trow = min(t0 + (lane & 31), N - 1);
    const f16 * qr = q + ((int64_t)b * N + trow) * ld + (int64_t)h * D;
    const int64_t sbase = ((int64_t)b * H + h) * NP * KP;
    f32x16 acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[j][i] = 0.0f;
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
        const int d0 = kk * 16 + 8 * (lane >> 5);
        f16x8 af;
        if (vec && d0 + 8 <= D) {
            af = *reinterpret_cast<const f16x8 *>(qr + d0);
#pragma unroll
            for (int e = 0; e < 8; ++e) af[e] = af[e] > (f16)0.0f ? af[e] : (f16)0.0f;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const f16 x = d0 + e < D ? qr[d0 + e] : (f16)0.0f;
                af[e] = x > (f16)0.0f ? x : (f16)0.0f;
            }
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int64_t off = sbase + (int64_t)(j * 32 + (lane & 31)) * KP + kk * 16 + 8 * (lane >> 5);
            const f16x8 bh = *reinterpret_cast<const f16x8 *>(shi + off);
            const f16x8 bl = *reinterpret_cast<const f16x8 *>(slo + off);
            acc[j] = mfma_32x32x16(af, bh, acc[j]);
            acc[j] = mfma_32x32x16(af, bl, acc[j]);
        }
    }
    // Lane holds column r = 32 j + (lane & 31), rows t0 + 8*(i/4) + 4*(lane/32) + i%4.
    // The denominator is column D, held by lane (lane & 32) | (D % 32) of tile D / 32.
    const int jd = D >> 5, cd = D & 31;
    const float eps = ldexpf(1e-15f, la_state_exponent(la_bound(pmax + ((int64_t)b * H + h) * nch, nch)));
    float den[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        float v = 0.0f;
#pragma unroll
        for (int j = 0; j < NT; ++j)
            if (j == jd) v = acc[j][i];
        den[i] = __shfl(v, (lane & 32) | cd, 64) + eps;
    }
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int r = j * 32 + (lane & 31);
        if (r >= D) continue;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int t = t0 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
            if (t < N) out[((int64_t)b * N + t) * ldo + (int64_t)h * D + r] = (f16)(acc[j][i] / den[i]);
        }
    }
}

// la_fused_kernel: the whole linear attention of one (b, h) with head_dim 32
// in one workgroup of 8 waves, from the kGemmQKV layouts (relu already
// applied to q and k; K^T and V^T token-contiguous per channel).
//   1. Wave w sums its token range: S^T[d][r] += relu(K)^T[d][t..t+15] .
//      V^T[r][t..t+15]^T and ksum[d] += relu(K)^T[d][t..] . 1 on
//      v_mfma_f32_32x32x16_f16, both operands straight from global memory
//      (8 consecutive tokens per lane: one 16-byte load).
//   2. The 8 partial states are summed in LDS in wave order (bit-reproducible)
//      and stored as an fp16 hi/lo pair, 2^k S = hi + lo, k from the sum of
//      the 8 partials' maxima (the range rule of the chunked paths).
//   3. Wave w applies it to its tokens transposed, O^T[r][t] = [S | ksum] .
//      relu(q)^T, so each lane holds four consecutive head dims of one token
//      (8-byte stores); the denominator is row 0 of the ksum tile.
// With `splits` > 1, `splits` workgroups share one (b, h): each builds the
// whole (small) state and applies it to its own 1/splits of the tokens, so
// B*H*splits workgroups cover the CUs when B*H alone does not.
// out[t][r] = O^T[r][t] / (den[t] + 2^k 1e-15), as src/transformer_ops.cpp:496-537.
constexpr int kLfWaves = 8;
constexpr int kLfSrow = 40;  // halves per LDS row of the hi/lo state (80 B rows)

// Per-wave output staging of 32 tokens x 32 head dims: 64-byte token rows whose
// four 16-byte chunks are stored at chunk ^ ((token >> 2) & 3).  The 8-byte
// writes (lane = token, dims 8 i4 + 4 hh) and the 16-byte row reads (four
// lanes per token) then run at gfx950's conflict-free LDS rates (measured: the
// reads take a third of the cycles of unswizzled 80-byte rows).
SANA_DEV int la_ost_chunk(int token, int chunk) { return chunk ^ ((token >> 2) & 3); }

__global__ __launch_bounds__(64 * kLfWaves) void la_fused_kernel(const f16 * __restrict__ q, int64_t ldq,
                                                        const f16 * __restrict__ kt, const f16 * __restrict__ vt,
                                                        f16 * __restrict__ out, int64_t ldo, int N, int H,
                                                        int splits) {
    __shared__ float part[kLfWaves][33][32];                       // per-wave S^T (rows d) + ksum row
    __shared__ __attribute__((aligned(16))) f16 sh[2][2][32][kLfSrow];  // [S|ksum tile][hi|lo][row][d]
    __shared__ __attribute__((aligned(16))) f16 ost[kLfWaves][32][32];  // per-wave output staging [token][dim chunk]
    __shared__ float pmax[kLfWaves];                                   // max |entry| of each wave's partial
    // XCD-aware order: workgroup ids are dealt round-robin to the 8 XCDs, so id
    // goes to position (id % 8) * (n / 8) + id / 8 and the `splits` workgroups of
    // one (b, h), which read the same K^T / V^T, run on one XCD and share its L2.
    const int nwg = (int)gridDim.x, per = nwg / 8, id = (int)blockIdx.x;
    const int pos = id < per * 8 ? (id % 8) * per + id / 8 : id;
    const int bh = pos / splits, sp = pos - bh * splits, b = bh / H, h = bh - b * H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hh = lane >> 5;
    const f16 * K = kt + ((int64_t)b * H + h) * 32 * N;  // rows d = 0..31, N tokens each
    const f16 * V = vt + ((int64_t)b * H + h) * 32 * N;
    const int span = (N / kLfWaves + 15) / 16 * 16;      // state tokens per wave, multiple of 16
    const int tb = w * span, te = min(N, tb + span);
    // apply range [ta, tz) of this wave within the workgroup's token share
    const int per_split = (N + splits - 1) / splits;
    const int T0 = min(N, sp * per_split), T1 = min(N, T0 + per_split);
    const int span3 = ((T1 - T0 + kLfWaves - 1) / kLfWaves + 15) / 16 * 16;
    const int ta = min(T1, T0 + w * span3), tz = min(T1, ta + span3);

    // query fragments of the first kQpf apply steps are independent of the
    // state: issue them before anything else
    constexpr int kQpf = 4;
    const f16 * qbase = q + (int64_t)b * N * ldq + (int64_t)h * 32 + 8 * hh;
    f16x8 qpf[kQpf][2];
#pragma unroll
    for (int j = 0; j < kQpf; ++j) {
        const int tq = min(ta + 32 * j + (lane & 31), N - 1);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) qpf[j][kk] = *reinterpret_cast<const f16x8 *>(qbase + (int64_t)tq * ldq + kk * 16);
    }

    // 1. partial state: each group's loads (kG steps of 16 tokens) are all
    // issued before its MFMAs
    f32x16 s, ks;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = ks[i] = 0.0f;
    f16x8 ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = (f16)1.0f;
    const f16 * krow = K + (int64_t)(lane & 31) * N + 8 * hh;
    const f16 * vrow = V + (int64_t)(lane & 31) * N + 8 * hh;
    constexpr int kG = 8;
    for (int g0 = tb; g0 < te; g0 += 16 * kG) {
        f16x8 ka[kG], va[kG];
#pragma unroll
        for (int u = 0; u < kG; ++u) {
            const int t = g0 + 16 * u;
            if (t < te) {
                ka[u] = *reinterpret_cast<const f16x8 *>(krow + t);
                va[u] = *reinterpret_cast<const f16x8 *>(vrow + t);
            }
        }
#pragma unroll
        for (int u = 0; u < kG; ++u) {
            if (g0 + 16 * u < te) {
                s = mfma_32x32x16(ka[u], va[u], s);
                ks = mfma_32x32x16(ka[u], ones, ks);
            }
        }
    }
    // lane holds column r = lane & 31 and rows d = 8*(i/4) + 4*hh + i%4
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int d = 8 * (i >> 2) + 4 * hh + (i & 3);
        part[w][d][lane & 31] = s[i];
        if ((lane & 31) == 0) part[w][32][d] = ks[i];
    }
    {
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) m = fmaxf(m, fmaxf(fabsf(s[i]), ks[i]));
        m = wave_max(m);
        if (lane == 0) pmax[w] = m;
    }
    __syncthreads();
    const int kexp = la_state_exponent(la_bound(pmax, kLfWaves));
    const float scale = ldexpf(1.0f, kexp), eps = ldexpf(1e-15f, kexp);

    // 2. fixed-order sum of the partials -> hi/lo state tiles.  Tile 0 row r
    // holds S[r][d]; tile 1 row 0 holds ksum[d], rows 1..31 are zero.
    for (int e = tid; e < 2 * 32 * 32; e += 64 * kLfWaves) {
        // consecutive threads take consecutive r: conflict-free reads of part[.][d][r]
        const int tile = e >> 10, d = (e >> 5) & 31, r = e & 31;
        float acc = 0.0f;
        if (tile == 0) {
            for (int ww = 0; ww < kLfWaves; ++ww) acc += part[ww][d][r];
        } else if (r == 0) {
            for (int ww = 0; ww < kLfWaves; ++ww) acc += part[ww][32][d];
        }
        // tile 1, r > 0: zero rows
        acc *= scale;
        const f16 hi = (f16)acc;
        sh[tile][0][r][d] = hi;
        sh[tile][1][r][d] = (f16)(acc - (float)hi);
    }
    __syncthreads();

    // 3. apply, 32 tokens per step
    const f16 * srow0 = &sh[0][0][lane & 31][8 * hh];
    f16x8 sa[2][2][2];  // [tile][hi|lo][k-step]
#pragma unroll
    for (int tile = 0; tile < 2; ++tile)
#pragma unroll
        for (int hl = 0; hl < 2; ++hl)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
                sa[tile][hl][kk] = *reinterpret_cast<const f16x8 *>(srow0 + (tile * 2 + hl) * 32 * kLfSrow + kk * 16);
    // two 32-token steps per iteration: four independent MFMA chains
    // Output of 32 tokens: staged in this wave's LDS tile [token][dim] (the lane
    // holds token lane & 31, dims 8*i4 + 4*hh + {0..3}), then written as full
    // 64-byte token rows, four lanes per token, 16 tokens per store instruction.
    auto apply_store = [&](int t0, const f32x16 & o, const f32x16 & dn) {
        // the denominator of token column (lane & 31) is row 0: i = 0 on the hh = 0 lane
        const float rden = 1.0f / (__shfl(dn[0], lane & 31, 64) + eps);
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
            f16x4 v4;
#pragma unroll
            for (int u = 0; u < 4; ++u) v4[u] = (f16)(o[4 * i4 + u] * rden);
            *reinterpret_cast<f16x4 *>(&ost[w][lane & 31][8 * la_ost_chunk(lane & 31, i4) + 4 * hh]) = v4;
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int tl = half * 16 + (lane >> 2), c8 = (lane & 3) * 8;
            const f16x8 v8 = *reinterpret_cast<const f16x8 *>(&ost[w][tl][8 * la_ost_chunk(tl, lane & 3)]);
            const int t = t0 + tl;
            if (t < tz) *reinterpret_cast<f16x8 *>(out + ((int64_t)b * N + t) * ldo + (int64_t)h * 32 + c8) = v8;
        }
        __builtin_amdgcn_wave_barrier();
    };
    auto load_q = [&](int t0, f16x8 (&qf)[2]) {
        const int tq = min(t0 + (lane & 31), N - 1);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) qf[kk] = *reinterpret_cast<const f16x8 *>(qbase + (int64_t)tq * ldq + kk * 16);
    };
    for (int j = 0, t0 = ta; t0 < tz; j += 2, t0 += 64) {
        f16x8 qa[2], qb[2];
        if (j + 1 < kQpf) {
#pragma unroll
            for (int jj = 0; jj + 1 < kQpf; jj += 2)
                if (jj == j) {
#pragma unroll
                    for (int kk = 0; kk < 2; ++kk) {
                        qa[kk] = qpf[jj][kk];
                        qb[kk] = qpf[jj + 1][kk];
                    }
                }
        } else {
            load_q(t0, qa);
            load_q(t0 + 32, qb);
        }
        f32x16 oa, da, ob, db;
#pragma unroll
        for (int i = 0; i < 16; ++i) oa[i] = da[i] = ob[i] = db[i] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int hl = 0; hl < 2; ++hl) {
                oa = mfma_32x32x16(sa[0][hl][kk], qa[kk], oa);
                ob = mfma_32x32x16(sa[0][hl][kk], qb[kk], ob);
                da = mfma_32x32x16(sa[1][hl][kk], qa[kk], da);
                db = mfma_32x32x16(sa[1][hl][kk], qb[kk], db);
            }
        apply_store(t0, oa, da);
        if (t0 + 32 < tz) apply_store(t0 + 32, ob, db);
    }
}

// la_chunk_kernel: the chunk partial states of the chunked path for head_dim
// 32, from the kGemmQKV layouts (relu(K)^T and V^T token-contiguous per
// channel).  One workgroup of 8 waves per (token chunk, b, h): each wave sums
// its share of the chunk as la_fused_kernel's step 1 does (MFMA operands
// straight from global memory), the 8 partials are added in LDS in wave order
// and the chunk's (D+1) x D partial is written in la_state_kernel's layout
// (part[r * D + d] = S[r][d], ksum in row D) with its max |entry|, which
// la_reduce_apply32_kernel reduces and applies.
__global__ __launch_bounds__(64 * kLfWaves) void la_chunk_kernel(const f16 * __restrict__ kt,
                                                                 const f16 * __restrict__ vt, int N, int T, int nch,
                                                                 float * __restrict__ part,
                                                                 float * __restrict__ pmax) {
    __shared__ float sp[kLfWaves][33][33];  // per-wave S^T (rows d) + ksum row, padded rows
    __shared__ float wmax[kLfWaves];
    const int c = blockIdx.x, bh = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hh = lane >> 5;
    const f16 * K = kt + (int64_t)bh * 32 * N;
    const f16 * V = vt + (int64_t)bh * 32 * N;
    const int cb = c * T, ce = min(N, cb + T);
    const int span = ((ce - cb + kLfWaves - 1) / kLfWaves + 15) / 16 * 16;
    const int tb = min(ce, cb + w * span), te = min(ce, tb + span);
    f32x16 sacc, ks;
#pragma unroll
    for (int i = 0; i < 16; ++i) sacc[i] = ks[i] = 0.0f;
    f16x8 ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = (f16)1.0f;
    const f16 * krow = K + (int64_t)(lane & 31) * N + 8 * hh;
    const f16 * vrow = V + (int64_t)(lane & 31) * N + 8 * hh;
    constexpr int kG = 8;
    for (int g0 = tb; g0 < te; g0 += 16 * kG) {
        f16x8 ka[kG], va[kG];
#pragma unroll
        for (int u = 0; u < kG; ++u) {
            const int t = g0 + 16 * u;
            if (t < te) {
                ka[u] = *reinterpret_cast<const f16x8 *>(krow + t);
                va[u] = *reinterpret_cast<const f16x8 *>(vrow + t);
            }
        }
#pragma unroll
        for (int u = 0; u < kG; ++u) {
            if (g0 + 16 * u < te) {
                sacc = mfma_32x32x16(ka[u], va[u], sacc);
                ks = mfma_32x32x16(ka[u], ones, ks);
            }
        }
    }
    // lane holds column r = lane & 31 and rows d = 8*(i/4) + 4*hh + i%4
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int d = 8 * (i >> 2) + 4 * hh + (i & 3);
        sp[w][d][lane & 31] = sacc[i];
        if ((lane & 31) == 0) sp[w][32][d] = ks[i];
    }
    __syncthreads();
    float * out = part + ((int64_t)bh * nch + c) * (33 * 32);
    float m = 0.0f;
    for (int e = tid; e < 33 * 32; e += 64 * kLfWaves) {
        const int r = e >> 5, d = e & 31;
        float a = 0.0f;
        if (r < 32) {
            for (int ww = 0; ww < kLfWaves; ++ww) a += sp[ww][d][r];
        } else {
            for (int ww = 0; ww < kLfWaves; ++ww) a += sp[ww][32][d];
        }
        out[e] = a;
        m = fmaxf(m, fabsf(a));
    }
    m = wave_max(m);
    if (lane == 0) wmax[w] = m;
    __syncthreads();
    if (tid == 0) {
        float mm = 0.0f;
        for (int ww = 0; ww < kLfWaves; ++ww) mm = fmaxf(mm, wmax[ww]);
        pmax[(int64_t)bh * nch + c] = mm;
    }
}

// la_apply32_kernel: the apply step of the chunked path for head_dim 32 as
// la_fused_kernel's step 3: O^T[r][t] = [S | ksum] . relu(q)^T with the
// reduced hi/lo state (la_reduce_kernel's [64][32] layout: rows 0..31 S,
// row 32 ksum) as the A operand, so each lane holds four consecutive head dims
// of one token and 32-token blocks leave through LDS as 64-byte token rows.
// Workgroup: 8 waves over `span` tokens of one (b, h), 64 tokens per step.
__global__ __launch_bounds__(64 * kLfWaves) void la_apply32_kernel(const f16 * __restrict__ q, int64_t ldq,
                                                                   const f16 * __restrict__ shi,
                                                                   const f16 * __restrict__ slo,
                                                                   const float * __restrict__ pmax, int nch,
                                                                   f16 * __restrict__ out, int64_t ldo, int N,
                                                                   int H, int span) {
    __shared__ __attribute__((aligned(16))) f16 ost[kLfWaves][32][32];
    const int bh = blockIdx.y, b = bh / H, h = bh - b * H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hh = lane >> 5;
    const int wspan = span / kLfWaves;  // a multiple of 64
    const int ta = min(N, blockIdx.x * span + w * wspan), tz = min(N, ta + wspan);
    const float eps = ldexpf(1e-15f, la_state_exponent(la_bound(pmax + (int64_t)bh * nch, nch)));
    constexpr int KP = 32;
    const int64_t sb = (int64_t)bh * 64 * KP + (lane & 31) * KP + 8 * hh;
    f16x8 sa[2][2][2];  // [tile][hi|lo][k-step]
#pragma unroll
    for (int tile = 0; tile < 2; ++tile)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            sa[tile][0][kk] = *reinterpret_cast<const f16x8 *>(shi + sb + tile * 32 * KP + kk * 16);
            sa[tile][1][kk] = *reinterpret_cast<const f16x8 *>(slo + sb + tile * 32 * KP + kk * 16);
        }
    const f16 * qbase = q + (int64_t)b * N * ldq + (int64_t)h * 32 + 8 * hh;
    auto load_q = [&](int t0, f16x8 (&qf)[2]) {
        const int tq = min(t0 + (lane & 31), N - 1);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            qf[kk] = *reinterpret_cast<const f16x8 *>(qbase + (int64_t)tq * ldq + kk * 16);
#pragma unroll
            for (int e = 0; e < 8; ++e) qf[kk][e] = qf[kk][e] > (f16)0.0f ? qf[kk][e] : (f16)0.0f;
        }
    };
    auto apply_store = [&](int t0, const f32x16 & o, const f32x16 & dn) {
        const float rden = 1.0f / (__shfl(dn[0], lane & 31, 64) + eps);
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
            f16x4 v4;
#pragma unroll
            for (int u = 0; u < 4; ++u) v4[u] = (f16)(o[4 * i4 + u] * rden);
            *reinterpret_cast<f16x4 *>(&ost[w][lane & 31][8 * la_ost_chunk(lane & 31, i4) + 4 * hh]) = v4;
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int tl = half * 16 + (lane >> 2), c8 = (lane & 3) * 8;
            const f16x8 v8 = *reinterpret_cast<const f16x8 *>(&ost[w][tl][8 * la_ost_chunk(tl, lane & 3)]);
            const int t = t0 + tl;
            if (t < tz) *reinterpret_cast<f16x8 *>(out + ((int64_t)b * N + t) * ldo + (int64_t)h * 32 + c8) = v8;
        }
        __builtin_amdgcn_wave_barrier();
    };
    f16x8 qa[2], qb[2];
    if (ta < tz) {
        load_q(ta, qa);
        load_q(ta + 32, qb);
    }
    for (int t0 = ta; t0 < tz; t0 += 64) {
        f32x16 oa, da, ob, db;
#pragma unroll
        for (int i = 0; i < 16; ++i) oa[i] = da[i] = ob[i] = db[i] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int hl = 0; hl < 2; ++hl) {
                oa = mfma_32x32x16(sa[0][hl][kk], qa[kk], oa);
                ob = mfma_32x32x16(sa[0][hl][kk], qb[kk], ob);
                da = mfma_32x32x16(sa[1][hl][kk], qa[kk], da);
                db = mfma_32x32x16(sa[1][hl][kk], qb[kk], db);
            }
        // the next step's queries are requested before this step's stores
        if (t0 + 64 < tz) {
            load_q(t0 + 64, qa);
            load_q(t0 + 96, qb);
        }
        apply_store(t0, oa, da);
        if (t0 + 32 < tz) apply_store(t0 + 32, ob, db);
    }
}

// la_reduce_apply32_kernel: la_reduce_kernel and la_apply32_kernel in one
// launch for head_dim 32.  Each workgroup first sums the nch chunk partials of
// its (b, h) in chunk order, scales them by the same 2^k and splits them into
// the same fp16 hi/lo pair as la_reduce_kernel (so the results are the same
// bits), but into LDS; then its 8 waves apply the state to `span` tokens as
// la_apply32_kernel does.  The partials (4.2 KB per chunk) come from L2 for
// every workgroup of a head, so `span` is large (2048 tokens) to keep the
// re-reads small next to the q and output bytes.
__global__ __launch_bounds__(64 * kLfWaves) void la_reduce_apply32_kernel(const f16 * __restrict__ q, int64_t ldq,
                                                                          const float * __restrict__ part,
                                                                          const float * __restrict__ pmax, int nch,
                                                                          f16 * __restrict__ out, int64_t ldo, int N,
                                                                          int H, int span) {
    constexpr int KP = 32, NP = 64, E = 33 * 32;
    __shared__ __attribute__((aligned(16))) f16 sst[2][NP * KP];  // [hi|lo][r][d]
    __shared__ __attribute__((aligned(16))) f16 ost[kLfWaves][32][32];
    // XCD-aware order: workgroup ids are dealt round-robin to the 8 XCDs, so id
    // goes to position (id % 8) * (n / 8) + id / 8 of the head-major order and
    // the token blocks of one head, which read the same partials, share an L2
    const int nb = (int)gridDim.x, nwg = nb * (int)gridDim.y, per = nwg / 8;
    const int id = (int)blockIdx.x + nb * (int)blockIdx.y;
    const int pos = id < per * 8 ? (id % 8) * per + id / 8 : id;
    const int bh = pos / nb, blk = pos - bh * nb, b = bh / H, h = bh - b * H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hh = lane >> 5;
    const int wspan = span / kLfWaves;  // a multiple of 64
    const int ta = min(N, blk * span + w * wspan), tz = min(N, ta + wspan);
    const f16 * qbase = q + (int64_t)b * N * ldq + (int64_t)h * 32 + 8 * hh;
    auto load_q = [&](int t0, f16x8 (&qf)[2]) {
        const int tq = min(t0 + (lane & 31), N - 1);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            qf[kk] = *reinterpret_cast<const f16x8 *>(qbase + (int64_t)tq * ldq + kk * 16);
#pragma unroll
            for (int e = 0; e < 8; ++e) qf[kk][e] = qf[kk][e] > (f16)0.0f ? qf[kk][e] : (f16)0.0f;
        }
    };
    // the first step's queries do not depend on the state
    f16x8 qa[2], qb[2];
    if (ta < tz) {
        load_q(ta, qa);
        load_q(ta + 32, qb);
    }
    // 1. the state, as la_reduce_kernel computes it
    const float * pmh = pmax + (int64_t)bh * nch;
    const int kexp = la_state_exponent(la_bound(pmh, nch));
    const float scale = ldexpf(1.0f, kexp), eps = ldexpf(1e-15f, kexp);
    for (int e = tid; e < NP * KP; e += 64 * kLfWaves) {
        const int r = e / KP, d = e - r * KP;
        float s = 0.0f;
        if (e < E) {  // rows 0 .. 32 (S, then ksum), d < 32
            const float * p = part + (int64_t)bh * nch * E + r * 32 + d;
            int c = 0;
            for (; c + 8 <= nch; c += 8) {
                float x[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) x[u] = p[(int64_t)(c + u) * E];
#pragma unroll
                for (int u = 0; u < 8; ++u) s += x[u];
            }
            for (; c < nch; ++c) s += p[(int64_t)c * E];
        }
        s *= scale;
        const f16 hv = (f16)s;
        sst[0][e] = hv;
        sst[1][e] = (f16)(s - (float)hv);
    }
    __syncthreads();
    // 2. apply (la_apply32_kernel's loop)
    const int sb = (lane & 31) * KP + 8 * hh;
    f16x8 sa[2][2][2];  // [tile][hi|lo][k-step]
#pragma unroll
    for (int tile = 0; tile < 2; ++tile)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            sa[tile][0][kk] = *reinterpret_cast<const f16x8 *>(&sst[0][sb + tile * 32 * KP + kk * 16]);
            sa[tile][1][kk] = *reinterpret_cast<const f16x8 *>(&sst[1][sb + tile * 32 * KP + kk * 16]);
        }
    auto apply_store = [&](int t0, const f32x16 & o, const f32x16 & dn) {
        const float rden = 1.0f / (__shfl(dn[0], lane & 31, 64) + eps);
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
            f16x4 v4;
#pragma unroll
            for (int u = 0; u < 4; ++u) v4[u] = (f16)(o[4 * i4 + u] * rden);
            *reinterpret_cast<f16x4 *>(&ost[w][lane & 31][8 * la_ost_chunk(lane & 31, i4) + 4 * hh]) = v4;
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int tl = half * 16 + (lane >> 2), c8 = (lane & 3) * 8;
            const f16x8 v8 = *reinterpret_cast<const f16x8 *>(&ost[w][tl][8 * la_ost_chunk(tl, lane & 3)]);
            const int t = t0 + tl;
            if (t < tz) *reinterpret_cast<f16x8 *>(out + ((int64_t)b * N + t) * ldo + (int64_t)h * 32 + c8) = v8;
        }
        __builtin_amdgcn_wave_barrier();
    };
    for (int t0 = ta; t0 < tz; t0 += 64) {
        f32x16 oa, da, ob, db;
#pragma unroll
        for (int i = 0; i < 16; ++i) oa[i] = da[i] = ob[i] = db[i] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int hl = 0; hl < 2; ++hl) {
                oa = mfma_32x32x16(sa[0][hl][kk], qa[kk], oa);
                ob = mfma_32x32x16(sa[0][hl][kk], qb[kk], ob);
                da = mfma_32x32x16(sa[1][hl][kk], qa[kk], da);
                db = mfma_32x32x16(sa[1][hl][kk], qb[kk], db);
            }
        if (t0 + 64 < tz) {
            load_q(t0 + 64, qa);
            load_q(t0 + 96, qb);
        }
        apply_store(t0, oa, da);
        if (t0 + 32 < tz) apply_store(t0 + 32, ob, db);
    }
}

// la_applyT_kernel: the transposed apply of la_apply32_kernel for other head
// dims (D % 8 == 0, D + 1 <= 96): O^T[r][t] = [S | ksum] . relu(q)^T with NT
// 32-row tiles of the reduced hi/lo state as the A operand (rows 0..D-1 S,
// row D ksum) and KS 16-deep steps over d; 32 tokens per step, staged in LDS
// and stored as 16-byte pieces of the token rows.
template <int NT, int KS>
__global__ __launch_bounds__(64 * kLfWaves) void la_applyT_kernel(const f16 * __restrict__ q, int64_t ldq,
                                                                  const f16 * __restrict__ shi,
                                                                  const f16 * __restrict__ slo,
                                                                  const float * __restrict__ pmax, int nch,
                                                                  f16 * __restrict__ out, int64_t ldo, int N, int H,
                                                                  int D, int span) {
    constexpr int KP = KS * 16, NP = NT * 32, SROW = NP + 8;  // SROW: halves per staged token row
    __shared__ __attribute__((aligned(16))) f16 ost[kLfWaves][32][SROW];
    const int bh = blockIdx.y, b = bh / H, h = bh - b * H;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hh = lane >> 5;
    const int wspan = span / kLfWaves;  // a multiple of 32
    const int ta = min(N, blockIdx.x * span + w * wspan), tz = min(N, ta + wspan);
    const float eps = ldexpf(1e-15f, la_state_exponent(la_bound(pmax + (int64_t)bh * nch, nch)));
    const int64_t sb = (int64_t)bh * NP * KP + (lane & 31) * KP + 8 * hh;
    f16x8 sa[NT][2][KS];  // [tile][hi|lo][k-step]
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            sa[j][0][kk] = *reinterpret_cast<const f16x8 *>(shi + sb + j * 32 * KP + kk * 16);
            sa[j][1][kk] = *reinterpret_cast<const f16x8 *>(slo + sb + j * 32 * KP + kk * 16);
        }
    // the denominator row D: tile D / 32, element (D % 32) of the lane layout
    const int jd = D >> 5, rd = D & 31;
    const int id = 4 * (rd >> 3) + (rd & 3), hd = (rd >> 2) & 1;
    const f16 * qbase = q + (int64_t)b * N * ldq + (int64_t)h * D + 8 * hh;
    const int G = D / 8;  // 16-byte pieces per token row
    f16x8 qf[KS];
    auto load_q = [&](int t0) {
        const int tq = min(t0 + (lane & 31), N - 1);
#pragma unroll
        for (int kk = 0; kk < KS; ++kk) {
            if (kk * 16 + 8 * hh < D) {
                qf[kk] = *reinterpret_cast<const f16x8 *>(qbase + (int64_t)tq * ldq + kk * 16);
#pragma unroll
                for (int e = 0; e < 8; ++e) qf[kk][e] = qf[kk][e] > (f16)0.0f ? qf[kk][e] : (f16)0.0f;
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) qf[kk][e] = (f16)0.0f;
            }
        }
    };
    if (ta < tz) load_q(ta);
    for (int t0 = ta; t0 < tz; t0 += 32) {
        f32x16 o[NT];
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int i = 0; i < 16; ++i) o[j][i] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < KS; ++kk)
#pragma unroll
            for (int hl = 0; hl < 2; ++hl)
#pragma unroll
                for (int j = 0; j < NT; ++j) o[j] = mfma_32x32x16(sa[j][hl][kk], qf[kk], o[j]);
        // the next step's queries are requested before this step's stores
        if (t0 + 32 < tz) load_q(t0 + 32);
        float dv = 0.0f;
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int i = 0; i < 16; ++i)
                if (j == jd && i == id) dv = o[j][i];
        const float rden = 1.0f / (__shfl(dv, (lane & 31) | (hd << 5), 64) + eps);
        // lane: token lane & 31, rows 32 j + 8 i4 + 4 hh + {0..3}
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                f16x4 v4;
#pragma unroll
                for (int u = 0; u < 4; ++u) v4[u] = (f16)(o[j][4 * i4 + u] * rden);
                *reinterpret_cast<f16x4 *>(&ost[w][lane & 31][32 * j + 8 * i4 + 4 * hh]) = v4;
            }
        __builtin_amdgcn_wave_barrier();
        for (int it = lane; it < 32 * G; it += 64) {
            const int tl = it / G, g = it - (it / G) * G;
            const int t = t0 + tl;
            if (t < tz)
                *reinterpret_cast<f16x8 *>(out + ((int64_t)b * N + t) * ldo + (int64_t)h * D + 8 * g) =
                    *reinterpret_cast<const f16x8 *>(&ost[w][tl][8 * g]);
        }
        __builtin_amdgcn_wave_barrier();
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

// Fast path of K4 for L <= 32 * LT (<= 320 keys), D <= 96, D % 8 == 0.
//
// One workgroup of 8 waves per (head, 128 queries, batch row).  The grid is
// head-major (blockIdx.x = head): consecutive workgroup ids go to different
// XCDs, so each XCD's L2 holds the K/V of H/8 heads instead of all of them.
//
// The head's K [keys][dims] and V^T [dims][keys] (XaCfg layouts) are staged in LDS once and
// shared by the 8 waves; wave w takes query group w & 3 (32 queries) and key
// half w >> 2.  Scores are computed transposed, S^T = K . Q^T on
// v_mfma_f32_32x32x16_f16, so each lane holds one query column and the
// softmax max is in-lane plus one cross-half shuffle.  exp(S^T) in fp16 feeds
// O^T = V^T . P^T straight from registers as the B operand: in each 16-key
// step lane half hh holds keys 4hh..4hh+3 and 8+4hh..8+4hh+3 (the rows the
// score MFMA leaves in it), and V^T is staged with its keys permuted the same
// way inside every 16-key group, so the A operand is one 16-byte LDS read.
// When D is not a multiple of 32, the last staged V^T row (a padding row of
// the last 32-dim tile) holds 1 for every key < L, so the same MFMA also
// produces the softmax denominator sum_k p_k.  The two key halves' (max, O^T) are merged
// through LDS: O = O_0 2^(m_0 - m) + O_1 2^(m_1 - m), m = max(m_0, m_1).
//
// With FLASH (long sequences) each wave instead takes 32 queries of each of
// `qblocks` 256-query blocks in turn and both key halves itself, with a
// running max (online softmax), so one staging of the head serves many queries
// and no merge is needed.
//
// Staging issues every 16-byte load (Q, K, V^T) up front, unconditionally and
// in bounds (clamped rows and chunks, masked afterwards with dword ANDs), with
// a power-of-two thread -> (row, chunk) map.  Measured slower: writing V^T to
// LDS only after the softmax (+0.5 us), and a dense map that loads only the
// head's own chunks with every lane busy (+0.5 us, though 40 % fewer bytes).
// Without a key bias and with the ones row, the softmax takes the max
// of the raw scores and needs no bias add: keys past L repeat key L - 1 and
// meet zeroed V^T columns and ones-row entries.
constexpr int kXaQ = 128;  // queries per workgroup
constexpr float kLog2e = 1.4426950408889634f;

// Two LDS layouts of the staged head, both free of bank conflicts for the
// 16-lane fragment reads (16 consecutive rows at one 16-byte chunk) and for
// the staging writes:
//  * padded (PACK false): K [LP][KS * 16 + 8] and V^T [DP][LP + 8] halves;
//  * packed (PACK true):  K as 2 KS chunk planes of [LP][8] halves with row r
//    of plane c in slot r ^ c (a staging write covers one row's chunks, which
//    then land in distinct bank groups; a fragment read covers 16 rows of one
//    plane, a permutation of 16 consecutive slots), and V^T [DP][LP] with
//    chunk c of row r in slot c ^ (r & 15) when a row has a multiple of 16
//    chunks, else c ^ ((r >> 1) & 7) (the row stride is then 8 chunks mod 16,
//    so row parity picks the half of the 64 banks).
// gfx950 allocates LDS per workgroup in 1280-byte granules (128 of them per
// CU): a 64 x 64 GEMM workgroup's 49152 bytes take 39, leaving 89 = 113920
// bytes.  The packed head of 300 keys x 72 dims is exactly that (the padded
// one 120576), so the key-split path's workgroups share CUs with the other CFG
// branch's 64 x 64 GEMM workgroups: 1024 px forward 5.234 -> 5.047 ms in one
// process, while a 114080-byte variant (16-byte gaps between the K planes)
// gained only 0.03 ms.  The online-softmax path keeps the padded layout: its
// loop re-reads K and V^T for every query block, and the per-lane swizzle
// there costs VALU work that path has no room for (40.7 -> 73.5 us per
// 16384-token launch with it), and its 16384-row GEMM neighbours take 64-80 KB.
template <int LT, int KS, bool PACK = false>
struct XaCfg {
    static constexpr int LP = LT * 32;              // keys, padded to the score tile
    static constexpr int KROW = KS * 16 + 8;        // halves per padded K row (72, 88, 104: conflict-free reads)
    static constexpr int KCH = KS * 2;              // 16-byte chunks per K row (< 16)
    static constexpr int DT = (KS * 16 + 31) / 32;  // 32-wide output dim tiles
    static constexpr int DP = DT * 32;              // staged V^T rows
    static constexpr int VROW = PACK ? LP : LP + 8; // halves per staged V^T row
    static constexpr bool V16 = (LP / 8) % 16 == 0;
    static_assert(!PACK || (LP / 8) % 8 == 0, "V^T swizzle permutes aligned groups of 8 chunks");
    // V^T slot swizzle of row r (depends on r's low five bits only)
    static SANA_DEV int vx(int r) { return PACK ? (V16 ? (r & 15) : ((r >> 1) & 7)) : 0; }
    // offsets in halves of chunk c of K row r and of V^T row r
    // (packed: k_at(r0 + r, c) = k_at(r, c) + 8 r0 for r0 a multiple of 32)
    static SANA_DEV int k_at(int r, int c) { return PACK ? (c * LP + (r ^ c)) * 8 : r * KROW + c * 8; }
    static SANA_DEV int v_at(int r, int c) { return r * VROW + (c ^ vx(r)) * 8; }
    static constexpr int K_BYTES = (PACK ? KCH * LP * 8 : LP * KROW) * 2;
    static_assert(!PACK || (KCH <= 16 && LP % 16 == 0), "K row swizzle stays inside a 16-row group");
    static constexpr int V_BYTES = DP * VROW * 2;
    static constexpr int MERGE_BYTES = 4 * (DT * 16 + 2) * 64 * 4;
    static constexpr int STAGE_BYTES = K_BYTES + V_BYTES + LP * 4;
    static constexpr int LDS_BYTES = STAGE_BYTES > MERGE_BYTES ? STAGE_BYTES : MERGE_BYTES;
};

template <int LT, int KS, bool ONES, bool FLASH>
__global__ __launch_bounds__(512) void xattn_lds_kernel(const f16 * __restrict__ q, int64_t ldq,
                                                        const f16 * __restrict__ k, int64_t ldk,
                                                        const f16 * __restrict__ vt, int64_t ldvt,
                                                        const float * __restrict__ bias, f16 * __restrict__ out,
                                                        int64_t ldo, int N, int L, int D, float scale, int qblocks) {
    using X = XaCfg<LT, KS, !FLASH>;
    static_assert(LT % 2 == 0, "key tiles split in two halves");
    static_assert(X::DP <= 128 && X::LP / 8 <= 64, "staging map");
    constexpr int LTH = LT / 2;
    constexpr int LP = X::LP, DT = X::DT, DP = X::DP;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    f16 * Ks = reinterpret_cast<f16 *>(smem);                          // K, X::k_at
    f16 * Vs = reinterpret_cast<f16 *>(smem + X::K_BYTES);             // V^T, keys permuted, X::v_at
    float * bs = reinterpret_cast<float *>(smem + X::K_BYTES + X::V_BYTES);  // [LP] log2-scaled bias, -inf past L
    // (head, query block) from an XCD-aware order: workgroups are dealt
    // round-robin to the 8 XCDs, so id goes to position (id % 8) * (n / 8) +
    // id / 8 of the head-major order and each XCD runs a contiguous range of
    // heads -- the query blocks of a head share its staged K / V in one L2, and
    // neighbouring heads, whose query and output rows share 128-byte lines
    // (head_dim 72 is not a multiple of 64), mostly share it too
    const int H = gridDim.x, b = blockIdx.z;
    const int nwg = H * (int)gridDim.y, per = nwg / 8, id = (int)blockIdx.x + H * (int)blockIdx.y;
    const int pos = id < per * 8 ? (id % 8) * per + id / 8 : id;
    const int h = pos / (int)gridDim.y, qy = pos - h * (int)gridDim.y;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = w & 3, kh = w >> 2;
    const int hh = lane >> 5;
    constexpr bool ones_row = ONES;  // D < DP: the last V^T row carries the denominator

    // query fragments (B operand of the score MFMA): query (lane & 31), dims 16 ks + 8 hh ..
    f16x8 qf[KS];
    auto load_q = [&](int q0) {
        const int qcol = min(q0 + (lane & 31), N - 1);
        const f16 * qr = q + ((int64_t)b * N + qcol) * ldq + (int64_t)h * D;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int d0 = ks * 16 + 8 * hh;
            const f16x8 v = *reinterpret_cast<const f16x8 *>(qr + min(d0, D - 8));
            uint32_t w[4];
            __builtin_memcpy(w, &v, 16);
            const uint32_t m = d0 < D ? 0xffffffffu : 0u;  // dims past D are zero
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] &= m;
            __builtin_memcpy(&qf[ks], w, 16);
        }
    };
    const int q0 = qy * kXaQ + g * 32;  // key-split path: this wave's query group
    // this wave's first query block (online-softmax path: of the first 256-query block)
    const int qw0 = FLASH ? (qy * qblocks * 8 + w) * 32 : q0;
    load_q(qw0);  // in flight during the K/V staging (rows clamped into range)

    // K staging: thread -> chunk kc = tid & 15 (8 dims), rows kr0 + 32 j.  Every
    // load is in bounds and unconditional: rows past L repeat row L - 1 and
    // chunks past D repeat the head's last chunk, so every staged value is real
    // (finite) data.  A repeated key scores like key L - 1 (the max is
    // unchanged) and its V^T column and ones-row entries are staged as zeros,
    // so it adds nothing to O or to the denominator; dims past D meet zero
    // query dims.
    const int kc = tid & 15, kr0 = tid >> 4;
    const bool kc_live = kc < KS * 2;  // chunks 0 .. 2 KS - 1 are staged
    const f16 * kp = k + (int64_t)b * L * ldk + (int64_t)h * D + min(kc, (D - 1) >> 3) * 8;
    f16x8 kreg[LT];
#pragma unroll
    for (int j = 0; j < LT; ++j)
        kreg[j] = *reinterpret_cast<const f16x8 *>(kp + (int64_t)min(kr0 + 32 * j, L - 1) * ldk);
    // V^T staging: thread -> 8-key chunk vc = tid & 63, dims vd0 + 8 j (vd0 = the
    // wave index).  Chunks past L repeat the last chunk and dims past D repeat
    // dim D - 1 (output dims past D are never stored); keys past L are then
    // zeroed with per-dword masks.
    constexpr int VJ = DP / 8;
    const int vc = tid & 63;
    const int vd0 = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool vc_live = vc < LP / 8;
    const f16 * vp = vt + ((int64_t)b * H * D + (int64_t)h * D) * ldvt + min(vc, (L - 1) >> 3) * 8;
    f16x8 vreg[VJ];
#pragma unroll
    for (int j = 0; j < VJ; ++j)
        vreg[j] = *reinterpret_cast<const f16x8 *>(vp + (int64_t)min(vd0 + 8 * j, D - 1) * ldvt);
    uint32_t km[4];  // keys 8 vc + 2 e and 8 vc + 2 e + 1 below L
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int k0 = vc * 8 + 2 * e;
        km[e] = k0 + 1 < L ? 0xffffffffu : (k0 < L ? 0x0000ffffu : 0u);
    }
    // log2-scaled key bias; keys past L repeat key L - 1's, or are -inf where no
    // ones row masks the denominator (D a multiple of 32)
    for (int key = tid; key < LP; key += 512) {
        const int kb = min(key, L - 1);
        const float bv = bias ? bias[(int64_t)b * L + kb] * kLog2e : 0.0f;
        bs[key] = (ONES || key < L) ? bv : -INFINITY;
    }
    if (kc_live) {
#pragma unroll
        for (int j = 0; j < LT; ++j)
            *reinterpret_cast<f16x8 *>(Ks + X::k_at(kr0 + 32 * j, kc)) = kreg[j];
    }
    if (vc_live) {
        // keys 8 vc .. 8 vc + 7: the first four go to positions 16 (vc >> 1) + 4 (vc & 1),
        // the last four 8 positions further
        const int pos = 16 * (vc >> 1) + 4 * (vc & 1);
#pragma unroll
        for (int j = 0; j < VJ; ++j) {
            const int d = vd0 + 8 * j;
            uint32_t w[4];
            __builtin_memcpy(w, &vreg[j], 16);
            if (ONES && j == VJ - 1 && vd0 == 7) {  // d == DP - 1: the ones row
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = 0x3c003c00u;
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] &= km[e];
            if constexpr (!FLASH) {
                // positions pos and pos + 8: offset pos & 7 of chunks pos >> 3 and (pos >> 3) + 1
                *reinterpret_cast<uint2 *>(Vs + X::v_at(d, pos >> 3) + (pos & 7)) = make_uint2(w[0], w[1]);
                *reinterpret_cast<uint2 *>(Vs + X::v_at(d, (pos >> 3) + 1) + (pos & 7)) = make_uint2(w[2], w[3]);
            } else {
                *reinterpret_cast<uint2 *>(Vs + d * X::VROW + pos) = make_uint2(w[0], w[1]);
                *reinterpret_cast<uint2 *>(Vs + d * X::VROW + pos + 8) = make_uint2(w[2], w[3]);
            }
        }
    }
    __syncthreads();

    if constexpr (FLASH) {
        // Long sequences: the staged head serves `qblocks` blocks of 256 queries.
        // Each wave takes 32 queries per block and both key halves in turn with
        // a running max (online softmax), so no cross-wave merge is needed and
        // the waves never synchronise after the staging.
        const float scale2 = scale * kLog2e;
        for (int qb = 0; qb < qblocks; ++qb) {
            const int qw = ((qy * qblocks + qb) * 8 + w) * 32;
            if (qw >= N) break;
            // qf holds this block's queries: requested before the staging for
            // the first block, during the previous block's softmax otherwise
            const int qn = qw + 8 * 32;  // this wave's queries in the next 256-query block
            const bool next = qb + 1 < qblocks && qn < N;
            f32x16 o[DT];
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) o[dt][i] = 0.0f;
            float m = -INFINITY, sum = 0.0f;
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int tb = half * LTH;
                f32x16 st[LTH];
#pragma unroll
                for (int t = 0; t < LTH; ++t)
#pragma unroll
                    for (int i = 0; i < 16; ++i) st[t][i] = 0.0f;
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const int d0 = ks * 16 + 8 * hh;
#pragma unroll
                    for (int t = 0; t < LTH; ++t) {
                        const f16x8 kf =
                            *reinterpret_cast<const f16x8 *>(Ks + ((tb + t) * 32 + (lane & 31)) * X::KROW + d0);
                        st[t] = mfma_32x32x16(kf, qf[ks], st[t]);
                    }
                }
                // the second half's scores are the last use of qf: the next
                // block's queries load into it behind this block's softmax and P.V
                if (half == 1 && next) load_q(qn);
                float mh = -INFINITY;
                const bool raw = ONES && !bias;
                if (raw) {
#pragma unroll
                    for (int t = 0; t < LTH; ++t)
#pragma unroll
                        for (int i = 0; i < 16; ++i) mh = fmaxf(mh, st[t][i]);
                    mh = fmaxf(mh, __shfl_xor(mh, 32, 64)) * scale2;
                } else {
#pragma unroll
                    for (int t = 0; t < LTH; ++t)
#pragma unroll
                        for (int i4 = 0; i4 < 4; ++i4) {
                            const f32x4 b4 = *reinterpret_cast<const f32x4 *>(bs + (tb + t) * 32 + 8 * i4 + 4 * hh);
#pragma unroll
                            for (int u = 0; u < 4; ++u) {
                                const float sv = st[t][4 * i4 + u] * scale2 + b4[u];
                                st[t][4 * i4 + u] = sv;
                                mh = fmaxf(mh, sv);
                            }
                        }
                    mh = fmaxf(mh, __shfl_xor(mh, 32, 64));
                }
                const float mn = fmaxf(m, mh);
                // all keys so far at -inf: keep their probabilities at exp2(-inf) = 0
                const float mref = mn == -INFINITY ? 0.0f : mn;
                if (half == 1) {
                    const float a = __builtin_amdgcn_exp2f(m - mref);
#pragma unroll
                    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                        for (int i = 0; i < 16; ++i) o[dt][i] *= a;
                    sum *= a;
                }
                f16x8 pf[LTH][2];
                // one fma per score on both paths: raw scores are scaled here,
                // biased ones were scaled above and fma(s, 1, -m) rounds as s - m
                // (a per-score select between the two forms costs a v_sub and a
                // v_cndmask per score once the compiler if-converts it)
                const float esc = raw ? scale2 : 1.0f;
#pragma unroll
                for (int t = 0; t < LTH; ++t)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const float e = __builtin_amdgcn_exp2f(fmaf(st[t][i], esc, -mref));
                        if constexpr (!ones_row) sum += e;
                        pf[t][i >> 3][i & 7] = (f16)e;
                    }
#pragma unroll
                for (int t = 0; t < LTH; ++t)
#pragma unroll
                    for (int s2 = 0; s2 < 2; ++s2) {
                        const int kpos = (tb + t) * 32 + 16 * s2 + 8 * hh;
#pragma unroll
                        for (int dt = 0; dt < DT; ++dt) {
                            const f16x8 af =
                                *reinterpret_cast<const f16x8 *>(Vs + (dt * 32 + (lane & 31)) * X::VROW + kpos);
                            o[dt] = mfma_32x32x16(af, pf[t][s2], o[dt]);
                        }
                    }
                m = mn;
            }
            float den;
            if constexpr (ones_row) {
                den = __shfl(o[DT - 1][15], (lane & 31) + 32, 64);
            } else {
                den = sum + __shfl_xor(sum, 32, 64);
            }
            const float rs = 1.0f / den;
            const int qq = qw + (lane & 31);
            if (qq < N) {
                f16 * orow = out + ((int64_t)b * N + qq) * ldo + (int64_t)h * D;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                    for (int i4 = 0; i4 < 4; ++i4) {
                        const int dim = dt * 32 + 8 * i4 + 4 * hh;
                        if (dim < D) {
                            f16x4 v4;
#pragma unroll
                            for (int u = 0; u < 4; ++u) v4[u] = (f16)(o[dt][4 * i4 + u] * rs);
                            *reinterpret_cast<f16x4 *>(orow + dim) = v4;
                        }
                    }
            }
        }
        return;
    }

    // scores of this wave's key half: tile t is global key tile kh * LTH + t
    const int tb = kh * LTH;
    f32x16 st[LTH];
#pragma unroll
    for (int t = 0; t < LTH; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) st[t][i] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        // chunk 2 ks + hh of row lane & 31; tile tb + t adds (tb + t) * 32 rows
        const int kof = X::k_at(lane & 31, 2 * ks + hh);
#pragma unroll
        for (int t = 0; t < LTH; ++t) {
            const f16x8 kf = *reinterpret_cast<const f16x8 *>(Ks + kof + (tb + t) * 32 * 8);
            st[t] = mfma_32x32x16(kf, qf[ks], st[t]);
        }
    }
    const float scale2 = scale * kLog2e;
    float mx = -INFINITY;
    f16x8 pf[LTH][2];
    float sum = 0.0f;
    if (ONES && !bias) {
        // no bias to add: the max of the raw scores, then 2^(s scale2 - max scale2)
#pragma unroll
        for (int t = 0; t < LTH; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, st[t][i]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * scale2;
#pragma unroll
        for (int t = 0; t < LTH; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) pf[t][i >> 3][i & 7] = (f16)__builtin_amdgcn_exp2f(fmaf(st[t][i], scale2, -mx));
    } else {
#pragma unroll
        for (int t = 0; t < LTH; ++t)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const f32x4 b4 = *reinterpret_cast<const f32x4 *>(bs + (tb + t) * 32 + 8 * i4 + 4 * hh);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const float sv = st[t][4 * i4 + u] * scale2 + b4[u];
                    st[t][4 * i4 + u] = sv;
                    mx = fmaxf(mx, sv);
                }
            }
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        // a half whose keys are all -inf has mx = -inf: its probabilities are exp2(-inf) = 0
        const float mref = mx == -INFINITY ? 0.0f : mx;
#pragma unroll
        for (int t = 0; t < LTH; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float e = __builtin_amdgcn_exp2f(st[t][i] - mref);
                if constexpr (!ones_row) sum += e;
                pf[t][i >> 3][i & 7] = (f16)e;
            }
    }

    f32x16 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] = 0.0f;
    // this lane's V^T fragment offsets (row lane & 31 of the first dim tile);
    // row dt * 32 + r swizzles as row r, so tile dt adds dt * 32 rows
    int vof[LTH][2];
#pragma unroll
    for (int t = 0; t < LTH; ++t)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) vof[t][s2] = X::v_at(lane & 31, ((tb + t) * 32 + 16 * s2 + 8 * hh) >> 3);
#pragma unroll
    for (int t = 0; t < LTH; ++t)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const f16x8 af = *reinterpret_cast<const f16x8 *>(Vs + dt * 32 * X::VROW + vof[t][s2]);
                o[dt] = mfma_32x32x16(af, pf[t][s2], o[dt]);
            }
        }
    // denominator of this half: the last row (31) of the last O^T tile, held by
    // the upper lane half in register 15 -- or the in-lane sum
    if constexpr (ones_row) {
        sum = __shfl(o[DT - 1][15], (lane & 31) + 32, 64);
    } else {
        sum += __shfl_xor(sum, 32, 64);
    }

    // merge the two key halves through LDS (the staged K/V are no longer read)
    __syncthreads();
    constexpr int NV = DT * 16 + 2;
    float * part = reinterpret_cast<float *>(smem) + g * NV * 64 + lane;  // [g][NV values][64 lanes]
    if (kh == 1) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i = 0; i < 16; ++i) part[(dt * 16 + i) * 64] = o[dt][i];
        part[DT * 16 * 64] = mx;
        part[(DT * 16 + 1) * 64] = sum;
    }
    __syncthreads();
    if (kh == 1) return;
    const float m1 = part[DT * 16 * 64], l1 = part[(DT * 16 + 1) * 64];
    const float m = fmaxf(mx, m1);
    const float a0 = __builtin_amdgcn_exp2f(mx - m), a1 = __builtin_amdgcn_exp2f(m1 - m);
    const float rs = 1.0f / (sum * a0 + l1 * a1);
    const float c0 = a0 * rs, c1 = a1 * rs;

    const int qq = q0 + (lane & 31);
    if (qq < N) {
        f16 * orow = out + ((int64_t)b * N + qq) * ldo + (int64_t)h * D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const int dim = dt * 32 + 8 * i4 + 4 * hh;
                if (dim < D) {
                    f16x4 v4;
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int i = 4 * i4 + u;
                        v4[u] = (f16)(o[dt][i] * c0 + part[(dt * 16 + i) * 64] * c1);
                    }
                    *reinterpret_cast<f16x4 *>(orow + dim) = v4;
                }
            }
    }
}

// Queries per image from which one staging of a head serves several 256-query
// blocks (the online-softmax path of xattn_lds_kernel, for 320 staged keys).
// Measured per 300-key, 16 x 72-head launch: 14.3 against 18.6 us at 4096
// queries, 40.5 against 68.8 us at 16384; at 1024 the key-split path's
// 128-query workgroups win (9.4 against 12.0 us).
constexpr int kXaFlashTokens = 4096;

template <int LT, int KS, bool ONES, bool FLASH>
hipError_t launch_xattn_lds2(const f16 * q, int64_t ldq, const f16 * k, int64_t ldk, const f16 * vt, int64_t ldvt,
                             const float * bias, f16 * out, int64_t ldo, int B, int N, int L, int H, int D,
                             float scale, hipStream_t s) {
    using X = XaCfg<LT, KS, !FLASH>;
    static const bool attr =
        hipFuncSetAttribute(reinterpret_cast<const void *>(&xattn_lds_kernel<LT, KS, ONES, FLASH>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, X::LDS_BYTES) == hipSuccess;
    (void)attr;
    static const std::string name = "xattn_lds_kernel<" + std::to_string(LT) + ", " + std::to_string(KS) + ", " +
                                    (ONES ? "true" : "false") + (FLASH ? ", true>" : ", false>");
    note_kernel(name.c_str());
    dim3 grid(H, (N + kXaQ - 1) / kXaQ, B);
    int qblocks = 1;
    if (FLASH) {
        // blocks of 256 queries per workgroup: about 256 workgroups in all
        const int64_t nqb = (N + 255) / 256;
        qblocks = (int)std::max<int64_t>(1, nqb * H * B / 256);
        grid.y = (unsigned)((nqb + qblocks - 1) / qblocks);
    }
    hipLaunchKernelGGL((xattn_lds_kernel<LT, KS, ONES, FLASH>), grid, dim3(512), X::LDS_BYTES, s, q, ldq, k, ldk, vt,
                       ldvt, bias, out, ldo, N, L, D, scale, qblocks);
    return hipGetLastError();
}

template <int LT, int KS, bool ONES>
hipError_t launch_xattn_lds1(const f16 * q, int64_t ldq, const f16 * k, int64_t ldk, const f16 * vt, int64_t ldvt,
                             const float * bias, f16 * out, int64_t ldo, int B, int N, int L, int H, int D,
                             float scale, hipStream_t s) {
    if constexpr (LT == 10) {
        if (N >= kXaFlashTokens)
            return launch_xattn_lds2<LT, KS, ONES, true>(q, ldq, k, ldk, vt, ldvt, bias, out, ldo, B, N, L, H, D,
                                                         scale, s);
    }
    return launch_xattn_lds2<LT, KS, ONES, false>(q, ldq, k, ldk, vt, ldvt, bias, out, ldo, B, N, L, H, D, scale, s);
}

template <int LT, int KS>
hipError_t launch_xattn_lds(const f16 * q, int64_t ldq, const f16 * k, int64_t ldk, const f16 * vt, int64_t ldvt,
                            const float * bias, f16 * out, int64_t ldo, int B, int N, int L, int H, int D,
                            float scale, hipStream_t s) {
    if (D < XaCfg<LT, KS>::DP)
        return launch_xattn_lds1<LT, KS, true>(q, ldq, k, ldk, vt, ldvt, bias, out, ldo, B, N, L, H, D, scale, s);
    return launch_xattn_lds1<LT, KS, false>(q, ldq, k, ldk, vt, ldvt, bias, out, ldo, B, N, L, H, D, scale, s);
}

template <int LT>
hipError_t launch_xattn_lds_d(const f16 * q, int64_t ldq, const f16 * k, int64_t ldk, const f16 * vt, int64_t ldvt,
                              const float * bias, f16 * out, int64_t ldo, int B, int N, int L, int H, int D,
                              float scale, hipStream_t s) {
    switch ((D + 15) / 16) {
        case 1:
        case 2: return launch_xattn_lds<LT, 2>(q, ldq, k, ldk, vt, ldvt, bias, out, ldo, B, N, L, H, D, scale, s);
        case 3:
        case 4: return launch_xattn_lds<LT, 4>(q, ldq, k, ldk, vt, ldvt, bias, out, ldo, B, N, L, H, D, scale, s);
        case 5: return launch_xattn_lds<LT, 5>(q, ldq, k, ldk, vt, ldvt, bias, out, ldo, B, N, L, H, D, scale, s);
        default: return launch_xattn_lds<LT, 6>(q, ldq, k, ldk, vt, ldvt, bias, out, ldo, B, N, L, H, D, scale, s);
    }
}

template <int LT>
hipError_t launch_xattn(const f16 * q, int64_t ldq, const f16 * k, int64_t ldk, const f16 * vt, int64_t ldvt,
                        const float * bias, f16 * out, int64_t ldo, int B, int N, int L, int H, int D, float scale,
                        int vec, hipStream_t s) {
    static const std::string name = "xattn_kernel<" + std::to_string(LT) + ">";
    note_kernel(name.c_str());
    hipLaunchKernelGGL((xattn_kernel<LT>), dim3((N + 63) / 64, H, B), dim3(256), 0, s, q, ldq, k, ldk, vt, ldvt, bias,
                       out, ldo, N, L, H, D, scale, vec);
    return hipGetLastError();
}

}  // namespace

namespace {
int la_chunk_tokens(int N) {
    // sub-chunk multiple giving at most kLaChunks partial states per (b, h)
    const int per = (N + kLaChunks - 1) / kLaChunks;
    return (per + kLaSub - 1) / kLaSub * kLaSub;
}
}  // namespace

bool linear_attention_fused_ok(int N, int D) { return D == 32 && N > 0 && N % 16 == 0; }


hipError_t linear_attention_fused(const half_t * q, int64_t ldq, const half_t * kt, const half_t * vt, half_t * out,
                                  int64_t ldo, int B, int N, int H, int D, hipStream_t s, int co) {
    if (!linear_attention_fused_ok(N, D) || B <= 0 || H <= 0 || ldq < (int64_t)H * D || ldo < (int64_t)H * D ||
        ldq % 8 || ldo % 8 || (int64_t)B * H > 65535 ||
        ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kt) | reinterpret_cast<uintptr_t>(vt)) & 15) ||
        (reinterpret_cast<uintptr_t>(out) & 15))
        return hipErrorInvalidValue;
    // enough workgroups for the 256 CUs: (b, h) pairs times token splits
    const int splits = (int)std::max<int64_t>(1, std::min<int64_t>(8, 256 / ((int64_t)B * H * std::max(co, 1))));
    note_kernel("la_fused_kernel");
    hipLaunchKernelGGL(la_fused_kernel, dim3((unsigned)(B * H * splits)), dim3(64 * kLfWaves), 0, s,
                       reinterpret_cast<const f16 *>(q), ldq, reinterpret_cast<const f16 *>(kt),
                       reinterpret_cast<const f16 *>(vt), reinterpret_cast<f16 *>(out), ldo, N, H, splits);
    return hipGetLastError();
}

hipError_t linear_attention_chunked(const half_t * q, int64_t ldq, const half_t * kt, const half_t * vt,
                                    half_t * out, int64_t ldo, int B, int N, int H, int D, float * ws, hipStream_t s) {
    if (!linear_attention_fused_ok(N, D) || B <= 0 || H <= 0 || ldq < (int64_t)H * D || ldo < (int64_t)H * D ||
        ldq % 8 || ldo % 8 || (int64_t)B * H > 65535 || !ws ||
        ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kt) | reinterpret_cast<uintptr_t>(vt) |
          reinterpret_cast<uintptr_t>(out)) & 15))
        return hipErrorInvalidValue;
    const int T = la_chunk_tokens(N);
    const int nch = (N + T - 1) / T;
    constexpr int E = 33 * 32, NP = 64, KP = 32;  // NT = 2 column tiles of [S | ksum], KS = 2 steps over d
    float * part = ws;
    f16 * shi = reinterpret_cast<f16 *>(ws + ((size_t)B * H * E * nch + 3) / 4 * 4);
    f16 * slo = shi + (size_t)B * H * NP * KP;
    float * pmax = reinterpret_cast<float *>(slo + (size_t)B * H * NP * KP);
    (void)shi;
    (void)slo;
    note_kernel("la_chunk_kernel + la_reduce_apply32_kernel");
    hipLaunchKernelGGL(la_chunk_kernel, dim3((unsigned)nch, (unsigned)(B * H)), dim3(64 * kLfWaves), 0, s,
                       reinterpret_cast<const f16 *>(kt), reinterpret_cast<const f16 *>(vt), N, T, nch, part, pmax);
    // reduce + apply: 8 waves x kRaSpan / 8 tokens per workgroup
    constexpr int kRaSpan = 2048;
    hipLaunchKernelGGL(la_reduce_apply32_kernel, dim3((unsigned)((N + kRaSpan - 1) / kRaSpan), (unsigned)(B * H)),
                       dim3(64 * kLfWaves), 0, s, reinterpret_cast<const f16 *>(q), ldq, part, pmax, nch,
                       reinterpret_cast<f16 *>(out), ldo, N, H, kRaSpan);
    return hipGetLastError();
}

size_t linattn_workspace_floats(int B, int N, int H, int D) {
    const int T = la_chunk_tokens(N);
    const size_t nch = (size_t)(N + T - 1) / T;
    const size_t E = (size_t)(D + 1) * D;
    const size_t NP = (size_t)(D + 1 + 31) / 32 * 32, KP = (size_t)(D + 15) / 16 * 16;
    // partial states (fp32, rounded up to 16 bytes) + the hi/lo fp16 state pair (counted in floats)
    // + the partials' maxima
    return ((size_t)B * H * E * nch + 3) / 4 * 4 + (size_t)B * H * NP * KP + (size_t)B * H * nch;
}

hipError_t linear_attention(const half_t * q, const half_t * k, const half_t * v, int64_t ld, half_t * out,
                            int64_t ldo, int B, int N, int H, int D, float * ws, hipStream_t s) {
    if (B <= 0 || N <= 0 || H <= 0 || D <= 0 || D > 112 || ld < (int64_t)H * D || ldo < (int64_t)H * D || !ws ||
        (int64_t)B * H > 65535)  // B * H workgroup rows of the reduction and the head_dim-32 apply
        return hipErrorInvalidValue;
    const int T = la_chunk_tokens(N);
    const int nch = (N + T - 1) / T;
    const int E = (D + 1) * D;
    const int NT = (D + 1 + 31) / 32, KS = (D + 15) / 16;
    const int NP = NT * 32, KP = KS * 16;
    float * part = ws;
    f16 * shi = reinterpret_cast<f16 *>(ws + ((size_t)B * H * E * nch + 3) / 4 * 4);
    f16 * slo = shi + (size_t)B * H * NP * KP;
    float * pmax = reinterpret_cast<float *>(slo + (size_t)B * H * NP * KP);
    const f16 * qq = reinterpret_cast<const f16 *>(q);
    const f16 * kq = reinterpret_cast<const f16 *>(k);
    const f16 * vq = reinterpret_cast<const f16 *>(v);
    const auto al16 = [](const void * p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const int vec_kv = (D % 8 == 0 && ld % 8 == 0 && al16(k) && al16(v)) ? 1 : 0;
    const int vec_q = (D % 8 == 0 && ld % 8 == 0 && al16(q)) ? 1 : 0;
    const dim3 g1(nch, H, B);
    // head_dim 32: the transposed apply with 64-byte token-row stores
    const bool apply32 = D == 32 && vec_q && ldo % 8 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
    note_kernel(apply32 ? "la_state_kernel + la_reduce_kernel + la_apply32_kernel"
                        : "la_state_kernel + la_reduce_kernel + la_apply_kernel");
    const int td = (D + 31) / 32;
    const dim3 t1(64 * kLsWaves);
    if (td == 1) hipLaunchKernelGGL((la_state_kernel<1>), g1, t1, 0, s, kq, vq, ld, N, H, D, T, nch, vec_kv, part, pmax);
    else if (td == 2) hipLaunchKernelGGL((la_state_kernel<2>), g1, t1, 0, s, kq, vq, ld, N, H, D, T, nch, vec_kv, part, pmax);
    else if (td == 3) hipLaunchKernelGGL((la_state_kernel<3>), g1, t1, 0, s, kq, vq, ld, N, H, D, T, nch, vec_kv, part, pmax);
    else hipLaunchKernelGGL((la_state_kernel<4>), g1, t1, 0, s, kq, vq, ld, N, H, D, T, nch, vec_kv, part, pmax);
    hipLaunchKernelGGL(la_reduce_kernel, dim3((NP * KP + 255) / 256, B * H), dim3(256), 0, s, part, pmax, nch, D,
                       NP, KP, shi, slo);
    f16 * oo = reinterpret_cast<f16 *>(out);
    if (apply32) {
        constexpr int kSpan = 64 * kLfWaves;
        hipLaunchKernelGGL(la_apply32_kernel, dim3((unsigned)((N + kSpan - 1) / kSpan), (unsigned)(B * H)),
                           dim3(64 * kLfWaves), 0, s, qq, ld, shi, slo, pmax, nch, oo, ldo, N, H, kSpan);
        return hipGetLastError();
    }
    if (D % 8 == 0 && D + 1 <= 96 && vec_q && ldo % 8 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0) {
        // transposed apply with 16-byte stores of the token rows: 8 waves x 64 tokens
        constexpr int kSpan = 64 * kLfWaves;
        const dim3 gt((unsigned)((N + kSpan - 1) / kSpan), (unsigned)(B * H));
        const dim3 tt(64 * kLfWaves);
#define SANA_LA_APPLYT(nt, ks)                                                                                    \
    if (NT == nt && KS == ks) {                                                                                   \
        hipLaunchKernelGGL((la_applyT_kernel<nt, ks>), gt, tt, 0, s, qq, ld, shi, slo, pmax, nch, oo, ldo, N, H, D, \
                           kSpan);                                                                                \
        return hipGetLastError();                                                                                 \
    }
        // (NT, KS) of D = 8..88 in steps of 8
        SANA_LA_APPLYT(1, 1) SANA_LA_APPLYT(1, 2) SANA_LA_APPLYT(2, 2) SANA_LA_APPLYT(2, 3) SANA_LA_APPLYT(2, 4)
        SANA_LA_APPLYT(3, 4) SANA_LA_APPLYT(3, 5) SANA_LA_APPLYT(3, 6)
#undef SANA_LA_APPLYT
    }
    const dim3 g3((N + 127) / 128, H, B);
#define SANA_LA_APPLY(nt, ks)                                                                                     \
    hipLaunchKernelGGL((la_apply_kernel<nt, ks>), g3, dim3(256), 0, s, qq, ld, shi, slo, pmax, nch, oo, ldo, N, H, \
                       D, vec_q)
    // NT = ceil((D + 1) / 32) in 1..4, KS = ceil(D / 16) in 1..7
    if (NT == 1) {
        if (KS == 1) SANA_LA_APPLY(1, 1); else SANA_LA_APPLY(1, 2);
    } else if (NT == 2) {
        if (KS == 2) SANA_LA_APPLY(2, 2); else if (KS == 3) SANA_LA_APPLY(2, 3); else SANA_LA_APPLY(2, 4);
    } else if (NT == 3) {
        if (KS == 4) SANA_LA_APPLY(3, 4); else if (KS == 5) SANA_LA_APPLY(3, 5); else SANA_LA_APPLY(3, 6);
    } else {
        if (KS == 6) SANA_LA_APPLY(4, 6); else SANA_LA_APPLY(4, 7);
    }
#undef SANA_LA_APPLY
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
    // LDS-staged head, transposed scores (ldvt >= the 32-padded key count)
    const int lt32 = (L + 31) / 32;
    const bool out_vec = ldo % 8 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;  // 8-byte output stores
    if (vec && out_vec && D <= 96 && lt32 <= 10 && ldvt >= (int64_t)lt32 * 32) {
        if (lt32 <= 2) return launch_xattn_lds_d<2>(qq, ldq, kk, ldk, vv, ldvt, bias, oo, ldo, B, N, L, H, D, scale, s);
        if (lt32 <= 4) return launch_xattn_lds_d<4>(qq, ldq, kk, ldk, vv, ldvt, bias, oo, ldo, B, N, L, H, D, scale, s);
        if (lt32 <= 6) return launch_xattn_lds_d<6>(qq, ldq, kk, ldk, vv, ldvt, bias, oo, ldo, B, N, L, H, D, scale, s);
        return launch_xattn_lds_d<10>(qq, ldq, kk, ldk, vv, ldvt, bias, oo, ldo, B, N, L, H, D, scale, s);
    }
    const int lt = (L + 15) / 16;
    if (lt <= 2) return launch_xattn<2>(qq, ldq, kk, ldk, vv, ldvt, bias, oo, ldo, B, N, L, H, D, scale, vec, s);
    if (lt <= 8) return launch_xattn<8>(qq, ldq, kk, ldk, vv, ldvt, bias, oo, ldo, B, N, L, H, D, scale, vec, s);
    if (lt <= 20) return launch_xattn<20>(qq, ldq, kk, ldk, vv, ldvt, bias, oo, ldo, B, N, L, H, D, scale, vec, s);
    return launch_xattn<32>(qq, ldq, kk, ldk, vv, ldvt, bias, oo, ldo, B, N, L, H, D, scale, vec, s);
}

}  // namespace sana
