// fp32 kernels behind the op-level API of the drop-in (the declarations of the
// reference's src/common_ops.h and src/transformer_ops.h): a batched GEMM on
// MFMA (v_mfma_f32_32x32x2f32: fp32 products, fp32 accumulation), row
// softmax with scale and key bias, SiLU / GELU-tanh, RMSNorm, k x k depthwise
// convolution, the GLU of the split channels, ReLU linear attention, and the
// head layout moves.  Every buffer is fp32 and in the reference's layouts.
// These serve API-level calls on host tensors; the DiT forward itself runs on
// the fused fp16-operand kernels of gemm.hip / attention.hip / ffn.hip / norm.hip.
#include <cmath>
#include <string>

#include "../../include/sana_dit.h"
#include "hip_common.h"

namespace sana {
void set_last_error(const std::string & m);
}

namespace {

struct OpGemm {
    const float * A;
    const float * B;
    const float * bias;
    float * C;
    int64_t lda, ldb, ldc, sA, sB, sC;
    int M, N, K, b_trans, bias_mode, accumulate;
};

constexpr int kTM = 64, kTN = 64, kTK = 16;

// C[z] (+)= A[z] . op(B[z]) (+ bias), A [M, K] row-major, op(B) = B [K, N] or
// B^T with B [N, K].  Block tile 64 x 64, four waves of 32 x 32, K staged 16
// at a time through LDS with zero fill at the edges.  The bias is added after
// the products (bias_mode 1: per column, 2: per row).
__global__ __launch_bounds__(256) void gemm_f32_kernel(OpGemm p) {
    __shared__ float As[kTK][kTM + 1];
    __shared__ float Bs[kTK][kTN + 1];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int wm = (w >> 1) * 32, wn = (w & 1) * 32;
    const int m0 = blockIdx.y * kTM, n0 = blockIdx.x * kTN;
    const float * A = p.A + (int64_t)blockIdx.z * p.sA;
    const float * B = p.B + (int64_t)blockIdx.z * p.sB;
    float * C = p.C + (int64_t)blockIdx.z * p.sC;
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    for (int k0 = 0; k0 < p.K; k0 += kTK) {
#pragma unroll
        for (int pass = 0; pass < 4; ++pass) {
            const int r = (tid >> 4) + 16 * pass, k = tid & 15;
            const int gm = m0 + r, gk = k0 + k;
            As[k][r] = (gm < p.M && gk < p.K) ? A[(int64_t)gm * p.lda + gk] : 0.0f;
        }
        if (p.b_trans) {
#pragma unroll
            for (int pass = 0; pass < 4; ++pass) {
                const int n = (tid >> 4) + 16 * pass, k = tid & 15;
                const int gn = n0 + n, gk = k0 + k;
                Bs[k][n] = (gn < p.N && gk < p.K) ? B[(int64_t)gn * p.ldb + gk] : 0.0f;
            }
        } else {
#pragma unroll
            for (int pass = 0; pass < 4; ++pass) {
                const int k = (tid >> 6) + 4 * pass, n = tid & 63;
                const int gn = n0 + n, gk = k0 + k;
                Bs[k][n] = (gn < p.N && gk < p.K) ? B[(int64_t)gk * p.ldb + gn] : 0.0f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kTK; kk += 2) {
            const float a = As[kk + (lane >> 5)][wm + (lane & 31)];
            const float b = Bs[kk + (lane >> 5)][wn + (lane & 31)];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
        }
        __syncthreads();
    }
    const int col = n0 + wn + (lane & 31);
    if (col >= p.N) return;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int row = m0 + wm + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        if (row >= p.M) continue;
        float v = acc[i];
        if (p.bias) v = (p.bias_mode == 2 ? p.bias[row] : p.bias[col]) + v;
        float * dst = C + (int64_t)row * p.ldc + col;
        *dst = p.accumulate ? *dst + v : v;
    }
}

__global__ void unary_f32_kernel(const float * __restrict__ x, float * __restrict__ y, int64_t n, int op) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    y[i] = op == SANA_OP_SILU ? silu_f(v) : (op == SANA_OP_GELU_TANH ? gelu_tanh_f(v) : fmaxf(v, 0.0f));
}

// One wave per row: v = x * scale (+ bias[(row / bias_div) * cols + col]);
// y = exp(v - max) * (1 / sum exp(v - max)).
__global__ __launch_bounds__(256) void softmax_f32_kernel(const float * __restrict__ x, float * __restrict__ y,
                                                          int64_t rows, int cols, float scale,
                                                          const float * __restrict__ bias, int64_t bias_div) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float * xr = x + row * cols;
    const float * br = bias ? bias + (row / bias_div) * cols : nullptr;
    float * yr = y + row * cols;
    float mx = -INFINITY;
    for (int c = lane; c < cols; c += 64) {
        float v = xr[c] * scale;
        if (br) v += br[c];
        yr[c] = v;
        mx = fmaxf(mx, v);
    }
    mx = wave_max(mx);
    float sum = 0.0f;
    for (int c = lane; c < cols; c += 64) {
        const float e = expf(yr[c] - mx);
        yr[c] = e;
        sum += e;
    }
    const float recip = 1.0f / wave_sum(sum);
    for (int c = lane; c < cols; c += 64) yr[c] *= recip;
}

// One wave per row: y = x / sqrt(mean(x^2) + eps) (* w).
__global__ __launch_bounds__(256) void rms_norm_f32_kernel(const float * __restrict__ x, const float * __restrict__ w,
                                                           float * __restrict__ y, int64_t rows, int cols, float eps) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float * xr = x + row * cols;
    float * yr = y + row * cols;
    float ss = 0.0f;
    for (int c = lane; c < cols; c += 64) ss += xr[c] * xr[c];
    const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)cols + eps);
    for (int c = lane; c < cols; c += 64) {
        float v = xr[c] * inv;
        if (w) v *= w[c];
        yr[c] = v;
    }
}

// k x k depthwise convolution, zero padding k/2, NCHW; taps in (ky, kx)
// order, then the bias.  One thread per output element.
__global__ void dwconv_f32_kernel(const float * __restrict__ x, const float * __restrict__ w,
                                  const float * __restrict__ bias, float * __restrict__ y, int64_t planes, int C,
                                  int H, int W, int ks) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t HW = (int64_t)H * W;
    if (i >= planes * HW) return;
    const int64_t plane = i / HW;
    const int c = (int)(plane % C);
    const int yy = (int)((i % HW) / W), xx = (int)(i % W);
    const float * xp = x + plane * HW;
    const float * wc = w + (int64_t)c * ks * ks;
    const int pad = ks / 2;
    float sum = 0.0f;
    for (int ky = 0; ky < ks; ++ky) {
        const int iy = yy + ky - pad;
        if (iy < 0 || iy >= H) continue;
        for (int kx = 0; kx < ks; ++kx) {
            const int ix = xx + kx - pad;
            if (ix >= 0 && ix < W) sum += xp[(int64_t)iy * W + ix] * wc[ky * ks + kx];
        }
    }
    if (bias) sum += bias[c];
    y[i] = sum;
}

// y[b, c, s] = x[b, c, s] * silu(x[b, F + c, s]) for x [B, 2F, S].
__global__ void glu_f32_kernel(const float * __restrict__ x, float * __restrict__ y, int64_t B, int64_t F,
                               int64_t S) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= B * F * S) return;
    const int64_t b = i / (F * S), r = i % (F * S);
    const float * xb = x + b * 2 * F * S;
    y[i] = xb[r] * silu_f(xb[F * S + r]);
}

// Linear-attention state of one (batch*head, entry): entries r < D are
// S[r][d] = sum_t v[t][r] * relu(k[t][d]); entry r = D is ksum[d] =
// sum_t relu(k[t][d]).  Tokens are summed in order.  state: [BH][D + 1][D].
__global__ void linattn_state_f32_kernel(const float * __restrict__ k, const float * __restrict__ v,
                                         float * __restrict__ state, int N, int D) {
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t bh = blockIdx.y;
    if (e >= (D + 1) * D) return;
    const int r = e / D, d = e % D;
    const float * kb = k + bh * N * D;
    const float * vb = v + bh * N * D;
    float s = 0.0f;
    for (int t = 0; t < N; ++t) {
        const float kv = fmaxf(kb[(int64_t)t * D + d], 0.0f);
        s += (r < D ? vb[(int64_t)t * D + r] : 1.0f) * kv;
    }
    state[bh * (D + 1) * D + e] = s;
}

// out[t][r] = sum_d S[r][d] relu(q[t][d]) / (sum_d ksum[d] relu(q[t][d]) + 1e-15).
__global__ void linattn_apply_f32_kernel(const float * __restrict__ q, const float * __restrict__ state,
                                         float * __restrict__ out, int Nq, int D) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t bh = blockIdx.y;
    if (i >= (int64_t)Nq * D) return;
    const int t = (int)(i / D), r = (int)(i % D);
    const float * qr = q + (bh * Nq + t) * D;
    const float * S = state + bh * (D + 1) * D;
    float num = 0.0f, den = 0.0f;
    for (int d = 0; d < D; ++d) {
        const float qv = fmaxf(qr[d], 0.0f);
        num += S[r * D + d] * qv;
        den += S[D * D + d] * qv;
    }
    out[(bh * Nq + t) * D + r] = num / (den + 1e-15f);
}

// split = 1: y[b][h][t][d] = x[b][t][h*D + d]; split = 0: the inverse.
__global__ void heads_f32_kernel(const float * __restrict__ x, float * __restrict__ y, int64_t B, int64_t N,
                                 int64_t H, int64_t D, int split) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= B * N * H * D) return;
    // i indexes the [B, N, H*D] layout
    const int64_t d = i % D, h = (i / D) % H, t = (i / (D * H)) % N, b = i / (D * H * N);
    const int64_t j = ((b * H + h) * N + t) * D + d;
    if (split)
        y[j] = x[i];
    else
        y[i] = x[j];
}

int fail(const char * what) {
    sana::set_last_error(what);
    return SANA_ERR_INVALID_ARGUMENT;
}

int launched(const char * what) {
    const hipError_t e = hipGetLastError();
    if (e == hipSuccess) return SANA_OK;
    sana::set_last_error(std::string(what) + ": " + hipGetErrorString(e));
    return SANA_ERR_HIP;
}

unsigned blocks_for(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

extern "C" {

int sana_op_gemm_f32(const float * A, int64_t lda, int64_t strideA, const float * B, int64_t ldb, int64_t strideB,
                     int b_transposed, const float * bias, int bias_mode, float * C, int64_t ldc, int64_t strideC,
                     int64_t M, int64_t N, int64_t K, int64_t batch, int accumulate, void * stream) {
    if (!A || !B || !C) return fail("null operand");
    if (M <= 0 || N <= 0 || K < 0 || batch <= 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX ||
        batch > 65535)
        return fail("gemm dimensions out of range");
    if (lda < K || ldb < (b_transposed ? K : N) || ldc < N) return fail("gemm leading dimension too small");
    if (bias && bias_mode != 1 && bias_mode != 2) return fail("bias_mode must be 1 (per column) or 2 (per row)");
    OpGemm p{A, B, bias, C, lda, ldb, ldc, strideA, strideB, strideC, (int)M, (int)N, (int)K,
             b_transposed ? 1 : 0, bias_mode, accumulate ? 1 : 0};
    const dim3 grid((unsigned)((N + kTN - 1) / kTN), (unsigned)((M + kTM - 1) / kTM), (unsigned)batch);
    if (grid.y > 65535) return fail("gemm M too large");
    hipLaunchKernelGGL(gemm_f32_kernel, grid, dim3(256), 0, static_cast<hipStream_t>(stream), p);
    return launched("gemm_f32");
}

int sana_op_unary_f32(const float * x, float * y, int64_t n, int op, void * stream) {
    if (!x || !y || n < 0) return fail("bad unary arguments");
    if (op != SANA_OP_SILU && op != SANA_OP_GELU_TANH && op != SANA_OP_RELU) return fail("unknown unary op");
    if (n == 0) return SANA_OK;
    hipLaunchKernelGGL(unary_f32_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, static_cast<hipStream_t>(stream), x,
                       y, n, op);
    return launched("unary_f32");
}

int sana_op_softmax_f32(const float * x, float * y, int64_t rows, int64_t cols, float scale, const float * bias,
                        int64_t bias_div, void * stream) {
    if (!x || !y || rows < 0 || cols <= 0 || cols > INT32_MAX) return fail("bad softmax arguments");
    if (bias && bias_div <= 0) return fail("softmax bias_div must be positive");
    if (rows == 0) return SANA_OK;
    hipLaunchKernelGGL(softmax_f32_kernel, dim3(blocks_for(rows, 4)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       x, y, rows, (int)cols, scale, bias, bias_div);
    return launched("softmax_f32");
}

int sana_op_rms_norm_f32(const float * x, const float * w, float * y, int64_t rows, int64_t cols, float eps,
                         void * stream) {
    if (!x || !y || rows < 0 || cols <= 0 || cols > INT32_MAX) return fail("bad rms_norm arguments");
    if (rows == 0) return SANA_OK;
    hipLaunchKernelGGL(rms_norm_f32_kernel, dim3(blocks_for(rows, 4)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), x, w, y, rows, (int)cols, eps);
    return launched("rms_norm_f32");
}

int sana_op_dwconv_f32(const float * x, const float * w, const float * bias, float * y, int64_t B, int64_t C,
                       int64_t H, int64_t W, int64_t ksize, void * stream) {
    if (!x || !w || !y || B < 0 || C <= 0 || H <= 0 || W <= 0 || (ksize != 3 && ksize != 5) || C > INT32_MAX ||
        H > INT32_MAX || W > INT32_MAX)
        return fail("bad depthwise conv arguments");
    const int64_t n = B * C * H * W;
    if (n == 0) return SANA_OK;
    hipLaunchKernelGGL(dwconv_f32_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, static_cast<hipStream_t>(stream), x,
                       w, bias, y, B * C, (int)C, (int)H, (int)W, (int)ksize);
    return launched("dwconv_f32");
}

int sana_op_glu_f32(const float * x, float * y, int64_t B, int64_t F, int64_t S, void * stream) {
    if (!x || !y || B < 0 || F < 0 || S < 0) return fail("bad glu arguments");
    const int64_t n = B * F * S;
    if (n == 0) return SANA_OK;
    hipLaunchKernelGGL(glu_f32_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, static_cast<hipStream_t>(stream), x, y,
                       B, F, S);
    return launched("glu_f32");
}

int sana_op_linear_attention_f32(const float * q, const float * k, const float * v, float * out, int64_t BH,
                                 int64_t Nq, int64_t Nk, int64_t D, float * state, void * stream) {
    if (!q || !k || !v || !out || !state || BH < 0 || Nq < 0 || Nk < 0 || D <= 0 || D > 4096 || BH > 65535 ||
        Nq > INT32_MAX || Nk > INT32_MAX)
        return fail("bad linear attention arguments");
    if (BH == 0) return SANA_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(linattn_state_f32_kernel, dim3(blocks_for((D + 1) * D, 256), (unsigned)BH), dim3(256), 0, s,
                       k, v, state, (int)Nk, (int)D);
    int rc = launched("linattn_state_f32");
    if (rc != SANA_OK || Nq == 0) return rc;
    hipLaunchKernelGGL(linattn_apply_f32_kernel, dim3(blocks_for(Nq * D, 256), (unsigned)BH), dim3(256), 0, s, q,
                       state, out, (int)Nq, (int)D);
    return launched("linattn_apply_f32");
}

int sana_op_heads_f32(const float * x, float * y, int64_t B, int64_t N, int64_t H, int64_t D, int split,
                      void * stream) {
    if (!x || !y || B < 0 || N < 0 || H <= 0 || D < 0) return fail("bad head layout arguments");
    const int64_t n = B * N * H * D;
    if (n == 0) return SANA_OK;
    hipLaunchKernelGGL(heads_f32_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, static_cast<hipStream_t>(stream), x,
                       y, B, N, H, D, split ? 1 : 0);
    return launched("heads_f32");
}

}  // extern "C"
