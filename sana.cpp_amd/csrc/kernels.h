// Host-side launchers of the gfx950 kernels.  Every launcher validates the
// shapes its kernel assumes and returns hipErrorInvalidValue instead of
// launching when they do not hold, so no kernel runs out of bounds.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sana {

typedef _Float16 half_t;

enum GemmMode {
    kGemmStore = 0,     // out16/out32[m, n] = act(acc + bias[n])
    kGemmResidual = 1,  // out32[m, n] += gate(m, n) * (acc + bias[n]); out16 = f16(out32) if set
    kGemmVT = 2,        // transposed-batched store of V^T (see GemmParams::vt_*)
    kGemmQKV = 3,       // fused q|k|v split for linear attention (see GemmParams::qkv_*)
};

// kActGeglu (plain stores to out16 only): W rows interleaved as gate / up
// pairs, out16[m, n / 2] = f16(gelu_tanh(acc[m, n]) * acc[m, n + 1]) for even n.
enum GemmAct { kActNone = 0, kActSilu = 1, kActGelu = 2, kActGeglu = 3 };

// C[m, n] = sum_k A[m, k] * W[n, k]; fp16 operands, fp32 accumulation.
// K must be a multiple of 64 and both lda and ldw >= K, multiples of 8.
struct GemmParams {
    const half_t * A = nullptr;
    int64_t lda = 0;
    const half_t * W = nullptr;
    int64_t ldw = 0;
    int M = 0, N = 0, K = 0;
    const float * bias = nullptr;     // [N] (kGemmVT: [M], per output row)
    int mode = kGemmStore;
    int act = kActNone;
    half_t * out16 = nullptr;
    int64_t ldo16 = 0;
    float * out32 = nullptr;
    int64_t ldo32 = 0;
    // Residual gate: gate(m, n) = gate_a[(m / rows_per_batch) * gate_stride + n] + gate_t[n]
    // (t_mod row slice + scale_shift_table row); gate_a == nullptr means gate 1.
    const float * gate_a = nullptr;
    const float * gate_t = nullptr;
    int64_t gate_stride = 0;
    int rows_per_batch = 1;
    // kGemmVT: element (m, n) with m = blk * vt_rows + r, n = b * vt_cols + j is
    // stored at out16[((blk * vt_batch + b) * vt_rows + r) * vt_ld + j].
    int vt_rows = 0, vt_cols = 0, vt_batch = 0;
    int64_t vt_ld = 0;
    // kGemmQKV: output column n of section s = n / qkv_c (q, k, v), channel
    // c = n % qkv_c, row m = b * qkv_n + t:
    //   q: out16[m * ldo16 + c] = relu(acc + bias)        (token-major)
    //   k: kt16[(b * qkv_c + c) * qkv_n + t] = relu(acc + bias)   (token-contiguous)
    //   v: vt16[(b * qkv_c + c) * qkv_n + t] = acc + bias
    half_t * kt16 = nullptr;
    half_t * vt16 = nullptr;
    int qkv_c = 0, qkv_n = 0;
    // Implicit 3x3 "same" convolution (conv = 1), optionally on the nearest-2x
    // upsample of its input (conv = 2).  Output pixel m = (b * conv_h + y) *
    // conv_w + x of a conv_h x conv_w grid; A is the input in NHWC fp16 with a
    // one-pixel zero border ([B][(ih + 2) * (iw + 2)][lda], ih x iw = the
    // output grid, or half of it for conv = 2), lda = channels per tap (a
    // multiple of 64), K = 9 * lda with tap-major weights W[n][(ky * 3 + kx) *
    // lda + c].  With out16_pad the fp16 output goes to the interior of a
    // bordered [B][(conv_h + 2) * (conv_w + 2)][ldo16] buffer.
    int conv = 0, conv_h = 0, conv_w = 0, out16_pad = 0;
    // conv = 2, residual mode: with up_src set, the residual is not read from
    // out32 but starts as the pixel-shuffled channel-repeat shortcut of the
    // low-resolution input up_src (fp32 NHWC, up_c channels): output pixel
    // (y, x), channel n takes up_src[(y/2, x/2)][(4n + 2(y%2) + x%2) / up_rep].
    const float * up_src = nullptr;
    int up_c = 0, up_rep = 1;
    // Batched plain stores (mode kGemmStore, conv 0): `batch` independent
    // products in one launch; product z reads A + z * batch_a, W + (z / batch_w_div)
    // * batch_w (grouped heads share a W) and writes out16 + z * batch_o16 and
    // out32 + z * batch_o32 (element offsets).
    int batch = 1, batch_w_div = 1;
    int64_t batch_a = 0, batch_w = 0, batch_o16 = 0, batch_o32 = 0;
    // Launches of this shape that run concurrently with this one (on other
    // streams or graph branches); the tile choice sizes its grid for the CUs
    // it shares with them.
    int co = 1;
    int vec = 0;  // set by gemm(): 16-byte epilogue accesses are aligned
};

hipError_t gemm(const GemmParams & p, hipStream_t s);

// Name of the last kernel (instantiation) a launcher on this thread launched,
// as rocprofv3 prints it, for the measurement hooks; launchers record it with
// note_kernel (a pointer to storage that outlives the call).
void note_kernel(const char * name);
const char * last_kernel();

// LayerNorm (eps, optional gamma/beta) + adaLN modulate, fp32 in, fp16 out:
// out[m, c] = f16(ln(x)[m, c] * (1 + scale) + shift), with
// shift = mod_a[b * mod_stride + shift_off + c] + mod_t[shift_off + c] (same for scale; mod_t may be null).
// Device ranges a launch reads on the side to pull them into the 256 MB
// last-level cache before a later kernel needs them (the next GEMMs' weights):
// `workgroups` extra workgroups stream the n ranges (16-byte multiples,
// 16-byte aligned) and discard the data.
struct CacheWarm {
    static constexpr int kMax = 6;
    const void * p[kMax] = {};
    int64_t bytes[kMax] = {};
    int n = 0, workgroups = 0;
};
// warm: optional cache warm-up carried by the same launch (vectorised rows only).
hipError_t ln_modulate(const float * x, int64_t ldx, half_t * out, int64_t ldo, int M, int C, int rows_per_batch,
                       float eps, const float * gamma, const float * beta, const float * mod_a, const float * mod_t,
                       int64_t mod_stride, int64_t shift_off, int64_t scale_off, hipStream_t s,
                       const CacheWarm * warm = nullptr);

// comb[l][b][i] = tmod[b][i] + tables[l][i] (l < L, b < B, i < W).
hipError_t mod_combine(const float * tmod, const float * tables, int L, int B, int W, float * comb, hipStream_t s);

// RMSNorm (eps, weight) fp32 -> fp16 (and optionally fp32 [M, C] into out32).
hipError_t rms_norm_f16(const float * x, int64_t ldx, const float * weight, half_t * out, int64_t ldo, float * out32,
                        int M, int C, float eps, hipStream_t s);

// fp32 -> fp16 copy of a [M, C] matrix into a buffer with leading dim ldo
// (columns C..ldo-1 are written as zero).
hipError_t to_f16_padded(const float * x, int M, int C, half_t * out, int64_t ldo, hipStream_t s);

// Time MLP pieces (fp32).
// out[b, n] = bias[n] + sum_k act_in(in[b, k]) * W[n, k] (W fp32 [N, K]); act_in: 0 none, 1 silu.
hipError_t gemv_f32(const float * in, const float * W, const float * bias, float * out, int B, int K, int N,
                    int act_in, hipStream_t s);
// gemv_f32 of the sinusoid [cos(t_b f_i), sin(t_b f_i)] of B timesteps t read
// from device memory, f_i = freq[i] for i < K / 2 (K % 8 == 0).
hipError_t gemv_sinusoid_f32(const float * t, const float * freq, const float * W, const float * bias, float * out,
                             int B, int K, int N, hipStream_t s);
// gemv_f32 that also writes comb[l][b][n] = out[b, n] + tables[l][n] for the L tables.
hipError_t gemv_comb_f32(const float * in, const float * W, const float * bias, float * out, const float * tables,
                         int L, float * comb, int B, int K, int N, int act_in, hipStream_t s);

// Patch embed: NCHW latent [Bl, Cl, S] (batch b reads latent batch b % Bl) -> tokens [B, S, C] fp32.
hipError_t patch_embed(const float * latent, int Bl, int B, int Cl, int S, const float * W, const float * bias,
                       float * out, int C, hipStream_t s);

// Final layer: LN(eps, no affine) + modulate(shift = emb + T[0], scale = emb + T[1])
// into y [B*S, C] fp32 (workspace), then proj (Wt [C, Cl] fp32, bias [Cl],
// Cl <= 32) stored NCHW [B, Cl, S].  With C % 384 == 0 and S % 32 == 0 both
// run in one kernel and y is not written.
hipError_t final_layer(const float * x, const float * emb, const float * table, const float * Wt, const float * bias,
                       float * y, float * out, int B, int S, int C, int Cl, float eps, hipStream_t s);

// ReLU linear attention.  q/k/v fp16 token-major with row stride ld (head h at
// columns h*D..), out fp16 with row stride ldo.  Workspace: partial states.
size_t linattn_workspace_floats(int B, int N, int H, int D);
// Whole linear attention in one launch for head_dim 32, from the kGemmQKV
// layouts: relu(q) token-major [B*N, ldq], relu(K)^T and V^T [B][H*32][N].
bool linear_attention_fused_ok(int N, int D);
// co: launches of this shape running concurrently (sizes the token splits).
hipError_t linear_attention_fused(const half_t * q, int64_t ldq, const half_t * kt, const half_t * vt, half_t * out,
                                  int64_t ldo, int B, int N, int H, int D, hipStream_t s, int co = 1);
// The same from the kGemmQKV layouts in three kernels (chunk states straight
// from relu(K)^T and V^T, the fixed-order reduction, the apply), for long
// sequences where rebuilding the state per token split does not pay; head_dim
// 32, workspace of linattn_workspace_floats(B, N, H, 32) floats.
hipError_t linear_attention_chunked(const half_t * q, int64_t ldq, const half_t * kt, const half_t * vt,
                                    half_t * out, int64_t ldo, int B, int N, int H, int D, float * workspace,
                                    hipStream_t s);
hipError_t linear_attention(const half_t * q, const half_t * k, const half_t * v, int64_t ld, half_t * out,
                            int64_t ldo, int B, int N, int H, int D, float * workspace, hipStream_t s);

// Softmax cross attention.  q fp16 [B*N, ldq]; k fp16 rows (b*L + j) with stride
// ldk (head h at columns h*D..); vt fp16 [B][H*D][ldvt] (keys contiguous);
// bias fp32 [B, L] or null; out fp16 [B*N, ldo].
hipError_t cross_attention(const half_t * q, int64_t ldq, const half_t * k, int64_t ldk, const half_t * vt,
                           int64_t ldvt, const float * bias, half_t * out, int64_t ldo, int B, int N, int L, int H,
                           int D, hipStream_t s);

// Depthwise 3x3 (zero pad, bias) + GLU gate on a token-major grid:
// x fp16 [B, H*W, ldx] (E = 2F channels), wt fp32 tap-major [9][E], bias [E],
// out[b, t, c] = f16(d(c) * silu(d(F + c))), out fp16 [B*H*W, ldo].
hipError_t dwconv_glu(const half_t * x, int64_t ldx, const float * wt, const float * bias, half_t * out, int64_t ldo,
                      int B, int Hh, int Ww, int F, hipStream_t s);

// Measured MFMA ceiling: `workgroups` x 256 threads of independent fp16
// 32x32x16 MFMA chains, `iters` steps; sink holds workgroups * 256 floats.
hipError_t mfma_peak(int workgroups, int iters, bool zero_operands, float * sink, hipStream_t s);
double mfma_peak_flops(int workgroups, int iters);
// Measured HBM ceiling: streams `bytes` (a multiple of 16) from src, into dst
// (copy) or, with dst null, into per-thread sums in sink (read only; sink holds
// hbm_peak_workgroups() * 256 floats).
int hbm_peak_workgroups();
hipError_t hbm_peak(const void * src, void * dst, int64_t bytes, float * sink, hipStream_t s);

}  // namespace sana
