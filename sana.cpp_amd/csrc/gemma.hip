// Gemma-2 text encoder (the stage before the denoiser: src/gemma_encoder.cpp,
// which runs llama.cpp's Gemma-2 graph in embeddings mode) on one MI355X,
// and its C ABI.
//
// Per layer, with T tokens (rows), hidden H, nh query heads and nkv kv heads
// of dimension d, FFN width F:
//   a16  = rmsnorm(x) * attn_norm                        gemma_norm_kernel
//   qkv  = a16 [Wq; Wk; Wv]^T                            one MFMA GEMM, fp32 out
//   q16, k16 = rope(q) * query_scale, rope(k); V^T       gemma_qkv_kernel
//   S_h  = q16_h k16_kv(h)^T                             all heads in one batched GEMM
//   P_h  = softmax(causal / window mask, soft-cap)       gemma_softmax_kernel
//   o16_h = P_h V_kv(h)                                  all heads in one batched GEMM (B = V^T)
//   x   += rmsnorm(o16 Wo^T) * post_attention_norm       split-K GEMM + gemma_norm_kernel
//   a16  = rmsnorm(x) * ffn_norm
//   g16  = gelu_tanh(a16 Wgate^T) * (a16 Wup^T)        one GEMM, gate / up rows
//                                                        interleaved, gated in its epilogue
//   x   += rmsnorm(g16 Wdown^T) * post_ffw_norm          split-K GEMM + gemma_norm_kernel
// Each post-norm residual add and the pre-norm after it are one launch.
// The layers of one encode run as one cached graph per sequence-length list.
// out = rmsnorm(x) * output_norm.  Activations are token-major; GEMM operands
// fp16 with fp32 accumulation; the residual stream, norms, softmax and RoPE
// in fp32.  RMSNorm weights are taken as stored in the GGUF (1 + w).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/sana_dit.h"
#include "gguf.h"
#include "hip_common.h"
#include "host_util.h"
#include "kernels.h"

using sana::half_t;
using namespace sana_host;

namespace {

unsigned blocks_for(int64_t n, int per = 256) { return (unsigned)((n + per - 1) / per); }

// x32[t][c] = embed[token[t]][c] * scale (token ids checked on the host).
__global__ void gemma_embed_kernel(const int32_t * __restrict__ tok, const f16 * __restrict__ emb,
                                   float * __restrict__ x, int T, int H, float scale) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)T * H) return;
    const int t = (int)(i / H), c = (int)(i - (int64_t)t * H);
    x[i] = (float)emb[(int64_t)tok[t] * H + c] * scale;
}

// One workgroup of 256 threads per row of C (<= 1024 * NC4) channels:
// v = y / sqrt(mean(y^2) + eps) * w, y the fixed-order sum of `parts` split-K
// partials part_stride floats apart; the sum of squares is reduced over the
// four waves through LDS.  mode 0: out16 = fp16(v); 1: x += v (post-norm
// residual, out32 = x); 2: out32 = v; 3: x += v as mode 1, then the next
// pre-norm of the new row, out16 = fp16(x / sqrt(mean(x^2) + eps) * w2), with
// the same summation order as a separate mode-0 launch on x.
template <int NC4>
__global__ __launch_bounds__(256) void gemma_norm_kernel(const float * __restrict__ y, int parts,
                                                         int64_t part_stride, int C, int M,
                                                         const float * __restrict__ w, float eps, int mode,
                                                         f16 * __restrict__ out16, float * __restrict__ out32,
                                                         const float * __restrict__ w2) {
    __shared__ float wsum[4];
    const int row = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63;
    const int n4 = C >> 2;
    const float4 * yr = reinterpret_cast<const float4 *>(y + (int64_t)row * C);
    float4 v[NC4];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NC4; ++i) {
        const int c4 = tid + 256 * i;
        v[i] = c4 < n4 ? yr[c4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int z = 1; z < parts; ++z) {
            if (c4 >= n4) break;
            const float4 u = reinterpret_cast<const float4 *>(y + z * part_stride + (int64_t)row * C)[c4];
            v[i] = make_float4(v[i].x + u.x, v[i].y + u.y, v[i].z + u.z, v[i].w + u.w);
        }
        ss += (v[i].x * v[i].x + v[i].y * v[i].y) + (v[i].z * v[i].z + v[i].w * v[i].w);
    }
    ss = wave_sum(ss);
    if (lane == 0) wsum[tid >> 6] = ss;
    __syncthreads();
    const float tot = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    const float inv = 1.0f / sqrtf(tot / (float)C + eps);
    float ss2 = 0.0f;
#pragma unroll
    for (int i = 0; i < NC4; ++i) {
        const int c4 = tid + 256 * i;
        if (c4 >= n4) continue;
        const float4 g = reinterpret_cast<const float4 *>(w)[c4];
        float o[4] = {v[i].x * inv * g.x, v[i].y * inv * g.y, v[i].z * inv * g.z, v[i].w * inv * g.w};
        if (mode == 0) {
            f16x4 h;
#pragma unroll
            for (int e = 0; e < 4; ++e) h[e] = (f16)o[e];
            *reinterpret_cast<f16x4 *>(out16 + (int64_t)row * C + 4 * c4) = h;
        } else {
            float4 * xr = reinterpret_cast<float4 *>(out32 + (int64_t)row * C) + c4;
            if (mode == 1 || mode == 3) {
                const float4 x = *xr;
                const float4 xn = make_float4(x.x + o[0], x.y + o[1], x.z + o[2], x.w + o[3]);
                *xr = xn;
                v[i] = xn;  // the new residual row, for mode 3's second norm
                ss2 += (xn.x * xn.x + xn.y * xn.y) + (xn.z * xn.z + xn.w * xn.w);
            } else {
                *xr = make_float4(o[0], o[1], o[2], o[3]);
            }
        }
    }
    if (mode != 3) return;
    ss2 = wave_sum(ss2);
    __syncthreads();  // every wave has read wsum
    if (lane == 0) wsum[tid >> 6] = ss2;
    __syncthreads();
    const float tot2 = (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
    const float inv2 = 1.0f / sqrtf(tot2 / (float)C + eps);
#pragma unroll
    for (int i = 0; i < NC4; ++i) {
        const int c4 = tid + 256 * i;
        if (c4 >= n4) continue;
        const float4 g = reinterpret_cast<const float4 *>(w2)[c4];
        f16x4 h;
        h[0] = (f16)(v[i].x * inv2 * g.x);
        h[1] = (f16)(v[i].y * inv2 * g.y);
        h[2] = (f16)(v[i].z * inv2 * g.z);
        h[3] = (f16)(v[i].w * inv2 * g.w);
        *reinterpret_cast<f16x4 *>(out16 + (int64_t)row * C + 4 * c4) = h;
    }
}

// qkv32 [T][(nh + 2 nkv) d] -> q16 [T][nh d] = rope(q) * qscale, k16 [T][nkv d]
// = rope(k), vt16 [nkv][d][Tp] = V^T (tokens T..Tp-1 zero).  NeoX RoPE: pair
// (i, i + d/2) of a head rotated by t * theta^(-2i/d).  One thread per
// (token, rotation pair) of the q and k heads, and per (token, channel) of v.
__global__ void gemma_qkv_kernel(const float * __restrict__ qkv, int T, int Tp, int nh, int nkv, int d,
                                 float theta, float qscale, f16 * __restrict__ q16, f16 * __restrict__ k16,
                                 f16 * __restrict__ vt16) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int half = d / 2, ld = (nh + 2 * nkv) * d;
    const int64_t nrot = (int64_t)T * (nh + nkv) * half;
    if (i < nrot) {
        const int t = (int)(i / ((nh + nkv) * half));
        const int r = (int)(i - (int64_t)t * (nh + nkv) * half);
        const int head = r / half, p = r - head * half;  // heads 0..nh-1 are q, then k
        const float inv = powf(theta, -2.0f * (float)p / (float)d);
        float sn, cs;
        sincosf((float)t * inv, &sn, &cs);
        const float * src = qkv + (int64_t)t * ld + head * d;
        const float a = src[p], b = src[p + half];
        float oa = a * cs - b * sn, ob = b * cs + a * sn;
        if (head < nh) {
            f16 * dst = q16 + (int64_t)t * nh * d + head * d;
            dst[p] = (f16)(oa * qscale);
            dst[p + half] = (f16)(ob * qscale);
        } else {
            f16 * dst = k16 + (int64_t)t * nkv * d + (head - nh) * d;
            dst[p] = (f16)oa;
            dst[p + half] = (f16)ob;
        }
        return;
    }
    const int64_t j = i - nrot;
    if (j >= (int64_t)nkv * d * Tp) return;
    const int t = (int)(j % Tp), ch = (int)(j / Tp);  // ch = kvhead * d + dim
    vt16[j] = t < T ? (f16)qkv[(int64_t)t * ld + (nh + nkv) * d + ch] : (f16)0.0f;
}

// Rows (head, t) of S [nh][T][Tp]: s = cap * tanh(S / cap) over keys j <= t
// (and j > t - window when window > 0), softmax in fp32 -> P fp16 [nh][T][Tp]
// with zeros for the masked and padding keys.  One wave per row; lane keeps
// keys lane + 64 k (k < NJ, Tp <= 64 NJ) in registers, so each soft-capped
// score and its exponential are computed once.
template <int NJ>
__global__ __launch_bounds__(256) void gemma_softmax_kernel(const float * __restrict__ S, f16 * __restrict__ P,
                                                            int nh, int T, int Tp, float cap, int window) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= nh * T) return;
    const int t = row % T;
    const int j0 = window > 0 ? max(0, t - window + 1) : 0;
    const float * sr = S + (int64_t)row * Tp;
    f16 * pr = P + (int64_t)row * Tp;
    float v[NJ];
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < NJ; ++k) {
        const int j = lane + 64 * k;
        v[k] = (j >= j0 && j <= t) ? cap * tanhf(sr[j] / cap) : -INFINITY;
        mx = fmaxf(mx, v[k]);
    }
    mx = wave_max(mx);
    float sum = 0.0f;
#pragma unroll
    for (int k = 0; k < NJ; ++k) {
        v[k] = v[k] == -INFINITY ? 0.0f : expf(v[k] - mx);
        sum += v[k];
    }
    sum = wave_sum(sum);
    const float rs = 1.0f / sum;
#pragma unroll
    for (int k = 0; k < NJ; ++k) {
        const int j = lane + 64 * k;
        if (j < Tp) pr[j] = (f16)(v[k] * rs);
    }
}

struct LayerDev {
    DevMem wqkv, wo, wgu, wdown;          // fp16, [out][in]; wgu rows gate_0, up_0, gate_1, up_1, ...
    DevMem n_attn, n_post_attn, n_ffn, n_post_ffw;  // fp32
};

}  // namespace

struct sana_gemma {
    sana_gemma_config cfg{};
    int64_t Dq = 0, Dkv = 0;
    std::vector<std::unique_ptr<LayerDev>> layers;
    DevMem emb16, out_norm;
    std::map<std::string, bool> loaded;
    std::vector<std::string> required;
    hipStream_t stream = nullptr;
    // second stream: the attention of every other sequence runs on it, beside
    // the first sequence's (fork after the q|k|v projection, join before the
    // output projection of each layer)
    hipStream_t stream2 = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
    // workspace: rows of all sequences of one encode, and the per-sequence
    // attention buffers (V^T, scores, probabilities) back to back
    int64_t ws_M = 0, ws_vt = 0, ws_att = 0;
    DevMem tok, x32, y32, a16, qkv32, q16, k16, vt16, s32, p16, o16, g16, out32;
    // the encoder's kernels as one graph per sequence-length list (workspace
    // and weight pointers are baked in: dropped when either is reallocated)
    std::map<std::vector<int64_t>, hipGraphExec_t> graphs;
    ~sana_gemma() {
        for (auto & kv : graphs) (void)hipGraphExecDestroy(kv.second);
        if (ev_fork) (void)hipEventDestroy(ev_fork);
        if (ev_join) (void)hipEventDestroy(ev_join);
        if (stream2) (void)hipStreamDestroy(stream2);
        if (stream) (void)hipStreamDestroy(stream);
    }
};

namespace {

void drop_graphs(sana_gemma * g) {
    for (auto & kv : g->graphs) (void)hipGraphExecDestroy(kv.second);
    g->graphs.clear();
}

void upload_bytes(DevMem & d, const void * src, size_t bytes) {
    d.ensure(bytes, false);
    copy_to_device(d.p, src, bytes, "upload gemma weight");
}

// fp32 -> fp16 operand rows; a value fp16 cannot hold fails with
// SANA_ERR_FORMAT naming the tensor.
void upload_f16_rows(DevMem & d, const float * src, size_t n, size_t total, size_t offset, const std::string & tensor) {
    if (!d.p) d.ensure(total * 2, false);
    std::vector<_Float16> h(n);
    for (size_t i = 0; i < n; ++i) h[i] = to_f16_checked(src[i], tensor, i);
    copy_to_device(static_cast<_Float16 *>(d.p) + offset, h.data(), n * 2, "upload gemma weight");
}

// Rows r of src ([n_rows][width] fp32) to rows 2 r + parity of d ([2 n_rows][width] fp16).
void upload_f16_rows_interleaved(DevMem & d, const float * src, size_t n_rows, size_t width, int parity,
                                 const std::string & tensor) {
    if (!d.p) d.ensure(2 * n_rows * width * 2, false);
    std::vector<_Float16> h(n_rows * width);
    for (size_t i = 0; i < h.size(); ++i) h[i] = to_f16_checked(src[i], tensor, i);
    hip_check(hipMemcpy2D(static_cast<_Float16 *>(d.p) + parity * width, 2 * width * 2, h.data(), width * 2,
                          width * 2, n_rows, hipMemcpyHostToDevice),
              "upload gemma weight");
    // a pageable copy may return before the data lands: h must outlive it, and
    // the encoder's non-blocking stream is not ordered after the null stream
    hip_check(hipStreamSynchronize(nullptr), "upload gemma weight");
}

void expect(const std::string & name, const int64_t * shape, int ndim, std::vector<int64_t> want) {
    bool ok = ndim == (int)want.size();
    for (int i = 0; ok && i < ndim; ++i) ok = shape[i] == want[i];
    if (!ok) {
        std::string got, exp;
        for (int i = 0; i < ndim; ++i) got += (i ? "," : "") + std::to_string(shape[i]);
        for (size_t i = 0; i < want.size(); ++i) exp += (i ? "," : "") + std::to_string(want[i]);
        throw_err(SANA_ERR_SHAPE, "gemma weight " + name + " has shape [" + got + "], expected [" + exp + "]");
    }
}

std::vector<std::string> required_names(const sana_gemma * g) {
    std::vector<std::string> r = {"token_embd.weight", "output_norm.weight"};
    for (int64_t l = 0; l < g->cfg.layers; ++l)
        for (const char * s : {"attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "post_attention_norm",
                               "ffn_norm", "ffn_gate", "ffn_up", "ffn_down", "post_ffw_norm"})
            r.push_back("blk." + std::to_string(l) + "." + s + ".weight");
    return r;
}

void set_weight(sana_gemma * g, const std::string & n, const float * d, const int64_t * sh, int nd) {
    drop_graphs(g);
    const sana_gemma_config & c = g->cfg;
    const int64_t H = c.hidden, F = c.ffn, Dq = g->Dq, Dkv = g->Dkv;
    if (n == "token_embd.weight") {
        expect(n, sh, nd, {c.vocab, H});
        upload_f16_rows(g->emb16, d, (size_t)(c.vocab * H), (size_t)(c.vocab * H), 0, n);
    } else if (n == "output_norm.weight") {
        expect(n, sh, nd, {H});
        upload_bytes(g->out_norm, d, (size_t)H * 4);
    } else {
        const std::string pre = "blk.";
        const size_t dot = n.find('.', pre.size());
        if (n.compare(0, pre.size(), pre) != 0 || dot == std::string::npos)
            throw_err(SANA_ERR_INVALID_ARGUMENT, "unknown gemma weight " + n);
        const int64_t l = std::stoll(n.substr(pre.size(), dot - pre.size()));
        if (l < 0 || l >= c.layers) throw_err(SANA_ERR_INVALID_ARGUMENT, "gemma layer index out of range: " + n);
        const std::string s = n.substr(dot + 1);
        LayerDev & L = *g->layers[l];
        const size_t qkv_rows = (size_t)(Dq + 2 * Dkv);
        if (s == "attn_q.weight") {
            expect(n, sh, nd, {Dq, H});
            upload_f16_rows(L.wqkv, d, (size_t)(Dq * H), qkv_rows * H, 0, n);
        } else if (s == "attn_k.weight") {
            expect(n, sh, nd, {Dkv, H});
            upload_f16_rows(L.wqkv, d, (size_t)(Dkv * H), qkv_rows * H, (size_t)(Dq * H), n);
        } else if (s == "attn_v.weight") {
            expect(n, sh, nd, {Dkv, H});
            upload_f16_rows(L.wqkv, d, (size_t)(Dkv * H), qkv_rows * H, (size_t)((Dq + Dkv) * H), n);
        } else if (s == "attn_output.weight") {
            expect(n, sh, nd, {H, Dq});
            upload_f16_rows(L.wo, d, (size_t)(H * Dq), (size_t)(H * Dq), 0, n);
        } else if (s == "ffn_gate.weight") {
            expect(n, sh, nd, {F, H});
            upload_f16_rows_interleaved(L.wgu, d, (size_t)F, (size_t)H, 0, n);
        } else if (s == "ffn_up.weight") {
            expect(n, sh, nd, {F, H});
            upload_f16_rows_interleaved(L.wgu, d, (size_t)F, (size_t)H, 1, n);
        } else if (s == "ffn_down.weight") {
            expect(n, sh, nd, {H, F});
            upload_f16_rows(L.wdown, d, (size_t)(H * F), (size_t)(H * F), 0, n);
        } else {
            DevMem * dst = s == "attn_norm.weight"             ? &L.n_attn
                           : s == "post_attention_norm.weight" ? &L.n_post_attn
                           : s == "ffn_norm.weight"            ? &L.n_ffn
                           : s == "post_ffw_norm.weight"       ? &L.n_post_ffw
                                                               : nullptr;
            if (!dst) throw_err(SANA_ERR_INVALID_ARGUMENT, "unknown gemma weight " + n);
            expect(n, sh, nd, {H});
            upload_bytes(*dst, d, (size_t)H * 4);
        }
    }
    g->loaded[n] = true;
}

void check_ready(const sana_gemma * g) {
    for (const std::string & n : g->required)
        if (!g->loaded.count(n)) throw_err(SANA_ERR_STATE, "gemma weight not set: " + n);
}

// One sequence of an encode: its rows [row0, row0 + T) of the token-major
// buffers and its offsets into the per-sequence attention buffers.
struct Seq {
    int64_t row0, T, Tp, vt_off, att_off;
};

std::vector<Seq> layout(const sana_gemma * g, const std::vector<int64_t> & lens) {
    std::vector<Seq> q;
    int64_t row = 0, vt = 0, att = 0;
    for (int64_t T : lens) {
        const int64_t Tp = round_up(T, 64);
        q.push_back({row, T, Tp, vt, att});
        row += T;
        vt += g->Dkv * Tp;
        att += g->cfg.heads * T * Tp;
    }
    return q;
}

void ensure_workspace(sana_gemma * g, const std::vector<Seq> & q) {
    const Seq & e = q.back();
    const int64_t M = e.row0 + e.T, vt = e.vt_off + g->Dkv * e.Tp, att = e.att_off + g->cfg.heads * e.T * e.Tp;
    if (M <= g->ws_M && vt <= g->ws_vt && att <= g->ws_att) return;
    drop_graphs(g);
    const sana_gemma_config & c = g->cfg;
    const int64_t H = c.hidden;
    g->ws_M = std::max(g->ws_M, M);
    g->ws_vt = std::max(g->ws_vt, vt);
    g->ws_att = std::max(g->ws_att, att);
    const size_t R = (size_t)g->ws_M;
    g->tok.ensure(R * 4, false);
    g->x32.ensure(R * H * 4, false);
    g->y32.ensure(R * H * 4 * 4, false);  // up to four split-K partials
    g->a16.ensure(R * H * 2, false);
    g->qkv32.ensure(R * (g->Dq + 2 * g->Dkv) * 4, false);
    g->q16.ensure(R * g->Dq * 2, false);
    g->k16.ensure(R * g->Dkv * 2, false);
    g->vt16.ensure((size_t)g->ws_vt * 2, false);
    g->s32.ensure((size_t)g->ws_att * 4, false);
    g->p16.ensure((size_t)g->ws_att * 2, false);
    g->o16.ensure(R * g->Dq * 2, false);
    g->g16.ensure(R * c.ffn * 2, false);
    g->out32.ensure(R * H * 4, false);
}

void gemm(const half_t * A, int64_t lda, const half_t * W, int64_t ldw, int64_t M, int64_t N, int64_t K,
          half_t * o16, int64_t ldo16, float * o32, int64_t ldo32, hipStream_t s, int act = sana::kActNone) {
    sana::GemmParams p;
    p.act = act;
    p.A = A;
    p.lda = lda;
    p.W = W;
    p.ldw = ldw;
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    p.out16 = o16;
    p.ldo16 = ldo16;
    p.out32 = o32;
    p.ldo32 = ldo32;
    launch_check(sana::gemm(p, s), "gemma gemm");
}

// `batch` products in one launch: product z reads A + z * sa and W + (z / wdiv) * sw,
// writes o16 + z * so16 / o32 + z * so32.
void gemm_batched(const half_t * A, int64_t lda, int64_t sa, const half_t * W, int64_t ldw, int64_t sw, int wdiv,
                  int64_t M, int64_t N, int64_t K, half_t * o16, int64_t ldo16, int64_t so16, float * o32,
                  int64_t ldo32, int64_t so32, int batch, hipStream_t s) {
    sana::GemmParams p;
    p.A = A;
    p.lda = lda;
    p.W = W;
    p.ldw = ldw;
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    p.out16 = o16;
    p.ldo16 = ldo16;
    p.out32 = o32;
    p.ldo32 = ldo32;
    p.batch = batch;
    p.batch_w_div = wdiv;
    p.batch_a = sa;
    p.batch_w = sw;
    p.batch_o16 = so16;
    p.batch_o32 = so32;
    launch_check(sana::gemm(p, s), "gemma batched gemm");
}

void norm(const sana_gemma * g, const float * y, int64_t M, const DevMem & w, int mode, half_t * o16, float * o32,
          hipStream_t s, int parts = 1, const DevMem * w2 = nullptr) {
    const int64_t C = g->cfg.hidden;
    const dim3 grid((unsigned)M), blk(256);
    f16 * h = reinterpret_cast<f16 *>(o16);
    const float eps = g->cfg.rms_eps;
    const int64_t pstride = M * C;
    const float * w2p = w2 ? w2->as<float>() : nullptr;
#define SANA_GEMMA_NORM(n4)                                                                                      \
    hipLaunchKernelGGL((gemma_norm_kernel<n4>), grid, blk, 0, s, y, parts, pstride, (int)C, (int)M, w.as<float>(), \
                       eps, mode, h, o32, w2p)
    if (C <= 1024) SANA_GEMMA_NORM(1);
    else if (C <= 2048) SANA_GEMMA_NORM(2);
    else SANA_GEMMA_NORM(4);
#undef SANA_GEMMA_NORM
    launch_check(hipGetLastError(), "gemma norm");
}

// Split-K factor of an M x H output with contraction K: the down and output
// projections have long K and few output tiles, so their K is cut into parts
// (multiples of 64) whose fp32 partials the following norm kernel sums in
// fixed order.  Four parts of at least 2048 (the 2B down projection: 66.6 ->
// 46.0 us for a 738-row prompt pair, 2 % slower for 438 + 300 rows encoded
// apart), else two of at least 512 (the output projection; 2B shapes encoded
// apart: 14.3 ms unsplit, 10.7 ms in two).  The factor depends on K only, so
// a row's sums do not depend on the other rows of the encode.
int split_k(int64_t K) {
    if (K % 256 == 0 && K / 4 >= 2048) return 4;
    return K % 128 == 0 && K / 2 >= 512 ? 2 : 1;
}

// decode_embeddings (src/gemma_encoder.cpp:95-152) on device token ids, for
// one or more independent sequences at once: their rows share every
// per-token kernel (norms, the projections, GeGLU) and only the attention
// (RoPE positions, scores, softmax, P.V) runs per sequence.  Each row's
// result is bit-identical to encoding its sequence alone: the per-row
// arithmetic and its order do not depend on the other rows.
void encode(sana_gemma * g, const std::vector<Seq> & seqs, hipStream_t s) {
    const sana_gemma_config & c = g->cfg;
    const int64_t H = c.hidden, F = c.ffn, d = c.head_dim, nh = c.heads, nkv = c.kv_heads;
    const int64_t Dq = g->Dq, Dkv = g->Dkv, Dqkv = Dq + 2 * Dkv, grp = nh / nkv;
    const int64_t M = seqs.back().row0 + seqs.back().T;
    hipLaunchKernelGGL(gemma_embed_kernel, dim3(blocks_for(M * H)), dim3(256), 0, s, g->tok.as<int32_t>(),
                       g->emb16.as<f16>(), g->x32.as<float>(), (int)M, (int)H, std::sqrt((float)H));
    launch_check(hipGetLastError(), "gemma embed");
    half_t * a16 = g->a16.as<half_t>();
    for (int64_t l = 0; l < c.layers; ++l) {
        LayerDev & L = *g->layers[l];
        // the pre-attention norm: layer 0 here, later layers in the previous
        // layer's last norm launch
        if (l == 0) norm(g, g->x32.as<float>(), M, L.n_attn, 0, a16, nullptr, s);
        gemm(a16, H, L.wqkv.as<half_t>(), H, M, Dqkv, H, nullptr, 0, g->qkv32.as<float>(), Dqkv, s);
        const int window = (c.sliding_window > 0 && l % 2 == 0) ? (int)c.sliding_window : 0;
        // sequences 1, 3, ... on the second stream (their buffers are disjoint)
        const bool two = seqs.size() > 1;
        if (two) {
            hip_check(hipEventRecord(g->ev_fork, s), "hipEventRecord");
            hip_check(hipStreamWaitEvent(g->stream2, g->ev_fork, 0), "hipStreamWaitEvent");
        }
        for (size_t si = 0; si < seqs.size(); ++si) {
            const Seq & q = seqs[si];
            const hipStream_t ss = (si & 1) ? g->stream2 : s;
            const int64_t T = q.T, Tp = q.Tp;
            half_t * q16 = g->q16.as<half_t>() + q.row0 * Dq;
            half_t * k16 = g->k16.as<half_t>() + q.row0 * Dkv;
            half_t * vt16 = g->vt16.as<half_t>() + q.vt_off;
            float * s32 = g->s32.as<float>() + q.att_off;
            half_t * p16 = g->p16.as<half_t>() + q.att_off;
            const int64_t n = T * (nh + nkv) * (d / 2) + nkv * d * Tp;
            hipLaunchKernelGGL(gemma_qkv_kernel, dim3(blocks_for(n)), dim3(256), 0, ss,
                               g->qkv32.as<float>() + q.row0 * Dqkv, (int)T, (int)Tp, (int)nh, (int)nkv, (int)d,
                               c.rope_theta, c.query_scale, reinterpret_cast<f16 *>(q16),
                               reinterpret_cast<f16 *>(k16), reinterpret_cast<f16 *>(vt16));
            launch_check(hipGetLastError(), "gemma qkv");
            // scores of all heads in one launch: head h uses K head h / grp
            gemm_batched(q16, Dq, d, k16, Dkv, d, (int)grp, T, T, d, nullptr, 0, 0, s32, Tp, T * Tp, (int)nh, ss);
            {
                const dim3 sg((unsigned)((nh * T + 3) / 4)), sb(256);
                f16 * pp = reinterpret_cast<f16 *>(p16);
#define SANA_GEMMA_SOFTMAX(nj)                                                                                 \
    hipLaunchKernelGGL((gemma_softmax_kernel<nj>), sg, sb, 0, ss, s32, pp, (int)nh, (int)T, (int)Tp, c.attn_softcap, \
                       window)
                // Tp <= 64 NJ (token counts up to 8192: Tp <= 8192)
                if (Tp <= 512) SANA_GEMMA_SOFTMAX(8);
                else if (Tp <= 1024) SANA_GEMMA_SOFTMAX(16);
                else if (Tp <= 2048) SANA_GEMMA_SOFTMAX(32);
                else if (Tp <= 4096) SANA_GEMMA_SOFTMAX(64);
                else SANA_GEMMA_SOFTMAX(128);
#undef SANA_GEMMA_SOFTMAX
                launch_check(hipGetLastError(), "gemma softmax");
            }
            gemm_batched(p16, Tp, T * Tp, vt16, Tp, d * Tp, (int)grp, T, d, Tp, g->o16.as<half_t>() + q.row0 * Dq,
                         Dq, d, nullptr, 0, 0, (int)nh, ss);
        }
        if (two) {
            hip_check(hipEventRecord(g->ev_join, g->stream2), "hipEventRecord");
            hip_check(hipStreamWaitEvent(s, g->ev_join, 0), "hipStreamWaitEvent");
        }
        const int so = split_k(Dq);
        gemm_batched(g->o16.as<half_t>(), Dq, Dq / so, L.wo.as<half_t>(), Dq, Dq / so, 1, M, H, Dq / so, nullptr, 0,
                     0, g->y32.as<float>(), H, M * H, so, s);
        // x += post-attention norm of the projection, then the pre-FFN norm
        norm(g, g->y32.as<float>(), M, L.n_post_attn, 3, a16, g->x32.as<float>(), s, so, &L.n_ffn);
        gemm(a16, H, L.wgu.as<half_t>(), H, M, 2 * F, H, g->g16.as<half_t>(), F, nullptr, 0, s, sana::kActGeglu);
        const int sd = split_k(F);
        gemm_batched(g->g16.as<half_t>(), F, F / sd, L.wdown.as<half_t>(), F, F / sd, 1, M, H, F / sd, nullptr, 0, 0,
                     g->y32.as<float>(), H, M * H, sd, s);
        // x += post-FFN norm, then the next layer's pre-attention norm
        if (l + 1 < c.layers)
            norm(g, g->y32.as<float>(), M, L.n_post_ffw, 3, a16, g->x32.as<float>(), s, sd,
                 &g->layers[l + 1]->n_attn);
        else
            norm(g, g->y32.as<float>(), M, L.n_post_ffw, 1, nullptr, g->x32.as<float>(), s, sd);
    }
    norm(g, g->x32.as<float>(), M, g->out_norm, 2, nullptr, g->out32.as<float>(), s);
}

// Encodes the token sequences seqs[i] (host ids, lengths lens[i]) into
// hidden[i] (host, lens[i] x hidden floats) through the cached graph of
// this length list.
void run_encode(sana_gemma * g, const std::vector<const int32_t *> & toks, const std::vector<int64_t> & lens,
                const std::vector<float *> & hidden) {
    hip_check(hipSetDevice(g->cfg.device), "hipSetDevice");
    check_ready(g);
    int64_t total = 0;
    for (size_t i = 0; i < lens.size(); ++i) {
        const int64_t n = lens[i];
        if (n <= 0 || n > 8192) throw_err(SANA_ERR_INVALID_ARGUMENT, "gemma token count must be in [1, 8192]");
        for (int64_t j = 0; j < n; ++j)
            if (toks[i][j] < 0 || toks[i][j] >= g->cfg.vocab)
                throw_err(SANA_ERR_INVALID_ARGUMENT, "gemma token id out of range at position " + std::to_string(j) +
                                                         (lens.size() > 1 ? " of sequence " + std::to_string(i) : ""));
        total += n;
    }
    if (total > 16384) throw_err(SANA_ERR_INVALID_ARGUMENT, "gemma token count of one encode must be <= 16384");
    const std::vector<Seq> seqs = layout(g, lens);
    ensure_workspace(g, seqs);
    for (size_t i = 0; i < lens.size(); ++i)
        hip_check(hipMemcpyAsync(g->tok.as<int32_t>() + seqs[i].row0, toks[i], (size_t)lens[i] * 4,
                                 hipMemcpyHostToDevice, g->stream),
                  "upload tokens");
    auto it = g->graphs.find(lens);
    if (it == g->graphs.end()) {
        if (g->graphs.size() >= 8) drop_graphs(g);
        hipGraph_t graph = nullptr;
        hip_check(hipStreamBeginCapture(g->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        try {
            encode(g, seqs, g->stream);
        } catch (...) {
            (void)hipStreamEndCapture(g->stream, &graph);
            if (graph) (void)hipGraphDestroy(graph);
            throw;
        }
        hip_check(hipStreamEndCapture(g->stream, &graph), "hipStreamEndCapture");
        hipGraphExec_t exec = nullptr;
        const hipError_t r = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        hip_check(r, "hipGraphInstantiate");
        it = g->graphs.emplace(lens, exec).first;
    }
    hip_check(hipGraphLaunch(it->second, g->stream), "hipGraphLaunch");
    for (size_t i = 0; i < lens.size(); ++i)
        hip_check(hipMemcpyAsync(hidden[i], g->out32.as<float>() + seqs[i].row0 * g->cfg.hidden,
                                 (size_t)lens[i] * g->cfg.hidden * 4, hipMemcpyDeviceToHost, g->stream),
                  "download hidden");
    hip_check(hipStreamSynchronize(g->stream), "gemma encode");
}

void validate_config(const sana_gemma_config * c) {
    auto bad = [](const char * m) { throw_err(SANA_ERR_INVALID_ARGUMENT, m); };
    if (c->vocab <= 0 || c->layers <= 0 || c->heads <= 0 || c->kv_heads <= 0) bad("gemma sizes must be positive");
    if (c->heads % c->kv_heads) bad("gemma query heads must be a multiple of the kv heads");
    if (c->hidden <= 0 || c->hidden % 64 || c->hidden > 4096) bad("gemma hidden size must be a multiple of 64 up to 4096");
    if (c->head_dim <= 0 || c->head_dim % 64) bad("gemma head dim must be a multiple of 64");
    if (c->ffn <= 0 || c->ffn % 64) bad("gemma FFN width must be a multiple of 64");
    if (!(c->rms_eps > 0.0f) || !(c->rope_theta > 0.0f) || !(c->attn_softcap > 0.0f) || !(c->query_scale > 0.0f))
        bad("gemma eps, rope theta, soft-cap and query scale must be positive");
    if (c->sliding_window < 0) bad("gemma sliding window must be >= 0");
}

}  // namespace

extern "C" {

int sana_gemma_create(const sana_gemma_config * cfg, sana_gemma ** out) {
    if (!cfg || !out) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    return guarded([&] {
        validate_config(cfg);
        int ndev = 0;
        hip_check(hipGetDeviceCount(&ndev), "hipGetDeviceCount");
        if (cfg->device < 0 || cfg->device >= ndev) throw_err(SANA_ERR_INVALID_ARGUMENT, "no such device");
        hip_check(hipSetDevice(cfg->device), "hipSetDevice");
        auto g = std::make_unique<sana_gemma>();
        g->cfg = *cfg;
        g->Dq = cfg->heads * cfg->head_dim;
        g->Dkv = cfg->kv_heads * cfg->head_dim;
        for (int64_t l = 0; l < cfg->layers; ++l) g->layers.push_back(std::make_unique<LayerDev>());
        g->required = required_names(g.get());
        hip_check(hipStreamCreateWithFlags(&g->stream, hipStreamNonBlocking), "hipStreamCreate");
        hip_check(hipStreamCreateWithFlags(&g->stream2, hipStreamNonBlocking), "hipStreamCreate");
        hip_check(hipEventCreateWithFlags(&g->ev_fork, hipEventDisableTiming), "hipEventCreate");
        hip_check(hipEventCreateWithFlags(&g->ev_join, hipEventDisableTiming), "hipEventCreate");
        *out = g.release();
    });
}

int sana_gemma_destroy(sana_gemma * g) {
    if (!g) return SANA_OK;
    (void)hipSetDevice(g->cfg.device);
    (void)hipDeviceSynchronize();
    delete g;
    return SANA_OK;
}

int sana_gemma_set_weight(sana_gemma * g, const char * name, const float * data, const int64_t * shape, int ndim) {
    if (!g || !name || !data || !shape) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    return guarded([&] {
        hip_check(hipSetDevice(g->cfg.device), "hipSetDevice");
        set_weight(g, name, data, shape, ndim);
    });
}

int sana_gemma_check_weights(sana_gemma * g) {
    if (!g) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    return guarded([&] { check_ready(g); });
}

int sana_gemma_load_gguf(sana_gemma * g, const char * path) {
    if (!g || !path) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    return guarded([&] {
        using namespace sana::gguf;
        hip_check(hipSetDevice(g->cfg.device), "hipSetDevice");
        Index idx;
        try {
            idx = read_index(path);
        } catch (const std::exception & e) {
            throw_err(SANA_ERR_IO, e.what());
        }
        MappedFile f(path);
        std::map<std::string, const TensorInfo *> by;
        for (const auto & t : idx.tensors) by[t.name] = &t;
        std::vector<float> tmp;
        for (const std::string & n : g->required) {
            auto it = by.find(n);
            if (it == by.end()) throw_err(SANA_ERR_INVALID_ARGUMENT, "weight name not found in weight index: " + n);
            const TensorInfo & t = *it->second;
            size_t cnt = 1;
            for (int64_t dd : t.shape) cnt *= (size_t)dd;
            const float * src;
            if (t.type == kF32) {
                src = reinterpret_cast<const float *>(f.data() + t.offset);
            } else if (t.type == kF16 || t.type == kBF16) {
                tmp.resize(cnt);
                const uint16_t * h = reinterpret_cast<const uint16_t *>(f.data() + t.offset);
                for (size_t i = 0; i < cnt; ++i) {
                    if (t.type == kF16) {
                        _Float16 x;
                        std::memcpy(&x, h + i, 2);
                        tmp[i] = (float)x;
                    } else {
                        const uint32_t u = (uint32_t)h[i] << 16;
                        std::memcpy(&tmp[i], &u, 4);
                    }
                }
                src = tmp.data();
            } else {
                throw_err(SANA_ERR_FORMAT, "unsupported gguf tensor type for " + t.name);
            }
            set_weight(g, n, src, t.shape.data(), (int)t.shape.size());
        }
    });
}

int sana_gemma_encode(sana_gemma * g, const int32_t * tokens, int64_t n, float * hidden) {
    if (!g || !tokens || !hidden) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    return guarded([&] { run_encode(g, {tokens}, {n}, {hidden}); });
}

int sana_gemma_encode_pair(sana_gemma * g, const int32_t * tokens_a, int64_t na, const int32_t * tokens_b,
                           int64_t nb, float * hidden_a, float * hidden_b) {
    if (!g || !tokens_a || !tokens_b || !hidden_a || !hidden_b)
        return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    return guarded([&] { run_encode(g, {tokens_a, tokens_b}, {na, nb}, {hidden_a, hidden_b}); });
}

}  // extern "C"
