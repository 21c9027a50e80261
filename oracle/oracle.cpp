// CPU restatement of sana.cpp's Linux DiT path -- TEST INFRASTRUCTURE ONLY.
// See oracle.h for the contract.  Each routine cites the reference lines whose
// loop and accumulation order it reproduces.  Build: oracle/Makefile
// (-O3 -ffp-contract=off, no -ffast-math, so nothing is contracted or
// re-associated and results match the reference bit for bit).
#include "oracle.h"
#include "model_spec.h"
#include "vae_spec.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <random>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace {

thread_local std::string g_err;
int g_threads = 0;

int fail(const std::string & m) {
    g_err = m;
    return -1;
}

int n_threads() {
    if (g_threads > 0) return g_threads;
    unsigned hc = std::thread::hardware_concurrency();
    return static_cast<int>(std::min(16u, std::max(1u, hc)));
}

// Run fn(begin, end) over [0, n) split into contiguous chunks, one per thread.
template <class F>
void parallel_rows(size_t n, F fn) {
    const int T = std::min<int>(n_threads(), static_cast<int>(std::max<size_t>(1, n / 8)));
    if (T <= 1 || n < 16) {
        fn(size_t(0), n);
        return;
    }
    std::vector<std::thread> th;
    const size_t chunk = (n + T - 1) / T;
    for (int t = 0; t < T; ++t) {
        const size_t b = t * chunk, e = std::min(n, b + chunk);
        if (b >= e) break;
        th.emplace_back([=] { fn(b, e); });
    }
    for (auto & x : th) x.join();
}

std::vector<float> transpose(const float * w, size_t rows, size_t cols) {
    std::vector<float> t(rows * cols);
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < cols; ++c) t[c * rows + r] = w[r * cols + c];
    return t;
}

// C[m, n] = (bias ? bias[n] : 0) then C[m, n] += A[m, k] * WT[k, n] for k = 0..K-1
// in order: the i-k-j loop of gemm_row_major (src/common_ops.cpp:49-64) and the
// bias-initialised tile of conv2d_1x1_blocked (:282-298).  Rows are blocked by 8
// and columns by 256 only to reuse cache; each C[m, n] still sees the same
// sequence of roundings.
void gemm_ikj(const float * A, size_t lda, const float * WT, const float * bias, float * C, size_t ldc,
              size_t M, size_t K, size_t N) {
    parallel_rows((M + 7) / 8, [&](size_t rb0, size_t rb1) {
        for (size_t rb = rb0; rb < rb1; ++rb) {
            const size_t m0 = rb * 8, m1 = std::min(M, m0 + 8);
            for (size_t n0 = 0; n0 < N; n0 += 256) {
                const size_t n1 = std::min(N, n0 + 256);
                for (size_t m = m0; m < m1; ++m)
                    for (size_t n = n0; n < n1; ++n) C[m * ldc + n] = bias ? bias[n] : 0.0f;
                for (size_t k = 0; k < K; ++k) {
                    const float * w = WT + k * N;
                    for (size_t m = m0; m < m1; ++m) {
                        const float a = A[m * lda + k];
                        float * c = C + m * ldc;
                        for (size_t n = n0; n < n1; ++n) c[n] += a * w[n];
                    }
                }
            }
        }
    });
}

// Linear with a PyTorch-order weight [N, K].
void linear(const float * in, const float * w, const float * bias, float * out, size_t M, size_t K, size_t N) {
    std::vector<float> wt = transpose(w, N, K);
    gemm_ikj(in, K, wt.data(), bias, out, N, M, K, N);
}

inline float silu(float x) { return x / (1.0f + std::exp(-x)); }  // src/tensor.cpp:551-555

inline float gelu_tanh(float x) {  // src/transformer_ops.cpp:15-18
    const float a = std::sqrt(2.0f / static_cast<float>(M_PI));
    return 0.5f * x * (1.0f + std::tanh(a * (x + 0.044715f * x * x * x)));
}

// src/tensor.cpp:235-268 (#else): sequential mean, two-pass variance.
void layer_norm(const float * x, const float * g, const float * b, float * out, size_t rows, size_t C, float eps) {
    parallel_rows(rows, [&](size_t r0, size_t r1) {
        for (size_t r = r0; r < r1; ++r) {
            const float * row = x + r * C;
            float * o = out + r * C;
            float mean = 0.0f;
            for (size_t h = 0; h < C; ++h) mean += row[h];
            mean /= static_cast<float>(C);
            float var = 0.0f;
            for (size_t h = 0; h < C; ++h) {
                const float d = row[h] - mean;
                var += d * d;
            }
            var /= static_cast<float>(C);
            const float inv = 1.0f / std::sqrt(var + eps);
            for (size_t h = 0; h < C; ++h) {
                float v = (row[h] - mean) * inv;
                if (g) v *= g[h];
                if (b) v += b[h];
                o[h] = v;
            }
        }
    });
}

// src/tensor.cpp:276-316.
void rms_norm(const float * x, const float * w, float * out, size_t rows, size_t C, float eps) {
    parallel_rows(rows, [&](size_t r0, size_t r1) {
        for (size_t r = r0; r < r1; ++r) {
            const float * row = x + r * C;
            float ms = 0.0f;
            for (size_t h = 0; h < C; ++h) ms += row[h] * row[h];
            ms /= static_cast<float>(C);
            const float inv = 1.0f / std::sqrt(ms + eps);
            for (size_t h = 0; h < C; ++h) {
                float v = row[h] * inv;
                if (w) v *= w[h];
                out[r * C + h] = v;
            }
        }
    });
}

// src/tensor.cpp:364-372; shift/scale rows are taken with stride `mod_stride`.
void modulate(const float * x, const float * shift, const float * scale, size_t mod_stride, float * out,
              size_t B, size_t N, size_t C) {
    for (size_t b = 0; b < B; ++b)
        for (size_t t = 0; t < N; ++t)
            for (size_t h = 0; h < C; ++h) {
                const size_t i = (b * N + t) * C + h;
                out[i] = x[i] * (1.0f + scale[b * mod_stride + h]) + shift[b * mod_stride + h];
            }
}

// src/transformer_ops.cpp:496-537 on token-major tensors with row stride ld.
void linear_attention(const float * q, const float * k, const float * v, float * out, size_t ld,
                      size_t B, size_t Nq, size_t Nkv, size_t H, size_t D) {
    parallel_rows(B * H, [&](size_t p0, size_t p1) {
        std::vector<float> S((D + 1) * D);
        for (size_t p = p0; p < p1; ++p) {
            const size_t b = p / H, h = p % H;
            std::fill(S.begin(), S.end(), 0.0f);
            for (size_t t = 0; t < Nkv; ++t) {
                const float * kr = k + (b * Nkv + t) * ld + h * D;
                const float * vr = v + (b * Nkv + t) * ld + h * D;
                for (size_t d = 0; d < D; ++d) {
                    const float kv = std::max(0.0f, kr[d]);
                    for (size_t r = 0; r < D; ++r) S[r * D + d] += vr[r] * kv;
                    S[D * D + d] += kv;
                }
            }
            for (size_t t = 0; t < Nq; ++t) {
                const float * qr = q + (b * Nq + t) * ld + h * D;
                float * o = out + (b * Nq + t) * ld + h * D;
                for (size_t r = 0; r < D; ++r) {
                    float num = 0.0f;
                    for (size_t d = 0; d < D; ++d) num += S[r * D + d] * std::max(0.0f, qr[d]);
                    o[r] = num;
                }
                float den = 0.0f;
                for (size_t d = 0; d < D; ++d) den += S[D * D + d] * std::max(0.0f, qr[d]);
                den += 1e-15f;
                for (size_t r = 0; r < D; ++r) o[r] /= den;
            }
        }
    });
}

// attention_4d: scores via gemm_row_major(b_transposed) (src/transformer_ops.cpp:178-225),
// * float(1/sqrt(double(D))) (:355, std::sqrt of an integer is double), + bias (:357-388),
// softmax (:318-335), P.V via gemm_row_major (:232-273).
void attention(const float * q, const float * k, const float * v, const float * bias, float * out,
               size_t ldq, size_t ldkv, size_t B, size_t Nq, size_t L, size_t H, size_t D) {
    const float scale = static_cast<float>(1.0f / std::sqrt(static_cast<double>(D)));
    parallel_rows(B * H * Nq, [&](size_t r0, size_t r1) {
        std::vector<float> s(L);
        for (size_t r = r0; r < r1; ++r) {
            const size_t b = r / (H * Nq), h = (r / Nq) % H, i = r % Nq;
            const float * qr = q + (b * Nq + i) * ldq + h * D;
            for (size_t j = 0; j < L; ++j) s[j] = 0.0f;
            for (size_t d = 0; d < D; ++d) {
                const float a = qr[d];
                for (size_t j = 0; j < L; ++j) s[j] += a * k[(b * L + j) * ldkv + h * D + d];
            }
            for (size_t j = 0; j < L; ++j) s[j] *= scale;
            if (bias)
                for (size_t j = 0; j < L; ++j) s[j] += bias[b * L + j];
            float mx = s[0];
            for (size_t j = 0; j < L; ++j)
                if (s[j] > mx) mx = s[j];
            float den = 0.0f;
            for (size_t j = 0; j < L; ++j) {
                const float e = std::exp(s[j] - mx);
                s[j] = e;
                den += e;
            }
            const float rc = 1.0f / den;
            for (size_t j = 0; j < L; ++j) s[j] *= rc;
            float * o = out + (b * Nq + i) * ldq + h * D;
            for (size_t d = 0; d < D; ++d) o[d] = 0.0f;
            for (size_t j = 0; j < L; ++j) {
                const float a = s[j];
                for (size_t d = 0; d < D; ++d) o[d] += a * v[(b * L + j) * ldkv + h * D + d];
            }
        }
    });
}

// src/common_ops.cpp:483-505: taps in (ky, kx) order, skipped outside the grid, bias last.
void depthwise3x3(const float * x, const float * w, const float * bias, float * out, size_t B, size_t Hh,
                  size_t Ww, size_t C) {
    parallel_rows(B * Hh, [&](size_t r0, size_t r1) {
        for (size_t r = r0; r < r1; ++r) {
            const size_t b = r / Hh, y = r % Hh;
            for (size_t xx = 0; xx < Ww; ++xx)
                for (size_t c = 0; c < C; ++c) {
                    float sum = 0.0f;
                    for (int ky = 0; ky < 3; ++ky)
                        for (int kx = 0; kx < 3; ++kx) {
                            const long iy = static_cast<long>(y) + ky - 1, ix = static_cast<long>(xx) + kx - 1;
                            if (iy >= 0 && iy < static_cast<long>(Hh) && ix >= 0 && ix < static_cast<long>(Ww))
                                sum += x[((b * Hh + iy) * Ww + ix) * C + c] * w[c * 9 + ky * 3 + kx];
                        }
                    if (bias) sum += bias[c];
                    out[((b * Hh + y) * Ww + xx) * C + c] = sum;
                }
        }
    });
}

// src/common_ops.cpp:733-761 in token-major layout (the grid transposes of
// src/transformer.cpp:765-774 are pure data movement).
void glumb_conv(const float * x, const float * inv_w, const float * inv_b, const float * dw_w,
                const float * dw_b, const float * pt_w, float * out, size_t B, size_t Hh, size_t Ww,
                size_t Cin, size_t E, size_t Cout) {
    const size_t M = B * Hh * Ww, F = E / 2;
    std::vector<float> hid(M * E), dw(M * E), glu(M * F);
    linear(x, inv_w, inv_b, hid.data(), M, Cin, E);
    for (float & v : hid) v = silu(v);
    depthwise3x3(hid.data(), dw_w, dw_b, dw.data(), B, Hh, Ww, E);
    for (size_t m = 0; m < M; ++m)
        for (size_t f = 0; f < F; ++f) glu[m * F + f] = dw[m * E + f] * silu(dw[m * E + F + f]);
    linear(glu.data(), pt_w, nullptr, out, M, F, Cout);
}

void caption_projection(const float * x, const float * w1, const float * b1, const float * w2, const float * b2,
                        const float * nw, float * out, size_t rows, size_t Cin, size_t C) {
    std::vector<float> h(rows * C), p(rows * C);
    linear(x, w1, b1, h.data(), rows, Cin, C);
    for (float & v : h) v = gelu_tanh(v);
    linear(h.data(), w2, b2, p.data(), rows, C, C);
    rms_norm(p.data(), nw, out, rows, C, 1e-5f);
}

// src/transformer.cpp:77-122 (#else).
void timestep_embedding(const float * t, float * out, size_t B, size_t dim) {
    const size_t half = dim / 2;
    std::vector<float> freq(half);
    const float ls = -std::log(10000.0f) / static_cast<float>(half);
    for (size_t i = 0; i < half; ++i) freq[i] = std::exp(static_cast<float>(i) * ls);
    for (size_t b = 0; b < B; ++b) {
        for (size_t i = 0; i < half; ++i) {
            const float v = t[b] * freq[i];
            out[b * dim + i] = std::cos(v);
            out[b * dim + half + i] = std::sin(v);
        }
        if (dim % 2 == 1) out[b * dim + dim - 1] = 0.0f;
    }
}

// src/transformer.cpp:726-778 on token-major tensors.
void block_forward(const oracle_block_weights & w, const float * x, const float * ctx, const float * t_mod,
                   const float * bias, size_t B, size_t N, size_t L, float * after_self, float * after_cross,
                   float * after_ff) {
    const size_t C = w.hidden, E = w.ffn, M = B * N;
    size_t side = static_cast<size_t>(std::sqrt(static_cast<double>(N)));
    if (side * side != N) throw std::invalid_argument("token count must form a square grid");
    // compute_sana_block_modulation (src/transformer.cpp:521-531)
    std::vector<float> mod(B * 6 * C);
    for (size_t b = 0; b < B; ++b)
        for (size_t i = 0; i < 6 * C; ++i) mod[b * 6 * C + i] = t_mod[b * 6 * C + i] + w.scale_shift_table[i];
    const float * m0 = mod.data();
    std::vector<float> xn(M * C), a(M * C), q(M * C), k(M * C), v(M * C), o(M * C), br(M * C);
    layer_norm(x, w.attn_norm_gamma, w.attn_norm_beta, xn.data(), M, C, 1e-6f);
    modulate(xn.data(), m0 + 0 * C, m0 + 1 * C, 6 * C, a.data(), B, N, C);
    linear(a.data(), w.q_w, w.q_b, q.data(), M, C, C);
    linear(a.data(), w.k_w, w.k_b, k.data(), M, C, C);
    linear(a.data(), w.v_w, w.v_b, v.data(), M, C, C);
    linear_attention(q.data(), k.data(), v.data(), o.data(), C, B, N, N, w.self_heads, C / w.self_heads);
    linear(o.data(), w.out_w, w.out_b, br.data(), M, C, C);
    for (size_t b = 0; b < B; ++b)
        for (size_t t = 0; t < N; ++t)
            for (size_t h = 0; h < C; ++h) br[(b * N + t) * C + h] *= m0[b * 6 * C + 2 * C + h];
    for (size_t i = 0; i < M * C; ++i) after_self[i] = x[i] + br[i];
    // cross attention (src/transformer_ops.cpp:572-608)
    std::vector<float> kc(B * L * C), vc(B * L * C);
    linear(after_self, w.cq_w, w.cq_b, q.data(), M, C, C);
    linear(ctx, w.ck_w, w.ck_b, kc.data(), B * L, C, C);
    linear(ctx, w.cv_w, w.cv_b, vc.data(), B * L, C, C);
    attention(q.data(), kc.data(), vc.data(), bias, o.data(), C, C, B, N, L, w.cross_heads, C / w.cross_heads);
    linear(o.data(), w.co_w, w.co_b, br.data(), M, C, C);
    for (size_t i = 0; i < M * C; ++i) after_cross[i] = after_self[i] + br[i];
    // Mix-FFN
    layer_norm(after_cross, w.mlp_norm_gamma, w.mlp_norm_beta, xn.data(), M, C, 1e-6f);
    modulate(xn.data(), m0 + 3 * C, m0 + 4 * C, 6 * C, a.data(), B, N, C);
    glumb_conv(a.data(), w.inv_w, w.inv_b, w.dw_w, w.dw_b, w.pt_w, br.data(), B, side, side, C, E, C);
    for (size_t b = 0; b < B; ++b)
        for (size_t t = 0; t < N; ++t)
            for (size_t h = 0; h < C; ++h) br[(b * N + t) * C + h] *= m0[b * 6 * C + 5 * C + h];
    for (size_t i = 0; i < M * C; ++i) after_ff[i] = after_cross[i] + br[i];
}

// attention_block_3d (src/transformer_ops.cpp:545-570).
void attention_block(const float * x, const float * wq, const float * bq, const float * wk, const float * bk,
                     const float * wv, const float * bv, const float * wo, const float * bo, float * out, size_t B,
                     size_t N, size_t C, size_t heads) {
    const size_t M = B * N;
    std::vector<float> q(M * C), k(M * C), v(M * C), o(M * C);
    linear(x, wq, bq, q.data(), M, C, C);
    linear(x, wk, bk, k.data(), M, C, C);
    linear(x, wv, bv, v.data(), M, C, C);
    linear_attention(q.data(), k.data(), v.data(), o.data(), C, B, N, N, heads, C / heads);
    linear(o.data(), wo, bo, out, M, C, C);
}

// cross_attention_block_3d (src/transformer_ops.cpp:572-608).
void cross_attention_block(const float * x, const float * ctx, const float * bias, const float * wq, const float * bq,
                           const float * wk, const float * bk, const float * wv, const float * bv, const float * wo,
                           const float * bo, float * out, size_t B, size_t N, size_t L, size_t C, size_t heads) {
    const size_t M = B * N;
    std::vector<float> q(M * C), k(B * L * C), v(B * L * C), o(M * C);
    linear(x, wq, bq, q.data(), M, C, C);
    linear(ctx, wk, bk, k.data(), B * L, C, C);
    linear(ctx, wv, bv, v.data(), B * L, C, C);
    attention(q.data(), k.data(), v.data(), bias, o.data(), C, C, B, N, L, heads, C / heads);
    linear(o.data(), wo, bo, out, M, C, C);
}

// ---------------------------------------------------------------- randn
// torch CPU randn as restated in src/torch_rng.cpp:14-68: one mt19937 draw per
// element mapped to a 24-bit uniform, then Box-Muller over blocks of 16
// (first 8 are u1, next 8 are u2); a ragged tail re-draws the last 16.
void normal16(float * d) {
    for (int j = 0; j < 8; ++j) {
        const float u1 = 1.0f - d[j];
        const float u2 = d[j + 8];
        const float rad = std::sqrt(-2.0f * std::log(u1));
        const float th = static_cast<float>(2.0 * 3.14159265358979323846 * static_cast<double>(u2));
        d[j] = rad * std::cos(th);
        d[j + 8] = rad * std::sin(th);
    }
}

inline float uniform24(std::mt19937 & e) {
    return static_cast<float>(static_cast<uint32_t>(e()) & ((1u << 24) - 1)) * (1.0f / static_cast<float>(1u << 24));
}

void randn(float * out, size_t n, uint64_t seed) {
    if (n < 16) throw std::invalid_argument("randn requires at least 16 elements");
    std::mt19937 e(static_cast<std::mt19937::result_type>(seed & 0xffffffffULL));
    for (size_t i = 0; i < n; ++i) out[i] = uniform24(e);
    size_t i = 0;
    for (; i + 16 <= n; i += 16) normal16(out + i);
    if (n % 16 != 0) {
        float * tail = out + n - 16;
        for (size_t j = 0; j < 16; ++j) tail[j] = uniform24(e);
        normal16(tail);
    }
}

// ---------------------------------------------------------------- scheduler
// src/scheduler.cpp:89-141 (flow sigmas, linspace, integer-truncated timesteps)
void schedule(size_t steps, std::vector<float> & ts, std::vector<float> & sig) {
    const float denom = 1000.0f, shift = 3.0f;
    std::vector<float> sh(steps + 1);
    for (size_t i = 0; i <= steps; ++i) {
        const float alpha = 1.0f + (1.0f / denom - 1.0f) * (static_cast<float>(i) / static_cast<float>(steps));
        const float s = 1.0f - alpha;
        sh[i] = shift * s / (1.0f + (shift - 1.0f) * s);
    }
    ts.clear();
    sig.clear();
    for (size_t i = 0; i < steps; ++i) {
        const float s = sh[steps - i];
        sig.push_back(s);
        ts.push_back(static_cast<float>(static_cast<int>(s * denom)));
    }
    sig.push_back(0.0f);
}

struct SchedState {
    std::vector<float> ts, sig;
    size_t step = 0, lower = 0;
    std::vector<std::vector<float>> prev;
};

float lambda_of(float sigma) {  // flow sigmas: alpha = 1 - sigma (src/scheduler.cpp:71-81)
    return std::log(1.0f - sigma) - std::log(sigma);
}

// convert_sana_scheduler_model_output (src/scheduler.cpp:155-173): x0 = sample - sigma * v.
void sched_convert(const float * mo, const float * sample, size_t n, float sigma, float * out) {
    for (size_t i = 0; i < n; ++i) out[i] = sample[i] - sigma * mo[i];
}

// sana_scheduler_first_order_update (src/scheduler.cpp:175-205).
void sched_first(const float * conv, const float * sample, size_t n, float st_v, float ss_v, float * out) {
    const float alpha_t = 1.0f - st_v, sigma_t = st_v, sigma_s = ss_v;
    const float h = lambda_of(st_v) - lambda_of(ss_v);
    const float a = sigma_t / sigma_s, bcoef = -alpha_t * (std::exp(-h) - 1.0f);
    for (size_t i = 0; i < n; ++i) out[i] = a * sample[i] + bcoef * conv[i];
}

// sana_scheduler_second_order_update, midpoint (src/scheduler.cpp:207-260).
void sched_second(const float * sample, const float * m0, const float * m1, size_t n, float st_v, float s0_v,
                  float s1_v, float * out) {
    const float alpha_t = 1.0f - st_v, sigma_t = st_v, sigma_s0 = s0_v;
    const float lt = lambda_of(st_v), l0 = lambda_of(s0_v), l1 = lambda_of(s1_v);
    const float h = lt - l0, h0 = l0 - l1, r0 = h0 / h;
    const float a = sigma_t / sigma_s0, bcoef = -alpha_t * (std::exp(-h) - 1.0f);
    const float ccoef = -0.5f * alpha_t * (std::exp(-h) - 1.0f);
    for (size_t i = 0; i < n; ++i) {
        const float d1 = (1.0f / r0) * (m0[i] - m1[i]);
        out[i] = a * sample[i] + bcoef * m0[i] + ccoef * d1;
    }
}

// step_sana_scheduler (src/scheduler.cpp:272-318) with order 2, midpoint,
// lower_order_final: first order at the first and last step, second order
// otherwise (the "lower_order_second" branch also takes the second-order path).
std::vector<float> sched_step(const std::vector<float> & model_out, const std::vector<float> & sample, SchedState & st) {
    const size_t n = sample.size();
    std::vector<float> conv(n);
    sched_convert(model_out.data(), sample.data(), n, st.sig[st.step], conv.data());
    st.prev.push_back(conv);
    if (st.prev.size() > 2) st.prev.erase(st.prev.begin());
    const bool last = st.step == st.ts.size() - 1;
    std::vector<float> out(n);
    if (st.lower < 1 || last) {
        sched_first(conv.data(), sample.data(), n, st.sig[st.step + 1], st.sig[st.step], out.data());
    } else {
        const std::vector<float> & m0 = st.prev.back();
        const std::vector<float> & m1 = st.prev[st.prev.size() - 2];
        sched_second(sample.data(), m0.data(), m1.data(), n, st.sig[st.step + 1], st.sig[st.step],
                     st.sig[st.step - 1], out.data());
    }
    if (st.lower < 2) st.lower += 1;
    st.step += 1;
    return out;
}

}  // namespace

// ================================================================= model
struct oracle_model {
    size_t layers, C, E, Ccap, Cl, self_heads, cross_heads;
    std::map<std::string, std::vector<float>> t;
    std::vector<float> ones, zeros;

    const float * p(const std::string & n) const {
        auto it = t.find(n);
        if (it == t.end()) throw std::invalid_argument("weight not set: " + n);
        return it->second.data();
    }
    oracle_block_weights block(size_t i) const {
        const std::string b = "transformer_blocks." + std::to_string(i) + ".";
        oracle_block_weights w;
        w.scale_shift_table = p(b + "scale_shift_table");
        w.attn_norm_gamma = ones.data();
        w.attn_norm_beta = zeros.data();
        w.q_w = p(b + "attn1.to_q.weight");
        w.k_w = p(b + "attn1.to_k.weight");
        w.v_w = p(b + "attn1.to_v.weight");
        w.q_b = w.k_b = w.v_b = zeros.data();
        w.out_w = p(b + "attn1.to_out.0.weight");
        w.out_b = p(b + "attn1.to_out.0.bias");
        w.cq_w = p(b + "attn2.to_q.weight");
        w.cq_b = p(b + "attn2.to_q.bias");
        w.ck_w = p(b + "attn2.to_k.weight");
        w.ck_b = p(b + "attn2.to_k.bias");
        w.cv_w = p(b + "attn2.to_v.weight");
        w.cv_b = p(b + "attn2.to_v.bias");
        w.co_w = p(b + "attn2.to_out.0.weight");
        w.co_b = p(b + "attn2.to_out.0.bias");
        w.mlp_norm_gamma = ones.data();
        w.mlp_norm_beta = zeros.data();
        w.inv_w = p(b + "ff.conv_inverted.weight");
        w.inv_b = p(b + "ff.conv_inverted.bias");
        w.dw_w = p(b + "ff.conv_depth.weight");
        w.dw_b = p(b + "ff.conv_depth.bias");
        w.pt_w = p(b + "ff.conv_point.weight");
        w.hidden = C;
        w.ffn = E;
        w.self_heads = self_heads;
        w.cross_heads = cross_heads;
        return w;
    }
    sana_spec::Dims dims() const {
        sana_spec::Dims d;
        d.layers = layers;
        d.hidden = C;
        d.ffn = E;
        d.caption = Ccap;
        d.latent = Cl;
        return d;
    }
};

namespace {

void model_time(const oracle_model & m, const float * t, size_t B, float * emb, float * tmod) {
    const size_t C = m.C;
    std::vector<float> tp(B * 256), h(B * C), e2(B * C);
    timestep_embedding(t, tp.data(), B, 256);
    linear(tp.data(), m.p("time_embed.emb.timestep_embedder.linear_1.weight"),
           m.p("time_embed.emb.timestep_embedder.linear_1.bias"), h.data(), B, 256, C);
    for (float & v : h) v = silu(v);
    linear(h.data(), m.p("time_embed.emb.timestep_embedder.linear_2.weight"),
           m.p("time_embed.emb.timestep_embedder.linear_2.bias"), emb, B, C, C);
    for (size_t i = 0; i < B * C; ++i) e2[i] = silu(emb[i]);
    linear(e2.data(), m.p("time_embed.linear.weight"), m.p("time_embed.linear.bias"), tmod, B, C, 6 * C);
}

// conv2d_1x1 patch embed (src/common_ops.cpp:390-403) written token-major.
void model_patch(const oracle_model & m, const float * lat, size_t B, size_t Hh, size_t Ww, float * tok) {
    const size_t S = Hh * Ww, Cl = m.Cl, C = m.C;
    std::vector<float> xt(B * S * Cl);
    for (size_t b = 0; b < B; ++b)
        for (size_t c = 0; c < Cl; ++c)
            for (size_t s = 0; s < S; ++s) xt[(b * S + s) * Cl + c] = lat[(b * Cl + c) * S + s];
    linear(xt.data(), m.p("patch_embed.proj.weight"), m.p("patch_embed.proj.bias"), tok, B * S, Cl, C);
}

void model_forward(const oracle_model & m, const float * latent, size_t Bl, size_t Hh, size_t Ww,
                   const float * ctx, size_t L, const float * bias, float t, float * np_out) {
    const size_t B = 2 * Bl, N = Hh * Ww, C = m.C, Cl = m.Cl, M = B * N;
    std::vector<float> lat(B * Cl * N);
    for (size_t r = 0; r < 2; ++r) std::copy(latent, latent + Bl * Cl * N, lat.begin() + r * Bl * Cl * N);
    std::vector<float> x(M * C), y(M * C), s1(M * C), s2(M * C), emb(B * C), tmod(B * 6 * C), tv(B, t);
    model_patch(m, lat.data(), B, Hh, Ww, x.data());
    model_time(m, tv.data(), B, emb.data(), tmod.data());
    for (size_t i = 0; i < m.layers; ++i) {
        oracle_block_weights w = m.block(i);
        block_forward(w, x.data(), ctx, tmod.data(), bias, B, N, L, s1.data(), s2.data(), y.data());
        std::swap(x, y);
    }
    // final layer (src/transformer.cpp:668-681)
    std::vector<float> nrm(M * C), sh(B * C), sc(B * C), md(M * C), pr(M * Cl);
    layer_norm(x.data(), nullptr, nullptr, nrm.data(), M, C, 1e-6f);
    const float * T = m.p("scale_shift_table");
    for (size_t b = 0; b < B; ++b)
        for (size_t c = 0; c < C; ++c) {
            sh[b * C + c] = emb[b * C + c] + T[c];
            sc[b * C + c] = emb[b * C + c] + T[C + c];
        }
    modulate(nrm.data(), sh.data(), sc.data(), C, md.data(), B, N, C);
    linear(md.data(), m.p("proj_out.weight"), m.p("proj_out.bias"), pr.data(), M, C, Cl);
    for (size_t b = 0; b < B; ++b)
        for (size_t s = 0; s < N; ++s)
            for (size_t c = 0; c < Cl; ++c) np_out[(b * Cl + c) * N + s] = pr[(b * N + s) * Cl + c];
}


// ================================================================ VAE decoder
// NCHW fp32, as the reference's src/vae.cpp and src/vae_ops.cpp (Linux #else
// branches).  Every output element sees the reference's sequence of fp32
// roundings; zero-padding taps are skipped, which leaves every sum unchanged
// (adding a +-0 product to a running sum that starts at +0 or at a bias never
// changes it).

// 3x3 same conv.  conv2d_3x3_same_dispatch (src/vae_ops.cpp:196-222) picks
// im2col + gemm_row_major (:18-95: sum from 0 over k = (ic, ky, kx), bias added
// after) when Cin*9*H*W <= 9e8, else tap accumulation (:104-194: bias first,
// taps (ky, kx) outer, input channels inner).
void vae_conv3x3(const float * in, const float * w, const float * bias, float * out, size_t B, size_t Cin,
                 size_t Cout, size_t Hh, size_t Ww, int order = -1) {
    const size_t S = Hh * Ww;
    const bool tap_order = order < 0 ? Cin * 9 * S > 900000000ULL : order == 1;
    parallel_rows(B * Cout, [&](size_t r0, size_t r1) {
        for (size_t r = r0; r < r1; ++r) {
            const size_t b = r / Cout, oc = r % Cout;
            float * o = out + r * S;
            const float * xb = in + b * Cin * S;
            const float init = (tap_order && bias) ? bias[oc] : 0.0f;
            for (size_t i = 0; i < S; ++i) o[i] = init;
            auto add_tap = [&](size_t ic, int ky, int kx) {
                const float a = w[((oc * Cin + ic) * 3 + ky) * 3 + kx];
                const float * xc = xb + ic * S;
                for (size_t y = 0; y < Hh; ++y) {
                    const long iy = static_cast<long>(y) + ky - 1;
                    if (iy < 0 || iy >= static_cast<long>(Hh)) continue;
                    const size_t x0 = kx == 0 ? 1 : 0, x1 = kx == 2 ? Ww - 1 : Ww;
                    const float * src = xc + iy * Ww + (kx - 1);
                    float * dst = o + y * Ww;
                    for (size_t x = x0; x < x1; ++x) dst[x] += a * src[x];
                }
            };
            if (!tap_order) {
                for (size_t ic = 0; ic < Cin; ++ic)
                    for (int ky = 0; ky < 3; ++ky)
                        for (int kx = 0; kx < 3; ++kx) add_tap(ic, ky, kx);
                if (bias)
                    for (size_t i = 0; i < S; ++i) o[i] += bias[oc];
            } else {
                for (int ky = 0; ky < 3; ++ky)
                    for (int kx = 0; kx < 3; ++kx)
                        for (size_t ic = 0; ic < Cin; ++ic) add_tap(ic, ky, kx);
            }
        }
    });
}

// conv2d_1x1 (src/common_ops.cpp:247-309, conv2d_1x1_blocked): bias first, then
// input channels in order.
void vae_conv1x1(const float * in, const float * w, const float * bias, float * out, size_t B, size_t Cin,
                 size_t Cout, size_t S) {
    parallel_rows(B * Cout, [&](size_t r0, size_t r1) {
        for (size_t r = r0; r < r1; ++r) {
            const size_t b = r / Cout, oc = r % Cout;
            float * o = out + r * S;
            const float init = bias ? bias[oc] : 0.0f;
            for (size_t i = 0; i < S; ++i) o[i] = init;
            for (size_t ic = 0; ic < Cin; ++ic) {
                const float a = w[oc * Cin + ic];
                const float * x = in + (b * Cin + ic) * S;
                for (size_t i = 0; i < S; ++i) o[i] += a * x[i];
            }
        }
    });
}

// grouped_conv2d_1x1 (src/vae_ops.cpp:243-300): per group gemm_row_major from 0.
void vae_grouped1x1(const float * in, const float * w, float * out, size_t B, size_t Cin, size_t Cout,
                    size_t groups, size_t S) {
    const size_t ipg = Cin / groups, opg = Cout / groups;
    parallel_rows(B * Cout, [&](size_t r0, size_t r1) {
        for (size_t r = r0; r < r1; ++r) {
            const size_t b = r / Cout, oc = r % Cout, g = oc / opg;
            float * o = out + r * S;
            for (size_t i = 0; i < S; ++i) o[i] = 0.0f;
            for (size_t k = 0; k < ipg; ++k) {
                const float a = w[oc * ipg + k];
                const float * x = in + (b * Cin + g * ipg + k) * S;
                for (size_t i = 0; i < S; ++i) o[i] += a * x[i];
            }
        }
    });
}

// depthwise_conv5x5_process_plane (src/common_ops.cpp:628-649): per output the
// 25 taps in (ky, kx) order skipping the outside, bias last.
void vae_dw5x5(const float * in, const float * w, const float * bias, float * out, size_t B, size_t C, size_t Hh,
               size_t Ww) {
    parallel_rows(B * C, [&](size_t r0, size_t r1) {
        for (size_t r = r0; r < r1; ++r) {
            const size_t c = r % C;
            const float * x = in + r * Hh * Ww;
            float * o = out + r * Hh * Ww;
            for (size_t y = 0; y < Hh; ++y)
                for (size_t xx = 0; xx < Ww; ++xx) {
                    float sum = 0.0f;
                    for (int ky = 0; ky < 5; ++ky)
                        for (int kx = 0; kx < 5; ++kx) {
                            const long iy = static_cast<long>(y) + ky - 2, ix = static_cast<long>(xx) + kx - 2;
                            if (iy >= 0 && iy < static_cast<long>(Hh) && ix >= 0 && ix < static_cast<long>(Ww))
                                sum += x[iy * Ww + ix] * w[(c * 5 + ky) * 5 + kx];
                        }
                    if (bias) sum += bias[c];
                    o[y * Ww + xx] = sum;
                }
        }
    });
}

// rms_norm_4d_channelwise (src/vae_ops.cpp:476-560): per pixel sum of squares
// over channels with std::fma in channel order, 1 / sqrt(sum * (1/C) + eps),
// then (x * inv) * w (+ b).
void vae_rms_norm(const float * in, const float * w, const float * bias, float * out, size_t B, size_t C, size_t S,
                  float eps) {
    const float inv_c = 1.0f / static_cast<float>(C);
    parallel_rows(B * ((S + 63) / 64), [&](size_t r0, size_t r1) {
        for (size_t r = r0; r < r1; ++r) {
            const size_t nb = (S + 63) / 64, b = r / nb, s0 = (r % nb) * 64, s1 = std::min(S, s0 + 64);
            float ss[64], inv[64];
            for (size_t i = s0; i < s1; ++i) ss[i - s0] = 0.0f;
            for (size_t c = 0; c < C; ++c) {
                const float * x = in + (b * C + c) * S;
                for (size_t i = s0; i < s1; ++i) ss[i - s0] = std::fma(x[i], x[i], ss[i - s0]);
            }
            for (size_t i = s0; i < s1; ++i) inv[i - s0] = 1.0f / std::sqrt(ss[i - s0] * inv_c + eps);
            for (size_t c = 0; c < C; ++c) {
                const float * x = in + (b * C + c) * S;
                float * o = out + (b * C + c) * S;
                for (size_t i = s0; i < s1; ++i) {
                    float v = x[i] * inv[i - s0] * w[c];
                    if (bias) v += bias[c];
                    o[i] = v;
                }
            }
        }
    });
}

// run_vae_upsample_block (src/vae_ops.cpp:808-821): nearest 2x (:330-375), the
// 3x3 conv, then add_upsample_shortcut_2x_inplace (:386-445):
// out[oc, 2y+i, 2x+j] += in[(4 oc + 2i + j) / repeats, y, x].
void vae_upsample(const float * in, const float * w, const float * bias, float * out, size_t B, size_t Cin,
                  size_t Cout, size_t Hh, size_t Ww, bool shortcut) {
    const size_t H2 = 2 * Hh, W2 = 2 * Ww;
    std::vector<float> up(B * Cin * H2 * W2);
    for (size_t r = 0; r < B * Cin; ++r)
        for (size_t y = 0; y < H2; ++y)
            for (size_t x = 0; x < W2; ++x) up[(r * H2 + y) * W2 + x] = in[(r * Hh + y / 2) * Ww + x / 2];
    vae_conv3x3(up.data(), w, bias, out, B, Cin, Cout, H2, W2);
    if (!shortcut) return;
    if ((Cout * 4) % Cin != 0) throw std::invalid_argument("VAE upsample shortcut channel ratio is invalid");
    const size_t rep = Cout * 4 / Cin;
    for (size_t b = 0; b < B; ++b)
        for (size_t oc = 0; oc < Cout; ++oc)
            for (size_t y = 0; y < Hh; ++y)
                for (size_t x = 0; x < Ww; ++x)
                    for (size_t q = 0; q < 4; ++q) {
                        const size_t ic = (oc * 4 + q) / rep;
                        out[((b * Cout + oc) * H2 + 2 * y + q / 2) * W2 + 2 * x + q % 2] +=
                            in[((b * Cin + ic) * Hh + y) * Ww + x];
                    }
}

// NCHW <-> token-major for the GLUMBConv restatement (pure data movement).
void nchw_to_tokens(const float * in, float * out, size_t B, size_t C, size_t S) {
    for (size_t b = 0; b < B; ++b)
        for (size_t c = 0; c < C; ++c)
            for (size_t i = 0; i < S; ++i) out[(b * S + i) * C + c] = in[(b * C + c) * S + i];
}
void tokens_to_nchw(const float * in, float * out, size_t B, size_t C, size_t S) {
    for (size_t b = 0; b < B; ++b)
        for (size_t c = 0; c < C; ++c)
            for (size_t i = 0; i < S; ++i) out[(b * C + c) * S + i] = in[(b * S + i) * C + c];
}

struct VaeModel {
    std::vector<size_t> ch;
    std::vector<bool> attn;
    size_t latent = 32, head_dim = 32, expand = 4;
    float scaling = 0.41407f;
    std::map<std::string, std::vector<float>> w;
    std::map<std::string, std::vector<size_t>> shape;
    const float * p(const std::string & n) const {
        auto it = w.find(n);
        if (it == w.end()) throw std::invalid_argument("missing vae weight " + n);
        return it->second.data();
    }
};

// run_vae_res_block (src/vae_ops.cpp:570-583)
void vae_res_block(const VaeModel & m, const std::string & q, const float * in, float * out, size_t B, size_t C,
                   size_t Hh, size_t Ww) {
    const size_t n = B * C * Hh * Ww;
    std::vector<float> h(n), h2(n);
    vae_conv3x3(in, m.p(q + "conv1.weight"), m.p(q + "conv1.bias"), h.data(), B, C, C, Hh, Ww);
    for (float & v : h) v = silu(v);
    vae_conv3x3(h.data(), m.p(q + "conv2.weight"), nullptr, h2.data(), B, C, C, Hh, Ww);
    vae_rms_norm(h2.data(), m.p(q + "norm.weight"), m.p(q + "norm.bias"), out, B, C, Hh * Ww, 1e-5f);
    for (size_t i = 0; i < n; ++i) out[i] += in[i];
}

// run_vae_glumb_conv (src/vae_ops.cpp:585-607): glumb_conv (src/common_ops.cpp:733-761), RMSNorm, + input.
void vae_glumb_block(const VaeModel & m, const std::string & q, const float * in, float * out, size_t B, size_t C,
                     size_t Hh, size_t Ww) {
    const size_t S = Hh * Ww, n = B * C * S, E = 2 * m.expand * C;
    std::vector<float> tok(n), gt(n), g(n);
    nchw_to_tokens(in, tok.data(), B, C, S);
    glumb_conv(tok.data(), m.p(q + "conv_out.conv_inverted.weight"), m.p(q + "conv_out.conv_inverted.bias"),
               m.p(q + "conv_out.conv_depth.weight"), m.p(q + "conv_out.conv_depth.bias"),
               m.p(q + "conv_out.conv_point.weight"), gt.data(), B, Hh, Ww, C, E, C);
    tokens_to_nchw(gt.data(), g.data(), B, C, S);
    vae_rms_norm(g.data(), m.p(q + "conv_out.norm.weight"), m.p(q + "conv_out.norm.bias"), out, B, C, S, 1e-5f);
    for (size_t i = 0; i < n; ++i) out[i] += in[i];
}

// run_vae_multiscale_attention (src/vae_ops.cpp:640-806).  Channel groups of
// 3 * D consecutive channels (of q|k|v concatenated, then of the multiscale
// branch) are the heads: q = the group's first D channels, k the next D, v the
// last D.  Per head: scores[r][d] = sum_t vp[r][t] relu(k)[d][t] over t in
// order (vp = v with a row of ones appended), hidden[r][t] = sum_d
// scores[r][d] relu(q)[d][t] over d in order, out = hidden[d] / (hidden[D] + 1e-15).
void vae_msattn(const VaeModel & m, const std::string & q, const float * in, float * out, size_t B, size_t C,
                size_t Hh, size_t Ww) {
    const size_t S = Hh * Ww, D = m.head_dim, inner = C, heads = inner / D;
    std::vector<float> qkv(B * 3 * inner * S), ms(B * 3 * inner * S), dw(B * 3 * inner * S);
    {
        std::vector<float> t(B * inner * S);
        const char * names[3] = {"attn.to_q.weight", "attn.to_k.weight", "attn.to_v.weight"};
        for (int j = 0; j < 3; ++j) {
            vae_conv1x1(in, m.p(q + names[j]), nullptr, t.data(), B, C, inner, S);
            for (size_t b = 0; b < B; ++b)
                std::copy(t.begin() + b * inner * S, t.begin() + (b + 1) * inner * S,
                          qkv.begin() + (b * 3 + j) * inner * S);
        }
    }
    vae_dw5x5(qkv.data(), m.p(q + "attn.to_qkv_multiscale.0.proj_in.weight"), nullptr, dw.data(), B, 3 * inner, Hh,
              Ww);
    vae_grouped1x1(dw.data(), m.p(q + "attn.to_qkv_multiscale.0.proj_out.weight"), ms.data(), B, 3 * inner,
                   3 * inner, 3 * heads, S);
    const size_t merged_heads = 2 * heads;
    std::vector<float> merged(B * merged_heads * D * S);
    parallel_rows(B * merged_heads, [&](size_t r0, size_t r1) {
        std::vector<float> qm(D * S), km(D * S), vm((D + 1) * S), sc((D + 1) * D), hid((D + 1) * S);
        for (size_t r = r0; r < r1; ++r) {
            const size_t b = r / merged_heads, g = r % merged_heads;
            const bool msb = g >= heads;
            const size_t lg = msb ? g - heads : g;
            const float * src = (msb ? ms.data() : qkv.data()) + (b * 3 * inner + lg * 3 * D) * S;
            for (size_t d = 0; d < D; ++d)
                for (size_t t = 0; t < S; ++t) {
                    qm[d * S + t] = std::max(0.0f, src[d * S + t]);
                    km[d * S + t] = std::max(0.0f, src[(D + d) * S + t]);
                    vm[d * S + t] = src[(2 * D + d) * S + t];
                }
            for (size_t t = 0; t < S; ++t) vm[D * S + t] = 1.0f;
            for (size_t rr = 0; rr <= D; ++rr) {
                float * srow = sc.data() + rr * D;
                for (size_t d = 0; d < D; ++d) srow[d] = 0.0f;
                for (size_t t = 0; t < S; ++t) {
                    const float a = vm[rr * S + t];
                    for (size_t d = 0; d < D; ++d) srow[d] += a * km[d * S + t];
                }
            }
            for (size_t rr = 0; rr <= D; ++rr) {
                float * h = hid.data() + rr * S;
                for (size_t t = 0; t < S; ++t) h[t] = 0.0f;
                for (size_t d = 0; d < D; ++d) {
                    const float a = sc[rr * D + d];
                    for (size_t t = 0; t < S; ++t) h[t] += a * qm[d * S + t];
                }
            }
            float * mg = merged.data() + (b * merged_heads + g) * D * S;
            for (size_t t = 0; t < S; ++t) {
                const float den = hid[D * S + t] + 1e-15f;
                for (size_t d = 0; d < D; ++d) mg[d * S + t] = hid[d * S + t] / den;
            }
        }
    });
    std::vector<float> o(B * C * S);
    vae_conv1x1(merged.data(), m.p(q + "attn.to_out.weight"), nullptr, o.data(), B, merged_heads * D, C, S);
    vae_rms_norm(o.data(), m.p(q + "attn.norm_out.weight"), m.p(q + "attn.norm_out.bias"), out, B, C, S, 1e-5f);
    for (size_t i = 0; i < B * C * S; ++i) out[i] += in[i];
}

// run_vae_decoder_input (src/vae.cpp:216-241): conv_in, then
// add_repeated_channels_inplace (src/vae_ops.cpp:451-471).
void vae_decoder_input(const VaeModel & m, const float * scaled, float * out, size_t B, size_t Hh, size_t Ww) {
    const size_t top = m.ch.back(), S = Hh * Ww, rep = top / m.latent;
    vae_conv3x3(scaled, m.p("decoder.conv_in.weight"), m.p("decoder.conv_in.bias"), out, B, m.latent, top, Hh, Ww);
    for (size_t b = 0; b < B; ++b)
        for (size_t c = 0; c < m.latent; ++c)
            for (size_t r = 0; r < rep; ++r) {
                float * o = out + (b * top + c * rep + r) * S;
                const float * x = scaled + (b * m.latent + c) * S;
                for (size_t i = 0; i < S; ++i) o[i] += x[i];
            }
}

// run_vae_decode (src/vae.cpp:243-325).
void vae_decode(const VaeModel & m, const float * latent, float * image, size_t B, size_t Hh, size_t Ww) {
    const size_t L = m.ch.size();
    std::vector<float> scaled(latent, latent + B * m.latent * Hh * Ww);
    const float inv = 1.0f / m.scaling;
    for (float & v : scaled) v *= inv;
    size_t C = m.ch.back(), h = Hh, w = Ww;
    std::vector<float> cur(B * C * h * w), nxt;
    vae_decoder_input(m, scaled.data(), cur.data(), B, Hh, Ww);
    for (size_t lv = L; lv-- > 0;) {
        const std::string p = "decoder.up_blocks." + std::to_string(lv) + ".";
        size_t base = 0;
        if (lv + 1 < L) {
            const size_t Co = m.ch[lv];
            nxt.assign(B * Co * 4 * h * w, 0.0f);
            vae_upsample(cur.data(), m.p(p + "0.conv.weight"), m.p(p + "0.conv.bias"), nxt.data(), B, C, Co, h, w,
                         true);
            cur.swap(nxt);
            C = Co;
            h *= 2;
            w *= 2;
            base = 1;
        }
        for (size_t l = base; l < base + 3; ++l) {
            const std::string q = p + std::to_string(l) + ".";
            nxt.assign(cur.size(), 0.0f);
            if (!m.attn[lv]) {
                vae_res_block(m, q, cur.data(), nxt.data(), B, C, h, w);
                cur.swap(nxt);
            } else {
                vae_msattn(m, q, cur.data(), nxt.data(), B, C, h, w);
                cur.swap(nxt);
                vae_glumb_block(m, q, cur.data(), nxt.data(), B, C, h, w);
                cur.swap(nxt);
            }
        }
    }
    nxt.assign(cur.size(), 0.0f);
    vae_rms_norm(cur.data(), m.p("decoder.norm_out.weight"), m.p("decoder.norm_out.bias"), nxt.data(), B, C, h * w,
                 1e-5f);
    for (float & v : nxt) v = std::max(0.0f, v);
    vae_conv3x3(nxt.data(), m.p("decoder.conv_out.weight"), m.p("decoder.conv_out.bias"), image, B, C, 3, h, w);
}

template <class F>
int guard(F f) {
    try {
        f();
        return 0;
    } catch (const std::exception & e) {
        return fail(e.what());
    }
}

}  // namespace

extern "C" {

const char * oracle_last_error(void) { return g_err.c_str(); }
void oracle_set_threads(int n) { g_threads = n; }

int oracle_randn(float * out, size_t n, uint64_t seed) {
    if (n < 16) return fail("randn requires at least 16 elements");
    randn(out, n, seed);
    return 0;
}

int oracle_linear(const float * in, const float * w, const float * bias, float * out, size_t M, size_t K, size_t N) {
    return guard([&] { linear(in, w, bias, out, M, K, N); });
}

int oracle_layer_norm(const float * x, const float * g, const float * b, float * out, size_t rows, size_t C, float eps) {
    return guard([&] { layer_norm(x, g, b, out, rows, C, eps); });
}

int oracle_rms_norm(const float * x, const float * w, float * out, size_t rows, size_t C, float eps) {
    return guard([&] { rms_norm(x, w, out, rows, C, eps); });
}

int oracle_modulate(const float * x, const float * shift, const float * scale, float * out, size_t B, size_t N,
                    size_t C) {
    return guard([&] { modulate(x, shift, scale, C, out, B, N, C); });
}

int oracle_linear_attention(const float * q, const float * k, const float * v, float * out, size_t B, size_t Nq,
                            size_t Nkv, size_t H, size_t D) {
    if (Nq != Nkv) return fail("token-major layout needs Nq == Nkv");
    return guard([&] { linear_attention(q, k, v, out, H * D, B, Nq, Nkv, H, D); });
}

int oracle_attention(const float * q, const float * k, const float * v, const float * bias, float * out, size_t B,
                     size_t Nq, size_t L, size_t H, size_t D) {
    return guard([&] { attention(q, k, v, bias, out, H * D, H * D, B, Nq, L, H, D); });
}

int oracle_depthwise3x3(const float * x, const float * w, const float * bias, float * out, size_t B, size_t Hh,
                        size_t Ww, size_t C) {
    return guard([&] { depthwise3x3(x, w, bias, out, B, Hh, Ww, C); });
}

int oracle_glumb_conv(const float * x, const float * inv_w, const float * inv_b, const float * dw_w,
                      const float * dw_b, const float * pt_w, float * out, size_t B, size_t Hh, size_t Ww,
                      size_t Cin, size_t E, size_t Cout) {
    if (E % 2 != 0) return fail("expanded channel count must be even");
    return guard([&] { glumb_conv(x, inv_w, inv_b, dw_w, dw_b, pt_w, out, B, Hh, Ww, Cin, E, Cout); });
}

int oracle_caption_projection(const float * x, const float * w1, const float * b1, const float * w2,
                              const float * b2, const float * nw, float * out, size_t rows, size_t Cin, size_t C) {
    return guard([&] { caption_projection(x, w1, b1, w2, b2, nw, out, rows, Cin, C); });
}

int oracle_timestep_embedding(const float * t, float * out, size_t B, size_t dim) {
    return guard([&] { timestep_embedding(t, out, B, dim); });
}

int oracle_cfg(const float * np, float * out, size_t n, float g) {
    for (size_t i = 0; i < n; ++i) out[i] = np[i] + g * (np[n + i] - np[i]);
    return 0;
}

int oracle_block_forward(const oracle_block_weights * w, const float * x, const float * ctx, const float * t_mod,
                         const float * bias, size_t B, size_t N, size_t L, float * a, float * c, float * f) {
    if (!w || w->self_heads == 0 || w->cross_heads == 0 || w->hidden % w->self_heads || w->hidden % w->cross_heads)
        return fail("bad block weights");
    return guard([&] { block_forward(*w, x, ctx, t_mod, bias, B, N, L, a, c, f); });
}

int oracle_attention_block(const float * x, const float * wq, const float * bq, const float * wk, const float * bk,
                           const float * wv, const float * bv, const float * wo, const float * bo, float * out,
                           size_t B, size_t N, size_t C, size_t heads) {
    if (heads == 0 || C % heads != 0) return fail("hidden size must be divisible by num_heads");
    return guard([&] { attention_block(x, wq, bq, wk, bk, wv, bv, wo, bo, out, B, N, C, heads); });
}

int oracle_cross_attention_block(const float * x, const float * ctx, const float * bias, const float * wq,
                                 const float * bq, const float * wk, const float * bk, const float * wv,
                                 const float * bv, const float * wo, const float * bo, float * out, size_t B,
                                 size_t N, size_t L, size_t C, size_t heads) {
    if (heads == 0 || C % heads != 0) return fail("hidden size must be divisible by num_heads");
    return guard([&] { cross_attention_block(x, ctx, bias, wq, bq, wk, bk, wv, bv, wo, bo, out, B, N, L, C, heads); });
}

int oracle_sched_convert(const float * mo, const float * sample, size_t n, float sigma, float * out) {
    sched_convert(mo, sample, n, sigma, out);
    return 0;
}

int oracle_sched_first_order(const float * conv, const float * sample, size_t n, float st, float ss, float * out) {
    sched_first(conv, sample, n, st, ss, out);
    return 0;
}

int oracle_sched_second_order(const float * sample, const float * m0, const float * m1, size_t n, float st,
                              float s0, float s1, float * out) {
    sched_second(sample, m0, m1, n, st, s0, s1, out);
    return 0;
}

oracle_model * oracle_model_create(size_t layers, size_t hidden, size_t ffn, size_t caption_dim, size_t latent,
                                   size_t self_heads, size_t cross_heads) {
    auto * m = new oracle_model();
    m->layers = layers;
    m->C = hidden;
    m->E = ffn;
    m->Ccap = caption_dim;
    m->Cl = latent;
    m->self_heads = self_heads;
    m->cross_heads = cross_heads;
    m->ones.assign(hidden, 1.0f);
    m->zeros.assign(hidden, 0.0f);
    return m;
}

void oracle_model_destroy(oracle_model * m) { delete m; }

int oracle_model_set(oracle_model * m, const char * name, const float * data, size_t n) {
    m->t[name].assign(data, data + n);
    return 0;
}

int oracle_model_generate(oracle_model * m) {
    return guard([&] {
        for (const sana_spec::Entry & e : sana_spec::manifest(m->dims())) {
            std::vector<float> v(sana_spec::numel(e.shape));
            if (e.ones) {
                std::fill(v.begin(), v.end(), 1.0f);
            } else if (v.size() >= 16) {
                randn(v.data(), v.size(), e.seed);
                for (float & x : v) x *= 0.02f;
            } else {
                // randn needs >= 16 values (src/torch_rng.cpp:39-41); tiny test
                // shapes take the first values of a 16-value draw.
                float t16[16];
                randn(t16, 16, e.seed);
                for (size_t i = 0; i < v.size(); ++i) v[i] = t16[i] * 0.02f;
            }
            m->t[e.name] = std::move(v);
        }
    });
}

int oracle_model_get(const oracle_model * m, const char * name, float * out, size_t n) {
    auto it = m->t.find(name);
    if (it == m->t.end()) return fail(std::string("weight not set: ") + name);
    if (it->second.size() != n) return fail("size mismatch");
    std::copy(it->second.begin(), it->second.end(), out);
    return 0;
}

uint64_t oracle_digest(const float * data, size_t n) {
    uint64_t h = 14695981039346656037ULL;
    const unsigned char * p = reinterpret_cast<const unsigned char *>(data);
    for (size_t i = 0; i < n * 4; ++i) {
        h ^= p[i];
        h *= 1099511628211ULL;
    }
    return h;
}

int oracle_model_project_caption(const oracle_model * m, const float * cap, size_t B, size_t L, float * ctx) {
    return guard([&] {
        caption_projection(cap, m->p("caption_projection.linear_1.weight"), m->p("caption_projection.linear_1.bias"),
                           m->p("caption_projection.linear_2.weight"), m->p("caption_projection.linear_2.bias"),
                           m->p("caption_norm.weight"), ctx, B * L, m->Ccap, m->C);
    });
}

int oracle_model_time(const oracle_model * m, const float * t, size_t B, float * emb, float * tmod) {
    return guard([&] { model_time(*m, t, B, emb, tmod); });
}

int oracle_model_patch_embed(const oracle_model * m, const float * lat, size_t B, size_t Hh, size_t Ww, float * tok) {
    return guard([&] { model_patch(*m, lat, B, Hh, Ww, tok); });
}

int oracle_model_block(const oracle_model * m, size_t i, const float * x, const float * ctx, const float * tmod,
                       const float * bias, size_t B, size_t N, size_t L, float * a, float * c, float * f) {
    if (i >= m->layers) return fail("block index out of range");
    return guard([&] {
        oracle_block_weights w = m->block(i);
        block_forward(w, x, ctx, tmod, bias, B, N, L, a, c, f);
    });
}

int oracle_model_forward(const oracle_model * m, const float * latent, size_t Bl, size_t Hh, size_t Ww,
                         const float * ctx, size_t L, const float * bias, float t, float * np) {
    return guard([&] { model_forward(*m, latent, Bl, Hh, Ww, ctx, L, bias, t, np); });
}

int oracle_model_loop(const oracle_model * m, const float * latent, size_t Bl, size_t Hh, size_t Ww,
                      const float * cap, size_t L, const float * bias, size_t steps, float g, float * fin) {
    return guard([&] {
        const size_t B = 2 * Bl, n = Bl * m->Cl * Hh * Ww;
        std::vector<float> ctx(B * L * m->C), np(2 * n), guided(n);
        caption_projection(cap, m->p("caption_projection.linear_1.weight"), m->p("caption_projection.linear_1.bias"),
                           m->p("caption_projection.linear_2.weight"), m->p("caption_projection.linear_2.bias"),
                           m->p("caption_norm.weight"), ctx.data(), B * L, m->Ccap, m->C);
        SchedState st;
        schedule(steps, st.ts, st.sig);
        std::vector<float> lat(latent, latent + n);
        while (st.step < st.ts.size()) {
            model_forward(*m, lat.data(), Bl, Hh, Ww, ctx.data(), L, bias, st.ts[st.step], np.data());
            for (size_t i = 0; i < n; ++i) guided[i] = np[i] + g * (np[n + i] - np[i]);
            lat = sched_step(guided, lat, st);
        }
        std::copy(lat.begin(), lat.end(), fin);
    });
}

int oracle_scheduler_timesteps(size_t steps, float * ts, float * sig) {
    if (steps == 0) return fail("num_inference_steps must be positive");
    std::vector<float> t, s;
    schedule(steps, t, s);
    std::copy(t.begin(), t.end(), ts);
    std::copy(s.begin(), s.end(), sig);
    return 0;
}


// ---------------------------------------------------------------- VAE API
struct oracle_vae : VaeModel {};

int oracle_vae_conv3x3(const float * in, const float * w, const float * bias, float * out, size_t B, size_t Cin,
                       size_t Cout, size_t Hh, size_t Ww, int order) {
    if (order < -1 || order > 1) return fail("order must be -1 (as the reference dispatches), 0 (im2col) or 1 (taps)");
    return guard([&] { vae_conv3x3(in, w, bias, out, B, Cin, Cout, Hh, Ww, order); });
}
int oracle_vae_conv1x1(const float * in, const float * w, const float * bias, float * out, size_t B, size_t Cin,
                       size_t Cout, size_t S) {
    return guard([&] { vae_conv1x1(in, w, bias, out, B, Cin, Cout, S); });
}
int oracle_vae_grouped_conv1x1(const float * in, const float * w, float * out, size_t B, size_t Cin, size_t Cout,
                               size_t groups, size_t S) {
    if (groups == 0 || Cin % groups || Cout % groups) return fail("channels must be divisible by groups");
    return guard([&] { vae_grouped1x1(in, w, out, B, Cin, Cout, groups, S); });
}
int oracle_vae_dw5x5(const float * in, const float * w, const float * bias, float * out, size_t B, size_t C,
                     size_t Hh, size_t Ww) {
    return guard([&] { vae_dw5x5(in, w, bias, out, B, C, Hh, Ww); });
}
int oracle_vae_rms_norm(const float * in, const float * w, const float * bias, float * out, size_t B, size_t C,
                        size_t S, float eps) {
    return guard([&] { vae_rms_norm(in, w, bias, out, B, C, S, eps); });
}
int oracle_vae_upsample(const float * in, const float * w, const float * bias, float * out, size_t B, size_t Cin,
                        size_t Cout, size_t Hh, size_t Ww, int shortcut) {
    return guard([&] { vae_upsample(in, w, bias, out, B, Cin, Cout, Hh, Ww, shortcut != 0); });
}

oracle_vae * oracle_vae_create_config(size_t latent, size_t levels, const size_t * channels, const int * attn) {
    vae_spec::Config c;
    c.latent = latent;
    for (size_t i = 0; i < levels; ++i) {
        c.channels.push_back(channels[i]);
        c.attn.push_back(attn[i] != 0);
    }
    auto * m = new oracle_vae();
    m->ch = c.channels;
    m->attn = c.attn;
    m->latent = c.latent;
    m->head_dim = c.head_dim;
    m->expand = c.expand;
    for (const vae_spec::Entry & e : vae_spec::manifest(c)) {
        m->shape[e.name] = e.shape;
        m->w[e.name].assign(vae_spec::numel(e.shape), 0.0f);
    }
    return m;
}

oracle_vae * oracle_vae_create(int full) {
    auto * m = new oracle_vae();
    const vae_spec::Config c = full ? vae_spec::full_config() : vae_spec::small_config();
    m->ch = c.channels;
    m->attn = c.attn;
    m->latent = c.latent;
    m->head_dim = c.head_dim;
    m->expand = c.expand;
    for (const vae_spec::Entry & e : vae_spec::manifest(c)) {
        m->shape[e.name] = e.shape;
        m->w[e.name].assign(vae_spec::numel(e.shape), 0.0f);
    }
    return m;
}
void oracle_vae_destroy(oracle_vae * m) { delete m; }

int oracle_vae_generate(oracle_vae * m) {
    return guard([&] {
        vae_spec::Config c;
        c.latent = m->latent;
        c.channels = m->ch;
        c.attn = m->attn;
        c.head_dim = m->head_dim;
        c.expand = m->expand;
        for (const vae_spec::Entry & e : vae_spec::manifest(c)) {
            std::vector<float> & t = m->w.at(e.name);
            std::vector<float> r(std::max<size_t>(t.size(), 16));
            randn(r.data(), r.size(), e.seed);
            for (size_t i = 0; i < t.size(); ++i) t[i] = e.norm ? 1.0f + 0.1f * r[i] : 0.02f * r[i];
        }
    });
}
int oracle_vae_set(oracle_vae * m, const char * name, const float * data, size_t n) {
    auto it = m->w.find(name);
    if (it == m->w.end()) return fail(std::string("unknown vae weight ") + name);
    if (it->second.size() != n) return fail(std::string("size mismatch for ") + name);
    std::copy(data, data + n, it->second.begin());
    return 0;
}
int oracle_vae_get(const oracle_vae * m, const char * name, float * out, size_t n) {
    auto it = m->w.find(name);
    if (it == m->w.end()) return fail(std::string("unknown vae weight ") + name);
    if (it->second.size() != n) return fail(std::string("size mismatch for ") + name);
    std::copy(it->second.begin(), it->second.end(), out);
    return 0;
}
int oracle_vae_decoder_input(const oracle_vae * m, const float * latent, size_t B, size_t Hh, size_t Ww,
                             float * out) {
    return guard([&] {
        std::vector<float> sc(latent, latent + B * m->latent * Hh * Ww);
        const float inv = 1.0f / m->scaling;
        for (float & v : sc) v *= inv;
        vae_decoder_input(*m, sc.data(), out, B, Hh, Ww);
    });
}
int oracle_vae_res_block(const oracle_vae * m, size_t level, size_t layer, const float * in, float * out, size_t B,
                         size_t Hh, size_t Ww) {
    return guard([&] {
        const std::string q = "decoder.up_blocks." + std::to_string(level) + "." + std::to_string(layer) + ".";
        vae_res_block(*m, q, in, out, B, m->ch.at(level), Hh, Ww);
    });
}
int oracle_vae_attention(const oracle_vae * m, size_t level, size_t layer, const float * in, float * out,
                         size_t B, size_t Hh, size_t Ww) {
    return guard([&] {
        const std::string q = "decoder.up_blocks." + std::to_string(level) + "." + std::to_string(layer) + ".";
        vae_msattn(*m, q, in, out, B, m->ch.at(level), Hh, Ww);
    });
}
int oracle_vae_glumb(const oracle_vae * m, size_t level, size_t layer, const float * in, float * out, size_t B,
                     size_t Hh, size_t Ww) {
    return guard([&] {
        const std::string q = "decoder.up_blocks." + std::to_string(level) + "." + std::to_string(layer) + ".";
        vae_glumb_block(*m, q, in, out, B, m->ch.at(level), Hh, Ww);
    });
}
int oracle_vae_decode(const oracle_vae * m, const float * latent, size_t B, size_t Hh, size_t Ww, float * image) {
    return guard([&] { vae_decode(*m, latent, image, B, Hh, Ww); });
}

}  // extern "C"
