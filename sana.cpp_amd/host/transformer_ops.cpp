// Op-level attention API (src/transformer_ops.h) on the GPU.  Checks and
// messages follow src/transformer_ops.cpp:64-608; composite blocks keep their
// intermediates on the device.
#include "transformer_ops.h"

#include <cmath>
#include <stdexcept>

#include "../../include/sana_dit.h"
#include "ops_device.h"

using namespace sana_host;

namespace {

struct Dims4 {
    size_t b, h, t, d;
};

Dims4 dims4(const Tensor & x) { return {x.dim_size(0), x.dim_size(1), x.dim_size(2), x.dim_size(3)}; }

// [B, N, H*D] -> [B, H, N, D] on the device
DeviceArray dev_split(const DeviceArray & x, size_t B, size_t N, size_t H, size_t D) {
    DeviceArray y(B * N * H * D);
    op_check(sana_op_heads_f32(x.get(), y.get(), (int64_t)B, (int64_t)N, (int64_t)H, (int64_t)D, 1, nullptr));
    return y;
}

DeviceArray dev_merge(const DeviceArray & x, size_t B, size_t N, size_t H, size_t D) {
    DeviceArray y(B * N * H * D);
    op_check(sana_op_heads_f32(x.get(), y.get(), (int64_t)B, (int64_t)N, (int64_t)H, (int64_t)D, 0, nullptr));
    return y;
}

// scores[z] = q[z] . k[z]^T for z < B*H: [Nq, D] x [Nk, D]^T
DeviceArray dev_scores(const DeviceArray & q, const DeviceArray & k, size_t BH, size_t Nq, size_t Nk, size_t D) {
    DeviceArray s(BH * Nq * Nk);
    if (BH && Nq && Nk)
        op_check(sana_op_gemm_f32(q.get(), (int64_t)D, (int64_t)(Nq * D), k.get(), (int64_t)D, (int64_t)(Nk * D), 1,
                                  nullptr, 1, s.get(), (int64_t)Nk, (int64_t)(Nq * Nk), (int64_t)Nq, (int64_t)Nk,
                                  (int64_t)D, (int64_t)BH, 0, nullptr));
    return s;
}

// out[z] = w[z] . v[z]: [Nq, Nk] x [Nk, D]
DeviceArray dev_values(const DeviceArray & w, const DeviceArray & v, size_t BH, size_t Nq, size_t Nk, size_t D) {
    DeviceArray o(BH * Nq * D);
    if (BH && Nq && D)
        op_check(sana_op_gemm_f32(w.get(), (int64_t)Nk, (int64_t)(Nq * Nk), v.get(), (int64_t)D, (int64_t)(Nk * D), 0,
                                  nullptr, 1, o.get(), (int64_t)D, (int64_t)(Nq * D), (int64_t)Nq, (int64_t)D,
                                  (int64_t)Nk, (int64_t)BH, 0, nullptr));
    return o;
}

// softmax(scores * scale + bias[b, 0, :]) over the last axis, in place
void dev_softmax(DeviceArray & s, size_t rows, size_t cols, float scale, const DeviceArray * bias, size_t rows_per_b) {
    if (rows && cols)
        op_check(sana_op_softmax_f32(s.get(), s.get(), (int64_t)rows, (int64_t)cols, scale, opt(bias),
                                     (int64_t)rows_per_b, nullptr));
}

// 1 / sqrt(head_dim) as the reference computes it: the size_t argument takes
// the double overload of std::sqrt, then the quotient is rounded to float.
float attention_scale(size_t head_dim) { return static_cast<float>(1.0f / std::sqrt(static_cast<double>(head_dim))); }

DeviceArray dev_attention(const DeviceArray & q, const DeviceArray & k, const DeviceArray & v, size_t B, size_t H,
                          size_t Nq, size_t Nk, size_t D, const Tensor * bias) {
    DeviceArray s = dev_scores(q, k, B * H, Nq, Nk, D);
    std::unique_ptr<DeviceArray> b = upload_opt(bias);
    dev_softmax(s, B * H * Nq, Nk, attention_scale(D), b.get(), H * Nq);
    return dev_values(s, v, B * H, Nq, Nk, D);
}

DeviceArray dev_linear_attention(const DeviceArray & q, const DeviceArray & k, const DeviceArray & v, size_t BH,
                                 size_t Nq, size_t Nk, size_t D) {
    DeviceArray o(BH * Nq * D), state(BH * (D + 1) * D);
    if (BH && D)
        op_check(sana_op_linear_attention_f32(q.get(), k.get(), v.get(), o.get(), (int64_t)BH, (int64_t)Nq,
                                              (int64_t)Nk, (int64_t)D, state.get(), nullptr));
    return o;
}

void check_attention_bias(const Tensor * bias, size_t batch, size_t keys) {
    if (bias && (bias->rank() != 3 || bias->dim_size(0) != batch || bias->dim_size(1) != 1 ||
                 bias->dim_size(2) != keys))
        throw std::invalid_argument("attention_bias shape must be {batch, 1, key_tokens}");
}

void check_heads(size_t hidden, size_t heads) {
    if (heads == 0) throw std::invalid_argument("num_heads must be greater than 0");
    if (hidden % heads != 0) throw std::invalid_argument("hidden size must be divisible by num_heads");
}

}  // namespace

Tensor project_caption_context(const Tensor & x, const Tensor & w1, const Tensor * b1, const Tensor & w2,
                               const Tensor * b2, const Tensor & norm_weight) {
    // linear -> GELU(tanh) -> linear -> RMSNorm(eps 1e-5, weight) (src/transformer_ops.cpp:64-76)
    if (x.rank() != 3) throw std::invalid_argument("input must be rank 3");
    check_linear_args(w1, b1, x.dim_size(2));
    check_linear_args(w2, b2, w1.dim_size(1));
    const size_t B = x.dim_size(0), L = x.dim_size(1), C = w2.dim_size(1);
    if (norm_weight.rank() != 1 || norm_weight.dim_size(0) != C)
        throw std::invalid_argument("weight must be 1D and match hidden size");
    DeviceArray h = dev_linear(DeviceArray(x), B * L, x.dim_size(2), w1, b1);
    dev_unary(h, SANA_OP_GELU_TANH);
    DeviceArray p = dev_linear(h, B * L, w1.dim_size(1), w2, b2);
    DeviceArray nw(norm_weight), out(B * L * C);
    if (B * L > 0 && C > 0)
        op_check(sana_op_rms_norm_f32(p.get(), nw.get(), out.get(), (int64_t)(B * L), (int64_t)C, 1e-5f, nullptr));
    return out.to_tensor({B, L, C});
}

Tensor split_heads_3d(const Tensor & input, size_t num_heads) {
    if (input.rank() != 3) throw std::invalid_argument("input must be rank 3");
    check_heads(input.dim_size(2), num_heads);
    const size_t B = input.dim_size(0), N = input.dim_size(1), D = input.dim_size(2) / num_heads;
    return dev_split(DeviceArray(input), B, N, num_heads, D).to_tensor({B, num_heads, N, D});
}

Tensor merge_heads_4d(const Tensor & input) {
    if (input.rank() != 4) throw std::invalid_argument("input must be rank 4");
    const Dims4 d = dims4(input);
    return dev_merge(DeviceArray(input), d.b, d.t, d.h, d.d).to_tensor({d.b, d.t, d.h * d.d});
}

Tensor attention_scores_4d(const Tensor & q, const Tensor & k) {
    if (q.rank() != 4) throw std::invalid_argument("q must be rank 4");
    if (k.rank() != 4) throw std::invalid_argument("k must be rank 4");
    if (q.dim_size(0) != k.dim_size(0)) throw std::invalid_argument("q and k batch size must match");
    if (q.dim_size(1) != k.dim_size(1)) throw std::invalid_argument("q and k head count must match");
    if (q.dim_size(3) != k.dim_size(3)) throw std::invalid_argument("q and k head_dim must match");
    const Dims4 a = dims4(q);
    const size_t Nk = k.dim_size(2);
    return dev_scores(DeviceArray(q), DeviceArray(k), a.b * a.h, a.t, Nk, a.d).to_tensor({a.b, a.h, a.t, Nk});
}

Tensor attention_values_4d(const Tensor & weights, const Tensor & v) {
    if (weights.rank() != 4) throw std::invalid_argument("weights must be rank 4");
    if (v.rank() != 4) throw std::invalid_argument("v must be rank 4");
    if (weights.dim_size(0) != v.dim_size(0)) throw std::invalid_argument("weights and v batch size must match");
    if (weights.dim_size(1) != v.dim_size(1)) throw std::invalid_argument("weights and v head count must match");
    if (weights.dim_size(3) != v.dim_size(2))
        throw std::invalid_argument("weights k_tokens must match v token count");
    const Dims4 w = dims4(weights);
    const size_t D = v.dim_size(3);
    return dev_values(DeviceArray(weights), DeviceArray(v), w.b * w.h, w.t, w.d, D).to_tensor({w.b, w.h, w.t, D});
}

Tensor softmax_lastdim_4d(const Tensor & input) {
    if (input.rank() != 4) throw std::invalid_argument("input must be rank 4");
    const Dims4 d = dims4(input);
    DeviceArray s(input);
    dev_softmax(s, d.b * d.h * d.t, d.d, 1.0f, nullptr, 1);
    return s.to_tensor(input.shape());
}

Tensor attention_4d(const Tensor & q, const Tensor & k, const Tensor & v, const Tensor * attention_bias) {
    if (q.rank() != 4) throw std::invalid_argument("q must be rank 4");
    if (k.rank() != 4) throw std::invalid_argument("k must be rank 4");
    if (q.dim_size(0) != k.dim_size(0)) throw std::invalid_argument("q and k batch size must match");
    if (q.dim_size(1) != k.dim_size(1)) throw std::invalid_argument("q and k head count must match");
    if (q.dim_size(3) != k.dim_size(3)) throw std::invalid_argument("q and k head_dim must match");
    check_attention_bias(attention_bias, q.dim_size(0), k.dim_size(2));
    if (v.rank() != 4) throw std::invalid_argument("v must be rank 4");
    if (q.dim_size(0) != v.dim_size(0)) throw std::invalid_argument("weights and v batch size must match");
    if (q.dim_size(1) != v.dim_size(1)) throw std::invalid_argument("weights and v head count must match");
    if (k.dim_size(2) != v.dim_size(2)) throw std::invalid_argument("weights k_tokens must match v token count");
    const Dims4 a = dims4(q);
    const size_t Nk = k.dim_size(2), Dv = v.dim_size(3);
    if (Dv != a.d) {
        // values of a different width: scores and softmax as usual, values with Dv columns
        DeviceArray s = dev_scores(DeviceArray(q), DeviceArray(k), a.b * a.h, a.t, Nk, a.d);
        std::unique_ptr<DeviceArray> b = upload_opt(attention_bias);
        dev_softmax(s, a.b * a.h * a.t, Nk, attention_scale(a.d), b.get(), a.h * a.t);
        return dev_values(s, DeviceArray(v), a.b * a.h, a.t, Nk, Dv).to_tensor({a.b, a.h, a.t, Dv});
    }
    return dev_attention(DeviceArray(q), DeviceArray(k), DeviceArray(v), a.b, a.h, a.t, Nk, a.d, attention_bias)
        .to_tensor({a.b, a.h, a.t, a.d});
}

Tensor linear_attention_4d(const Tensor & q, const Tensor & k, const Tensor & v) {
    if (q.rank() != 4 || k.rank() != 4 || v.rank() != 4)
        throw std::invalid_argument("q, k, and v must be rank 4");
    if (q.dim_size(0) != k.dim_size(0) || q.dim_size(0) != v.dim_size(0))
        throw std::invalid_argument("q, k, and v batch size must match");
    if (q.dim_size(1) != k.dim_size(1) || q.dim_size(1) != v.dim_size(1))
        throw std::invalid_argument("q, k, and v head count must match");
    if (q.dim_size(3) != k.dim_size(3) || q.dim_size(3) != v.dim_size(3))
        throw std::invalid_argument("q, k, and v head_dim must match");
    if (k.dim_size(2) != v.dim_size(2)) throw std::invalid_argument("k and v token count must match");
    const Dims4 a = dims4(q);
    return dev_linear_attention(DeviceArray(q), DeviceArray(k), DeviceArray(v), a.b * a.h, a.t, k.dim_size(2), a.d)
        .to_tensor(q.shape());
}

Tensor attention_block_3d(const Tensor & input, const Tensor & q_weight, const Tensor * q_bias,
                          const Tensor & k_weight, const Tensor * k_bias, const Tensor & v_weight,
                          const Tensor * v_bias, const Tensor & out_weight, const Tensor * out_bias,
                          size_t num_heads) {
    // q, k, v projections -> heads -> ReLU linear attention -> merge -> out projection
    // (src/transformer_ops.cpp:545-570)
    if (input.rank() != 3) throw std::invalid_argument("input must be rank 3");
    const size_t B = input.dim_size(0), N = input.dim_size(1), K = input.dim_size(2);
    for (const auto & wb : {std::make_pair(&q_weight, q_bias), std::make_pair(&k_weight, k_bias),
                            std::make_pair(&v_weight, v_bias)})
        check_linear_args(*wb.first, wb.second, K);
    const size_t C = q_weight.dim_size(1);
    if (k_weight.dim_size(1) != C || v_weight.dim_size(1) != C)
        throw std::invalid_argument("q, k, and v head_dim must match");
    check_heads(C, num_heads);
    check_linear_args(out_weight, out_bias, C);
    const size_t D = C / num_heads;
    DeviceArray x(input);
    DeviceArray q = dev_split(dev_linear(x, B * N, K, q_weight, q_bias), B, N, num_heads, D);
    DeviceArray k = dev_split(dev_linear(x, B * N, K, k_weight, k_bias), B, N, num_heads, D);
    DeviceArray v = dev_split(dev_linear(x, B * N, K, v_weight, v_bias), B, N, num_heads, D);
    DeviceArray o = dev_merge(dev_linear_attention(q, k, v, B * num_heads, N, N, D), B, N, num_heads, D);
    return dev_linear(o, B * N, C, out_weight, out_bias).to_tensor({B, N, out_weight.dim_size(1)});
}

Tensor cross_attention_block_3d(const Tensor & input, const Tensor & context, const Tensor * attention_bias,
                                const Tensor & q_weight, const Tensor * q_bias, const Tensor & k_weight,
                                const Tensor * k_bias, const Tensor & v_weight, const Tensor * v_bias,
                                const Tensor & out_weight, const Tensor * out_bias, size_t num_heads) {
    // (src/transformer_ops.cpp:572-608)
    if (input.rank() != 3) throw std::invalid_argument("input must be rank 3");
    if (context.rank() != 3) throw std::invalid_argument("context must be rank 3");
    if (input.dim_size(0) != context.dim_size(0))
        throw std::invalid_argument("input and context batch size must match");
    const size_t B = input.dim_size(0), N = input.dim_size(1), L = context.dim_size(1);
    check_linear_args(q_weight, q_bias, input.dim_size(2));
    check_linear_args(k_weight, k_bias, context.dim_size(2));
    check_linear_args(v_weight, v_bias, context.dim_size(2));
    const size_t C = q_weight.dim_size(1);
    if (k_weight.dim_size(1) != C || v_weight.dim_size(1) != C)
        throw std::invalid_argument("q and k head_dim must match");
    check_heads(C, num_heads);
    check_attention_bias(attention_bias, B, L);
    check_linear_args(out_weight, out_bias, C);
    const size_t D = C / num_heads;
    DeviceArray x(input), c(context);
    DeviceArray q = dev_split(dev_linear(x, B * N, input.dim_size(2), q_weight, q_bias), B, N, num_heads, D);
    DeviceArray k = dev_split(dev_linear(c, B * L, context.dim_size(2), k_weight, k_bias), B, L, num_heads, D);
    DeviceArray v = dev_split(dev_linear(c, B * L, context.dim_size(2), v_weight, v_bias), B, L, num_heads, D);
    DeviceArray o = dev_merge(dev_attention(q, k, v, B, num_heads, N, L, D, attention_bias), B, N, num_heads, D);
    return dev_linear(o, B * N, C, out_weight, out_bias).to_tensor({B, N, out_weight.dim_size(1)});
}
