// Op-level API (src/common_ops.h) on the GPU.  Argument checks and messages
// follow src/common_ops.cpp:114-761; the arithmetic is the fp32 MFMA GEMM and
// the fp32 kernels of ops32.hip (bias added after the products, as
// gemm_row_major's initialise-then-accumulate does).
#include "common_ops.h"

#include <stdexcept>

#include "../../include/sana_dit.h"
#include "ops_device.h"

namespace sana_host {

std::unique_ptr<DeviceArray> upload_opt(const Tensor * t) {
    return t ? std::make_unique<DeviceArray>(*t) : nullptr;
}

void check_linear_args(const Tensor & weight, const Tensor * bias, size_t in_features) {
    if (weight.rank() != 2) throw std::invalid_argument("weight must be rank 2");
    if (bias && bias->rank() != 1) throw std::invalid_argument("bias must be rank 1");
    if (in_features != weight.dim_size(0)) throw std::invalid_argument("inner dim must match for multiplication");
    if (bias && bias->dim_size(0) != weight.dim_size(1)) throw std::invalid_argument("dim for bias mismatch");
}

void check_conv1x1_args(const Tensor & weight, const Tensor * bias, size_t in_channels) {
    if (weight.rank() != 4) throw std::invalid_argument("weight must be rank 4");
    if (weight.dim_size(2) != 1 || weight.dim_size(3) != 1) throw std::invalid_argument("weight kernel must be 1x1");
    if (in_channels != weight.dim_size(1))
        throw std::invalid_argument("input channels must match weight in_channels");
    if (bias) {
        if (bias->rank() != 1) throw std::invalid_argument("bias must be rank 1");
        if (bias->dim_size(0) != weight.dim_size(0))
            throw std::invalid_argument("bias size must match out_channels");
    }
}

DeviceArray dev_linear(const DeviceArray & x, size_t rows, size_t K, const Tensor & weight, const Tensor * bias) {
    check_linear_args(weight, bias, K);
    const size_t N = weight.dim_size(1);
    DeviceArray w(weight), out(rows * N);
    auto b = upload_opt(bias);
    if (rows && N)
        op_check(sana_op_gemm_f32(x.get(), (int64_t)K, 0, w.get(), (int64_t)N, 0, 0, opt(b.get()), 1, out.get(),
                                  (int64_t)N, 0, (int64_t)rows, (int64_t)N, (int64_t)K, 1, 0, nullptr));
    return out;
}

void dev_unary(DeviceArray & x, int op) { op_check(sana_op_unary_f32(x.get(), x.get(), (int64_t)x.size(), op, nullptr)); }

DeviceArray dev_conv1x1(const DeviceArray & x, size_t B, size_t IC, size_t S, const Tensor & weight,
                        const Tensor * bias) {
    check_conv1x1_args(weight, bias, IC);
    const size_t OC = weight.dim_size(0);
    DeviceArray w(weight), out(B * OC * S);
    auto b = upload_opt(bias);
    // out[b] [OC, S] = W [OC, IC] . x[b] [IC, S] + bias[oc]
    if (B && OC && S)
        op_check(sana_op_gemm_f32(w.get(), (int64_t)IC, 0, x.get(), (int64_t)S, (int64_t)(IC * S), 0, opt(b.get()), 2,
                                  out.get(), (int64_t)S, (int64_t)(OC * S), (int64_t)OC, (int64_t)S, (int64_t)IC,
                                  (int64_t)B, 0, nullptr));
    return out;
}

}  // namespace sana_host

using namespace sana_host;

void gemm_row_major(const float * A, const float * B, const float * bias, float * C, size_t M, size_t K, size_t N,
                    bool b_transposed) {
    if (M == 0 || N == 0) return;
    DeviceArray a(A, M * K), b(B, K * N), c(M * N);
    std::unique_ptr<DeviceArray> bb = bias ? std::make_unique<DeviceArray>(bias, N) : nullptr;
    op_check(sana_op_gemm_f32(a.get(), (int64_t)K, 0, b.get(), (int64_t)(b_transposed ? K : N), 0, b_transposed ? 1 : 0,
                              opt(bb.get()), 1, c.get(), (int64_t)N, 0, (int64_t)M, (int64_t)N, (int64_t)K, 1, 0,
                              nullptr));
    c.download(C, M * N);
}

void gemm_accumulate_row_major(const float * A, const float * B, float * C, size_t M, size_t K, size_t N) {
    if (M == 0 || N == 0) return;
    DeviceArray a(A, M * K), b(B, K * N), c(C, M * N);
    op_check(sana_op_gemm_f32(a.get(), (int64_t)K, 0, b.get(), (int64_t)N, 0, 0, nullptr, 1, c.get(), (int64_t)N, 0,
                              (int64_t)M, (int64_t)N, (int64_t)K, 1, 1, nullptr));
    c.download(C, M * N);
}

Tensor linear_2d(const Tensor & input, const Tensor & weight, const Tensor * bias) {
    if (input.rank() != 2) throw std::invalid_argument("input must be rank 2");
    check_linear_args(weight, bias, input.dim_size(1));
    const size_t rows = input.dim_size(0), K = input.dim_size(1);
    return dev_linear(DeviceArray(input), rows, K, weight, bias).to_tensor({rows, weight.dim_size(1)});
}

Tensor mlp_2d(const Tensor & input, const Tensor & up_weight, const Tensor * up_bias, const Tensor & down_weight,
              const Tensor * down_bias) {
    if (input.rank() != 2) throw std::invalid_argument("input must be rank 2");
    check_linear_args(up_weight, up_bias, input.dim_size(1));
    check_linear_args(down_weight, down_bias, up_weight.dim_size(1));
    const size_t rows = input.dim_size(0);
    DeviceArray h = dev_linear(DeviceArray(input), rows, input.dim_size(1), up_weight, up_bias);
    dev_unary(h, SANA_OP_SILU);
    return dev_linear(h, rows, up_weight.dim_size(1), down_weight, down_bias).to_tensor({rows, down_weight.dim_size(1)});
}

Tensor linear_3d_lastdim(const Tensor & input, const Tensor & weight, const Tensor * bias) {
    if (input.rank() != 3) throw std::invalid_argument("input must be rank 3");
    check_linear_args(weight, bias, input.dim_size(2));
    const size_t B = input.dim_size(0), T = input.dim_size(1);
    return dev_linear(DeviceArray(input), B * T, input.dim_size(2), weight, bias).to_tensor({B, T, weight.dim_size(1)});
}

Tensor mlp_3d_lastdim(const Tensor & input, const Tensor & up_weight, const Tensor * up_bias,
                      const Tensor & down_weight, const Tensor * down_bias) {
    if (input.rank() != 3) throw std::invalid_argument("input must be rank 3");
    check_linear_args(up_weight, up_bias, input.dim_size(2));
    check_linear_args(down_weight, down_bias, up_weight.dim_size(1));
    const size_t B = input.dim_size(0), T = input.dim_size(1);
    DeviceArray h = dev_linear(DeviceArray(input), B * T, input.dim_size(2), up_weight, up_bias);
    dev_unary(h, SANA_OP_SILU);
    return dev_linear(h, B * T, up_weight.dim_size(1), down_weight, down_bias)
        .to_tensor({B, T, down_weight.dim_size(1)});
}

Tensor conv2d_1x1(const Tensor & input, const Tensor & weight, const Tensor * bias) {
    if (input.rank() != 4) throw std::invalid_argument("input must be rank 4");
    check_conv1x1_args(weight, bias, input.dim_size(1));
    const size_t B = input.dim_size(0), H = input.dim_size(2), W = input.dim_size(3);
    return dev_conv1x1(DeviceArray(input), B, input.dim_size(1), H * W, weight, bias)
        .to_tensor({B, weight.dim_size(0), H, W});
}

namespace {

Tensor depthwise(const Tensor & input, const Tensor & weight, const Tensor * bias, size_t ks) {
    if (input.rank() != 4) throw std::invalid_argument("input must be rank 4");
    if (weight.rank() != 4) throw std::invalid_argument("weight must be rank 4");
    if (weight.dim_size(1) != 1 || weight.dim_size(2) != ks || weight.dim_size(3) != ks)
        throw std::invalid_argument(ks == 3 ? "weight shape must be {channels, 1, 3, 3}"
                                            : "weight shape must be {channels, 1, 5, 5}");
    const size_t C = input.dim_size(1);
    if (weight.dim_size(0) != C) throw std::invalid_argument("weight channels must match input channels");
    if (bias) {
        if (bias->rank() != 1) throw std::invalid_argument("bias must be rank 1");
        if (bias->dim_size(0) != C) throw std::invalid_argument("bias size must match channels");
    }
    const size_t B = input.dim_size(0), H = input.dim_size(2), W = input.dim_size(3);
    if (B * C * H * W == 0) return Tensor(input.shape());
    DeviceArray x(input), w(weight), y(input.numel());
    auto b = upload_opt(bias);
    op_check(sana_op_dwconv_f32(x.get(), w.get(), opt(b.get()), y.get(), (int64_t)B, (int64_t)C, (int64_t)H,
                                (int64_t)W, (int64_t)ks, nullptr));
    return y.to_tensor(input.shape());
}

}  // namespace

Tensor depthwise_conv2d_3x3(const Tensor & input, const Tensor & weight, const Tensor * bias) {
    return depthwise(input, weight, bias, 3);
}

Tensor depthwise_conv2d_5x5(const Tensor & input, const Tensor & weight, const Tensor * bias) {
    return depthwise(input, weight, bias, 5);
}

Tensor glumb_conv(const Tensor & input, const Tensor & inv_w, const Tensor * inv_b, const Tensor & dw_w,
                  const Tensor * dw_b, const Tensor & pt_w) {
    // conv1x1 -> SiLU -> depthwise 3x3 -> data * SiLU(gate) -> conv1x1 (src/common_ops.cpp:733-761)
    if (input.rank() != 4) throw std::invalid_argument("input must be rank 4");
    check_conv1x1_args(inv_w, inv_b, input.dim_size(1));
    const size_t B = input.dim_size(0), H = input.dim_size(2), W = input.dim_size(3), S = H * W;
    const size_t E = inv_w.dim_size(0);
    if (dw_w.rank() != 4) throw std::invalid_argument("weight must be rank 4");
    if (dw_w.dim_size(1) != 1 || dw_w.dim_size(2) != 3 || dw_w.dim_size(3) != 3)
        throw std::invalid_argument("weight shape must be {channels, 1, 3, 3}");
    if (dw_w.dim_size(0) != E) throw std::invalid_argument("weight channels must match input channels");
    if (dw_b && (dw_b->rank() != 1 || dw_b->dim_size(0) != E))
        throw std::invalid_argument(dw_b->rank() != 1 ? "bias must be rank 1" : "bias size must match channels");
    if (E % 2 != 0) throw std::invalid_argument("channel count must be even");
    check_conv1x1_args(pt_w, nullptr, E / 2);
    DeviceArray h = dev_conv1x1(DeviceArray(input), B, input.dim_size(1), S, inv_w, inv_b);
    dev_unary(h, SANA_OP_SILU);
    DeviceArray d(h.size()), g(B * (E / 2) * S);
    {
        DeviceArray w(dw_w);
        auto b = upload_opt(dw_b);
        if (h.size())
            op_check(sana_op_dwconv_f32(h.get(), w.get(), opt(b.get()), d.get(), (int64_t)B, (int64_t)E, (int64_t)H,
                                        (int64_t)W, 3, nullptr));
    }
    op_check(sana_op_glu_f32(d.get(), g.get(), (int64_t)B, (int64_t)(E / 2), (int64_t)S, nullptr));
    return dev_conv1x1(g, B, E / 2, S, pt_w, nullptr).to_tensor({B, pt_w.dim_size(0), H, W});
}
