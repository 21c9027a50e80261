// Device-resident building blocks shared by common_ops.cpp and
// transformer_ops.cpp: each takes and returns DeviceArrays so composite ops
// (MLPs, GLUMBConv, attention blocks) keep their intermediates on the GPU.
#pragma once

#include <cstddef>
#include <memory>

#include "device_array.h"
#include "tensor.h"

namespace sana_host {

// x [rows, K] . W [K, N] (+ bias [N]); argument checks as linear_3d_lastdim.
DeviceArray dev_linear(const DeviceArray & x, size_t rows, size_t K, const Tensor & weight, const Tensor * bias);
// In place: op = SANA_OP_SILU / SANA_OP_GELU_TANH / SANA_OP_RELU.
void dev_unary(DeviceArray & x, int op);
// NCHW 1x1 convolution: W [OC, IC, 1, 1] over x [B, IC, S] (+ bias [OC]).
DeviceArray dev_conv1x1(const DeviceArray & x, size_t B, size_t IC, size_t S, const Tensor & weight,
                        const Tensor * bias);
// The weight / bias checks of linear_2d / linear_3d_lastdim.
void check_linear_args(const Tensor & weight, const Tensor * bias, size_t in_features);
// Checks of conv2d_1x1 for an input of `in_channels` channels.
void check_conv1x1_args(const Tensor & weight, const Tensor * bias, size_t in_channels);

std::unique_ptr<DeviceArray> upload_opt(const Tensor * t);

}  // namespace sana_host
