// Host tensor of the drop-in C++ API.  Semantics (layouts, broadcast rules,
// exception types) follow the reference's src/tensor.cpp:12-593; the
// implementations are plain loops of this library's own.
#include "tensor.h"

#include <cmath>
#include <numeric>
#include <stdexcept>

Tensor::Tensor(std::vector<size_t> shape) : shape_(std::move(shape)) { data_.assign(numel(), 0.0f); }

const std::vector<size_t> & Tensor::shape() const { return shape_; }
std::vector<float> & Tensor::data() { return data_; }
const std::vector<float> & Tensor::data() const { return data_; }

float & Tensor::at(size_t i) {
    if (i >= data_.size()) throw std::out_of_range("index out of range");
    return data_[i];
}

const float & Tensor::at(size_t i) const {
    if (i >= data_.size()) throw std::out_of_range("index out of range");
    return data_[i];
}

float & Tensor::at(const std::vector<size_t> & idx) { return at(flat_index(idx)); }
const float & Tensor::at(const std::vector<size_t> & idx) const { return at(flat_index(idx)); }

void Tensor::fill(float v) { std::fill(data_.begin(), data_.end(), v); }

bool Tensor::same_shape(const Tensor & o) const { return shape_ == o.shape_; }

size_t Tensor::flat_index(const std::vector<size_t> & idx) const {
    if (idx.size() != shape_.size()) throw std::out_of_range("indices must give one index per dimension");
    size_t flat = 0;
    for (size_t d = 0; d < shape_.size(); ++d) {
        if (idx[d] >= shape_[d]) throw std::out_of_range("index exceeds the tensor dimension");
        flat = flat * shape_[d] + idx[d];
    }
    return flat;
}

size_t Tensor::rank() const { return shape_.size(); }

size_t Tensor::numel() const {
    return std::accumulate(shape_.begin(), shape_.end(), size_t(1), [](size_t a, size_t b) { return a * b; });
}

size_t Tensor::dim_size(size_t axis) const {
    if (axis >= shape_.size()) throw std::out_of_range("tensor dimension axis out of range");
    return shape_[axis];
}

void Tensor::add_inplace(const Tensor & o) {
    if (!same_shape(o)) throw std::invalid_argument("cannot add two tensors with different shapes");
    for (size_t i = 0; i < data_.size(); ++i) data_[i] += o.data_[i];
}

void Tensor::mul_inplace_scalar(float s) {
    for (float & v : data_) v *= s;
}

void Tensor::mul_inplace_broadcast_lastdim(const Tensor & gate) {
    if (rank() != 3) throw std::invalid_argument("input must be rank 3");
    if (gate.rank() != 3) throw std::invalid_argument("gate must be rank 3");
    const size_t B = shape_[0], N = shape_[1], C = shape_[2];
    if (gate.shape_[0] != B || gate.shape_[1] != 1 || gate.shape_[2] != C)
        throw std::invalid_argument("gate must have shape {batch, 1, hidden}");
    for (size_t b = 0; b < B; ++b)
        for (size_t t = 0; t < N; ++t)
            for (size_t c = 0; c < C; ++c) data_[(b * N + t) * C + c] *= gate.data_[b * C + c];
}

Tensor Tensor::transpose_2d() const {
    if (rank() != 2) throw std::invalid_argument("rank is not 2");
    const size_t R = shape_[0], C = shape_[1];
    Tensor out({C, R});
    for (size_t r = 0; r < R; ++r)
        for (size_t c = 0; c < C; ++c) out.data_[c * R + r] = data_[r * C + c];
    return out;
}

Tensor Tensor::layer_norm_3d_lastdim(float eps, const Tensor * gamma, const Tensor * beta) const {
    if (rank() != 3) throw std::invalid_argument("tensor must be 3d");
    const size_t C = shape_[2], rows = shape_[0] * shape_[1];
    if (gamma && (gamma->rank() != 1 || gamma->shape_[0] != C))
        throw std::invalid_argument("gamma must be 1D and match hidden size");
    if (beta && (beta->rank() != 1 || beta->shape_[0] != C))
        throw std::invalid_argument("beta must be 1D and match hidden size");
    Tensor out(shape_);
    for (size_t r = 0; r < rows; ++r) {
        const float * x = data_.data() + r * C;
        float mean = 0.0f, var = 0.0f;
        for (size_t c = 0; c < C; ++c) mean += x[c];
        mean /= static_cast<float>(C);
        for (size_t c = 0; c < C; ++c) var += (x[c] - mean) * (x[c] - mean);
        var /= static_cast<float>(C);
        const float inv = 1.0f / std::sqrt(var + eps);
        for (size_t c = 0; c < C; ++c) {
            float y = (x[c] - mean) * inv;
            if (gamma) y *= gamma->data_[c];
            if (beta) y += beta->data_[c];
            out.data_[r * C + c] = y;
        }
    }
    return out;
}

Tensor Tensor::rms_norm_3d_lastdim(float eps, const Tensor * weight) const {
    if (rank() != 3) throw std::invalid_argument("tensor must be 3d");
    const size_t C = shape_[2], rows = shape_[0] * shape_[1];
    if (weight && (weight->rank() != 1 || weight->shape_[0] != C))
        throw std::invalid_argument("weight must be 1D and match hidden size");
    Tensor out(shape_);
    for (size_t r = 0; r < rows; ++r) {
        const float * x = data_.data() + r * C;
        float ms = 0.0f;
        for (size_t c = 0; c < C; ++c) ms += x[c] * x[c];
        const float inv = 1.0f / std::sqrt(ms / static_cast<float>(C) + eps);
        for (size_t c = 0; c < C; ++c) out.data_[r * C + c] = x[c] * inv * (weight ? weight->data_[c] : 1.0f);
    }
    return out;
}

Tensor Tensor::modulate_3d_lastdim(const Tensor & shift, const Tensor & scale) const {
    if (rank() != 3) throw std::invalid_argument("input must be rank 3");
    if (shift.rank() != 3 || scale.rank() != 3) throw std::invalid_argument("shift and scale must be rank 3");
    const size_t B = shape_[0], N = shape_[1], C = shape_[2];
    if (shift.shape_[0] != B || shift.shape_[1] != 1 || shift.shape_[2] != C)
        throw std::invalid_argument("shift must have shape {batch, 1, hidden}");
    if (scale.shape_[0] != B || scale.shape_[1] != 1 || scale.shape_[2] != C)
        throw std::invalid_argument("scale must have shape {batch, 1, hidden}");
    Tensor out(shape_);
    for (size_t b = 0; b < B; ++b)
        for (size_t t = 0; t < N; ++t)
            for (size_t c = 0; c < C; ++c) {
                const size_t i = (b * N + t) * C + c;
                out.data_[i] = data_[i] * (1.0f + scale.data_[b * C + c]) + shift.data_[b * C + c];
            }
    return out;
}

Tensor Tensor::tokens_to_grid_4d(size_t height, size_t width) const {
    if (rank() != 3) throw std::invalid_argument("input must be rank 3");
    if (height == 0 || width == 0) throw std::invalid_argument("height and width must be greater than 0");
    const size_t B = shape_[0], N = shape_[1], C = shape_[2];
    if (N != height * width) throw std::invalid_argument("tokens must equal height * width");
    Tensor out({B, C, height, width});
    for (size_t b = 0; b < B; ++b)
        for (size_t t = 0; t < N; ++t)
            for (size_t c = 0; c < C; ++c) out.data_[(b * C + c) * N + t] = data_[(b * N + t) * C + c];
    return out;
}

Tensor Tensor::grid_to_tokens_3d() const {
    const size_t B = dim_size(0), C = dim_size(1), N = dim_size(2) * dim_size(3);
    Tensor out({B, N, C});
    for (size_t b = 0; b < B; ++b)
        for (size_t c = 0; c < C; ++c)
            for (size_t t = 0; t < N; ++t) out.data_[(b * N + t) * C + c] = data_[(b * C + c) * N + t];
    return out;
}

std::pair<Tensor, Tensor> Tensor::split_channels_4d() const {
    if (rank() != 4) throw std::invalid_argument("input must be rank 4");
    const size_t B = shape_[0], C = shape_[1], S = shape_[2] * shape_[3];
    if (C % 2 != 0) throw std::invalid_argument("channel count must be even");
    const size_t H = C / 2;
    Tensor a({B, H, shape_[2], shape_[3]}), g({B, H, shape_[2], shape_[3]});
    for (size_t b = 0; b < B; ++b)
        for (size_t c = 0; c < H; ++c)
            for (size_t s = 0; s < S; ++s) {
                a.data_[(b * H + c) * S + s] = data_[(b * C + c) * S + s];
                g.data_[(b * H + c) * S + s] = data_[(b * C + H + c) * S + s];
            }
    return {a, g};
}

std::tuple<Tensor, Tensor, Tensor, Tensor, Tensor, Tensor> Tensor::split_six_way_3d() const {
    if (rank() != 3) throw std::invalid_argument("input must be rank 3");
    if (shape_[1] != 6) throw std::invalid_argument("second dimension must be exactly 6");
    const size_t B = shape_[0], C = shape_[2];
    std::vector<Tensor> parts(6, Tensor({B, 1, C}));
    for (size_t p = 0; p < 6; ++p)
        for (size_t b = 0; b < B; ++b)
            for (size_t c = 0; c < C; ++c) parts[p].data_[b * C + c] = data_[(b * 6 + p) * C + c];
    return {parts[0], parts[1], parts[2], parts[3], parts[4], parts[5]};
}

void Tensor::silu_inplace() {
    for (float & v : data_) v = v / (1.0f + std::exp(-v));
}

void Tensor::relu_inplace() {
    for (float & v : data_) v = v > 0.0f ? v : 0.0f;
}

float Tensor::max_abs_diff(const Tensor & o) const {
    if (!same_shape(o)) throw std::invalid_argument("shape mismatch");
    float m = 0.0f;
    for (size_t i = 0; i < data_.size(); ++i) m = std::max(m, std::fabs(data_[i] - o.data_[i]));
    return m;
}

float Tensor::mean_abs_diff(const Tensor & o) const {
    if (!same_shape(o)) throw std::invalid_argument("shape mismatch");
    if (data_.empty()) return 0.0f;
    double s = 0.0;
    for (size_t i = 0; i < data_.size(); ++i) s += std::fabs(data_[i] - o.data_[i]);
    return static_cast<float>(s / static_cast<double>(data_.size()));
}
