// Drop-in denoiser API on the HIP gfx950 path.
//
// Host side: the loaders and validators keep the reference's checks, messages
// and exception types (src/transformer.cpp:167-498, :780-884).  Device side:
// block_forward, run_model_blocks, the CFG step and the CFG loop upload the
// weights once into a sana_dit context (sana_dit.h) and run the forward there.
// Contexts are cached per weights object (its address, plus a fingerprint of
// every tensor's storage address, shape and sampled values, so a reallocated
// or refilled weights object is uploaded again); at most kMaxModels stay
// resident, least recently used first out.  Calls are serialised by one mutex.
//
// Limits of the device path (std::invalid_argument when exceeded): hidden size
// <= 2048, self head_dim <= 100, latent channels <= 32, caption length <= 512,
// the same head counts in every block.
#include "transformer.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>

#include "../../include/sana_dit.h"
#include "../csrc/gguf.h"
#include "fingerprint.h"

namespace {

// ---------------------------------------------------------------- errors

[[noreturn]] void raise_abi(int rc) {
    const std::string msg = sana_dit_last_error();
    if (rc == SANA_ERR_INVALID_ARGUMENT || rc == SANA_ERR_SHAPE) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

void ck(int rc) {
    if (rc != SANA_OK) raise_abi(rc);
}

// ---------------------------------------------------------------- host helpers

size_t square_side(size_t tokens) {  // infer_square_side, src/transformer.cpp:18-24
    const size_t side = static_cast<size_t>(std::sqrt(static_cast<double>(tokens)));
    if (side * side != tokens) throw std::invalid_argument("token count must form a square grid");
    return side;
}

bool all_equal(const Tensor & t, float v) {
    for (float x : t.data())
        if (x != v) return false;
    return true;
}

std::vector<int64_t> shape64(const Tensor & t) {
    std::vector<int64_t> s;
    for (size_t d : t.shape()) s.push_back(static_cast<int64_t>(d));
    return s;
}

// ---------------------------------------------------------------- fingerprints

using sana_fp::mix;

uint64_t block_fingerprint(const SanaBlockWeights * blocks, size_t count) {
    uint64_t h = sana_fp::kSeed;
    mix(h, count);
    for (size_t i = 0; i < count; ++i) {
        const SanaBlockWeights & w = blocks[i];
        for (const Tensor * t :
             {&w.scale_shift_table, &w.attn_norm_gamma, &w.attn_norm_beta, &w.q_weight, &w.q_bias, &w.k_weight,
              &w.k_bias, &w.v_weight, &w.v_bias, &w.out_weight, &w.out_bias, &w.cross_q_weight, &w.cross_q_bias,
              &w.cross_k_weight, &w.cross_k_bias, &w.cross_v_weight, &w.cross_v_bias, &w.cross_out_weight,
              &w.cross_out_bias, &w.mlp_norm_gamma, &w.mlp_norm_beta, &w.ff_inverted_weight, &w.ff_inverted_bias,
              &w.ff_depth_weight, &w.ff_depth_bias, &w.ff_point_weight})
            sana_fp::tensor(h, *t);
        mix(h, w.self_num_heads);
        mix(h, w.cross_num_heads);
    }
    return h;
}

uint64_t top_fingerprint(const SanaDenoiserWeights & w) {
    uint64_t h = sana_fp::kSeed;
    for (const Tensor * t :
         {&w.caption.linear_1_weight, &w.caption.linear_1_bias, &w.caption.linear_2_weight, &w.caption.linear_2_bias,
          &w.patch_embed_weight, &w.patch_embed_bias, &w.time_embed_linear_1_weight, &w.time_embed_linear_1_bias,
          &w.time_embed_linear_2_weight, &w.time_embed_linear_2_bias, &w.time_projection_weight,
          &w.time_projection_bias, &w.caption_norm_weight, &w.final_scale_shift_table, &w.proj_out_weight,
          &w.proj_out_bias})
        sana_fp::tensor(h, *t);
    return h;
}

// ---------------------------------------------------------------- device models

struct DeviceModel {
    sana_dit * ctx = nullptr;
    uint64_t blocks_fp = 0;
    std::pair<int64_t, int64_t> dims{0, 0};  // caption width, latent channels of the context
    bool top_loaded = false;
    uint64_t top_fp = 0;
    uint64_t last_use = 0;
    // conditioning currently set on the context
    bool ctx_valid = false;
    int ctx_projected = 0;
    std::vector<size_t> ctx_shape;
    std::vector<float> ctx_data, ctx_bias;
    bool ctx_has_bias = false;

    DeviceModel() = default;
    DeviceModel(const DeviceModel &) = delete;
    DeviceModel & operator=(const DeviceModel &) = delete;
    ~DeviceModel() {
        if (ctx) sana_dit_destroy(ctx);
    }
};

constexpr size_t kMaxModels = 4;
std::mutex g_mutex;
std::map<std::pair<int, const void *>, std::unique_ptr<DeviceModel>> g_models;
uint64_t g_clock = 0;

int hip_device() {
    const char * e = std::getenv("SANA_HIP_DEVICE");
    return e ? std::atoi(e) : 0;
}

void put_block_tensor(sana_dit * c, int64_t blk, const char * suffix, const Tensor & t, int transposed) {
    const std::vector<int64_t> s = shape64(t);
    ck(sana_dit_set_block_weight(c, blk, suffix, t.data().data(), s.data(), static_cast<int>(s.size()), transposed));
}

void put_norm(sana_dit * c, int64_t blk, int which, const Tensor & gamma, const Tensor & beta, size_t hidden) {
    if (gamma.rank() != 1 || gamma.dim_size(0) != hidden)
        throw std::invalid_argument("gamma must be 1D and match hidden size");
    if (beta.rank() != 1 || beta.dim_size(0) != hidden)
        throw std::invalid_argument("beta must be 1D and match hidden size");
    if (all_equal(gamma, 1.0f) && all_equal(beta, 0.0f)) return;  // the kernels' default affine
    ck(sana_dit_set_block_norm(c, blk, which, gamma.data().data(), beta.data().data()));
}

void upload_block(sana_dit * c, int64_t i, const SanaBlockWeights & w, size_t hidden) {
    put_block_tensor(c, i, "scale_shift_table", w.scale_shift_table, 0);
    put_norm(c, i, 0, w.attn_norm_gamma, w.attn_norm_beta, hidden);
    put_norm(c, i, 1, w.mlp_norm_gamma, w.mlp_norm_beta, hidden);
    put_block_tensor(c, i, "attn1.to_q.weight", w.q_weight, 1);
    put_block_tensor(c, i, "attn1.to_k.weight", w.k_weight, 1);
    put_block_tensor(c, i, "attn1.to_v.weight", w.v_weight, 1);
    if (!all_equal(w.q_bias, 0.0f) || !all_equal(w.k_bias, 0.0f) || !all_equal(w.v_bias, 0.0f)) {
        put_block_tensor(c, i, "attn1.to_q.bias", w.q_bias, 0);
        put_block_tensor(c, i, "attn1.to_k.bias", w.k_bias, 0);
        put_block_tensor(c, i, "attn1.to_v.bias", w.v_bias, 0);
    }
    put_block_tensor(c, i, "attn1.to_out.0.weight", w.out_weight, 1);
    put_block_tensor(c, i, "attn1.to_out.0.bias", w.out_bias, 0);
    put_block_tensor(c, i, "attn2.to_q.weight", w.cross_q_weight, 1);
    put_block_tensor(c, i, "attn2.to_q.bias", w.cross_q_bias, 0);
    put_block_tensor(c, i, "attn2.to_k.weight", w.cross_k_weight, 1);
    put_block_tensor(c, i, "attn2.to_k.bias", w.cross_k_bias, 0);
    put_block_tensor(c, i, "attn2.to_v.weight", w.cross_v_weight, 1);
    put_block_tensor(c, i, "attn2.to_v.bias", w.cross_v_bias, 0);
    put_block_tensor(c, i, "attn2.to_out.0.weight", w.cross_out_weight, 1);
    put_block_tensor(c, i, "attn2.to_out.0.bias", w.cross_out_bias, 0);
    put_block_tensor(c, i, "ff.conv_inverted.weight", w.ff_inverted_weight, 0);
    put_block_tensor(c, i, "ff.conv_inverted.bias", w.ff_inverted_bias, 0);
    put_block_tensor(c, i, "ff.conv_depth.weight", w.ff_depth_weight, 0);
    put_block_tensor(c, i, "ff.conv_depth.bias", w.ff_depth_bias, 0);
    put_block_tensor(c, i, "ff.conv_point.weight", w.ff_point_weight, 0);
}

void put_top(sana_dit * c, const char * name, const Tensor & t, int transposed) {
    const std::vector<int64_t> s = shape64(t);
    ck(sana_dit_set_weight(c, name, t.data().data(), s.data(), static_cast<int>(s.size()), transposed));
}

void upload_top(sana_dit * c, const SanaDenoiserWeights & w) {
    put_top(c, "caption_projection.linear_1.weight", w.caption.linear_1_weight, 1);
    put_top(c, "caption_projection.linear_1.bias", w.caption.linear_1_bias, 0);
    put_top(c, "caption_projection.linear_2.weight", w.caption.linear_2_weight, 1);
    put_top(c, "caption_projection.linear_2.bias", w.caption.linear_2_bias, 0);
    put_top(c, "patch_embed.proj.weight", w.patch_embed_weight, 0);
    put_top(c, "patch_embed.proj.bias", w.patch_embed_bias, 0);
    put_top(c, "time_embed.emb.timestep_embedder.linear_1.weight", w.time_embed_linear_1_weight, 1);
    put_top(c, "time_embed.emb.timestep_embedder.linear_1.bias", w.time_embed_linear_1_bias, 0);
    put_top(c, "time_embed.emb.timestep_embedder.linear_2.weight", w.time_embed_linear_2_weight, 1);
    put_top(c, "time_embed.emb.timestep_embedder.linear_2.bias", w.time_embed_linear_2_bias, 0);
    put_top(c, "time_embed.linear.weight", w.time_projection_weight, 1);
    put_top(c, "time_embed.linear.bias", w.time_projection_bias, 0);
    put_top(c, "caption_norm.weight", w.caption_norm_weight, 0);
    put_top(c, "scale_shift_table", w.final_scale_shift_table, 0);
    put_top(c, "proj_out.weight", w.proj_out_weight, 1);
    put_top(c, "proj_out.bias", w.proj_out_bias, 0);
    ck(sana_dit_check_weights(c));
}

size_t block_hidden(const SanaBlockWeights & w) {
    if (w.scale_shift_table.rank() != 2 || w.scale_shift_table.dim_size(0) != 6)
        throw std::invalid_argument("scale_shift_table must have shape {6, hidden}");
    return w.scale_shift_table.dim_size(1);
}

// Caption width and latent channels a context is created with: from the
// top-level weights where they have the expected ranks (run_model_blocks does
// not need them), else placeholders.
std::pair<int64_t, int64_t> top_dims(const SanaDenoiserWeights * top, size_t hidden) {
    int64_t caption = static_cast<int64_t>(hidden), latent = 1;
    if (top && top->caption.linear_1_weight.rank() == 2)
        caption = static_cast<int64_t>(top->caption.linear_1_weight.dim_size(0));
    if (top && top->patch_embed_weight.rank() == 4)
        latent = static_cast<int64_t>(top->patch_embed_weight.dim_size(1));
    return {caption, latent};
}

// Device context holding `count` blocks, created or refreshed as the
// fingerprints require; with need_top the top-level weights of `top` are
// uploaded too.
DeviceModel & device_model(int kind, const void * key, const SanaBlockWeights * blocks, size_t count,
                           const SanaDenoiserWeights * top, bool need_top) {
    if (count == 0) throw std::invalid_argument("model must contain at least one block");
    const SanaBlockWeights & b0 = blocks[0];
    const size_t hidden = block_hidden(b0);
    const std::pair<int64_t, int64_t> dims = top_dims(top, hidden);
    const uint64_t bfp = block_fingerprint(blocks, count);
    auto & slot = g_models[{kind, key}];
    if (slot && (slot->blocks_fp != bfp || (need_top && slot->dims != dims))) slot.reset();
    if (!slot) {
        if (g_models.size() > kMaxModels) {
            auto victim = g_models.end();
            for (auto it = g_models.begin(); it != g_models.end(); ++it)
                if (it->second && (victim == g_models.end() || it->second->last_use < victim->second->last_use))
                    victim = it;
            if (victim != g_models.end()) g_models.erase(victim);
        }
        for (size_t i = 1; i < count; ++i)
            if (blocks[i].self_num_heads != b0.self_num_heads || blocks[i].cross_num_heads != b0.cross_num_heads)
                throw std::invalid_argument("all model blocks must use the same head counts on this device path");
        if (b0.ff_inverted_weight.rank() != 4) throw std::invalid_argument("ff conv weights must be rank 4");
        if (b0.self_num_heads == 0) throw std::invalid_argument("self_num_heads must be greater than 0");
        if (b0.cross_num_heads == 0) throw std::invalid_argument("cross_num_heads must be greater than 0");
        auto dm = std::make_unique<DeviceModel>();
        sana_dit_config cfg{};
        cfg.layers = static_cast<int64_t>(count);
        cfg.hidden = static_cast<int64_t>(hidden);
        cfg.ffn = static_cast<int64_t>(b0.ff_inverted_weight.dim_size(0));
        cfg.caption_dim = dims.first;
        cfg.latent_channels = dims.second;
        cfg.self_heads = static_cast<int64_t>(b0.self_num_heads);
        cfg.cross_heads = static_cast<int64_t>(b0.cross_num_heads);
        cfg.device = hip_device();
        ck(sana_dit_create(&cfg, &dm->ctx));
        for (size_t i = 0; i < count; ++i) upload_block(dm->ctx, static_cast<int64_t>(i), blocks[i], hidden);
        dm->blocks_fp = bfp;
        dm->dims = dims;
        slot = std::move(dm);
    }
    DeviceModel & m = *slot;
    if (need_top) {
        const uint64_t tfp = top_fingerprint(*top);
        if (!m.top_loaded || m.top_fp != tfp) {
            m.top_loaded = false;
            upload_top(m.ctx, *top);
            m.top_loaded = true;
            m.top_fp = tfp;
            m.ctx_valid = false;
        }
    }
    m.last_use = ++g_clock;
    return m;
}

// Sets the conditioning unless the same data is already set.  bias is the
// [B, 1, L] additive key mask or null.
void set_conditioning(DeviceModel & m, const Tensor & data, int projected, const Tensor * bias) {
    const bool same = m.ctx_valid && m.ctx_projected == projected && m.ctx_shape == data.shape() &&
                      m.ctx_has_bias == (bias != nullptr) && m.ctx_data == data.data() &&
                      (!bias || m.ctx_bias == bias->data());
    if (same) return;
    m.ctx_valid = false;
    const int64_t B = static_cast<int64_t>(data.dim_size(0)), L = static_cast<int64_t>(data.dim_size(1));
    const int64_t dim = static_cast<int64_t>(data.dim_size(2));
    ck(sana_dit_set_context(m.ctx, data.data().data(), B, L, dim, projected, bias ? bias->data().data() : nullptr));
    m.ctx_projected = projected;
    m.ctx_shape = data.shape();
    m.ctx_data = data.data();
    m.ctx_has_bias = bias != nullptr;
    m.ctx_bias = bias ? bias->data() : std::vector<float>();
    m.ctx_valid = true;
}

void check_bias(const Tensor * bias, size_t batch, size_t keys) {
    if (!bias) return;
    if (bias->rank() != 3 || bias->dim_size(0) != batch || bias->dim_size(1) != 1 || bias->dim_size(2) != keys)
        throw std::invalid_argument("attention_bias shape must be {batch, 1, key_tokens}");
}

// The shape checks block_forward's host ops apply to (input, context,
// timestep) before any compute (src/transformer.cpp:733-760 and the ops it calls).
void check_block_inputs(const Tensor & input, const Tensor & context, const Tensor & timestep, size_t hidden,
                        const Tensor * bias) {
    if (timestep.rank() != 2) throw std::invalid_argument("timestep must be rank 2");
    if (timestep.dim_size(1) != 6 * hidden) throw std::invalid_argument("timestep width must equal 6 * hidden");
    if (input.rank() != 3) throw std::invalid_argument("tensor must be 3d");
    if (input.dim_size(2) != hidden) throw std::invalid_argument("gamma must be 1D and match hidden size");
    if (timestep.dim_size(0) != input.dim_size(0))
        throw std::invalid_argument("shift must have shape {batch, 1, hidden}");
    if (context.rank() != 3) throw std::invalid_argument("context must be rank 3");
    if (input.dim_size(0) != context.dim_size(0))
        throw std::invalid_argument("input and context batch size must match");
    if (context.dim_size(2) != hidden)
        throw std::invalid_argument("context hidden size must match the cross-attention key/value weights");
    check_bias(bias, input.dim_size(0), context.dim_size(1));
    square_side(input.dim_size(1));
}

bool default_solver(const SanaSchedulerConfig & c) {
    return c.use_flow_sigmas && c.solver_order == 2 && c.lower_order_final && c.prediction_type == "flow_prediction" &&
           c.algorithm_type == "dpmsolver++" && c.solver_type == "midpoint" && c.final_sigmas_type == "zero";
}

void check_dims(const std::vector<size_t> & shape, std::initializer_list<size_t> want, const char * msg) {
    if (shape != std::vector<size_t>(want)) throw std::invalid_argument(msg);
}

// Tensor names of load_block_weights (src/transformer.cpp:214-308), by the
// member they fill.  linear = 1: stored [out, in], loaded transposed to [in, out].
struct BlockTensorName {
    const char * suffix;
    Tensor SanaBlockWeights::*member;
    int linear;
};

const BlockTensorName kBlockNames[] = {
    {"scale_shift_table", &SanaBlockWeights::scale_shift_table, 0},
    {"attn1.to_q.weight", &SanaBlockWeights::q_weight, 1},
    {"attn1.to_k.weight", &SanaBlockWeights::k_weight, 1},
    {"attn1.to_v.weight", &SanaBlockWeights::v_weight, 1},
    {"attn1.to_out.0.weight", &SanaBlockWeights::out_weight, 1},
    {"attn1.to_out.0.bias", &SanaBlockWeights::out_bias, 0},
    {"attn2.to_q.weight", &SanaBlockWeights::cross_q_weight, 1},
    {"attn2.to_q.bias", &SanaBlockWeights::cross_q_bias, 0},
    {"attn2.to_k.weight", &SanaBlockWeights::cross_k_weight, 1},
    {"attn2.to_k.bias", &SanaBlockWeights::cross_k_bias, 0},
    {"attn2.to_v.weight", &SanaBlockWeights::cross_v_weight, 1},
    {"attn2.to_v.bias", &SanaBlockWeights::cross_v_bias, 0},
    {"attn2.to_out.0.weight", &SanaBlockWeights::cross_out_weight, 1},
    {"attn2.to_out.0.bias", &SanaBlockWeights::cross_out_bias, 0},
    {"ff.conv_inverted.weight", &SanaBlockWeights::ff_inverted_weight, 0},
    {"ff.conv_inverted.bias", &SanaBlockWeights::ff_inverted_bias, 0},
    {"ff.conv_depth.weight", &SanaBlockWeights::ff_depth_weight, 0},
    {"ff.conv_depth.bias", &SanaBlockWeights::ff_depth_bias, 0},
    {"ff.conv_point.weight", &SanaBlockWeights::ff_point_weight, 0},
};

}  // namespace

// ---------------------------------------------------------------- loading

SanaCaptionWeights load_caption_weights(const std::string & dir,
                                        const std::unordered_map<std::string, SavedWeightInfo> & index) {
    return SanaCaptionWeights{
        load_linear_weight_tensor(dir, index, "caption_projection.linear_1.weight"),
        load_weight_tensor(dir, index, "caption_projection.linear_1.bias"),
        load_linear_weight_tensor(dir, index, "caption_projection.linear_2.weight"),
        load_weight_tensor(dir, index, "caption_projection.linear_2.bias"),
    };
}

SanaBlockWeights load_block_weights(const std::string & dir,
                                    const std::unordered_map<std::string, SavedWeightInfo> & index,
                                    const std::string & prefix, size_t self_num_heads, size_t cross_num_heads) {
    if (self_num_heads == 0) throw std::invalid_argument("self_num_heads must be greater than 0");
    if (cross_num_heads == 0) throw std::invalid_argument("cross_num_heads must be greater than 0");
    // Placeholders for the members the checkpoint does not hold; every tensor
    // member is assigned below.
    const Tensor none({0});
    SanaBlockWeights w{none, none, none, none, none, none, none, none, none, none, none, none, none, none,
                       none, none, none, none, none, none, none, none, none, none, none, none, self_num_heads,
                       cross_num_heads};
    for (const BlockTensorName & n : kBlockNames) {
        const std::string name = prefix.empty() ? n.suffix : prefix + "." + n.suffix;
        w.*n.member = n.linear ? load_linear_weight_tensor(dir, index, name) : load_weight_tensor(dir, index, name);
    }
    // Shape checks of src/transformer.cpp:308-360, same order and messages.
    if (w.scale_shift_table.rank() != 2 || w.scale_shift_table.dim_size(0) != 6)
        throw std::runtime_error("scale_shift_table must have shape {6, hidden}");
    if (w.q_weight.rank() != 2 || w.k_weight.rank() != 2 || w.v_weight.rank() != 2 || w.out_weight.rank() != 2)
        throw std::runtime_error("attn1 projection weights must be rank 2");
    if (w.out_bias.rank() != 1) throw std::runtime_error("attn1 output bias must be rank 1");
    if (w.cross_q_weight.rank() != 2 || w.cross_k_weight.rank() != 2 || w.cross_v_weight.rank() != 2 ||
        w.cross_out_weight.rank() != 2)
        throw std::runtime_error("attn2 projection weights must be rank 2");
    if (w.cross_q_bias.rank() != 1 || w.cross_k_bias.rank() != 1 || w.cross_v_bias.rank() != 1 ||
        w.cross_out_bias.rank() != 1)
        throw std::runtime_error("attn2 biases must be rank 1");
    if (w.ff_inverted_weight.rank() != 4 || w.ff_depth_weight.rank() != 4 || w.ff_point_weight.rank() != 4)
        throw std::runtime_error("ff conv weights must be rank 4");
    if (w.ff_inverted_bias.rank() != 1 || w.ff_depth_bias.rank() != 1)
        throw std::runtime_error("ff conv biases must be rank 1");
    const size_t hidden = w.q_weight.dim_size(1);
    if (w.scale_shift_table.dim_size(1) != hidden)
        throw std::runtime_error("scale_shift_table hidden size must match attention hidden size");
    if (hidden % self_num_heads != 0)
        throw std::runtime_error("self attention hidden size must be divisible by self_num_heads");
    if (hidden % cross_num_heads != 0)
        throw std::runtime_error("cross attention hidden size must be divisible by cross_num_heads");
    if (w.cross_q_weight.dim_size(1) != hidden || w.cross_out_weight.dim_size(0) != hidden)
        throw std::runtime_error("attn2 hidden size must match block hidden size");
    if (w.cross_q_bias.dim_size(0) != hidden || w.cross_out_bias.dim_size(0) != hidden)
        throw std::runtime_error("attn2 q/out bias size must match block hidden size");
    if (w.ff_inverted_weight.dim_size(1) != hidden || w.ff_point_weight.dim_size(0) != hidden)
        throw std::runtime_error("ff hidden size must match block hidden size");
    const size_t expanded = w.ff_inverted_weight.dim_size(0);
    if (w.ff_inverted_bias.dim_size(0) != expanded || w.ff_depth_weight.dim_size(0) != expanded ||
        w.ff_depth_bias.dim_size(0) != expanded)
        throw std::runtime_error("ff expanded channel sizes must match");
    if (w.ff_point_weight.dim_size(1) * 2 != expanded)
        throw std::runtime_error("ff point conv input channels must match split GLUMB width");
    // Sana's blocks have no q/k/v biases and non-affine norms: zeros and ones
    // (src/transformer.cpp:361-398).
    Tensor zeros({hidden}), ones({hidden});
    ones.fill(1.0f);
    w.q_bias = w.k_bias = w.v_bias = zeros;
    w.attn_norm_gamma = w.mlp_norm_gamma = ones;
    w.attn_norm_beta = w.mlp_norm_beta = zeros;
    return w;
}

std::vector<std::string> find_block_prefixes(const std::unordered_map<std::string, SavedWeightInfo> & index) {
    std::vector<std::string> names;
    names.reserve(index.size());
    for (const auto & kv : index) names.push_back(kv.first);
    return sana::gguf::block_prefixes(names);
}

std::vector<SanaBlockWeights> load_model_block_weights(const std::string & dir,
                                                       const std::unordered_map<std::string, SavedWeightInfo> & index,
                                                       size_t self_num_heads, size_t cross_num_heads) {
    const std::vector<std::string> prefixes = find_block_prefixes(index);
    if (prefixes.empty()) throw std::invalid_argument("weight index does not contain any prefixed model blocks");
    std::vector<SanaBlockWeights> blocks;
    blocks.reserve(prefixes.size());
    for (const std::string & p : prefixes)
        blocks.push_back(load_block_weights(dir, index, p, self_num_heads, cross_num_heads));
    return blocks;
}

SanaDenoiserWeights load_denoiser_weights(const std::string & block_dir,
                                          const std::unordered_map<std::string, SavedWeightInfo> & block_index,
                                          const std::string & caption_dir,
                                          const std::unordered_map<std::string, SavedWeightInfo> & caption_index,
                                          const std::string & dir,
                                          const std::unordered_map<std::string, SavedWeightInfo> & index,
                                          size_t self_num_heads, size_t cross_num_heads) {
    SanaCaptionWeights caption = load_caption_weights(caption_dir, caption_index);
    std::vector<SanaBlockWeights> blocks = load_model_block_weights(block_dir, block_index, self_num_heads,
                                                                     cross_num_heads);
    auto plain = [&](const char * n) { return load_weight_tensor(dir, index, n); };
    auto linear = [&](const char * n) { return load_linear_weight_tensor(dir, index, n); };
    SanaDenoiserWeights w{
        std::move(caption),
        std::move(blocks),
        plain("patch_embed.proj.weight"),
        plain("patch_embed.proj.bias"),
        linear("time_embed.emb.timestep_embedder.linear_1.weight"),
        plain("time_embed.emb.timestep_embedder.linear_1.bias"),
        linear("time_embed.emb.timestep_embedder.linear_2.weight"),
        plain("time_embed.emb.timestep_embedder.linear_2.bias"),
        linear("time_embed.linear.weight"),
        plain("time_embed.linear.bias"),
        plain("caption_norm.weight"),
        plain("scale_shift_table"),
        linear("proj_out.weight"),
        plain("proj_out.bias"),
    };
    validate_denoiser_weights(w);
    return w;
}

// ---------------------------------------------------------------- validation

void validate_model_block_sequence(const std::vector<SanaBlockWeights> & blocks) {
    if (blocks.empty()) throw std::invalid_argument("model must contain at least one block");
    const size_t hidden = blocks[0].scale_shift_table.dim_size(1);
    for (const SanaBlockWeights & b : blocks) {
        if (b.scale_shift_table.rank() != 2 || b.scale_shift_table.dim_size(0) != 6)
            throw std::invalid_argument("each block scale_shift_table must have shape {6, hidden}");
        if (b.scale_shift_table.dim_size(1) != hidden)
            throw std::invalid_argument("all model blocks must use the same hidden size");
        if (b.q_weight.shape() != std::vector<size_t>{hidden, hidden})
            throw std::invalid_argument("each block q_weight must have shape {hidden, hidden}");
        if (b.cross_out_bias.shape() != std::vector<size_t>{hidden})
            throw std::invalid_argument("each block cross_out_bias must match hidden size");
        if (b.ff_point_weight.rank() != 4 || b.ff_point_weight.dim_size(0) != hidden)
            throw std::invalid_argument("each block ff_point_weight output channels must match hidden size");
    }
}

void validate_denoiser_weights(const SanaDenoiserWeights & w) {
    validate_model_block_sequence(w.blocks);
    const SanaCaptionWeights & cap = w.caption;
    if (cap.linear_1_weight.rank() != 2 || cap.linear_2_weight.rank() != 2 || cap.linear_1_bias.rank() != 1 ||
        cap.linear_2_bias.rank() != 1)
        throw std::invalid_argument("caption weights must use expected linear tensor ranks");
    if (cap.linear_1_weight.dim_size(1) != cap.linear_1_bias.dim_size(0) ||
        cap.linear_2_weight.dim_size(0) != cap.linear_2_bias.dim_size(0))
        throw std::invalid_argument("caption weight dimensions must be internally consistent");
    const size_t hidden = w.blocks[0].scale_shift_table.dim_size(1);
    if (cap.linear_2_weight.dim_size(1) != hidden)
        throw std::invalid_argument("caption output hidden size must match model block hidden size");
    const size_t latent = w.patch_embed_weight.dim_size(1);
    if (w.patch_embed_weight.rank() != 4 || w.patch_embed_weight.dim_size(0) != hidden ||
        w.patch_embed_weight.dim_size(2) != 1 || w.patch_embed_weight.dim_size(3) != 1)
        throw std::invalid_argument("patch_embed_weight must have shape {hidden, latent_channels, 1, 1}");
    check_dims(w.patch_embed_bias.shape(), {hidden}, "patch_embed_bias must match hidden size");
    check_dims(w.time_embed_linear_1_weight.shape(), {256, hidden},
               "time_embed_linear_1_weight must have shape {256, hidden}");
    check_dims(w.time_embed_linear_1_bias.shape(), {hidden}, "time_embed_linear_1_bias must match hidden size");
    check_dims(w.time_embed_linear_2_weight.shape(), {hidden, hidden},
               "time_embed_linear_2_weight must have shape {hidden, hidden}");
    check_dims(w.time_embed_linear_2_bias.shape(), {hidden}, "time_embed_linear_2_bias must match hidden size");
    check_dims(w.time_projection_weight.shape(), {hidden, 6 * hidden},
               "time_projection_weight must have shape {hidden, 6 * hidden}");
    check_dims(w.time_projection_bias.shape(), {6 * hidden}, "time_projection_bias must match 6 * hidden");
    check_dims(w.caption_norm_weight.shape(), {hidden}, "caption_norm_weight must match hidden size");
    check_dims(w.final_scale_shift_table.shape(), {2, hidden}, "final_scale_shift_table must have shape {2, hidden}");
    check_dims(w.proj_out_weight.shape(), {hidden, latent}, "proj_out_weight must have shape {hidden, latent_channels}");
    check_dims(w.proj_out_bias.shape(), {latent}, "proj_out_bias must match latent channel count");
}

// ---------------------------------------------------------------- compute

SanaBlockModulation compute_sana_block_modulation(const Tensor & timestep, const Tensor & table) {
    if (timestep.rank() != 2) throw std::invalid_argument("timestep must be rank 2");
    if (table.rank() != 2) throw std::invalid_argument("scale_shift_table must be rank 2");
    if (table.dim_size(0) != 6) throw std::invalid_argument("scale_shift_table must have shape {6, hidden}");
    const size_t B = timestep.dim_size(0), C = table.dim_size(1);
    if (timestep.dim_size(1) != 6 * C) throw std::invalid_argument("timestep width must equal 6 * hidden");
    Tensor combined({B, 6, C});
    for (size_t b = 0; b < B; ++b)
        for (size_t i = 0; i < 6 * C; ++i)
            combined.data()[b * 6 * C + i] = timestep.data()[b * 6 * C + i] + table.data()[i];
    auto parts = combined.split_six_way_3d();
    return {std::get<0>(parts), std::get<1>(parts), std::get<2>(parts),
            std::get<3>(parts), std::get<4>(parts), std::get<5>(parts)};
}

namespace {
void drop_device_models(const void * key) {
    std::lock_guard<std::mutex> lock(g_mutex);
    for (auto it = g_models.begin(); it != g_models.end();)
        it = (!key || it->first.second == key) ? g_models.erase(it) : std::next(it);
}
}  // namespace

void invalidate_device_weights(const SanaDenoiserWeights & weights) { drop_device_models(&weights); }
void invalidate_device_weights(const SanaBlockWeights & weights) { drop_device_models(&weights); }
void invalidate_all_device_weights() { drop_device_models(nullptr); }

SanaBlockStageOutputs block_forward(const Tensor & input, const Tensor & context, const Tensor & timestep,
                                    const SanaBlockWeights & weights, const Tensor * bias) {
    if (timestep.rank() != 2) throw std::invalid_argument("timestep must be rank 2");
    const size_t hidden = block_hidden(weights);
    check_block_inputs(input, context, timestep, hidden, bias);
    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceModel & m = device_model(1, &weights, &weights, 1, nullptr, false);
    set_conditioning(m, context, 1, bias);
    SanaBlockStageOutputs out{Tensor(input.shape()), Tensor(input.shape()), Tensor(input.shape())};
    ck(sana_dit_block_forward(m.ctx, 0, input.data().data(), timestep.data().data(),
                              static_cast<int64_t>(input.dim_size(0)), static_cast<int64_t>(input.dim_size(1)),
                              out.after_self.data().data(), out.after_cross.data().data(),
                              out.after_ff.data().data()));
    return out;
}

Tensor run_model_blocks(const Tensor & input, const Tensor & context, const Tensor & timestep,
                        const SanaDenoiserWeights & weights, size_t begin, size_t end, const Tensor * bias) {
    if (begin > end || end > weights.blocks.size()) throw std::invalid_argument("invalid model block range");
    if (begin == end) return input;
    const size_t hidden = block_hidden(weights.blocks[0]);
    check_block_inputs(input, context, timestep, hidden, bias);
    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceModel & m = device_model(0, &weights, weights.blocks.data(), weights.blocks.size(), &weights, false);
    set_conditioning(m, context, 1, bias);
    Tensor out(input.shape());
    ck(sana_dit_run_blocks(m.ctx, static_cast<int64_t>(begin), static_cast<int64_t>(end), input.data().data(),
                           timestep.data().data(), static_cast<int64_t>(input.dim_size(0)),
                           static_cast<int64_t>(input.dim_size(1)), out.data().data()));
    return out;
}

Tensor apply_classifier_free_guidance(const Tensor & noise_pred, float guidance_scale) {
    if (noise_pred.rank() != 4) throw std::invalid_argument("noise_pred must be rank 4");
    if (noise_pred.dim_size(0) % 2 != 0)
        throw std::invalid_argument("noise_pred batch size must be even for classifier-free guidance");
    const std::vector<size_t> & s = noise_pred.shape();
    Tensor out({s[0] / 2, s[1], s[2], s[3]});
    const size_t n = out.numel();
    const float * uncond = noise_pred.data().data();
    const float * text = uncond + n;
    for (size_t i = 0; i < n; ++i) out.data()[i] = uncond[i] + guidance_scale * (text[i] - uncond[i]);
    return out;
}

namespace {

void check_latents(const Tensor & latents, size_t latent_channels) {
    if (latents.rank() != 4) throw std::invalid_argument("repeat_batch_4d_local expects a rank-4 tensor");
    if (latents.dim_size(1) != latent_channels)
        throw std::invalid_argument("latent channels must match patch_embed_weight input channels");
    square_side(latents.dim_size(2) * latents.dim_size(3));
}

// Forward of one CFG step on the device (conditioning already set): noise_pred [2B, Cl, H, W].
Tensor device_noise_pred(DeviceModel & m, const Tensor & latents, float t) {
    const std::vector<size_t> & s = latents.shape();
    Tensor np({2 * s[0], s[1], s[2], s[3]});
    ck(sana_dit_forward(m.ctx, latents.data().data(), static_cast<int64_t>(s[0]), static_cast<int64_t>(s[2]),
                        static_cast<int64_t>(s[3]), t, np.data().data()));
    return np;
}

}  // namespace

Tensor run_full_denoising_step_with_cfg(const Tensor & latents, const Tensor & context, float guidance_scale,
                                        SanaSchedulerState & state, const SanaSchedulerConfig & config,
                                        const SanaDenoiserWeights & weights, const Tensor * bias) {
    if (state.step_index >= state.schedule.timesteps.size())
        throw std::invalid_argument("scheduler step_index is out of range");
    if (context.rank() != 3) throw std::invalid_argument("context must be rank 3");
    if (latents.rank() != 4) throw std::invalid_argument("repeat_batch_4d_local expects a rank-4 tensor");
    if (context.dim_size(0) != latents.dim_size(0) * 2)
        throw std::invalid_argument("context batch size must equal 2 * latent batch size for CFG");
    if (bias && bias->dim_size(0) != latents.dim_size(0) * 2)
        throw std::invalid_argument("encoder_attention_bias batch size must equal 2 * latent batch size for CFG");
    validate_denoiser_weights(weights);
    const size_t hidden = weights.blocks[0].scale_shift_table.dim_size(1);
    check_latents(latents, weights.patch_embed_weight.dim_size(1));
    if (context.dim_size(2) != hidden)
        throw std::invalid_argument("context hidden size must match the cross-attention key/value weights");
    check_bias(bias, context.dim_size(0), context.dim_size(1));
    Tensor noise_pred({1});
    {
        std::lock_guard<std::mutex> lock(g_mutex);
        DeviceModel & m = device_model(0, &weights, weights.blocks.data(), weights.blocks.size(), &weights, true);
        set_conditioning(m, context, 1, bias);
        noise_pred = device_noise_pred(m, latents, state.schedule.timesteps[state.step_index]);
    }
    return step_sana_scheduler(apply_classifier_free_guidance(noise_pred, guidance_scale), latents, state, config);
}

Tensor run_full_denoising_loop_with_cfg(const Tensor & initial_latents, const Tensor & encoder_hidden_states,
                                        float guidance_scale, SanaSchedulerState & state,
                                        const SanaSchedulerConfig & config, const SanaDenoiserWeights & weights,
                                        const Tensor * bias) {
    validate_denoiser_weights(weights);
    if (encoder_hidden_states.rank() != 3) throw std::invalid_argument("input must be rank 3");
    if (encoder_hidden_states.dim_size(2) != weights.caption.linear_1_weight.dim_size(0))
        throw std::invalid_argument("caption feature width must match caption linear_1 input size");
    const size_t steps = state.schedule.timesteps.size();
    if (state.step_index >= steps) return initial_latents;
    check_latents(initial_latents, weights.patch_embed_weight.dim_size(1));
    if (encoder_hidden_states.dim_size(0) != initial_latents.dim_size(0) * 2)
        throw std::invalid_argument("context batch size must equal 2 * latent batch size for CFG");
    if (bias && bias->dim_size(0) != initial_latents.dim_size(0) * 2)
        throw std::invalid_argument("encoder_attention_bias batch size must equal 2 * latent batch size for CFG");
    check_bias(bias, encoder_hidden_states.dim_size(0), encoder_hidden_states.dim_size(1));

    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceModel & m = device_model(0, &weights, weights.blocks.data(), weights.blocks.size(), &weights, true);
    set_conditioning(m, encoder_hidden_states, 0, bias);  // caption projection runs on the device

    const std::vector<float> & ts = state.schedule.timesteps;
    const std::vector<float> & sg = state.schedule.sigmas;
    const bool fused = default_solver(config) && state.step_index == 0 && state.lower_order_step_count == 0 &&
                       state.previous_model_outputs.empty() && sg.size() == steps + 1;
    if (fused) {
        // Whole loop on the device: forward, CFG and the DPM-Solver++ update per step.
        const std::vector<size_t> & s = initial_latents.shape();
        Tensor out(s);
        ck(sana_dit_denoise_loop(m.ctx, initial_latents.data().data(), static_cast<int64_t>(s[0]),
                                 static_cast<int64_t>(s[2]), static_cast<int64_t>(s[3]), ts.data(), sg.data(),
                                 static_cast<int64_t>(steps), guidance_scale, out.data().data()));
        // Leave the scheduler state where the per-step path would
        // (src/scheduler.cpp:286-317): all steps taken, the last two converted outputs kept.
        Tensor x0_prev(s), x0_last(s);
        ck(sana_dit_loop_model_outputs(m.ctx, x0_prev.data().data(), x0_last.data().data()));
        state.previous_model_outputs.clear();
        if (steps >= 2) state.previous_model_outputs.push_back(x0_prev);
        state.previous_model_outputs.push_back(x0_last);
        state.lower_order_step_count = std::min<size_t>(steps, config.solver_order);
        state.step_index = steps;
        return out;
    }
    Tensor latents = initial_latents;
    while (state.step_index < steps) {
        Tensor np = device_noise_pred(m, latents, ts[state.step_index]);
        latents = step_sana_scheduler(apply_classifier_free_guidance(np, guidance_scale), latents, state, config);
    }
    return latents;
}
