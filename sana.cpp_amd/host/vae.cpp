// Drop-in DC-AE VAE decoder API on the HIP gfx950 path.
//
// Host side: the loaders and validators keep the reference's checks, messages
// and exception types (src/vae.cpp:10-209).  Device side: run_vae_decode and
// run_vae_decoder_input upload the decoder once into a sana_vae context
// (sana_dit.h) and run there.  Contexts are cached per decoder weights object
// (its address plus a fingerprint of every tensor's storage address, shape and
// sampled values, and the scaling factor); at most kMaxVaes stay resident,
// least recently used first out.  Calls are serialised by one mutex.
//
// Limits of the device path (std::invalid_argument when exceeded): at most 8
// up blocks, every block but the innermost starts with an upsample conv, each
// block holds three layers, channel counts are multiples of 64 up to 1024,
// attention head dim 32, at most 64 latent channels.
#include "vae.h"

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <stdexcept>
#include <utility>

#include "../../include/sana_dit.h"
#include "fingerprint.h"

namespace {

[[noreturn]] void raise_abi(int rc) {
    const std::string msg = sana_dit_last_error();
    if (rc == SANA_ERR_INVALID_ARGUMENT || rc == SANA_ERR_SHAPE) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

void ck(int rc) {
    if (rc != SANA_OK) raise_abi(rc);
}

using Index = std::unordered_map<std::string, SavedWeightInfo>;

// [out, in] linear weight as an [out, in, 1, 1] conv weight
// (linear_weight_to_conv1x1, src/vae_ops.cpp:592-599).
Tensor as_conv1x1(const Tensor & w) {
    if (w.rank() != 2) throw std::invalid_argument("linear_weight_to_conv1x1 expects rank-2 weight");
    Tensor out({w.dim_size(0), w.dim_size(1), 1, 1});
    out.data() = w.data();
    return out;
}

// ---------------------------------------------------------------- loaders (src/vae.cpp:10-118)

SanaVaeResBlockWeights load_res_block(const std::string & dir, const Index & index, const std::string & p) {
    auto get = [&](const char * s) { return load_weight_tensor(dir, index, p + s); };
    return SanaVaeResBlockWeights{get(".conv1.weight"), get(".conv1.bias"), get(".conv2.weight"), get(".norm.weight"),
                                  get(".norm.bias")};
}

SanaVaeAttnGlumbLayerWeights load_attn_glumb_layer(const std::string & dir, const Index & index,
                                                   const std::string & p) {
    auto get = [&](const char * s) { return load_weight_tensor(dir, index, p + s); };
    SanaVaeAttentionWeights a{as_conv1x1(get(".attn.to_q.weight")),
                              as_conv1x1(get(".attn.to_k.weight")),
                              as_conv1x1(get(".attn.to_v.weight")),
                              get(".attn.to_qkv_multiscale.0.proj_in.weight"),
                              get(".attn.to_qkv_multiscale.0.proj_out.weight"),
                              as_conv1x1(get(".attn.to_out.weight")),
                              get(".attn.norm_out.weight"),
                              get(".attn.norm_out.bias")};
    SanaVaeGlumbConvWeights g{get(".conv_out.conv_inverted.weight"), get(".conv_out.conv_inverted.bias"),
                              get(".conv_out.conv_depth.weight"),    get(".conv_out.conv_depth.bias"),
                              get(".conv_out.conv_point.weight"),    get(".conv_out.norm.weight"),
                              get(".conv_out.norm.bias")};
    return SanaVaeAttnGlumbLayerWeights{std::move(a), std::move(g)};
}

// An up block starts with an upsample conv when "<prefix>.0.conv.weight" is
// indexed; its layers are ResBlocks when the first layer after the upsample
// has conv1 (a block without upsample is always attention + GLUMBConv).
SanaVaeUpBlockWeights load_up_block(const std::string & dir, const Index & index, const std::string & prefix) {
    SanaVaeUpBlockWeights ub;
    const bool up = index.count(prefix + ".0.conv.weight") != 0;
    const size_t base = up ? 1 : 0;
    if (up) {
        ub.upsample_conv_weight = load_weight_tensor(dir, index, prefix + ".0.conv.weight");
        ub.upsample_conv_bias = load_weight_tensor(dir, index, prefix + ".0.conv.bias");
        ub.is_res_block = index.count(prefix + "." + std::to_string(base) + ".conv1.weight") != 0;
    }
    for (size_t l = base; l < base + 3; ++l) {
        const std::string p = prefix + "." + std::to_string(l);
        if (ub.is_res_block)
            ub.res_blocks.push_back(load_res_block(dir, index, p));
        else
            ub.attn_glumb_layers.push_back(load_attn_glumb_layer(dir, index, p));
    }
    return ub;
}

// ---------------------------------------------------------------- device contexts

struct DeviceVae {
    sana_vae * ctx = nullptr;
    uint64_t fp = 0;
    float scaling = 0.0f;
    uint64_t last_use = 0;

    DeviceVae() = default;
    DeviceVae(const DeviceVae &) = delete;
    DeviceVae & operator=(const DeviceVae &) = delete;
    ~DeviceVae() {
        if (ctx) sana_vae_destroy(ctx);
    }
};

constexpr size_t kMaxVaes = 2;
std::mutex g_mutex;
std::map<const void *, std::unique_ptr<DeviceVae>> g_vaes;
uint64_t g_clock = 0;

int hip_device() {
    const char * e = std::getenv("SANA_HIP_DEVICE");
    return e ? std::atoi(e) : 0;
}

uint64_t decoder_fingerprint(const SanaVaeDecoderWeights & d) {
    uint64_t h = sana_fp::kSeed;
    for (const Tensor * t : {&d.conv_in_weight, &d.conv_in_bias, &d.norm_out_weight, &d.norm_out_bias,
                             &d.conv_out_weight, &d.conv_out_bias})
        sana_fp::tensor(h, *t);
    sana_fp::mix(h, d.up_blocks.size());
    for (const SanaVaeUpBlockWeights & ub : d.up_blocks) {
        sana_fp::mix(h, ub.upsample_conv_weight.has_value());
        if (ub.upsample_conv_weight) sana_fp::tensor(h, *ub.upsample_conv_weight);
        if (ub.upsample_conv_bias) sana_fp::tensor(h, *ub.upsample_conv_bias);
        sana_fp::mix(h, ub.is_res_block);
        for (const SanaVaeResBlockWeights & r : ub.res_blocks)
            for (const Tensor * t : {&r.conv1_weight, &r.conv1_bias, &r.conv2_weight, &r.norm_weight, &r.norm_bias})
                sana_fp::tensor(h, *t);
        for (const SanaVaeAttnGlumbLayerWeights & l : ub.attn_glumb_layers) {
            const SanaVaeAttentionWeights & a = l.attention;
            const SanaVaeGlumbConvWeights & g = l.glumb;
            for (const Tensor * t :
                 {&a.to_q_weight_conv1x1, &a.to_k_weight_conv1x1, &a.to_v_weight_conv1x1, &a.proj_in_weight,
                  &a.proj_out_weight, &a.to_out_weight_conv1x1, &a.norm_out_weight, &a.norm_out_bias,
                  &g.conv_inverted_weight, &g.conv_inverted_bias, &g.conv_depth_weight, &g.conv_depth_bias,
                  &g.conv_point_weight, &g.norm_weight, &g.norm_bias})
                sana_fp::tensor(h, *t);
        }
    }
    return h;
}

size_t dim0(const Tensor & t, const char * what) {
    if (t.rank() < 1) throw std::invalid_argument(std::string("vae ") + what + " must have rank >= 1");
    return t.dim_size(0);
}

// Device config of a decoder (shapes are checked tensor by tensor on upload).
sana_vae_config device_config(const SanaVaeDecoderWeights & d, float scaling) {
    const size_t L = d.up_blocks.size();
    if (L > SANA_VAE_MAX_LEVELS)
        throw std::invalid_argument("vae decoder has more than 8 up blocks, the limit of this device path");
    sana_vae_config cfg{};
    cfg.latent_channels = static_cast<int64_t>(d.conv_in_weight.dim_size(1));
    cfg.levels = static_cast<int64_t>(L);
    cfg.head_dim = 32;
    cfg.expand = 4;
    cfg.scaling_factor = scaling;
    cfg.device = hip_device();
    for (size_t i = 0; i < L; ++i) {
        const SanaVaeUpBlockWeights & ub = d.up_blocks[i];
        if (ub.upsample_conv_weight.has_value() != (i + 1 < L) || ub.upsample_conv_bias.has_value() != (i + 1 < L))
            throw std::invalid_argument(
                "on this device path every vae up block but the innermost must start with an upsample conv");
        if (ub.is_res_block) {
            if (ub.res_blocks.size() != 3 || !ub.attn_glumb_layers.empty())
                throw std::invalid_argument("vae res up blocks must hold 3 res blocks on this device path");
            cfg.channels[i] = static_cast<int64_t>(dim0(ub.res_blocks[0].conv1_weight, "conv1.weight"));
        } else {
            if (ub.attn_glumb_layers.size() != 3 || !ub.res_blocks.empty())
                throw std::invalid_argument("vae attention up blocks must hold 3 layers on this device path");
            const size_t C = dim0(ub.attn_glumb_layers[0].attention.to_q_weight_conv1x1, "to_q weight");
            cfg.channels[i] = static_cast<int64_t>(C);
            const size_t inv = dim0(ub.attn_glumb_layers[0].glumb.conv_inverted_weight, "conv_inverted.weight");
            if (C == 0 || inv % (2 * C) != 0)
                throw std::invalid_argument("vae GLUMBConv conv_inverted channels must be an even multiple of C");
            cfg.expand = static_cast<int64_t>(inv / (2 * C));
        }
        cfg.attention[i] = ub.is_res_block ? 0 : 1;
    }
    return cfg;
}

void put(sana_vae * v, const std::string & name, const Tensor & t, size_t keep_dims = 0) {
    std::vector<int64_t> s;
    for (size_t d : t.shape()) s.push_back(static_cast<int64_t>(d));
    if (keep_dims) {  // [out, in, 1, 1] conv form of an attention linear -> [out, in]
        if (s.size() != 4 || s[2] != 1 || s[3] != 1)
            throw std::invalid_argument("vae attention 1x1 weight " + name + " must have shape [out, in, 1, 1]");
        s.resize(keep_dims);
    }
    ck(sana_vae_set_weight(v, name.c_str(), t.data().data(), s.data(), static_cast<int>(s.size())));
}

void upload(sana_vae * v, const SanaVaeDecoderWeights & d) {
    put(v, "decoder.conv_in.weight", d.conv_in_weight);
    put(v, "decoder.conv_in.bias", d.conv_in_bias);
    put(v, "decoder.norm_out.weight", d.norm_out_weight);
    put(v, "decoder.norm_out.bias", d.norm_out_bias);
    put(v, "decoder.conv_out.weight", d.conv_out_weight);
    put(v, "decoder.conv_out.bias", d.conv_out_bias);
    for (size_t i = 0; i < d.up_blocks.size(); ++i) {
        const SanaVaeUpBlockWeights & ub = d.up_blocks[i];
        const std::string p = "decoder.up_blocks." + std::to_string(i) + ".";
        size_t base = 0;
        if (ub.upsample_conv_weight) {
            put(v, p + "0.conv.weight", *ub.upsample_conv_weight);
            put(v, p + "0.conv.bias", *ub.upsample_conv_bias);
            base = 1;
        }
        for (size_t k = 0; k < 3; ++k) {
            const std::string q = p + std::to_string(base + k) + ".";
            if (ub.is_res_block) {
                const SanaVaeResBlockWeights & r = ub.res_blocks[k];
                put(v, q + "conv1.weight", r.conv1_weight);
                put(v, q + "conv1.bias", r.conv1_bias);
                put(v, q + "conv2.weight", r.conv2_weight);
                put(v, q + "norm.weight", r.norm_weight);
                put(v, q + "norm.bias", r.norm_bias);
            } else {
                const SanaVaeAttentionWeights & a = ub.attn_glumb_layers[k].attention;
                const SanaVaeGlumbConvWeights & g = ub.attn_glumb_layers[k].glumb;
                put(v, q + "attn.to_q.weight", a.to_q_weight_conv1x1, 2);
                put(v, q + "attn.to_k.weight", a.to_k_weight_conv1x1, 2);
                put(v, q + "attn.to_v.weight", a.to_v_weight_conv1x1, 2);
                put(v, q + "attn.to_qkv_multiscale.0.proj_in.weight", a.proj_in_weight);
                put(v, q + "attn.to_qkv_multiscale.0.proj_out.weight", a.proj_out_weight);
                put(v, q + "attn.to_out.weight", a.to_out_weight_conv1x1, 2);
                put(v, q + "attn.norm_out.weight", a.norm_out_weight);
                put(v, q + "attn.norm_out.bias", a.norm_out_bias);
                put(v, q + "conv_out.conv_inverted.weight", g.conv_inverted_weight);
                put(v, q + "conv_out.conv_inverted.bias", g.conv_inverted_bias);
                put(v, q + "conv_out.conv_depth.weight", g.conv_depth_weight);
                put(v, q + "conv_out.conv_depth.bias", g.conv_depth_bias);
                put(v, q + "conv_out.conv_point.weight", g.conv_point_weight);
                put(v, q + "conv_out.norm.weight", g.norm_weight);
                put(v, q + "conv_out.norm.bias", g.norm_bias);
            }
        }
    }
    ck(sana_vae_check_weights(v));
}

// The context of decoder `d`, created or re-uploaded as its fingerprint and
// scaling factor require.
DeviceVae & device_vae(const SanaVaeDecoderWeights & d, float scaling) {
    const uint64_t fp = decoder_fingerprint(d);
    auto & slot = g_vaes[&d];
    if (slot && (slot->fp != fp || slot->scaling != scaling)) slot.reset();
    if (!slot) {
        if (g_vaes.size() > kMaxVaes) {
            auto victim = g_vaes.end();
            for (auto it = g_vaes.begin(); it != g_vaes.end(); ++it)
                if (it->second && (victim == g_vaes.end() || it->second->last_use < victim->second->last_use))
                    victim = it;
            if (victim != g_vaes.end()) g_vaes.erase(victim);
        }
        const sana_vae_config cfg = device_config(d, scaling);
        auto dv = std::make_unique<DeviceVae>();
        ck(sana_vae_create(&cfg, &dv->ctx));
        upload(dv->ctx, d);
        dv->fp = fp;
        dv->scaling = scaling;
        g_vaes[&d] = std::move(dv);
    }
    DeviceVae & v = *g_vaes[&d];
    v.last_use = ++g_clock;
    return v;
}

}  // namespace

std::vector<std::string> find_vae_decoder_up_block_prefixes(const Index & index) {
    const std::string head = "decoder.up_blocks.";
    std::set<std::pair<size_t, std::string>> found;
    for (const auto & kv : index) {
        const std::string & n = kv.first;
        if (n.compare(0, head.size(), head) != 0) continue;
        const size_t dot = n.find('.', head.size());
        if (dot == std::string::npos || dot == head.size()) continue;
        const std::string digits = n.substr(head.size(), dot - head.size());
        if (!std::all_of(digits.begin(), digits.end(), [](char c) { return c >= '0' && c <= '9'; })) continue;
        found.insert({static_cast<size_t>(std::stoull(digits)), head + digits});
    }
    std::vector<std::string> out;
    for (const auto & f : found) out.push_back(f.second);
    return out;
}

SanaVaeWeights load_vae_weights(const std::string & weights_dir, const Index & index, float scaling_factor,
                                size_t spatial_compression_ratio) {
    auto get = [&](const char * n) { return load_weight_tensor(weights_dir, index, n); };
    SanaVaeDecoderWeights d{get("decoder.conv_in.weight"),  get("decoder.conv_in.bias"),
                            get("decoder.norm_out.weight"), get("decoder.norm_out.bias"),
                            get("decoder.conv_out.weight"), get("decoder.conv_out.bias"),
                            {}};
    for (const std::string & p : find_vae_decoder_up_block_prefixes(index))
        d.up_blocks.push_back(load_up_block(weights_dir, index, p));
    return SanaVaeWeights{std::move(d), scaling_factor, spatial_compression_ratio};
}

void validate_vae_decoder_weights(const SanaVaeDecoderWeights & w) {
    auto need = [](bool ok, const char * msg) {
        if (!ok) throw std::invalid_argument(msg);
    };
    need(w.conv_in_weight.rank() == 4, "vae decoder conv_in.weight must be rank 4");
    need(w.conv_in_bias.rank() == 1, "vae decoder conv_in.bias must be rank 1");
    need(w.norm_out_weight.rank() == 1, "vae decoder norm_out.weight must be rank 1");
    need(w.norm_out_bias.rank() == 1, "vae decoder norm_out.bias must be rank 1");
    need(w.conv_out_weight.rank() == 4, "vae decoder conv_out.weight must be rank 4");
    need(w.conv_out_bias.rank() == 1, "vae decoder conv_out.bias must be rank 1");
    need(!w.up_blocks.empty(), "vae decoder must contain at least one up block");
    need(w.conv_in_weight.dim_size(0) == w.conv_in_bias.dim_size(0),
         "vae decoder conv_in bias shape must match output channels");
    need(w.norm_out_weight.dim_size(0) == w.norm_out_bias.dim_size(0), "vae decoder norm_out bias shape must match");
    need(w.conv_out_weight.dim_size(0) == w.conv_out_bias.dim_size(0),
         "vae decoder conv_out bias shape must match output channels");
    need(w.norm_out_weight.dim_size(0) == w.conv_out_weight.dim_size(1),
         "vae decoder norm_out channels must match conv_out input channels");
}

void validate_vae_weights(const SanaVaeWeights & w) {
    validate_vae_decoder_weights(w.decoder);
    if (!(w.scaling_factor > 0.0f)) throw std::invalid_argument("vae scaling_factor must be positive");
    if (w.spatial_compression_ratio == 0) throw std::invalid_argument("vae spatial_compression_ratio must be positive");
}

Tensor run_vae_decoder_input(const Tensor & latents, const SanaVaeDecoderWeights & weights, bool in_shortcut) {
    validate_vae_decoder_weights(weights);
    if (latents.rank() != 4) throw std::invalid_argument("vae decoder input latents must be rank 4");
    if (latents.dim_size(1) != weights.conv_in_weight.dim_size(1))
        throw std::invalid_argument("vae decoder input channels must match conv_in.weight");
    const size_t B = latents.dim_size(0), C = weights.conv_in_weight.dim_size(0), H = latents.dim_size(2),
                 W = latents.dim_size(3);
    if (in_shortcut && C % latents.dim_size(1) != 0)
        throw std::invalid_argument("vae decoder conv_in output channels must be divisible by latent channels");
    Tensor out({B, C, H, W});
    if (out.numel() == 0) return out;
    std::lock_guard<std::mutex> lock(g_mutex);
    auto it = g_vaes.find(&weights);
    const float scaling = it != g_vaes.end() && it->second ? it->second->scaling : 1.0f;  // unused by this stage
    DeviceVae & v = device_vae(weights, scaling);
    ck(sana_vae_decoder_input(v.ctx, latents.data().data(), static_cast<int64_t>(B), static_cast<int64_t>(H),
                              static_cast<int64_t>(W), in_shortcut ? 1 : 0, out.data().data()));
    return out;
}

void invalidate_device_weights(const SanaVaeDecoderWeights & weights) {
    std::lock_guard<std::mutex> lock(g_mutex);
    g_vaes.erase(&weights);
}

void invalidate_device_weights(const SanaVaeWeights & weights) { invalidate_device_weights(weights.decoder); }

Tensor run_vae_decode(const Tensor & latents, const SanaVaeWeights & weights) {
    validate_vae_weights(weights);
    if (latents.rank() != 4) throw std::invalid_argument("vae decode latents must be rank 4");
    if (latents.dim_size(1) != weights.decoder.conv_in_weight.dim_size(1))
        throw std::invalid_argument("vae decode latent channels must match decoder conv_in input");
    const size_t B = latents.dim_size(0), H = latents.dim_size(2), W = latents.dim_size(3);
    const size_t up = size_t(1) << (weights.decoder.up_blocks.size() - 1);
    Tensor out({B, 3, H * up, W * up});
    if (out.numel() == 0) return out;
    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceVae & v = device_vae(weights.decoder, weights.scaling_factor);
    ck(sana_vae_decode(v.ctx, latents.data().data(), static_cast<int64_t>(B), static_cast<int64_t>(H),
                       static_cast<int64_t>(W), out.data().data()));
    return out;
}
