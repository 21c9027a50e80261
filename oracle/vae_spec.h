// Synthetic DC-AE decoder (the VAE after the denoising loop) weight manifest
// shared by the oracle, the reference harness and the GPU tests.  TEST
// INFRASTRUCTURE: nothing in the product path includes this file.
//
// Names and shapes are the GGUF tensor names and PyTorch-order shapes that the
// reference loader reads (src/vae.cpp:10-118, :155-167): conv_in / norm_out /
// conv_out, then per up block `decoder.up_blocks.{i}` an optional upsample conv
// (`.0.conv`) and exactly three layers, either ResBlocks (`conv1`, `conv2`,
// `norm`) or EfficientViT layers (`attn.*` multiscale linear attention and
// `conv_out.*` GLUMBConv).  The innermost (highest) block has no upsample.
//
// Values: randn_torch_cpu(shape, seed) with seed = 7000 + (index of the name in
// byte-wise sorted order), scaled by 0.02 -- except RMSNorm weights, which are
// 1 + 0.1 * randn so the norms neither vanish nor ignore their weight.  A
// tensor of fewer than 16 values (conv_out.bias) takes the first values of a
// 16-value draw, since the generator needs at least 16.
//
// Configs: "full" is the DC-AE f32c32 decoder of Sana 1.0 (latent 32 channels,
// levels 128/256/512/512/1024/1024, ResBlock x3 at the three outer levels,
// EfficientViT x3 at the three inner ones, head dim 32, GLUMBConv expansion 4,
// 5x5 multiscale kernel).  "small" keeps every op with 4 levels of 64/64/128/128.
#pragma once

#include <algorithm>
#include <cstddef>
#include <string>
#include <vector>

namespace vae_spec {

struct Entry {
    std::string name;
    std::vector<size_t> shape;   // PyTorch order
    bool norm;                   // RMSNorm weight: 1 + 0.1 randn
    unsigned long long seed;     // 7000 + sorted index
};

struct Config {
    size_t latent = 32;
    std::vector<size_t> channels;   // per level, level 0 = output resolution
    std::vector<bool> attn;         // per level: EfficientViT layers (else ResBlocks)
    size_t head_dim = 32;
    size_t expand = 4;              // GLUMBConv hidden = expand * C (inverted conv: 2x that)
};

inline Config full_config() {
    Config c;
    c.channels = {128, 256, 512, 512, 1024, 1024};
    c.attn = {false, false, false, true, true, true};
    return c;
}

inline Config small_config() {
    Config c;
    c.channels = {64, 64, 128, 128};
    c.attn = {false, false, true, true};
    return c;
}

inline std::vector<Entry> manifest(const Config & cfg) {
    std::vector<Entry> e;
    auto add = [&](const std::string & n, std::vector<size_t> s, bool norm = false) {
        e.push_back(Entry{n, std::move(s), norm, 0});
    };
    const size_t L = cfg.channels.size();
    const size_t top = cfg.channels[L - 1], out = cfg.channels[0];
    add("decoder.conv_in.weight", {top, cfg.latent, 3, 3});
    add("decoder.conv_in.bias", {top});
    add("decoder.norm_out.weight", {out}, true);
    add("decoder.norm_out.bias", {out});
    add("decoder.conv_out.weight", {3, out, 3, 3});
    add("decoder.conv_out.bias", {3});
    for (size_t i = 0; i < L; ++i) {
        const std::string p = "decoder.up_blocks." + std::to_string(i) + ".";
        const size_t C = cfg.channels[i];
        size_t base = 0;
        if (i + 1 < L) {
            add(p + "0.conv.weight", {C, cfg.channels[i + 1], 3, 3});
            add(p + "0.conv.bias", {C});
            base = 1;
        }
        for (size_t l = base; l < base + 3; ++l) {
            const std::string q = p + std::to_string(l) + ".";
            if (!cfg.attn[i]) {
                add(q + "conv1.weight", {C, C, 3, 3});
                add(q + "conv1.bias", {C});
                add(q + "conv2.weight", {C, C, 3, 3});
                add(q + "norm.weight", {C}, true);
                add(q + "norm.bias", {C});
            } else {
                const size_t Hd = cfg.expand * C;
                add(q + "attn.to_q.weight", {C, C});
                add(q + "attn.to_k.weight", {C, C});
                add(q + "attn.to_v.weight", {C, C});
                add(q + "attn.to_qkv_multiscale.0.proj_in.weight", {3 * C, 1, 5, 5});
                add(q + "attn.to_qkv_multiscale.0.proj_out.weight", {3 * C, cfg.head_dim, 1, 1});
                add(q + "attn.to_out.weight", {C, 2 * C});
                add(q + "attn.norm_out.weight", {C}, true);
                add(q + "attn.norm_out.bias", {C});
                add(q + "conv_out.conv_inverted.weight", {2 * Hd, C, 1, 1});
                add(q + "conv_out.conv_inverted.bias", {2 * Hd});
                add(q + "conv_out.conv_depth.weight", {2 * Hd, 1, 3, 3});
                add(q + "conv_out.conv_depth.bias", {2 * Hd});
                add(q + "conv_out.conv_point.weight", {C, Hd, 1, 1});
                add(q + "conv_out.norm.weight", {C}, true);
                add(q + "conv_out.norm.bias", {C});
            }
        }
    }
    std::sort(e.begin(), e.end(), [](const Entry & a, const Entry & b) { return a.name < b.name; });
    for (size_t i = 0; i < e.size(); ++i) e[i].seed = 7000ULL + i;
    return e;
}

inline size_t numel(const std::vector<size_t> & s) {
    size_t n = 1;
    for (size_t v : s) n *= v;
    return n;
}

}  // namespace vae_spec
