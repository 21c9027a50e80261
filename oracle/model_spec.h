// Synthetic Sana-0.6B weight manifest shared by the oracle, the reference
// harness and the GPU bench/tests.  TEST INFRASTRUCTURE: nothing in the
// product path includes this file.
//
// Names and shapes are the GGUF tensor names and PyTorch-order shapes that the
// reference loader expects (src/transformer.cpp:167-198 caption,
// :214-308 per block, :473-484 denoiser).  Every tensor is filled with
// 0.02 * randn_torch_cpu(shape, seed) where seed = 1000 + (index of the name
// in byte-wise sorted order over all three files).  The one deliberate
// deviation: caption_norm.weight is all ones, so the caption RMSNorm does not
// shrink the context to ~0.02 and trivialise cross-attention.
#pragma once

#include <algorithm>
#include <cstddef>
#include <string>
#include <vector>

namespace sana_spec {

enum WeightFile { kModelFile = 0, kCaptionFile = 1, kDenoiserFile = 2 };

struct Entry {
    std::string name;
    std::vector<size_t> shape;   // PyTorch order (GGUF ne reversed)
    int file;                    // WeightFile
    bool linear;                 // loader transposes it to [in, out]
    bool ones;                   // filled with 1.0 instead of noise
    unsigned long long seed;     // 1000 + sorted index
};

struct Dims {
    size_t layers = 28;
    size_t hidden = 1152;
    size_t ffn = 5760;           // expanded channels of the Mix-FFN (2 x 2880)
    size_t caption = 2304;
    size_t latent = 32;
    size_t time_freq = 256;
};

inline std::vector<Entry> manifest(const Dims & d) {
    std::vector<Entry> e;
    auto add = [&](const std::string & n, std::vector<size_t> s, int f, bool lin, bool ones = false) {
        e.push_back(Entry{n, std::move(s), f, lin, ones, 0});
    };
    const size_t C = d.hidden, E = d.ffn;
    for (size_t i = 0; i < d.layers; ++i) {
        const std::string p = "transformer_blocks." + std::to_string(i) + ".";
        add(p + "scale_shift_table", {6, C}, kModelFile, false);
        add(p + "attn1.to_q.weight", {C, C}, kModelFile, true);
        add(p + "attn1.to_k.weight", {C, C}, kModelFile, true);
        add(p + "attn1.to_v.weight", {C, C}, kModelFile, true);
        add(p + "attn1.to_out.0.weight", {C, C}, kModelFile, true);
        add(p + "attn1.to_out.0.bias", {C}, kModelFile, false);
        add(p + "attn2.to_q.weight", {C, C}, kModelFile, true);
        add(p + "attn2.to_q.bias", {C}, kModelFile, false);
        add(p + "attn2.to_k.weight", {C, C}, kModelFile, true);
        add(p + "attn2.to_k.bias", {C}, kModelFile, false);
        add(p + "attn2.to_v.weight", {C, C}, kModelFile, true);
        add(p + "attn2.to_v.bias", {C}, kModelFile, false);
        add(p + "attn2.to_out.0.weight", {C, C}, kModelFile, true);
        add(p + "attn2.to_out.0.bias", {C}, kModelFile, false);
        add(p + "ff.conv_inverted.weight", {E, C, 1, 1}, kModelFile, false);
        add(p + "ff.conv_inverted.bias", {E}, kModelFile, false);
        add(p + "ff.conv_depth.weight", {E, 1, 3, 3}, kModelFile, false);
        add(p + "ff.conv_depth.bias", {E}, kModelFile, false);
        add(p + "ff.conv_point.weight", {C, E / 2, 1, 1}, kModelFile, false);
    }
    add("caption_projection.linear_1.weight", {C, d.caption}, kCaptionFile, true);
    add("caption_projection.linear_1.bias", {C}, kCaptionFile, false);
    add("caption_projection.linear_2.weight", {C, C}, kCaptionFile, true);
    add("caption_projection.linear_2.bias", {C}, kCaptionFile, false);
    add("patch_embed.proj.weight", {C, d.latent, 1, 1}, kDenoiserFile, false);
    add("patch_embed.proj.bias", {C}, kDenoiserFile, false);
    add("time_embed.emb.timestep_embedder.linear_1.weight", {C, d.time_freq}, kDenoiserFile, true);
    add("time_embed.emb.timestep_embedder.linear_1.bias", {C}, kDenoiserFile, false);
    add("time_embed.emb.timestep_embedder.linear_2.weight", {C, C}, kDenoiserFile, true);
    add("time_embed.emb.timestep_embedder.linear_2.bias", {C}, kDenoiserFile, false);
    add("time_embed.linear.weight", {6 * C, C}, kDenoiserFile, true);
    add("time_embed.linear.bias", {6 * C}, kDenoiserFile, false);
    add("caption_norm.weight", {C}, kDenoiserFile, false, true);
    add("scale_shift_table", {2, C}, kDenoiserFile, false);
    add("proj_out.weight", {d.latent, C}, kDenoiserFile, true);
    add("proj_out.bias", {d.latent}, kDenoiserFile, false);

    std::sort(e.begin(), e.end(), [](const Entry & a, const Entry & b) { return a.name < b.name; });
    for (size_t i = 0; i < e.size(); ++i) {
        e[i].seed = 1000ULL + i;
    }
    return e;
}

inline size_t numel(const std::vector<size_t> & s) {
    size_t n = 1;
    for (size_t v : s) n *= v;
    return n;
}

}  // namespace sana_spec
