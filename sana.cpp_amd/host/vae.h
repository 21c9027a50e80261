// Drop-in DC-AE VAE decoder API: the declarations and weight structs of the
// reference's src/vae.h:11-92, with run_vae_decode / run_vae_decoder_input on
// the HIP gfx950 path (sana_vae_* of include/sana_dit.h).
#pragma once

#include <optional>
#include <string>
#include <unordered_map>
#include <vector>

#include "tensor.h"
#include "weights_io.h"

struct SanaVaeResBlockWeights {
    Tensor conv1_weight;
    Tensor conv1_bias;
    Tensor conv2_weight;
    Tensor norm_weight;
    Tensor norm_bias;
};

struct SanaVaeAttentionWeights {
    Tensor to_q_weight_conv1x1;
    Tensor to_k_weight_conv1x1;
    Tensor to_v_weight_conv1x1;
    Tensor proj_in_weight;
    Tensor proj_out_weight;
    Tensor to_out_weight_conv1x1;
    Tensor norm_out_weight;
    Tensor norm_out_bias;
};

struct SanaVaeGlumbConvWeights {
    Tensor conv_inverted_weight;
    Tensor conv_inverted_bias;
    Tensor conv_depth_weight;
    Tensor conv_depth_bias;
    Tensor conv_point_weight;
    Tensor norm_weight;
    Tensor norm_bias;
};

struct SanaVaeAttnGlumbLayerWeights {
    SanaVaeAttentionWeights attention;
    SanaVaeGlumbConvWeights glumb;
};

// An up block: an optional upsample conv, then three ResBlocks
// (is_res_block) or three attention + GLUMBConv layers.  The innermost block
// (highest index, run first) has no upsample.
struct SanaVaeUpBlockWeights {
    std::optional<Tensor> upsample_conv_weight;
    std::optional<Tensor> upsample_conv_bias;
    bool is_res_block = false;
    std::vector<SanaVaeResBlockWeights> res_blocks;
    std::vector<SanaVaeAttnGlumbLayerWeights> attn_glumb_layers;
};

struct SanaVaeDecoderWeights {
    Tensor conv_in_weight;
    Tensor conv_in_bias;
    Tensor norm_out_weight;
    Tensor norm_out_bias;
    Tensor conv_out_weight;
    Tensor conv_out_bias;
    std::vector<SanaVaeUpBlockWeights> up_blocks;
};

struct SanaVaeWeights {
    SanaVaeDecoderWeights decoder;
    float scaling_factor = 1.0f;
    size_t spatial_compression_ratio = 32;
};

// "decoder.up_blocks.<i>" prefixes present in the index, by ascending i.
std::vector<std::string> find_vae_decoder_up_block_prefixes(
    const std::unordered_map<std::string, SavedWeightInfo> & index);
SanaVaeWeights load_vae_weights(const std::string & weights_dir,
                                const std::unordered_map<std::string, SavedWeightInfo> & index,
                                float scaling_factor, size_t spatial_compression_ratio);
void validate_vae_decoder_weights(const SanaVaeDecoderWeights & weights);
void validate_vae_weights(const SanaVaeWeights & weights);
// conv_in of latents [B, Cl, H, W] (+ the channel-repeat shortcut) -> [B, C_top, H, W].
Tensor run_vae_decoder_input(const Tensor & latents, const SanaVaeDecoderWeights & weights, bool in_shortcut = true);
// latents [B, Cl, H, W] -> image [B, 3, H * 2^(blocks-1), W * 2^(blocks-1)].
Tensor run_vae_decode(const Tensor & latents, const SanaVaeWeights & weights);

// Device residency of the drop-in (no counterpart in the reference): a
// decoder's weights are uploaded on first use and reused while its address and
// fingerprint (tensor storage addresses, shapes, all values up to 4096 else 65
// spread samples) are unchanged.  After an in-place edit of tensor values,
// call invalidate_device_weights so the next decode uploads them again.
void invalidate_device_weights(const SanaVaeWeights & weights);
void invalidate_device_weights(const SanaVaeDecoderWeights & weights);
