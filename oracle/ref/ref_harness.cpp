// Driver around the REFERENCE's own CPU code (compiled from /root/reference/src
// by oracle/ref/Makefile into oracle/_ref/).  TEST INFRASTRUCTURE ONLY: it
// produces the golden vectors the oracle restatement and the HIP path are
// checked against, and it is the "reference" CPU baseline that bench.py times.
//
// It calls only exported reference functions (transformer.h, transformer_ops.h,
// common_ops.h, tensor.h, scheduler.h, torch_rng.h).  Three helpers that the
// reference keeps in an anonymous namespace are restated here so the forward
// can be stopped at the velocity (noise_pred) instead of the scheduler step:
//   repeat_batch            <- src/transformer.cpp:55-75
//   timestep_embedding      <- src/transformer.cpp:77-122 (#else branch)
//   final modulation        <- src/transformer.cpp:126-163 (#else branch)
// The "forward --check-step" mode proves the restatement bit-exact by running
// the reference's own run_full_denoising_step_with_cfg beside it.
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>
#include <algorithm>

#include "common_ops.h"
#include "scheduler.h"
#include "tensor.h"
#include "torch_rng.h"
#include "transformer.h"
#include "transformer_ops.h"
#include "vae.h"
#include "vae_ops.h"

#include "../model_spec.h"
#include "../vae_spec.h"

namespace {

using sana_spec::Entry;

struct Gen {
    std::unordered_map<std::string, Entry> by_name;
    explicit Gen(const sana_spec::Dims & d) {
        for (const Entry & e : sana_spec::manifest(d)) by_name[e.name] = e;
    }
    // Weight as stored in the GGUF (PyTorch order).
    Tensor raw(const std::string & name) const {
        auto it = by_name.find(name);
        if (it == by_name.end()) throw std::runtime_error("no such weight " + name);
        const Entry & e = it->second;
        if (e.ones) {
            Tensor t(e.shape);
            t.fill(1.0f);
            return t;
        }
        Tensor t = randn_torch_cpu(e.shape, e.seed);
        t.mul_inplace_scalar(0.02f);
        return t;
    }
    // Weight as the reference loader hands it to the model (linear -> [in,out]).
    Tensor loaded(const std::string & name) const {
        Tensor t = raw(name);
        if (by_name.at(name).linear) return t.transpose_2d();
        return t;
    }
};

Tensor filled(std::vector<size_t> shape, float v) {
    Tensor t(std::move(shape));
    t.fill(v);
    return t;
}

SanaBlockWeights make_block(const Gen & g, size_t i, size_t C, size_t self_heads, size_t cross_heads) {
    const std::string p = "transformer_blocks." + std::to_string(i) + ".";
    // Field order and injected tensors follow load_block_weights
    // (src/transformer.cpp:361-398): zero q/k/v bias, LN gamma=1 beta=0.
    return SanaBlockWeights{
        g.loaded(p + "scale_shift_table"),
        filled({C}, 1.0f), filled({C}, 0.0f),
        g.loaded(p + "attn1.to_q.weight"), filled({C}, 0.0f),
        g.loaded(p + "attn1.to_k.weight"), filled({C}, 0.0f),
        g.loaded(p + "attn1.to_v.weight"), filled({C}, 0.0f),
        g.loaded(p + "attn1.to_out.0.weight"), g.loaded(p + "attn1.to_out.0.bias"),
        g.loaded(p + "attn2.to_q.weight"), g.loaded(p + "attn2.to_q.bias"),
        g.loaded(p + "attn2.to_k.weight"), g.loaded(p + "attn2.to_k.bias"),
        g.loaded(p + "attn2.to_v.weight"), g.loaded(p + "attn2.to_v.bias"),
        g.loaded(p + "attn2.to_out.0.weight"), g.loaded(p + "attn2.to_out.0.bias"),
        filled({C}, 1.0f), filled({C}, 0.0f),
        g.loaded(p + "ff.conv_inverted.weight"), g.loaded(p + "ff.conv_inverted.bias"),
        g.loaded(p + "ff.conv_depth.weight"), g.loaded(p + "ff.conv_depth.bias"),
        g.loaded(p + "ff.conv_point.weight"),
        self_heads, cross_heads,
    };
}

SanaDenoiserWeights make_denoiser(const Gen & g, const sana_spec::Dims & d, size_t layers,
                                  size_t self_heads, size_t cross_heads) {
    std::vector<SanaBlockWeights> blocks;
    for (size_t i = 0; i < layers; ++i) blocks.push_back(make_block(g, i, d.hidden, self_heads, cross_heads));
    SanaCaptionWeights cap{
        g.loaded("caption_projection.linear_1.weight"), g.loaded("caption_projection.linear_1.bias"),
        g.loaded("caption_projection.linear_2.weight"), g.loaded("caption_projection.linear_2.bias"),
    };
    SanaDenoiserWeights w{
        cap, blocks,
        g.loaded("patch_embed.proj.weight"), g.loaded("patch_embed.proj.bias"),
        g.loaded("time_embed.emb.timestep_embedder.linear_1.weight"),
        g.loaded("time_embed.emb.timestep_embedder.linear_1.bias"),
        g.loaded("time_embed.emb.timestep_embedder.linear_2.weight"),
        g.loaded("time_embed.emb.timestep_embedder.linear_2.bias"),
        g.loaded("time_embed.linear.weight"), g.loaded("time_embed.linear.bias"),
        g.loaded("caption_norm.weight"), g.loaded("scale_shift_table"),
        g.loaded("proj_out.weight"), g.loaded("proj_out.bias"),
    };
    return w;
}

// Seeded DC-AE decoder weights as load_vae_weights (src/vae.cpp:140-167)
// would hand them over: linear attention weights reshaped to 1x1 convs by the
// reference's own linear_weight_to_conv1x1, everything else as stored.
struct VaeGen {
    std::unordered_map<std::string, vae_spec::Entry> by_name;
    explicit VaeGen(const vae_spec::Config & c) {
        for (const vae_spec::Entry & e : vae_spec::manifest(c)) by_name[e.name] = e;
    }
    Tensor operator()(const std::string & name) const {
        auto it = by_name.find(name);
        if (it == by_name.end()) throw std::runtime_error("no such vae weight " + name);
        const vae_spec::Entry & e = it->second;
        Tensor t(e.shape);
        const size_t n = t.numel();
        // randn_torch_cpu needs >= 16 values: smaller tensors take the head of a 16-value draw
        const Tensor r = randn_torch_cpu({std::max<size_t>(n, 16)}, e.seed);
        for (size_t i = 0; i < n; ++i) {
            const float v = r.data()[i];
            t.data()[i] = e.norm ? 1.0f + 0.1f * v : 0.02f * v;
        }
        return t;
    }
};

SanaVaeWeights make_vae(const vae_spec::Config & c) {
    VaeGen g(c);
    SanaVaeDecoderWeights dec{
        g("decoder.conv_in.weight"), g("decoder.conv_in.bias"), g("decoder.norm_out.weight"),
        g("decoder.norm_out.bias"), g("decoder.conv_out.weight"), g("decoder.conv_out.bias"), {}};
    const size_t L = c.channels.size();
    for (size_t i = 0; i < L; ++i) {
        const std::string p = "decoder.up_blocks." + std::to_string(i) + ".";
        SanaVaeUpBlockWeights ub;
        size_t base = 0;
        if (i + 1 < L) {
            ub.upsample_conv_weight = g(p + "0.conv.weight");
            ub.upsample_conv_bias = g(p + "0.conv.bias");
            ub.is_res_block = !c.attn[i];
            base = 1;
        }
        for (size_t l = base; l < base + 3; ++l) {
            const std::string q = p + std::to_string(l) + ".";
            if (ub.is_res_block) {
                ub.res_blocks.push_back(SanaVaeResBlockWeights{g(q + "conv1.weight"), g(q + "conv1.bias"),
                                                               g(q + "conv2.weight"), g(q + "norm.weight"),
                                                               g(q + "norm.bias")});
            } else {
                SanaVaeAttentionWeights a{
                    linear_weight_to_conv1x1(g(q + "attn.to_q.weight")),
                    linear_weight_to_conv1x1(g(q + "attn.to_k.weight")),
                    linear_weight_to_conv1x1(g(q + "attn.to_v.weight")),
                    g(q + "attn.to_qkv_multiscale.0.proj_in.weight"),
                    g(q + "attn.to_qkv_multiscale.0.proj_out.weight"),
                    linear_weight_to_conv1x1(g(q + "attn.to_out.weight")),
                    g(q + "attn.norm_out.weight"), g(q + "attn.norm_out.bias")};
                SanaVaeGlumbConvWeights m{
                    g(q + "conv_out.conv_inverted.weight"), g(q + "conv_out.conv_inverted.bias"),
                    g(q + "conv_out.conv_depth.weight"), g(q + "conv_out.conv_depth.bias"),
                    g(q + "conv_out.conv_point.weight"), g(q + "conv_out.norm.weight"),
                    g(q + "conv_out.norm.bias")};
                ub.attn_glumb_layers.push_back(SanaVaeAttnGlumbLayerWeights{a, m});
            }
        }
        dec.up_blocks.push_back(std::move(ub));
    }
    return SanaVaeWeights{std::move(dec), 0.41407f, (size_t)1 << (L - 1)};
}

Tensor repeat_batch(const Tensor & x, size_t r) {
    std::vector<size_t> s = x.shape();
    const size_t n = x.numel();
    s[0] *= r;
    Tensor out(s);
    for (size_t i = 0; i < r; ++i) std::copy(x.data().begin(), x.data().end(), out.data().begin() + i * n);
    return out;
}

Tensor timestep_embedding(const Tensor & t, size_t dim) {
    const size_t B = t.dim_size(0), half = dim / 2;
    Tensor out({B, dim});
    std::vector<float> freq(half);
    const float log_scale = -std::log(10000.0f) / static_cast<float>(half);
    for (size_t i = 0; i < half; ++i) freq[i] = std::exp(static_cast<float>(i) * log_scale);
    for (size_t b = 0; b < B; ++b) {
        for (size_t i = 0; i < half; ++i) {
            const float v = t.data()[b] * freq[i];
            out.data()[b * dim + i] = std::cos(v);
            out.data()[b * dim + half + i] = std::sin(v);
        }
    }
    return out;
}

struct TimeOut {
    Tensor embedded;   // pre-SiLU embedded timestep [B, C]
    Tensor t_mod;      // [B, 6C]
};

TimeOut time_mlp(const SanaDenoiserWeights & w, float t, size_t B) {
    Tensor tv({B});
    tv.fill(t);
    Tensor tp = timestep_embedding(tv, 256);
    Tensor e = linear_2d(tp, w.time_embed_linear_1_weight, &w.time_embed_linear_1_bias);
    e.silu_inplace();
    e = linear_2d(e, w.time_embed_linear_2_weight, &w.time_embed_linear_2_bias);
    Tensor h = e;
    h.silu_inplace();
    Tensor m = linear_2d(h, w.time_projection_weight, &w.time_projection_bias);
    return {e, m};
}

Tensor forward_noise_pred(const Tensor & latents, const Tensor & context, float t,
                          const SanaDenoiserWeights & w, const Tensor * bias) {
    Tensor lin = repeat_batch(latents, 2);
    Tensor grid = conv2d_1x1(lin, w.patch_embed_weight, &w.patch_embed_bias);
    Tensor tokens = grid.grid_to_tokens_3d();
    TimeOut to = time_mlp(w, t, lin.dim_size(0));
    Tensor h = run_model_blocks(tokens, context, to.t_mod, w, 0, w.blocks.size(), bias);
    Tensor n = h.layer_norm_3d_lastdim(1e-6f);
    const size_t B = to.embedded.dim_size(0), C = to.embedded.dim_size(1);
    Tensor shift({B, 1, C}), scale({B, 1, C});
    const float * T = w.final_scale_shift_table.data().data();
    for (size_t b = 0; b < B; ++b) {
        for (size_t c = 0; c < C; ++c) {
            shift.data()[b * C + c] = to.embedded.data()[b * C + c] + T[c];
            scale.data()[b * C + c] = to.embedded.data()[b * C + c] + T[C + c];
        }
    }
    Tensor mod = n.modulate_3d_lastdim(shift, scale);
    Tensor proj = linear_3d_lastdim(mod, w.proj_out_weight, &w.proj_out_bias);
    return proj.tokens_to_grid_4d(lin.dim_size(2), lin.dim_size(3));
}

Tensor make_mask_bias(size_t L, size_t uncond_real, size_t cond_real) {
    Tensor b({2, 1, L});
    for (size_t j = 0; j < L; ++j) {
        b.data()[j] = j < uncond_real ? 0.0f : -10000.0f;
        b.data()[L + j] = j < cond_real ? 0.0f : -10000.0f;
    }
    return b;
}

void dump(const std::string & dir, const std::string & name, const Tensor & t) {
    const std::string path = dir + "/" + name + ".f32";
    std::ofstream f(path, std::ios::binary);
    f.write(reinterpret_cast<const char *>(t.data().data()), static_cast<std::streamsize>(t.numel() * 4));
    if (!f) throw std::runtime_error("write failed: " + path);
    std::string shape;
    for (size_t s : t.shape()) shape += (shape.empty() ? "" : ",") + std::to_string(s);
    std::printf("wrote %s shape=[%s]\n", path.c_str(), shape.c_str());
    std::fflush(stdout);
}

double now_ms() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

int usage() {
    std::fprintf(stderr,
        "usage:\n"
        "  ref_harness digest\n"
        "  ref_harness block SELF_HEADS CROSS_HEADS SIDE T OUTDIR\n"
        "  ref_harness forward SELF_HEADS CROSS_HEADS SIDE T MASK CHECK_STEP OUTDIR\n"
        "  ref_harness forward-hw SELF_HEADS CROSS_HEADS H W T OUTDIR\n"
        "  ref_harness loop SELF_HEADS CROSS_HEADS SIDE STEPS GUIDANCE MASK OUTDIR\n"
        "  ref_harness time-block SELF_HEADS CROSS_HEADS BATCH SIDE REPS\n"
        "  ref_harness time-forward SELF_HEADS CROSS_HEADS SIDE\n"
        "  ref_harness time-micro SIDE REPS\n"
        "  ref_harness vae small|full SIDE OUTDIR\n"
        "  ref_harness vae-conv SIDE CIN COUT OUTDIR\n"
        "  ref_harness vae-digest small|full\n");
    return 2;
}

}  // namespace

int main(int argc, char ** argv) {
    if (argc < 2) return usage();
    const std::string mode = argv[1];
    sana_spec::Dims d;
    Gen g(d);
    try {
        if (mode == "digest") {
            // 64-bit FNV-1a of every generated tensor's fp32 bytes, PyTorch order.
            for (const Entry & e : sana_spec::manifest(d)) {
                Tensor t = g.raw(e.name);
                uint64_t h = 14695981039346656037ULL;
                const unsigned char * p = reinterpret_cast<const unsigned char *>(t.data().data());
                for (size_t i = 0; i < t.numel() * 4; ++i) { h ^= p[i]; h *= 1099511628211ULL; }
                std::printf("%s %016llx\n", e.name.c_str(), static_cast<unsigned long long>(h));
            }
            return 0;
        }
        if (mode == "block" && argc == 7) {
            const size_t sh = std::stoul(argv[2]), ch = std::stoul(argv[3]), side = std::stoul(argv[4]);
            const float t = std::stof(argv[5]);
            const std::string out = argv[6];
            SanaDenoiserWeights w = make_denoiser(g, d, 1, sh, ch);
            Tensor latent = randn_torch_cpu({1, d.latent, side, side}, 42);
            Tensor x = conv2d_1x1(latent, w.patch_embed_weight, &w.patch_embed_bias).grid_to_tokens_3d();
            TimeOut to = time_mlp(w, t, 1);
            Tensor ctx = randn_torch_cpu({1, 300, d.hidden}, 43);
            double t0 = now_ms();
            SanaBlockStageOutputs s = block_forward(x, ctx, to.t_mod, w.blocks[0], nullptr);
            std::printf("block_forward_ms %.3f\n", now_ms() - t0);
            dump(out, "x", x);
            dump(out, "t_mod", to.t_mod);
            dump(out, "after_self", s.after_self);
            dump(out, "after_cross", s.after_cross);
            dump(out, "after_ff", s.after_ff);
            return 0;
        }
        if (mode == "forward" && argc == 9) {
            const size_t sh = std::stoul(argv[2]), ch = std::stoul(argv[3]), side = std::stoul(argv[4]);
            const float t = std::stof(argv[5]);
            const bool mask = std::stoi(argv[6]) != 0, check = std::stoi(argv[7]) != 0;
            const std::string out = argv[8];
            SanaDenoiserWeights w = make_denoiser(g, d, d.layers, sh, ch);
            Tensor latent = randn_torch_cpu({1, d.latent, side, side}, 42);
            Tensor caption = randn_torch_cpu({2, 300, d.caption}, 43);
            Tensor bias = make_mask_bias(300, 1, 40);
            const Tensor * bp = mask ? &bias : nullptr;
            Tensor ctx = project_caption_context(caption, w.caption.linear_1_weight, &w.caption.linear_1_bias,
                                                 w.caption.linear_2_weight, &w.caption.linear_2_bias,
                                                 w.caption_norm_weight);
            dump(out, "context", ctx);
            double t0 = now_ms();
            Tensor np = forward_noise_pred(latent, ctx, t, w, bp);
            std::printf("forward_ms %.3f\n", now_ms() - t0);
            dump(out, "noise_pred", np);
            Tensor guided = apply_classifier_free_guidance(np, 4.5f);
            dump(out, "guided", guided);
            if (check) {
                SanaSchedulerConfig cfg = make_sana_scheduler_config();
                SanaSchedulerState s1 = init_sana_scheduler_state(20, cfg);
                SanaSchedulerState s2 = init_sana_scheduler_state(20, cfg);
                if (s1.schedule.timesteps[0] != t) throw std::runtime_error("check-step needs t == timesteps[0]");
                Tensor ref_step = run_full_denoising_step_with_cfg(latent, ctx, 4.5f, s1, cfg, w, bp);
                Tensor my_step = step_sana_scheduler(guided, latent, s2, cfg);
                const bool same = ref_step.data() == my_step.data();
                std::printf("check_step bit_exact=%d max_abs_diff=%g\n", same ? 1 : 0, ref_step.max_abs_diff(my_step));
                dump(out, "step0", ref_step);
                if (!same) return 1;
            }
            return 0;
        }
        if (mode == "forward-hw" && argc == 8) {
            // forward_noise_pred on an H x W latent (any H * W the reference
            // accepts: a perfect square), no mask
            const size_t sh = std::stoul(argv[2]), ch = std::stoul(argv[3]);
            const size_t hh = std::stoul(argv[4]), ww = std::stoul(argv[5]);
            const float t = std::stof(argv[6]);
            const std::string out = argv[7];
            SanaDenoiserWeights w = make_denoiser(g, d, d.layers, sh, ch);
            Tensor latent = randn_torch_cpu({1, d.latent, hh, ww}, 42);
            Tensor caption = randn_torch_cpu({2, 300, d.caption}, 43);
            Tensor ctx = project_caption_context(caption, w.caption.linear_1_weight, &w.caption.linear_1_bias,
                                                 w.caption.linear_2_weight, &w.caption.linear_2_bias,
                                                 w.caption_norm_weight);
            Tensor np = forward_noise_pred(latent, ctx, t, w, nullptr);
            dump(out, "noise_pred", np);
            return 0;
        }
        if (mode == "loop" && argc == 9) {
            const size_t sh = std::stoul(argv[2]), ch = std::stoul(argv[3]), side = std::stoul(argv[4]);
            const size_t steps = std::stoul(argv[5]);
            const float gs = std::stof(argv[6]);
            const bool mask = std::stoi(argv[7]) != 0;
            const std::string out = argv[8];
            SanaDenoiserWeights w = make_denoiser(g, d, d.layers, sh, ch);
            Tensor latent = randn_torch_cpu({1, d.latent, side, side}, 42);
            Tensor caption = randn_torch_cpu({2, 300, d.caption}, 43);
            Tensor bias = make_mask_bias(300, 1, 40);
            SanaSchedulerConfig cfg = make_sana_scheduler_config();
            SanaSchedulerState st = init_sana_scheduler_state(steps, cfg);
            double t0 = now_ms();
            Tensor fin = run_full_denoising_loop_with_cfg(latent, caption, gs, st, cfg, w, mask ? &bias : nullptr);
            std::printf("loop_ms %.3f\n", now_ms() - t0);
            dump(out, "final_latent", fin);
            return 0;
        }
        if (mode == "vae-conv" && argc == 6) {
            // both summation orders of the reference's 3x3 conv at one size
            const size_t side = std::stoul(argv[2]), cin = std::stoul(argv[3]), cout = std::stoul(argv[4]);
            const std::string out = argv[5];
            Tensor x = randn_torch_cpu({1, cin, side, side}, 51);
            Tensor w = randn_torch_cpu({cout, cin, 3, 3}, 52);
            w.mul_inplace_scalar(0.05f);
            Tensor b = randn_torch_cpu({std::max<size_t>(cout, 16)}, 53);
            Tensor bias({cout});
            for (size_t i = 0; i < cout; ++i) bias.data()[i] = b.data()[i];
            dump(out, "x", x);
            dump(out, "w", w);
            dump(out, "bias", bias);
            dump(out, "im2col", conv2d_3x3_im2col_gemm(x, w, &bias));
            dump(out, "tap", conv2d_3x3_tap_accumulate(x, w, &bias));
            return 0;
        }
        if ((mode == "vae" && argc == 5) || (mode == "vae-digest" && argc == 3)) {
            const std::string which = argv[2];
            const vae_spec::Config c = which == "full" ? vae_spec::full_config() : vae_spec::small_config();
            if (mode == "vae-digest") {
                VaeGen vg(c);
                for (const vae_spec::Entry & e : vae_spec::manifest(c)) {
                    Tensor t = vg(e.name);
                    uint64_t h = 14695981039346656037ULL;
                    const unsigned char * p = reinterpret_cast<const unsigned char *>(t.data().data());
                    for (size_t i = 0; i < t.numel() * 4; ++i) { h ^= p[i]; h *= 1099511628211ULL; }
                    std::printf("%s %016llx\n", e.name.c_str(), static_cast<unsigned long long>(h));
                }
                return 0;
            }
            const size_t side = std::stoul(argv[3]);
            const std::string out = argv[4];
            SanaVaeWeights w = make_vae(c);
            Tensor latent = randn_torch_cpu({1, c.latent, side, side}, 42);
            dump(out, "latent", latent);
            Tensor scaled = latent;
            scaled.mul_inplace_scalar(1.0f / w.scaling_factor);
            Tensor h0 = run_vae_decoder_input(scaled, w.decoder, true);
            dump(out, "decoder_input", h0);
            double t0 = now_ms();
            Tensor img = run_vae_decode(latent, w);
            std::printf("vae_decode_ms %.3f\n", now_ms() - t0);
            dump(out, "image", img);
            return 0;
        }
        if (mode == "time-forward" && argc == 5) {
            // one CFG step's forward as the reference runs it in its loop: the
            // caption projection (once per loop, src/transformer.cpp:701-708) and
            // the forward of run_full_denoising_step_with_cfg (:627-681)
            const size_t sh = std::stoul(argv[2]), ch = std::stoul(argv[3]), side = std::stoul(argv[4]);
            double t0 = now_ms();
            SanaDenoiserWeights w = make_denoiser(g, d, d.layers, sh, ch);
            Tensor latent = randn_torch_cpu({1, d.latent, side, side}, 42);
            Tensor caption = randn_torch_cpu({2, 300, d.caption}, 43);
            std::printf("setup_ms %.3f\n", now_ms() - t0);
            std::fflush(stdout);
            t0 = now_ms();
            Tensor ctx = project_caption_context(caption, w.caption.linear_1_weight, &w.caption.linear_1_bias,
                                                 w.caption.linear_2_weight, &w.caption.linear_2_bias,
                                                 w.caption_norm_weight);
            const double cap_ms = now_ms() - t0;
            std::printf("caption_projection_ms %.3f\n", cap_ms);
            std::fflush(stdout);
            t0 = now_ms();
            Tensor np = forward_noise_pred(latent, ctx, 999.0f, w, nullptr);
            const double fwd_ms = now_ms() - t0;
            std::printf("forward_ms %.3f\nstep_ms %.3f\n", fwd_ms, fwd_ms + cap_ms);
            return np.numel() ? 0 : 1;
        }
        if (mode == "time-micro" && argc == 4) {
            // linear_attention_4d on [2, 16, N, 72] and glumb_conv on [2, 1152, SIDE, SIDE]
            // (Mix-FFN 1152 -> 5760 -> 2880 -> 1152), inputs N(0, 1), weights N(0, 0.02)
            const size_t side = std::stoul(argv[2]), reps = std::stoul(argv[3]), N = side * side;
            Tensor q = randn_torch_cpu({2, 16, N, 72}, 61), k = randn_torch_cpu({2, 16, N, 72}, 62),
                   v = randn_torch_cpu({2, 16, N, 72}, 63);
            Tensor x = randn_torch_cpu({2, d.hidden, side, side}, 64);
            Tensor wi = randn_torch_cpu({d.ffn, d.hidden, 1, 1}, 65), bi = randn_torch_cpu({d.ffn}, 66);
            Tensor wd = randn_torch_cpu({d.ffn, 1, 3, 3}, 67), bd = randn_torch_cpu({d.ffn}, 68);
            Tensor wp = randn_torch_cpu({d.hidden, d.ffn / 2, 1, 1}, 69);
            for (Tensor * t : {&wi, &bi, &wd, &bd, &wp}) t->mul_inplace_scalar(0.02f);
            std::vector<double> la, ff;
            for (size_t r = 0; r < reps; ++r) {
                double t0 = now_ms();
                Tensor o = linear_attention_4d(q, k, v);
                la.push_back(now_ms() - t0);
                t0 = now_ms();
                Tensor y = glumb_conv(x, wi, &bi, wd, &bd, wp);
                ff.push_back(now_ms() - t0);
                if (!o.numel() || !y.numel()) return 1;
                std::printf("rep %zu linear_attention_ms %.3f mixffn_ms %.3f\n", r, la.back(), ff.back());
                std::fflush(stdout);
            }
            std::sort(la.begin(), la.end());
            std::sort(ff.begin(), ff.end());
            std::printf("median_linear_attention_ms %.3f\nmedian_mixffn_ms %.3f\n", la[la.size() / 2],
                        ff[ff.size() / 2]);
            return 0;
        }
        if (mode == "time-block" && argc == 7) {
            const size_t sh = std::stoul(argv[2]), ch = std::stoul(argv[3]);
            const size_t B = std::stoul(argv[4]), side = std::stoul(argv[5]), reps = std::stoul(argv[6]);
            SanaDenoiserWeights w = make_denoiser(g, d, 1, sh, ch);
            Tensor x = randn_torch_cpu({B, side * side, d.hidden}, 42);
            x.mul_inplace_scalar(0.1f);
            Tensor tm = randn_torch_cpu({B, 6 * d.hidden}, 44);
            tm.mul_inplace_scalar(0.05f);
            Tensor ctx = randn_torch_cpu({B, 300, d.hidden}, 43);
            std::vector<double> ms;
            for (size_t r = 0; r < reps; ++r) {
                double t0 = now_ms();
                SanaBlockStageOutputs s = block_forward(x, ctx, tm, w.blocks[0], nullptr);
                ms.push_back(now_ms() - t0);
                if (s.after_ff.numel() == 0) return 1;
                std::printf("rep %zu block_ms %.3f\n", r, ms.back());
                std::fflush(stdout);
            }
            std::sort(ms.begin(), ms.end());
            std::printf("median_block_ms %.3f\n", ms[ms.size() / 2]);
            return 0;
        }
    } catch (const std::exception & e) {
        std::fprintf(stderr, "error: %s\n", e.what());
        return 1;
    }
    return usage();
}
