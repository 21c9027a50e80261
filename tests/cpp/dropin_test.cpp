// Tests of the drop-in C++ API (sana.cpp_amd/host/*.h), written the way the
// reference's tests/test_tensor.cpp, tests/test_scheduler_main.cpp and
// tests/test_transformer.cpp are: known-answer values and exception types,
// plus whole-model parity of the device path against the CPU oracle (linked
// as the checker only).
//
//   dropin_test cpu          host-only checks; touches no GPU
//   dropin_test gpu          block known answers and small-model parity on the GPU
//   dropin_test gguf FILE [run]
//                            weights_io + loaders on FILE (a GGUF of the seeded
//                            small model) against the oracle's tensors; with
//                            `run`, also the denoise loop on the loaded weights
//                            (GPU) against the oracle's loop
//   dropin_test full-loop CAPTION LATENT STEPS OUT
//                            the denoise stage of sana_infer on the seeded
//                            Sana-0.6B model (28 blocks, 36/16 heads, guidance
//                            4.5): CAPTION [2,300,2304] and LATENT [1,32,32,32]
//                            raw fp32 in, final latent raw fp32 out
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

#include "oracle.h"
#include "scheduler.h"
#include "tensor.h"
#include "torch_rng.h"
#include "transformer.h"
#include "weights_io.h"

namespace {

int g_checks = 0, g_failures = 0;

void check(bool ok, const std::string & what) {
    ++g_checks;
    if (!ok) {
        ++g_failures;
        std::printf("FAIL %s\n", what.c_str());
        std::fflush(stdout);
    }
}

void near(float got, float want, float tol, const std::string & what) {
    check(std::fabs(got - want) <= tol, what + ": got " + std::to_string(got) + " want " + std::to_string(want));
}

template <class E>
void throws(const std::function<void()> & f, const std::string & what) {
    bool ok = false;
    try {
        f();
    } catch (const E &) {
        ok = true;
    } catch (const std::exception & e) {
        std::printf("  (%s threw another type: %s)\n", what.c_str(), e.what());
    }
    check(ok, what + " throws the reference's exception type");
}

double rel_l2(const std::vector<float> & a, const std::vector<float> & b) {
    double num = 0.0, den = 0.0;
    for (size_t i = 0; i < a.size() && i < b.size(); ++i) {
        num += (double(a[i]) - b[i]) * (double(a[i]) - b[i]);
        den += double(b[i]) * b[i];
    }
    if (a.size() != b.size()) return 1e30;
    return std::sqrt(num / (den > 0 ? den : 1.0));
}

void close_l2(const std::vector<float> & got, const std::vector<float> & want, double tol, const std::string & what) {
    const double e = rel_l2(got, want);
    std::printf("  %s: rel_l2 %.3e\n", what.c_str(), e);
    check(e < tol, what + " rel_l2 " + std::to_string(e));
}

Tensor t1(std::initializer_list<float> v) {
    Tensor t({v.size()});
    std::copy(v.begin(), v.end(), t.data().begin());
    return t;
}

Tensor filled(std::vector<size_t> shape, std::initializer_list<float> v) {
    Tensor t(std::move(shape));
    std::copy(v.begin(), v.end(), t.data().begin());
    return t;
}

// ---------------------------------------------------------------- tensor (tests/test_tensor.cpp)

void tensor_tests() {
    Tensor image({2, 3, 4});
    check(image.rank() == 3 && image.numel() == 24 && image.dim_size(2) == 4, "tensor shape");
    Tensor scalar({});
    check(scalar.rank() == 0 && scalar.numel() == 1, "rank-0 tensor holds one value");
    check(image.flat_index({1, 2, 3}) == 23 && image.flat_index({0, 1, 2}) == 6, "flat_index");
    throws<std::out_of_range>([&] { image.flat_index({2, 0, 0}); }, "flat_index out of range");
    throws<std::out_of_range>([&] { image.at(24); }, "at out of range");
    throws<std::invalid_argument>([&] { image.add_inplace(Tensor({2, 3})); }, "add_inplace shape mismatch");
    Tensor a = filled({2, 3}, {1, 2, 3, 4, 5, 6});
    Tensor t = a.transpose_2d();
    check(t.shape() == std::vector<size_t>({3, 2}) && t.at({0, 1}) == 4.0f && t.at({2, 0}) == 3.0f, "transpose_2d");
    Tensor n3 = filled({1, 2, 2}, {1, 3, 2, 4});
    Tensor ln = n3.layer_norm_3d_lastdim(0.0f);
    check(ln.at({0, 0, 0}) == -1.0f && ln.at({0, 1, 1}) == 1.0f, "layer_norm_3d_lastdim");
    Tensor g = t1({2, 3}), b = t1({1, -1});
    Tensor lna = n3.layer_norm_3d_lastdim(0.0f, &g, &b);
    check(lna.at({0, 0, 0}) == -1.0f && lna.at({0, 0, 1}) == 2.0f, "layer_norm affine");
    Tensor rms = filled({1, 2, 2}, {3, 4, 0, 5}).rms_norm_3d_lastdim(0.0f, &g);
    near(rms.at({0, 0, 0}), 1.6970563f, 1e-5f, "rms_norm[0]");
    near(rms.at({0, 1, 1}), 4.2426405f, 1e-5f, "rms_norm[3]");
    Tensor mod = filled({1, 2, 2}, {1, 2, 3, 4})
                     .modulate_3d_lastdim(filled({1, 1, 2}, {10, 20}), filled({1, 1, 2}, {0.5f, -0.5f}));
    check(mod.at({0, 0, 0}) == 11.5f && mod.at({0, 1, 1}) == 22.0f, "modulate_3d_lastdim");
    Tensor grid = filled({1, 4, 2}, {1, 2, 3, 4, 5, 6, 7, 8}).tokens_to_grid_4d(2, 2);
    check(grid.at({0, 0, 0, 1}) == 3.0f && grid.at({0, 1, 1, 0}) == 6.0f, "tokens_to_grid_4d");
    check(grid.grid_to_tokens_3d().at({0, 3, 1}) == 8.0f, "grid_to_tokens_3d");
}

// ---------------------------------------------------------------- scheduler (tests/test_scheduler_main.cpp)

void scheduler_tests() {
    const SanaSchedulerConfig config = make_sana_scheduler_config();
    check(config.num_train_timesteps == 1000 && config.solver_order == 2 && config.lower_order_final &&
              config.use_flow_sigmas && config.final_sigmas_type == "zero",
          "default scheduler config");
    const SanaSchedulerTimesteps s = build_sana_scheduler_timesteps(4, config);
    check(s.timesteps.size() == 4 && s.sigmas.size() == 5, "schedule sizes");
    const float ts[4] = {999, 899, 749, 499};
    const float sg[5] = {0.99966644f, 0.89963979f, 0.74962479f, 0.49966654f, 0.0f};
    for (int i = 0; i < 4; ++i) near(s.timesteps[i], ts[i], 1e-3f, "timestep " + std::to_string(i));
    for (int i = 0; i < 5; ++i) near(s.sigmas[i], sg[i], 1e-6f, "sigma " + std::to_string(i));
    throws<std::invalid_argument>([&] { build_sana_scheduler_timesteps(0, config); }, "zero steps");
    SanaSchedulerConfig bad = config;
    bad.use_flow_sigmas = false;
    throws<std::invalid_argument>([&] { build_sana_scheduler_timesteps(4, bad); }, "non-flow sigmas");
    bad = config;
    bad.solver_order = 0;
    throws<std::invalid_argument>([&] { init_sana_scheduler_state(4, bad); }, "solver_order 0");
    bad = config;
    bad.prediction_type = "epsilon";
    throws<std::invalid_argument>([&] { init_sana_scheduler_state(4, bad); }, "epsilon prediction");

    SanaSchedulerState st;
    st.schedule.timesteps = {800.0f, 500.0f, 200.0f};
    st.schedule.sigmas = {0.8f, 0.5f, 0.2f, 0.0f};
    const Tensor sample = t1({4.0f}), out = t1({2.0f});
    const Tensor conv = convert_sana_scheduler_model_output(out, sample, st, config);
    near(conv.at(0), 2.4f, 1e-6f, "convert");
    near(sana_scheduler_first_order_update(conv, sample, st, config).at(0), 3.4f, 1e-5f, "first order");
    SanaSchedulerState stepped = st;
    near(step_sana_scheduler(out, sample, stepped, config).at(0), 3.4f, 1e-5f, "step");
    check(stepped.step_index == 1 && stepped.lower_order_step_count == 1 &&
              stepped.previous_model_outputs.size() == 1,
          "state after a step");
    SanaSchedulerState so;
    so.schedule.timesteps.resize(16);
    so.schedule.sigmas = {0.8f,  0.5f,  0.2f,  0.1f,  0.09f, 0.08f,  0.07f, 0.06f, 0.05f,
                          0.04f, 0.03f, 0.02f, 0.015f, 0.01f, 0.005f, 0.001f, 0.0f};
    so.step_index = 1;
    so.lower_order_step_count = 1;
    so.previous_model_outputs = {t1({2.4f}), t1({2.0f})};
    near(sana_scheduler_second_order_update(t1({3.4f}), so, config).at(0), 2.44f, 1e-5f, "second order");
    step_sana_scheduler(t1({3.1f}), t1({3.4f}), so, config);
    check(so.step_index == 2 && so.lower_order_step_count == 2 && so.previous_model_outputs.size() == 2,
          "state after a second-order step");
}

// ---------------------------------------------------------------- transformer host side

SanaBlockWeights kat_block(const Tensor & proj) {
    // tests/test_transformer.cpp:373-431: hidden 2, one head, identity Mix-FFN
    Tensor sst({6, 2}), gamma = t1({1, 1}), beta = t1({0, 0}), bias = t1({0, 0});
    Tensor inv({4, 2, 1, 1}), inv_b({4}), dw({4, 1, 3, 3}), dw_b({4}), pt({2, 2, 1, 1});
    inv.at({0, 0, 0, 0}) = inv.at({1, 1, 0, 0}) = inv.at({2, 0, 0, 0}) = inv.at({3, 1, 0, 0}) = 1.0f;
    for (size_t e = 0; e < 4; ++e) dw.at({e, 0, 1, 1}) = 1.0f;
    pt.at({0, 0, 0, 0}) = pt.at({1, 1, 0, 0}) = 1.0f;
    return SanaBlockWeights{sst,  gamma, beta, proj, bias, proj, bias, proj, bias, proj,  bias, proj, bias, proj,
                            bias, proj,  bias, proj, bias, gamma, beta, inv,  inv_b, dw, dw_b, pt,   1,    1};
}

Tensor eye2() { return filled({2, 2}, {1, 0, 0, 1}); }

void transformer_host_tests() {
    Tensor tmod({1, 12});
    tmod.at({0, 4}) = tmod.at({0, 5}) = tmod.at({0, 10}) = tmod.at({0, 11}) = 1.0f;
    Tensor sst({6, 2});
    sst.at({1, 0}) = 0.5f;
    const SanaBlockModulation m = compute_sana_block_modulation(tmod, sst);
    check(m.shift_msa.shape() == std::vector<size_t>({1, 1, 2}), "modulation part shape");
    check(m.scale_msa.at(0) == 0.5f && m.gate_msa.at(0) == 1.0f && m.gate_mlp.at(1) == 1.0f,
          "modulation = timestep + table");
    throws<std::invalid_argument>([&] { compute_sana_block_modulation(Tensor({1, 11}), sst); }, "timestep width");

    Tensor np = filled({2, 1, 1, 2}, {1, 2, 3, 5});
    Tensor cfg = apply_classifier_free_guidance(np, 4.5f);
    check(cfg.shape() == std::vector<size_t>({1, 1, 1, 2}) && cfg.at(0) == 10.0f && cfg.at(1) == 15.5f, "cfg");
    throws<std::invalid_argument>([&] { apply_classifier_free_guidance(Tensor({3, 1, 1, 1}), 1.0f); },
                                  "cfg odd batch");

    // block_forward rejects bad shapes before any device work
    // (tests/test_transformer.cpp:606-612)
    const SanaBlockWeights w = kat_block(eye2());
    const Tensor lin({2, 3});
    throws<std::invalid_argument>([&] { block_forward(lin, lin, lin, w); }, "block_forward rank-2 inputs");
    Tensor x({1, 3, 2}), ctx({1, 2, 2});
    throws<std::invalid_argument>([&] { block_forward(x, ctx, tmod, w); }, "block_forward non-square tokens");
    Tensor bad_bias({1, 1, 3});
    throws<std::invalid_argument>([&] { block_forward(Tensor({1, 1, 2}), ctx, tmod, w, &bad_bias); },
                                  "block_forward bias shape");

    std::vector<SanaBlockWeights> none;
    throws<std::invalid_argument>([&] { validate_model_block_sequence(none); }, "empty block list");
}

void rng_tests() {
    // the same generator as the oracle's (pinned bit-exact against the
    // reference's randn_torch_cpu through the seeded weight digests)
    for (size_t n : {16u, 37u, 1000u}) {
        const Tensor t = randn_torch_cpu({n}, 42 + n);
        std::vector<float> ref(n);
        oracle_randn(ref.data(), n, 42 + n);
        check(std::memcmp(t.data().data(), ref.data(), n * 4) == 0, "randn_torch_cpu n=" + std::to_string(n));
    }
    throws<std::invalid_argument>([&] { randn_torch_cpu({15}, 1); }, "randn below 16 values");
}

// ---------------------------------------------------------------- small seeded model

struct SmallModel {
    size_t layers = 2, C = 128, E = 256, Ccap = 96, Cl = 8, Hs = 4, Hc = 2;
    oracle_model * om = nullptr;
    SmallModel(bool full = false) {
        if (full) {
            layers = 28;
            C = 1152;
            E = 5760;
            Ccap = 2304;
            Cl = 32;
            Hs = 36;
            Hc = 16;
        }
        om = oracle_model_create(layers, C, E, Ccap, Cl, Hs, Hc);
        if (!om || oracle_model_generate(om) != 0) throw std::runtime_error("oracle model");
    }
    ~SmallModel() { oracle_model_destroy(om); }
    Tensor get(const std::string & name, std::vector<size_t> shape) const {
        Tensor t(std::move(shape));
        if (oracle_model_get(om, name.c_str(), t.data().data(), t.numel()) != 0)
            throw std::runtime_error("oracle tensor " + name);
        return t;
    }
    Tensor lin(const std::string & name, size_t out, size_t in) const { return get(name, {out, in}).transpose_2d(); }
    SanaBlockWeights block(size_t i) const {
        const std::string p = "transformer_blocks." + std::to_string(i) + ".";
        Tensor zeros({C}), ones({C});
        ones.fill(1.0f);
        return SanaBlockWeights{get(p + "scale_shift_table", {6, C}),
                                ones,
                                zeros,
                                lin(p + "attn1.to_q.weight", C, C),
                                zeros,
                                lin(p + "attn1.to_k.weight", C, C),
                                zeros,
                                lin(p + "attn1.to_v.weight", C, C),
                                zeros,
                                lin(p + "attn1.to_out.0.weight", C, C),
                                get(p + "attn1.to_out.0.bias", {C}),
                                lin(p + "attn2.to_q.weight", C, C),
                                get(p + "attn2.to_q.bias", {C}),
                                lin(p + "attn2.to_k.weight", C, C),
                                get(p + "attn2.to_k.bias", {C}),
                                lin(p + "attn2.to_v.weight", C, C),
                                get(p + "attn2.to_v.bias", {C}),
                                lin(p + "attn2.to_out.0.weight", C, C),
                                get(p + "attn2.to_out.0.bias", {C}),
                                ones,
                                zeros,
                                get(p + "ff.conv_inverted.weight", {E, C, 1, 1}),
                                get(p + "ff.conv_inverted.bias", {E}),
                                get(p + "ff.conv_depth.weight", {E, 1, 3, 3}),
                                get(p + "ff.conv_depth.bias", {E}),
                                get(p + "ff.conv_point.weight", {C, E / 2, 1, 1}),
                                Hs,
                                Hc};
    }
    SanaDenoiserWeights weights() const {
        std::vector<SanaBlockWeights> blocks;
        for (size_t i = 0; i < layers; ++i) blocks.push_back(block(i));
        return SanaDenoiserWeights{
            {lin("caption_projection.linear_1.weight", C, Ccap), get("caption_projection.linear_1.bias", {C}),
             lin("caption_projection.linear_2.weight", C, C), get("caption_projection.linear_2.bias", {C})},
            blocks,
            get("patch_embed.proj.weight", {C, Cl, 1, 1}),
            get("patch_embed.proj.bias", {C}),
            lin("time_embed.emb.timestep_embedder.linear_1.weight", C, 256),
            get("time_embed.emb.timestep_embedder.linear_1.bias", {C}),
            lin("time_embed.emb.timestep_embedder.linear_2.weight", C, C),
            get("time_embed.emb.timestep_embedder.linear_2.bias", {C}),
            lin("time_embed.linear.weight", 6 * C, C),
            get("time_embed.linear.bias", {6 * C}),
            get("caption_norm.weight", {C}),
            get("scale_shift_table", {2, C}),
            lin("proj_out.weight", Cl, C),
            get("proj_out.bias", {Cl}),
        };
    }
};

void compare_weights(const SanaDenoiserWeights & a, const SanaDenoiserWeights & b) {
    auto same = [](const Tensor & x, const Tensor & y, const std::string & n) {
        check(x.shape() == y.shape() && x.data() == y.data(), "loaded tensor " + n);
    };
    same(a.caption.linear_1_weight, b.caption.linear_1_weight, "caption linear_1");
    same(a.caption.linear_2_bias, b.caption.linear_2_bias, "caption linear_2 bias");
    same(a.time_projection_weight, b.time_projection_weight, "time projection");
    same(a.proj_out_weight, b.proj_out_weight, "proj_out");
    same(a.final_scale_shift_table, b.final_scale_shift_table, "final table");
    check(a.blocks.size() == b.blocks.size(), "block count");
    for (size_t i = 0; i < a.blocks.size() && i < b.blocks.size(); ++i) {
        const std::string p = "block " + std::to_string(i) + " ";
        same(a.blocks[i].q_weight, b.blocks[i].q_weight, p + "q");
        same(a.blocks[i].cross_v_bias, b.blocks[i].cross_v_bias, p + "cross v bias");
        same(a.blocks[i].ff_depth_weight, b.blocks[i].ff_depth_weight, p + "depthwise");
        same(a.blocks[i].ff_point_weight, b.blocks[i].ff_point_weight, p + "point");
        check(a.blocks[i].self_num_heads == b.blocks[i].self_num_heads, p + "heads");
    }
}

int gguf_tests(const std::string & path, bool run) {
    const auto index = load_weight_index(path);
    const SmallModel sm;
    check(index.size() == sm.layers * 19 + 16, "tensor count " + std::to_string(index.size()));
    const auto it = index.find("transformer_blocks.1.attn1.to_q.weight");
    check(it != index.end() && it->second.shape == std::vector<size_t>({128, 128}) &&
              it->second.format == WeightFormat::Gguf && it->second.dtype == "float32",
          "index entry");
    check(find_block_prefixes(index) ==
              std::vector<std::string>({"transformer_blocks.0", "transformer_blocks.1"}),
          "block prefixes in numeric order");
    const SanaDenoiserWeights loaded = load_denoiser_weights(path, index, path, index, path, index, 4, 2);
    compare_weights(loaded, sm.weights());
    throws<std::invalid_argument>([&] { load_weight_tensor(path, index, "missing.weight"); }, "missing tensor");
    throws<std::runtime_error>([&] { load_weight_index(path + ".npy"); }, "non-gguf index");
    throws<std::invalid_argument>([&] { load_block_weights(path, index, "transformer_blocks.0", 0, 2); },
                                  "zero self heads");
    throws<std::runtime_error>([&] { load_block_weights(path, index, "transformer_blocks.0", 3, 2); },
                               "hidden not divisible by heads");
    if (run) {
        const Tensor caption = randn_torch_cpu({2, 16, sm.Ccap}, 43);
        const Tensor latent = randn_torch_cpu({1, sm.Cl, 8, 8}, 42);
        std::vector<float> ref(latent.numel());
        oracle_model_loop(sm.om, latent.data().data(), 1, 8, 8, caption.data().data(), 16, nullptr, 6, 4.5f,
                          ref.data());
        const SanaSchedulerConfig cfg = make_sana_scheduler_config();
        SanaSchedulerState st = init_sana_scheduler_state(6, cfg);
        close_l2(run_full_denoising_loop_with_cfg(latent, caption, 4.5f, st, cfg, loaded).data(), ref, 1e-2,
                 "loop on GGUF-loaded weights");
    }
    return 0;
}

// ---------------------------------------------------------------- device tests

void gpu_kat_tests() {
    // tests/test_transformer.cpp:373-484, at the fp16-operand tolerance of the
    // device path (2e-3 relative to max(1, |want|))
    Tensor x = filled({1, 1, 2}, {1, 0}), ctx = filled({1, 2, 2}, {2, 0, 0, 3});
    Tensor tmod({1, 12});
    tmod.at({0, 4}) = tmod.at({0, 5}) = tmod.at({0, 10}) = tmod.at({0, 11}) = 1.0f;
    const SanaBlockWeights w = kat_block(eye2());
    const SanaBlockStageOutputs o = block_forward(x, ctx, tmod, w);
    check(o.after_ff.shape() == std::vector<size_t>({1, 1, 2}), "block_forward shape");
    near(o.after_ff.at(0), 4.3467007f, 2e-3f * 4.35f, "block_forward[0]");
    near(o.after_ff.at(1), -0.9475632f, 2e-3f, "block_forward[1]");
    const SanaBlockWeights z = kat_block(Tensor({2, 2}));
    const Tensor r = block_forward(x, ctx, tmod, z).after_ff;
    near(r.at(0), 1.3607715f, 2e-3f * 1.37f, "residual-only block[0]");
    near(r.at(1), 0.0313307f, 2e-3f, "residual-only block[1]");
    // the first block's cached device copy must not be reused for the second
    const Tensor again = block_forward(x, ctx, tmod, w).after_ff;
    check(again.data() == o.after_ff.data(), "block_forward repeatable after another weights object");
}

void gpu_small_model_tests() {
    const SmallModel sm;
    const SanaDenoiserWeights w = sm.weights();
    validate_denoiser_weights(w);
    const size_t C = sm.C, L = 16, N = 64, B = 2;
    const Tensor caption = randn_torch_cpu({B, L, sm.Ccap}, 43);
    Tensor ctx({B, L, C});
    oracle_model_project_caption(sm.om, caption.data().data(), B, L, ctx.data().data());
    const Tensor x = randn_torch_cpu({B, N, C}, 7);
    Tensor emb({B, C}), tmod({B, 6 * C});
    const float tt[2] = {500.0f, 500.0f};
    oracle_model_time(sm.om, tt, B, emb.data().data(), tmod.data().data());
    Tensor bias({B, 1, L});
    bias.fill(-10000.0f);
    for (size_t l = 0; l < 5; ++l) bias.at({0, 0, l}) = 0.0f;
    for (size_t l = 0; l < 12; ++l) bias.at({1, 0, l}) = 0.0f;

    // block_forward: all three stages, masked
    std::vector<float> s1(B * N * C), s2(B * N * C), s3(B * N * C);
    oracle_model_block(sm.om, 1, x.data().data(), ctx.data().data(), tmod.data().data(), bias.data().data(), B, N, L,
                       s1.data(), s2.data(), s3.data());
    const SanaBlockStageOutputs o = block_forward(x, ctx, tmod, w.blocks[1], &bias);
    close_l2(o.after_self.data(), s1, 2e-3, "block_forward after_self");
    close_l2(o.after_cross.data(), s2, 2e-3, "block_forward after_cross");
    close_l2(o.after_ff.data(), s3, 2e-3, "block_forward after_ff");

    // run_model_blocks over both blocks
    std::vector<float> h0(B * N * C), a(B * N * C), b(B * N * C);
    oracle_model_block(sm.om, 0, x.data().data(), ctx.data().data(), tmod.data().data(), nullptr, B, N, L, a.data(),
                       b.data(), h0.data());
    std::vector<float> h1(B * N * C);
    oracle_model_block(sm.om, 1, h0.data(), ctx.data().data(), tmod.data().data(), nullptr, B, N, L, a.data(),
                       b.data(), h1.data());
    close_l2(run_model_blocks(x, ctx, tmod, w, 0, 2).data(), h1, 2e-3, "run_model_blocks [0, 2)");
    close_l2(run_model_blocks(x, ctx, tmod, w, 1, 2, &bias).data(), s3, 2e-3, "run_model_blocks [1, 2) masked");
    check(run_model_blocks(x, ctx, tmod, w, 1, 1).data() == x.data(), "empty block range returns the input");
    throws<std::invalid_argument>([&] { run_model_blocks(x, ctx, tmod, w, 2, 3); }, "block range past the end");

    // one CFG step against oracle forward + CFG + the host scheduler
    const SanaSchedulerConfig cfg = make_sana_scheduler_config();
    const Tensor latent = randn_torch_cpu({1, sm.Cl, 8, 8}, 42);
    SanaSchedulerState st = init_sana_scheduler_state(6, cfg);
    const Tensor stepped = run_full_denoising_step_with_cfg(latent, ctx, 4.5f, st, cfg, w, &bias);
    Tensor np({2, sm.Cl, 8, 8});
    oracle_model_forward(sm.om, latent.data().data(), 1, 8, 8, ctx.data().data(), L, bias.data().data(),
                         st.schedule.timesteps[0], np.data().data());
    SanaSchedulerState st_ref = init_sana_scheduler_state(6, cfg);
    const Tensor want = step_sana_scheduler(apply_classifier_free_guidance(np, 4.5f), latent, st_ref, cfg);
    close_l2(stepped.data(), want.data(), 2e-3, "run_full_denoising_step_with_cfg");
    check(st.step_index == 1, "step advances the scheduler");
    throws<std::invalid_argument>(
        [&] {
            SanaSchedulerState done = st;
            done.step_index = 6;
            run_full_denoising_step_with_cfg(latent, ctx, 4.5f, done, cfg, w);
        },
        "step past the schedule");
    throws<std::invalid_argument>(
        [&] { run_full_denoising_step_with_cfg(latent, Tensor({3, L, C}), 4.5f, st, cfg, w); },
        "context batch != 2 x latent batch");

    // whole loop: the fused device loop and the per-step path, against the oracle loop
    std::vector<float> ref(latent.numel());
    oracle_model_loop(sm.om, latent.data().data(), 1, 8, 8, caption.data().data(), L, bias.data().data(), 6, 4.5f,
                      ref.data());
    SanaSchedulerState s_fused = init_sana_scheduler_state(6, cfg);
    const Tensor fused = run_full_denoising_loop_with_cfg(latent, caption, 4.5f, s_fused, cfg, w, &bias);
    close_l2(fused.data(), ref, 1e-2, "run_full_denoising_loop_with_cfg (device loop)");
    SanaSchedulerState s_steps = init_sana_scheduler_state(6, cfg);
    Tensor lat = latent;
    while (s_steps.step_index < 6) lat = run_full_denoising_step_with_cfg(lat, ctx, 4.5f, s_steps, cfg, w, &bias);
    close_l2(lat.data(), ref, 1e-2, "per-step loop");
    check(s_fused.step_index == 6 && s_fused.lower_order_step_count == 2 &&
              s_fused.previous_model_outputs.size() == 2,
          "scheduler state after the device loop");
    if (s_fused.previous_model_outputs.size() == 2 && s_steps.previous_model_outputs.size() == 2) {
        close_l2(s_fused.previous_model_outputs[0].data(), s_steps.previous_model_outputs[0].data(), 2e-3,
                 "loop model output n-2");
        close_l2(s_fused.previous_model_outputs[1].data(), s_steps.previous_model_outputs[1].data(), 2e-3,
                 "loop model output n-1");
    }
    // a loop resumed mid-schedule takes the per-step path
    SanaSchedulerState s_mid = init_sana_scheduler_state(6, cfg);
    Tensor mid = run_full_denoising_step_with_cfg(latent, ctx, 4.5f, s_mid, cfg, w, &bias);
    mid = run_full_denoising_loop_with_cfg(mid, caption, 4.5f, s_mid, cfg, w, &bias);
    close_l2(mid.data(), ref, 1e-2, "loop resumed after one step");
}

std::vector<float> read_f32(const std::string & path, size_t n) {
    std::vector<float> v(n);
    std::ifstream f(path, std::ios::binary);
    f.read(reinterpret_cast<char *>(v.data()), static_cast<std::streamsize>(n * 4));
    if (!f) throw std::runtime_error("cannot read " + path);
    return v;
}

int full_loop(const std::string & caption_path, const std::string & latent_path, size_t steps,
              const std::string & out_path) {
    std::printf("generating the seeded 28-block weights\n");
    std::fflush(stdout);
    const SmallModel sm(true);
    const SanaDenoiserWeights w = sm.weights();
    Tensor caption({2, 300, 2304}), latent({1, 32, 32, 32});
    caption.data() = read_f32(caption_path, caption.numel());
    latent.data() = read_f32(latent_path, latent.numel());
    const SanaSchedulerConfig cfg = make_sana_scheduler_config();
    SanaSchedulerState st = init_sana_scheduler_state(steps, cfg);
    std::printf("running %zu steps\n", steps);
    std::fflush(stdout);
    const Tensor fin = run_full_denoising_loop_with_cfg(latent, caption, 4.5f, st, cfg, w);
    std::ofstream f(out_path, std::ios::binary);
    f.write(reinterpret_cast<const char *>(fin.data().data()), static_cast<std::streamsize>(fin.numel() * 4));
    check(static_cast<bool>(f), "final latent written");
    check(st.step_index == steps, "loop consumed the schedule");
    return 0;
}

}  // namespace

int main(int argc, char ** argv) {
    const std::string mode = argc > 1 ? argv[1] : "cpu";
    try {
        if (mode == "cpu") {
            tensor_tests();
            scheduler_tests();
            transformer_host_tests();
            rng_tests();
        } else if (mode == "gpu") {
            gpu_kat_tests();
            gpu_small_model_tests();
        } else if (mode == "gguf" && argc > 2) {
            gguf_tests(argv[2], argc > 3 && std::string(argv[3]) == "run");
        } else if (mode == "full-loop" && argc > 5) {
            full_loop(argv[2], argv[3], std::strtoul(argv[4], nullptr, 10), argv[5]);
        } else {
            std::fprintf(stderr, "usage: dropin_test cpu | gpu | gguf FILE [run] | full-loop CAPTION LATENT STEPS OUT\n");
            return 2;
        }
    } catch (const std::exception & e) {
        std::printf("FAIL uncaught exception: %s\n", e.what());
        return 1;
    }
    std::printf("%s: %d checks, %d failures\n", mode.c_str(), g_checks, g_failures);
    return g_failures ? 1 : 0;
}
