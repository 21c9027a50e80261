/* CPU restatement of sana.cpp's Linux DiT path -- TEST INFRASTRUCTURE.
 *
 * This library is the parity oracle: only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only as the checker.  The
 * product path (sana.cpp_amd/) never links or calls it.
 *
 * Every function follows the loop and accumulation order of the reference's
 * non-Apple (#else) branch it cites, so that, compiled with
 * -O3 -ffp-contract=off, it reproduces the reference's fp32 results bit for
 * bit.  Row-parallel threading is used only where each output row is an
 * independent computation, which leaves every output's operation sequence
 * unchanged.
 *
 * Layouts: activations are token-major [B, N, C]; linear weights are in
 * PyTorch/GGUF order [out, in] (the reference transposes them to [in, out]
 * at load, src/weights_io.cpp:367-377, which does not change any sum);
 * 1x1 conv weights [out, in]; depthwise weights [C, 3, 3].
 *
 * Return codes: 0 ok, -1 invalid argument (message via oracle_last_error()).
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char * oracle_last_error(void);
void oracle_set_threads(int n);

/* torch.randn(shape, generator=manual_seed(seed)) on CPU; n >= 16.
 * Follows src/torch_rng.cpp:14-68. */
int oracle_randn(float * out, size_t n, uint64_t seed);

/* out[M,N] = bias + in[M,K] . W[N,K]^T, i-k-j order of src/common_ops.cpp:49-64. */
int oracle_linear(const float * in, const float * w, const float * bias, float * out,
                  size_t M, size_t K, size_t N);
/* out[B,N,C] = LN(x) (eps, optional gamma/beta); src/tensor.cpp:235-268. */
int oracle_layer_norm(const float * x, const float * gamma, const float * beta, float * out,
                      size_t rows, size_t C, float eps);
/* src/tensor.cpp:276-316. */
int oracle_rms_norm(const float * x, const float * weight, float * out, size_t rows, size_t C, float eps);
/* out[b,t,h] = x*(1+scale[b,h]) + shift[b,h]; src/tensor.cpp:364-372. */
int oracle_modulate(const float * x, const float * shift, const float * scale, float * out,
                    size_t B, size_t N, size_t C);
/* ReLU linear attention on token-major q,k,v [B,N,H*D]; src/transformer_ops.cpp:496-537. */
int oracle_linear_attention(const float * q, const float * k, const float * v, float * out,
                            size_t B, size_t Nq, size_t Nkv, size_t H, size_t D);
/* Softmax attention, q [B,Nq,H*D], k/v [B,L,H*D], bias [B,L] or NULL;
 * src/transformer_ops.cpp:178-392. */
int oracle_attention(const float * q, const float * k, const float * v, const float * bias, float * out,
                     size_t B, size_t Nq, size_t L, size_t H, size_t D);
/* Depthwise 3x3 (zero pad) + bias on a token-major grid [B,H,W,C]; src/common_ops.cpp:483-505. */
int oracle_depthwise3x3(const float * x, const float * w, const float * bias, float * out,
                        size_t B, size_t Hh, size_t Ww, size_t C);
/* GLUMBConv on token-major x [B,H*W,Cin] -> [B,H*W,Cout]; src/common_ops.cpp:733-761. */
int oracle_glumb_conv(const float * x, const float * inv_w, const float * inv_b, const float * dw_w,
                      const float * dw_b, const float * pt_w, float * out, size_t B, size_t Hh, size_t Ww,
                      size_t Cin, size_t E, size_t Cout);
/* Caption MLP + RMSNorm; src/transformer_ops.cpp:64-76. */
int oracle_caption_projection(const float * x, const float * w1, const float * b1, const float * w2,
                              const float * b2, const float * norm_w, float * out, size_t rows,
                              size_t Cin, size_t C);
/* [B] timesteps -> [B, dim] sinusoid; src/transformer.cpp:77-122. */
int oracle_timestep_embedding(const float * t, float * out, size_t B, size_t dim);
/* u + g (c - u); src/transformer.cpp:570-602. */
int oracle_cfg(const float * noise_pred, float * out, size_t half_numel, float guidance);

/* attention_block_3d (src/transformer_ops.cpp:545-570): x [B,N,C]; linear
 * weights PyTorch order [C,C]; any bias may be NULL. */
int oracle_attention_block(const float * x, const float * wq, const float * bq, const float * wk, const float * bk,
                           const float * wv, const float * bv, const float * wo, const float * bo, float * out,
                           size_t B, size_t N, size_t C, size_t heads);
/* cross_attention_block_3d (src/transformer_ops.cpp:572-608): x [B,N,C],
 * context [B,L,C], bias [B,L] or NULL. */
int oracle_cross_attention_block(const float * x, const float * ctx, const float * bias, const float * wq,
                                 const float * bq, const float * wk, const float * bk, const float * wv,
                                 const float * bv, const float * wo, const float * bo, float * out, size_t B,
                                 size_t N, size_t L, size_t C, size_t heads);

/* DPM-Solver++ pieces of src/scheduler.cpp with explicit sigmas (flow sigmas:
 * alpha = 1 - sigma).  convert: :155-173; first order: :175-205; second
 * order (midpoint): :207-270. */
int oracle_sched_convert(const float * model_out, const float * sample, size_t n, float sigma, float * out);
int oracle_sched_first_order(const float * converted, const float * sample, size_t n, float sigma_t, float sigma_s,
                             float * out);
int oracle_sched_second_order(const float * sample, const float * m0, const float * m1, size_t n, float sigma_t,
                              float sigma_s0, float sigma_s1, float * out);

/* One DiT block with explicit weights (all 26 tensors of SanaBlockWeights,
 * src/transformer.h:26-55).  t_mod [B, 6C]; context [B, L, C]; bias [B, L] or NULL. */
typedef struct {
    const float * scale_shift_table;              /* [6, C] */
    const float * attn_norm_gamma, * attn_norm_beta;
    const float * q_w, * q_b, * k_w, * k_b, * v_w, * v_b, * out_w, * out_b;
    const float * cq_w, * cq_b, * ck_w, * ck_b, * cv_w, * cv_b, * co_w, * co_b;
    const float * mlp_norm_gamma, * mlp_norm_beta;
    const float * inv_w, * inv_b, * dw_w, * dw_b, * pt_w;
    size_t hidden, ffn, self_heads, cross_heads;
} oracle_block_weights;

int oracle_block_forward(const oracle_block_weights * w, const float * x, const float * context,
                         const float * t_mod, const float * bias, size_t B, size_t N, size_t L,
                         float * after_self, float * after_cross, float * after_ff);

/* Whole-model oracle.  Weights are registered by their GGUF tensor name
 * (shapes in PyTorch order); the model copies them. */
typedef struct oracle_model oracle_model;
oracle_model * oracle_model_create(size_t layers, size_t hidden, size_t ffn, size_t caption_dim,
                                   size_t latent_channels, size_t self_heads, size_t cross_heads);
void oracle_model_destroy(oracle_model * m);
int oracle_model_set(oracle_model * m, const char * name, const float * data, size_t numel);
/* Generate every tensor of the synthetic manifest (0.02 randn, seed 1000+sorted index). */
int oracle_model_generate(oracle_model * m);
/* Copy a registered tensor out (PyTorch order). */
int oracle_model_get(const oracle_model * m, const char * name, float * out, size_t numel);
/* 64-bit FNV-1a of a tensor's fp32 bytes. */
uint64_t oracle_digest(const float * data, size_t numel);

/* Caption projection of [B, L, caption_dim] -> context [B, L, C]. */
int oracle_model_project_caption(const oracle_model * m, const float * caption, size_t B, size_t L,
                                 float * context);
/* Time MLP for B timesteps: embedded [B,C] (pre-SiLU) and t_mod [B,6C]. */
int oracle_model_time(const oracle_model * m, const float * t, size_t B, float * embedded, float * t_mod);
/* Patch embed of NCHW latent [B, Cl, H, W] -> tokens [B, H*W, C]. */
int oracle_model_patch_embed(const oracle_model * m, const float * latent, size_t B, size_t Hh, size_t Ww,
                             float * tokens);
int oracle_model_block(const oracle_model * m, size_t block, const float * x, const float * context,
                       const float * t_mod, const float * bias, size_t B, size_t N, size_t L,
                       float * after_self, float * after_cross, float * after_ff);
/* The forward of run_full_denoising_step_with_cfg (src/transformer.cpp:627-681):
 * latent [Bl, Cl, H, W] is repeated x2, context [2Bl, L, C] (already projected),
 * bias [2Bl, L] or NULL -> noise_pred [2Bl, Cl, H, W]. */
int oracle_model_forward(const oracle_model * m, const float * latent, size_t Bl, size_t Hh, size_t Ww,
                         const float * context, size_t L, const float * bias, float t, float * noise_pred);
/* run_full_denoising_loop_with_cfg (src/transformer.cpp:692-724) with the
 * default scheduler config and `steps` steps; caption [2Bl, L, caption_dim]. */
int oracle_model_loop(const oracle_model * m, const float * latent, size_t Bl, size_t Hh, size_t Ww,
                      const float * caption, size_t L, const float * bias, size_t steps, float guidance,
                      float * final_latent);

/* Scheduler (src/scheduler.cpp).  Timesteps/sigmas of the default config. */
int oracle_scheduler_timesteps(size_t steps, float * timesteps, float * sigmas /* steps+1 */);

/* ---- DC-AE VAE decoder (src/vae.cpp, src/vae_ops.cpp), NCHW fp32 ----
 * Weights in PyTorch order (attention linears [out, in], convs [out, in, kh, kw]). */
/* 3x3 same conv.  order -1: the reference's size-dependent choice
 * (src/vae_ops.cpp:211-218); 0: im2col order (:18-95); 1: tap order (:104-194). */
int oracle_vae_conv3x3(const float * in, const float * w, const float * bias, float * out, size_t B, size_t Cin,
                       size_t Cout, size_t H, size_t W, int order);
int oracle_vae_conv1x1(const float * in, const float * w, const float * bias, float * out, size_t B, size_t Cin,
                       size_t Cout, size_t HW);
int oracle_vae_grouped_conv1x1(const float * in, const float * w, float * out, size_t B, size_t Cin, size_t Cout,
                               size_t groups, size_t HW);
int oracle_vae_dw5x5(const float * in, const float * w, const float * bias, float * out, size_t B, size_t C,
                     size_t H, size_t W);
/* Per-pixel RMSNorm over channels (eps), weight and optional bias. */
int oracle_vae_rms_norm(const float * in, const float * w, const float * bias, float * out, size_t B, size_t C,
                        size_t HW, float eps);
/* nearest 2x upsample, 3x3 conv, optional pixel-shuffled channel-repeat shortcut: out [B, Cout, 2H, 2W]. */
int oracle_vae_upsample(const float * in, const float * w, const float * bias, float * out, size_t B, size_t Cin,
                        size_t Cout, size_t H, size_t W, int shortcut);

/* Whole decoder with the synthetic weights of oracle/vae_spec.h (full = 1: the
 * Sana 1.0 DC-AE f32c32 decoder, 0: the small test decoder). */
typedef struct oracle_vae oracle_vae;
oracle_vae * oracle_vae_create(int full);
/* Any decoder shape (levels up to 8; head dim 32, expansion 4), same seeding rule. */
oracle_vae * oracle_vae_create_config(size_t latent, size_t levels, const size_t * channels, const int * attn);
void oracle_vae_destroy(oracle_vae * m);
int oracle_vae_generate(oracle_vae * m);
int oracle_vae_set(oracle_vae * m, const char * name, const float * data, size_t n);
int oracle_vae_get(const oracle_vae * m, const char * name, float * out, size_t n);
/* latent / scaling_factor -> conv_in + channel-repeat shortcut: out [B, top, H, W] */
int oracle_vae_decoder_input(const oracle_vae * m, const float * latent, size_t B, size_t H, size_t W, float * out);
/* one layer of up block `level` (ResBlock, attention, or GLUMBConv of an EfficientViT layer), NCHW in -> out */
int oracle_vae_res_block(const oracle_vae * m, size_t level, size_t layer, const float * in, float * out, size_t B,
                         size_t H, size_t W);
int oracle_vae_attention(const oracle_vae * m, size_t level, size_t layer, const float * in, float * out,
                         size_t B, size_t H, size_t W);
int oracle_vae_glumb(const oracle_vae * m, size_t level, size_t layer, const float * in, float * out, size_t B,
                     size_t H, size_t W);
/* run_vae_decode: latent [B, 32, H, W] -> image [B, 3, H * 2^(levels-1), W * 2^(levels-1)] */
int oracle_vae_decode(const oracle_vae * m, const float * latent, size_t B, size_t H, size_t W, float * image);

#ifdef __cplusplus
}
#endif
