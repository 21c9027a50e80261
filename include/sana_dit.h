/* sana_dit.h -- C ABI of the MI355X (gfx950) Sana-0.6B DiT forward.
 *
 * This is the drop-in boundary under the reference's C++ transformer API
 * (src/transformer.h:81-155).  Plain pointers and sizes only; no C++ or torch
 * types.  Host pointers are fp32 in the reference's layouts; *_device entry
 * points take device pointers and a hipStream_t passed as void*.
 *
 * Errors: every entry point returns SANA_OK (0) or a negative code; the
 * message of the last failure on the calling thread is sana_dit_last_error().
 * The C++ wrapper maps SANA_ERR_INVALID_ARGUMENT and SANA_ERR_SHAPE to
 * std::invalid_argument and the others to std::runtime_error, as the
 * reference throws them (src/transformer.cpp:500-514, :553-555, :574-579,
 * :613-624; src/weights_io.cpp:138-150, :336-354).
 *
 * Threading: a context is used by one host thread at a time; it owns a HIP
 * stream, the device weights, a workspace and cached HIP graphs.  All device
 * memory is allocated by create / weight upload / the first call at a new
 * shape, never inside a captured graph.
 */
#ifndef SANA_DIT_H
#define SANA_DIT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SANA_OK 0
#define SANA_ERR_INVALID_ARGUMENT (-1)
#define SANA_ERR_SHAPE (-2)
#define SANA_ERR_IO (-3)
#define SANA_ERR_FORMAT (-4)
#define SANA_ERR_HIP (-5)
#define SANA_ERR_OUT_OF_MEMORY (-6)
#define SANA_ERR_STATE (-7)

typedef struct sana_dit sana_dit;

typedef struct {
    int64_t layers;          /* transformer blocks (28) */
    int64_t hidden;          /* C (1152) */
    int64_t ffn;             /* expanded Mix-FFN channels E (5760 = 2 x 2880) */
    int64_t caption_dim;     /* caption feature width (2304) */
    int64_t latent_channels; /* Cl (32) */
    int64_t self_heads;      /* linear-attention heads (36 in sana_infer, src/infer_main.cpp:366) */
    int64_t cross_heads;     /* cross-attention heads (16, src/infer_main.cpp:367) */
    int device;              /* HIP device ordinal */
} sana_dit_config;

const char * sana_dit_last_error(void);

/* Replaces the model set-up of load_denoiser_weights (src/transformer.cpp:453-488). */
int sana_dit_create(const sana_dit_config * cfg, sana_dit ** out);
void sana_dit_destroy(sana_dit * ctx);

/* Upload one top-level tensor by its GGUF name (src/transformer.cpp:473-484,
 * :171-190): patch_embed.proj.*, time_embed.*, caption_projection.*,
 * caption_norm.weight, scale_shift_table, proj_out.*.  `shape` is the
 * PyTorch-order shape (GGUF ne reversed, src/weights_io.cpp:125-132).
 * transposed = 1 means a linear weight arrives as [in, out], the layout
 * load_linear_weight_tensor produces (src/weights_io.cpp:367-377). */
int sana_dit_set_weight(sana_dit * ctx, const char * name, const float * data, const int64_t * shape, int ndim,
                        int transposed);
/* Upload one tensor of block `block` by its suffix after the block prefix
 * (load_block_weights, src/transformer.cpp:214-308), e.g. "attn1.to_q.weight".
 * "attn1.to_{q,k,v}.bias" are optional (the reference loader injects zeros,
 * src/transformer.cpp:361-362; SanaBlockWeights built in memory may set them). */
int sana_dit_set_block_weight(sana_dit * ctx, int64_t block, const char * suffix, const float * data,
                              const int64_t * shape, int ndim, int transposed);
/* The linear weights run as fp16 GEMM operands: an fp32 value that fp16
 * cannot hold (|w| > 65504, inf or NaN) fails sana_dit_set_weight and
 * sana_dit_set_block_weight with SANA_ERR_FORMAT naming the tensor (the
 * reference keeps every weight in fp32, src/weights_io.cpp:340-355). */
/* The same two uploads for a linear weight given as IEEE fp16 bits, e.g. a
 * GGUF F16 payload as stored (the reference reads payloads as F32,
 * src/weights_io.cpp:325-365): the bits are copied into the fp16 operand
 * buffer with no fp32 round trip.  Only the 16-bit operand weights are
 * accepted -- attn1.to_{q,k,v,out.0}.weight, attn2.to_{q,k,v,out.0}.weight,
 * ff.conv_inverted.weight, ff.conv_point.weight and
 * caption_projection.linear_{1,2}.weight -- in their PyTorch-order shape (not
 * transposed); other names fail with SANA_ERR_INVALID_ARGUMENT, inf / NaN
 * with SANA_ERR_FORMAT. */
int sana_dit_set_weight_f16(sana_dit * ctx, const char * name, const uint16_t * data, const int64_t * shape,
                            int ndim);
int sana_dit_set_block_weight_f16(sana_dit * ctx, int64_t block, const char * suffix, const uint16_t * data,
                                  const int64_t * shape, int ndim);
/* Optional LayerNorm affine of a block (which = 0: attn norm, 1: mlp norm).
 * The reference loader injects gamma = 1, beta = 0 (src/transformer.cpp:364-398),
 * which is also the default here; NULL restores the default. */
int sana_dit_set_block_norm(sana_dit * ctx, int64_t block, int which, const float * gamma, const float * beta);
/* Checks that every tensor has been uploaded (validate_denoiser_weights,
 * src/transformer.cpp:807-884 checks the shapes; set_* already did). */
int sana_dit_check_weights(sana_dit * ctx);
/* Loads the three GGUF files of download_weights.sh (model, caption, denoiser)
 * (src/weights_io.cpp:134-164, :325-365) from a read-only mapping.  Payloads
 * may be F32, F16 or BF16 (the reference reads every payload as F32).  F16
 * linear weights are copied straight into the fp16 operand buffers
 * (sana_dit_set_*_f16); other 16-bit payloads are widened exactly to fp32 and
 * BF16 linear weights are then narrowed to fp16 under the range check above.
 * Other ggml types fail with SANA_ERR_FORMAT. */
int sana_dit_load_gguf(sana_dit * ctx, const char * model_path, const char * caption_path,
                       const char * denoiser_path);

/* Pre-packed device layouts cached on disk (the GGUF row's packed-layout
 * cache; no counterpart in the reference, which converts on every load).
 *
 * sana_dit_save_packed writes every weight of a fully loaded context, as the
 * device holds it (fp16 GEMM operands K-padded and fused, cross K/V stacked
 * over blocks, fp32 vectors), with the model dimensions, the caller's 64-bit
 * key of the source weights and a checksum per buffer.  The file appears
 * under `path` only when complete (written under a temporary name, then
 * renamed).  SANA_ERR_STATE if a weight is missing, SANA_ERR_IO on a write
 * failure.
 *
 * sana_dit_load_packed maps such a file and uploads it with one copy per
 * buffer.  The dimensions must equal the context's and `key` the saved one;
 * every buffer's size and checksum is verified before anything is uploaded,
 * so a refused image leaves the context unchanged.  SANA_ERR_IO if the file
 * cannot be opened, SANA_ERR_FORMAT for any mismatch or damage.  Set the
 * conditioning again after loading weights. */
int sana_dit_save_packed(sana_dit * ctx, const char * path, uint64_t key);
int sana_dit_load_packed(sana_dit * ctx, const char * path, uint64_t key);

/* sana_dit_load_gguf through a packed cache at cache_path: the key is derived
 * from the three GGUF files (path, size, modification time and the first MiB
 * of each).  A cache whose key, dimensions and checksums match is loaded
 * (*used_cache = 1); otherwise the GGUF files are loaded and the cache is
 * rewritten (*used_cache = 0).  Writing the cache is best effort: when it
 * fails the call still returns SANA_OK with the weights loaded.  used_cache
 * may be NULL. */
int sana_dit_load_gguf_cached(sana_dit * ctx, const char * model_path, const char * caption_path,
                              const char * denoiser_path, const char * cache_path, int * used_cache);

/* Conditioning for the following forwards.  projected = 0: data is the raw
 * caption [B, L, caption_dim] and the caption projection
 * (project_caption_context, src/transformer_ops.cpp:64-76) runs on the GPU;
 * projected = 1: data is the context [B, L, hidden].  bias is the additive
 * key mask [B, 1, L] (or NULL).  The cross-attention keys/values of all
 * blocks are computed here once, since they depend only on the context.
 * Uploading a weight they were computed from (the caption projection,
 * caption_norm, any block's attn2.to_k / attn2.to_v, or a packed image) drops
 * the conditioning: calls that need it fail with SANA_ERR_STATE until it is
 * set again.  Other weight uploads keep it. */
int sana_dit_set_context(sana_dit * ctx, const float * data, int64_t B, int64_t L, int64_t dim, int projected,
                         const float * bias);
/* Copy the projected context [B, L, hidden] (fp32 before the fp16 operand cast). */
int sana_dit_get_context(sana_dit * ctx, float * out);

/* The forward of run_full_denoising_step_with_cfg (src/transformer.cpp:627-681):
 * latent [Bl, Cl, H, W] (repeated x2 for CFG), timestep t for every batch row,
 * the context set above (batch 2*Bl) -> noise_pred [2*Bl, Cl, H, W].  H * W
 * must be a perfect square (infer_square_side, src/transformer.cpp:18-24). */
int sana_dit_forward(sana_dit * ctx, const float * latent, int64_t Bl, int64_t H, int64_t W, float t,
                     float * noise_pred);
/* Same with device pointers, asynchronous on `stream` (NULL = the context's stream). */
int sana_dit_forward_device(sana_dit * ctx, const float * d_latent, int64_t Bl, int64_t H, int64_t W, float t,
                            float * d_noise_pred, void * stream);
/* One whole step from raw inputs on the device: caption projection of
 * d_caption [2*Bl, L, caption_dim], cross K/V of all blocks, and the forward.
 * d_bias [2*Bl, L] or NULL.  Asynchronous on `stream`. */
int sana_dit_step_device(sana_dit * ctx, const float * d_caption, int64_t L, const float * d_bias,
                         const float * d_latent, int64_t Bl, int64_t H, int64_t W, float t, float * d_noise_pred,
                         void * stream);
/* block_forward (src/transformer.cpp:726-778) of one block on the context set
 * above: x [B, N, C], t_mod [B, 6C] -> the three stage outputs [B, N, C]. */
int sana_dit_block_forward(sana_dit * ctx, int64_t block, const float * x, const float * t_mod, int64_t B,
                           int64_t N, float * after_self, float * after_cross, float * after_ff);
/* run_model_blocks (src/transformer.cpp:544-568) on the context set above:
 * blocks [begin, end) applied to x [B, N, C] with t_mod [B, 6C] -> out [B, N, C]. */
int sana_dit_run_blocks(sana_dit * ctx, int64_t begin, int64_t end, const float * x, const float * t_mod, int64_t B,
                        int64_t N, float * out);
/* run_full_denoising_loop_with_cfg (src/transformer.cpp:692-724) with the
 * default scheduler (DPM-Solver++ order 2, midpoint, flow sigmas,
 * lower_order_final; src/scheduler.cpp:272-318) entirely on the device: per
 * step one forward at timesteps[i], classifier-free guidance (uncond = first
 * half of the context batch) and the solver update, fused.  timesteps [steps]
 * and sigmas [steps + 1] are the schedule of build_sana_scheduler_timesteps;
 * the context (caption projection and cross K/V) must be set.  latent and
 * final_latent are [Bl, Cl, H, W]. */
int sana_dit_denoise_loop(sana_dit * ctx, const float * latent, int64_t Bl, int64_t H, int64_t W,
                          const float * timesteps, const float * sigmas, int64_t steps, float guidance,
                          float * final_latent);
/* Same with device latent pointers, asynchronous on `stream` (timesteps and sigmas stay host arrays). */
int sana_dit_denoise_loop_device(sana_dit * ctx, const float * d_latent, int64_t Bl, int64_t H, int64_t W,
                                 const float * timesteps, const float * sigmas, int64_t steps, float guidance,
                                 float * d_final_latent, void * stream);
/* The converted model outputs (x0 = sample - sigma * guided prediction) of the
 * last two steps of the last denoise loop on this context, [Bl, Cl, H, W]
 * each: the previous_model_outputs a host scheduler state holds after the loop
 * (src/scheduler.cpp:286-290).  x0_prev is left untouched after a one-step loop.
 * The copies wait for the loop's last step on whatever stream the loop was
 * queued on, then return (blocking). */
int sana_dit_loop_model_outputs(sana_dit * ctx, float * x0_prev, float * x0_last);
/* Time MLP of the forward (src/transformer.cpp:638-656): B timesteps ->
 * embedded [B, C] (pre-SiLU) and t_mod [B, 6C]. */
int sana_dit_time_embed(sana_dit * ctx, const float * t, int64_t B, float * embedded, float * t_mod);
/* Measurement hook (no counterpart in the reference): average duration (ms)
 * over `iters` back-to-back eager launches of one kernel of the blocks, launched
 * exactly as the last forward launched it -- the same kernel instantiation and
 * shape (one batch row of a CFG pair per launch when the forward ran the pair as
 * two branches), on the forward's own buffers, which it overwrites.  Launch i
 * uses block i mod layers, so weights stream from HBM as in the forward.
 * which: 0 QKV GEMM, 1 attn-out GEMM (+ gated residual), 2 cross-q GEMM,
 * 3 cross-out GEMM (+ residual), 4 FFN inverted GEMM (+ SiLU), 5 FFN point GEMM
 * (+ gated residual), 6 LayerNorm + modulate, 7 linear attention, 8 cross
 * attention, 9 depthwise 3x3 + GLU.  Also returns the launch's algorithmic
 * flops (contractions) and bytes (interface tensors at their stored precision,
 * GEMM weights included, no re-reads), and in `name` (when not NULL, up to
 * name_cap bytes with the terminating 0) the launched kernel as rocprofv3
 * names it.  Needs a context and a forward. */
int sana_dit_time_kernel(sana_dit * ctx, int which, int iters, float * avg_ms, double * flops, double * bytes,
                         char * name, size_t name_cap);

/* ---- DC-AE VAE decoder: latent -> RGB (src/vae.h:11-92, src/vae.cpp) ----
 * Levels are indexed as the reference's decoder.up_blocks.{i} (level 0 = the
 * output resolution, the last level = the latent resolution, processed
 * first).  Every level holds three ResBlocks or three EfficientViT layers
 * (multiscale ReLU linear attention + GLUMBConv); every level but the last
 * starts with a nearest-2x upsample conv with a pixel-shuffled shortcut.
 * Channel counts must be multiples of 64 (<= 1024), head_dim 32. */
#define SANA_VAE_MAX_LEVELS 8
typedef struct sana_vae sana_vae;
typedef struct {
    int64_t latent_channels;                 /* 32 */
    int64_t levels;                          /* up blocks, <= SANA_VAE_MAX_LEVELS */
    int64_t channels[SANA_VAE_MAX_LEVELS];   /* per level */
    int32_t attention[SANA_VAE_MAX_LEVELS];  /* 1: EfficientViT layers, 0: ResBlocks */
    int64_t head_dim;                        /* 32 */
    int64_t expand;                          /* GLUMBConv expansion (hidden = expand * C) */
    float scaling_factor;                    /* SanaVaeWeights::scaling_factor, 0.41407 */
    int device;
} sana_vae_config;
int sana_vae_create(const sana_vae_config * cfg, sana_vae ** out);
int sana_vae_destroy(sana_vae * vae);
/* One tensor by its GGUF name and PyTorch-order shape (the names and shapes
 * load_vae_weights reads, src/vae.cpp:10-118,140-167; attention linears
 * [out, in]).  fp32 host data; converted and laid out for the device. */
int sana_vae_set_weight(sana_vae * vae, const char * name, const float * data, const int64_t * shape, int ndim);
/* SANA_ERR_STATE naming the first missing tensor, else SANA_OK. */
int sana_vae_check_weights(sana_vae * vae);
/* All tensors from one GGUF (F32, F16 or BF16 payloads). */
int sana_vae_load_gguf(sana_vae * vae, const char * path);
/* run_vae_decode (src/vae.cpp:243-325): latent [B, Cl, H, W] fp32 ->
 * image [B, 3, H * 2^(levels-1), W * 2^(levels-1)] fp32.  Host pointers. */
int sana_vae_decode(sana_vae * vae, const float * latent, int64_t B, int64_t H, int64_t W, float * image);
/* run_vae_decoder_input (src/vae.cpp:211-241): conv_in of latent [B, Cl, H, W]
 * (no scaling), plus the channel-repeat shortcut when in_shortcut != 0 ->
 * out [B, C_top, H, W] fp32.  Needs only the conv_in tensors.  Host pointers. */
int sana_vae_decoder_input(sana_vae * vae, const float * latent, int64_t B, int64_t H, int64_t W, int in_shortcut,
                           float * out);
/* Same on device pointers, asynchronous on `stream`. */
int sana_vae_decode_device(sana_vae * vae, const float * latent, int64_t B, int64_t H, int64_t W, float * image,
                           void * stream);

/* ---- Gemma-2 text encoder (the stage before the denoiser) ----
 * The decoder forward that src/gemma_encoder.cpp:95-152 runs through
 * llama.cpp in embeddings mode: token ids in, the per-token hidden states
 * after the final RMSNorm out.  Causal attention with grouped kv heads, NeoX
 * RoPE, logit soft-cap, a sliding window on the even layers, GELU-tanh gated
 * FFN, pre- and post-norms.  Sizes: hidden, head_dim and ffn multiples of 64
 * (hidden <= 4096), heads a multiple of kv_heads, up to 8192 tokens. */
typedef struct sana_gemma sana_gemma;
typedef struct {
    int64_t vocab, hidden, layers, heads, kv_heads, head_dim, ffn;  /* Gemma-2 2B: 256000 2304 26 8 4 256 9216 */
    int64_t sliding_window;                                           /* 4096; 0 = none */
    float rms_eps;                                                    /* 1e-6 */
    float rope_theta;                                                 /* 10000 */
    float attn_softcap;                                               /* 50 */
    float query_scale;                                                /* 1 / sqrt(head_dim) */
    int device;
} sana_gemma_config;
int sana_gemma_create(const sana_gemma_config * cfg, sana_gemma ** out);
int sana_gemma_destroy(sana_gemma * g);
/* One tensor by its GGUF name (token_embd, output_norm, blk.N.{attn_norm,
 * attn_q, attn_k, attn_v, attn_output, post_attention_norm, ffn_norm,
 * ffn_gate, ffn_up, ffn_down, post_ffw_norm}.weight) and PyTorch-order shape.
 * RMSNorm weights as the GGUF stores them (1 + w). fp32 host data. */
int sana_gemma_set_weight(sana_gemma * g, const char * name, const float * data, const int64_t * shape, int ndim);
/* SANA_ERR_STATE naming the first missing tensor, else SANA_OK. */
int sana_gemma_check_weights(sana_gemma * g);
/* All tensors from one GGUF (F32, F16 or BF16 payloads). */
int sana_gemma_load_gguf(sana_gemma * g, const char * path);
/* tokens [n] -> hidden [n, hidden] fp32 (host pointers). */
int sana_gemma_encode(sana_gemma * g, const int32_t * tokens, int64_t n, float * hidden);
/* Two independent sequences in one pass, as encode_prompt_pair
 * (src/gemma_encoder.cpp) needs for the prompt and the negative prompt: their
 * rows share the per-token kernels, attention stays within each sequence.
 * hidden_a / hidden_b equal what two sana_gemma_encode calls return, bit for
 * bit.  Each sequence up to 8192 tokens, na + nb <= 16384. */
int sana_gemma_encode_pair(sana_gemma * g, const int32_t * tokens_a, int64_t na, const int32_t * tokens_b,
                           int64_t nb, float * hidden_a, float * hidden_b);

/* Measured MFMA ceiling for roofline reports (no counterpart in the reference):
 * `workgroups` x 256 threads (4 waves) run `iters` steps of 8 independent fp16
 * v_mfma_f32_32x32x16 accumulators per wave (4 A x 2 B register fragments) with
 * no memory traffic, asynchronously on `stream`; `sink` (device, workgroups *
 * 256 floats) receives the sums; *flops is the work of the launch.  Operands
 * are fp16 values spread over [-1, 1) (as random weights are), or all zero
 * when `zero_operands` is nonzero: the part is power limited, and zeros run
 * faster.  The caller times it (e.g. with events); 1024 workgroups (4 waves
 * per SIMD) give the peak. */
int sana_hip_mfma_peak(int64_t workgroups, int64_t iters, int zero_operands, float * sink, void * stream,
                       double * flops);
/* Measured HBM ceiling (no counterpart in the reference): streams `bytes` (a
 * multiple of 16) from device buffer src into dst (copy: bytes read + bytes
 * written) or, with dst NULL, into per-thread sums in sink (read only; sink
 * holds *sink_floats floats, returned when sink is NULL and dst is NULL with
 * bytes 0).  Asynchronous on `stream`; the caller times it.  Use buffers far
 * larger than the 256 MB last-level cache. */
int sana_hip_hbm_peak(const void * src, void * dst, int64_t bytes, float * sink, int64_t * sink_floats,
                      void * stream);

/* torch.randn(shape, generator seeded with `seed`) on the CPU generator, into
 * out[0 .. n) (n >= 16; row-major over the shape): the seeded normals of
 * randn_torch_cpu (src/torch_rng.h:14, src/torch_rng.cpp:14-68), which
 * sana_infer uses for the initial latent.  Host only, no GPU needed. */
int sana_randn_torch_cpu(float * out, int64_t n, uint64_t seed);

/* GGUF index inspection (no GPU needed): number of tensors, and the name,
 * PyTorch-order shape (up to 4 dims), ggml type and absolute payload offset of
 * tensor i -- the fields load_gguf_weight_index records (src/weights_io.cpp:152-158). */
int sana_gguf_num_tensors(const char * path, int64_t * n);
int sana_gguf_tensor_info(const char * path, int64_t i, char * name, size_t name_cap, int64_t * shape, int * ndim,
                          int * type, uint64_t * offset);

/* ---- kernel-level launchers on device pointers (unit tests, op-level API) ---- */
/* out = act(A . W^T + bias): A fp16 [M, lda], W fp16 [N, ldw], K % 64 == 0;
 * act 0 none, 1 SiLU, 2 GELU-tanh, 3 gated pairs: W rows interleaved as
 * (gate, up), out16[m, n / 2] = gelu_tanh(gate) * up for even n (fp16 out only). */
int sana_hip_gemm(const void * A, int64_t lda, const void * W, int64_t ldw, int64_t M, int64_t N, int64_t K,
                  const float * bias, int act, void * out16, int64_t ldo16, float * out32, int64_t ldo32,
                  void * stream);
/* x[m, n] += gate(m, n) * (A . W^T + bias)[m, n]; gate = gate_a[(m / rows_per_batch) * gate_stride + n]
 * + gate_t[n] (gate_a NULL: gate 1); optional fp16 copy of the new x. */
int sana_hip_gemm_residual(const void * A, int64_t lda, const void * W, int64_t ldw, int64_t M, int64_t N,
                           int64_t K, const float * bias, const float * gate_a, const float * gate_t,
                           int64_t gate_stride, int64_t rows_per_batch, float * x, int64_t ldx, void * out16,
                           int64_t ldo16, void * stream);
int sana_hip_ln_modulate(const float * x, int64_t ldx, void * out16, int64_t ldo, int64_t M, int64_t C,
                         int64_t rows_per_batch, float eps, const float * gamma, const float * beta,
                         const float * mod_a, const float * mod_t, int64_t mod_stride, int64_t shift_off,
                         int64_t scale_off, void * stream);
/* ReLU linear attention (linear_attention_4d, src/transformer_ops.cpp:496-537)
 * on fp16 token-major q / k / v [B*N, ld] (head h at columns h*D..), out fp16
 * [B*N, ldo]; D <= 112, B * H <= 65535; workspace of
 * sana_hip_linear_attention_workspace(B, N, H, D) bytes. */
int sana_hip_linear_attention(const void * q, const void * k, const void * v, int64_t ld, void * out, int64_t ldo,
                              int64_t B, int64_t N, int64_t H, int64_t D, float * workspace, void * stream);
size_t sana_hip_linear_attention_workspace(int64_t B, int64_t N, int64_t H, int64_t D);
/* sana_hip_linear_attention without allocation or workspace argument.  No
 * counterpart in the reference: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The workspace is a static 16 MiB device array, one per GPU, kept
 * until the process ends; calls whose sana_hip_linear_attention_workspace size
 * exceeds it fail with SANA_ERR_INVALID_ARGUMENT (B=2, H=16, D=72 needs 11.7 MB
 * at any N).  Every call on a GPU shares that GPU's array: calls that overlap
 * on one GPU (two streams, two threads) race.  Runs on the current device; the
 * stream must belong to it.  Results equal sana_hip_linear_attention's.  The
 * array's device address is looked up once per device, on the first call; after
 * a hipDeviceReset the code object (and the array) is loaded anew, so this
 * entry point must not be called across a device reset in one process. */
int sana_hip_linear_attention_noalloc(const void * q, const void * k, const void * v, int64_t ld, void * out,
                                      int64_t ldo, int64_t B, int64_t N, int64_t H, int64_t D, void * stream);
int sana_hip_cross_attention(const void * q, int64_t ldq, const void * k, int64_t ldk, const void * vt,
                             int64_t ldvt, const float * bias, void * out, int64_t ldo, int64_t B, int64_t N,
                             int64_t L, int64_t H, int64_t D, void * stream);
int sana_hip_dwconv_glu(const void * x, int64_t ldx, const float * w_tapmajor, const float * bias, void * out,
                        int64_t ldo, int64_t B, int64_t H, int64_t W, int64_t F, void * stream);

/* ---- fp32 op launchers on device pointers: the op-level API of the drop-in
 * (src/common_ops.h:5-49, src/transformer_ops.h:5-50).  fp32 in, fp32 out, in
 * the reference's layouts; asynchronous on `stream`. ---- */
#define SANA_OP_SILU 0
#define SANA_OP_GELU_TANH 1
#define SANA_OP_RELU 2
/* C[z] (+)= A[z] . op(B[z]) + bias for z < batch (gemm_row_major,
 * src/common_ops.cpp:13-65, and its batched uses).  A [M, K] (lda), B [K, N]
 * (ldb) or, with b_transposed, [N, K]; bias_mode 1: bias[N] per column,
 * 2: bias[M] per row; accumulate = 1 adds into C (gemm_accumulate_row_major). */
int sana_op_gemm_f32(const float * A, int64_t lda, int64_t strideA, const float * B, int64_t ldb, int64_t strideB,
                     int b_transposed, const float * bias, int bias_mode, float * C, int64_t ldc, int64_t strideC,
                     int64_t M, int64_t N, int64_t K, int64_t batch, int accumulate, void * stream);
/* y = op(x) elementwise: SANA_OP_SILU, SANA_OP_GELU_TANH, SANA_OP_RELU. */
int sana_op_unary_f32(const float * x, float * y, int64_t n, int op, void * stream);
/* Row softmax of x * scale (+ bias[(row / bias_div) * cols + col]) (softmax_lastdim_4d
 * and attention_4d, src/transformer_ops.cpp:280-392). */
int sana_op_softmax_f32(const float * x, float * y, int64_t rows, int64_t cols, float scale, const float * bias,
                        int64_t bias_div, void * stream);
/* RMSNorm over rows (rms_norm_3d_lastdim, src/tensor.cpp:276-316); w may be NULL. */
int sana_op_rms_norm_f32(const float * x, const float * w, float * y, int64_t rows, int64_t cols, float eps,
                         void * stream);
/* Depthwise ksize x ksize (3 or 5) convolution, zero padding, NCHW
 * (depthwise_conv2d_3x3 / _5x5, src/common_ops.cpp:483-572, :576-718); bias may be NULL. */
int sana_op_dwconv_f32(const float * x, const float * w, const float * bias, float * y, int64_t B, int64_t C,
                       int64_t H, int64_t W, int64_t ksize, void * stream);
/* GLU of the split channels of x [B, 2F, S]: y = data * silu(gate) (glumb_conv,
 * src/common_ops.cpp:744-756). */
int sana_op_glu_f32(const float * x, float * y, int64_t B, int64_t F, int64_t S, void * stream);
/* linear_attention_4d (src/transformer_ops.cpp:402-543) on [BH, N, D] q / k / v;
 * state is a workspace of BH * (D + 1) * D floats. */
int sana_op_linear_attention_f32(const float * q, const float * k, const float * v, float * out, int64_t BH,
                                 int64_t Nq, int64_t Nk, int64_t D, float * state, void * stream);
/* split = 1: [B, N, H*D] -> [B, H, N, D] (split_heads_3d); split = 0: the
 * inverse (merge_heads_4d), src/transformer_ops.cpp:83-171. */
int sana_op_heads_f32(const float * x, float * y, int64_t B, int64_t N, int64_t H, int64_t D, int split,
                      void * stream);

#ifdef __cplusplus
}
#endif

#endif /* SANA_DIT_H */
