// Device model and C ABI of the Sana DiT forward on one MI355X.
//
// HBM layout (all device-resident after upload):
//   weights   fp16 [out, in] rows padded to a multiple of 64 in K (zeros), the
//             MFMA "TN" operand; attn1 q|k|v fused into one [3C, C] matrix;
//             attn2 k / v of all blocks stacked into [layers*C, C] each so the
//             step-invariant cross K/V of the whole model is two large GEMMs;
//             biases, adaLN tables, depthwise taps (tap-major [9][E]) and the
//             small time/patch/proj_out weights in fp32.
//   residual  fp32 [B*N, C] (token-major, the reference's [B, N, C]); every
//             GEMM A operand is an fp16 token-major copy with padded row stride.
//   context   fp16 [B*L, C]; cross K fp16 [B*L, layers*C]; cross V^T fp16
//             [layers][B][C][Lp] (keys contiguous for the P.V MFMA operand).
// No layout transposes remain: tokens_to_grid/grid_to_tokens/split_heads/
// merge_heads of the reference are address arithmetic here, and the CFG
// batch repeat is two batch rows reading the same latent.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/sana_dit.h"
#include "host_util.h"
#include "kernels.h"

using sana::half_t;

namespace {

using namespace sana_host;

struct BlockDev {
    DevMem w_qkv, b_qkv, w_out, b_out, w_cq, b_cq, w_co, b_co, w_inv, b_inv, w_dw, b_dw, w_pt;
    DevMem ln1_g, ln1_b, ln2_g, ln2_b;
    bool has_ln1 = false, has_ln2 = false;
    bool has_qkv_bias = false;  // attn1 q/k/v biases (zero in every checkpoint the loader reads)
};

__global__ void fill_kernel(float * p, int n, float v) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// Classifier-free guidance and one DPM-Solver++ update, fused, per latent element:
//   v  = u + g (c - u)                       (apply_classifier_free_guidance, src/transformer.cpp:586-598)
//   x0 = x - sigma_s v                        (convert_sana_scheduler_model_output, src/scheduler.cpp:155-173)
//   first order : x' = ca x + cb x0           (src/scheduler.cpp:175-205)
//   second order: x' = ca x + cb x0 + cc (x0 - x0_prev) / r0   (midpoint, :207-260)
// noise_pred holds the uncond half first, then the cond half (batch order of the context).
__global__ void cfg_dpm_kernel(const float * __restrict__ np, const float * __restrict__ x,
                               const float * __restrict__ x0_prev, float * __restrict__ x_out,
                               float * __restrict__ x0_out, int n, float g, float sigma_s, float ca, float cb, float cc,
                               float inv_r0, int second) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float u = np[i], c = np[n + i];
    const float v = u + g * (c - u);
    const float xi = x[i];
    const float x0 = xi - sigma_s * v;
    float out = ca * xi + cb * x0;
    if (second) out = ca * xi + cb * x0 + cc * (inv_r0 * (x0 - x0_prev[i]));
    x_out[i] = out;
    x0_out[i] = x0;
}

struct GraphEntry {
    hipGraphExec_t exec = nullptr;
};

}  // namespace

namespace sana {
void set_last_error(const std::string & m) { g_last_error = m; }
namespace {
thread_local const char * g_last_kernel = "";
}
void note_kernel(const char * name) { g_last_kernel = name; }
const char * last_kernel() { return g_last_kernel; }
}  // namespace sana

struct sana_dit {
    sana_dit_config cfg{};
    int64_t C = 0, E = 0, F = 0, Ccap = 0, Cl = 0, L_ = 0, Hs = 0, Hc = 0, Ds = 0, Dc = 0;
    int64_t Cp = 0, Fp = 0, Ccap_p = 0;  // K-padded row strides of GEMM operands
    hipStream_t stream = nullptr;
    // second branch of a CFG-split forward (the conditional batch row) and
    // its fork / join events; same (default) priority as `stream`
    hipStream_t stream2 = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
    hipEvent_t ev_head_fork = nullptr, ev_head_join = nullptr;  // forward head beside the step's context
    hipEvent_t ev_ctx = nullptr;                                 // context rows ready (cross V^T on stream2)
    // recorded on the stream of the last denoise loop after its last step, so
    // sana_dit_loop_model_outputs reads loop_x0 only once the loop has written it
    hipEvent_t ev_loop = nullptr;
    std::vector<std::unique_ptr<BlockDev>> blocks;
    DevMem w_k_all, b_k_all, w_v_all, b_v_all, sst_all;  // stacked over blocks
    DevMem w_cap1, b_cap1, w_cap2, b_cap2, cap_norm;
    DevMem w_patch_t, b_patch, w_t1, b_t1, w_t2, b_t2, w_tp, b_tp, sst_final, w_proj, b_proj, freq;
    std::map<std::string, int> have;  // uploaded tensor names
    // context
    int64_t ctx_B = 0, ctx_L = 0, ctx_Lp = 0;
    bool ctx_ready = false, ctx_bias = false;
    DevMem cap32, cap16, caph16, capf32, ctx32, ctx16, kc, vt, bias;
    // forward workspace
    int64_t ws_M = 0, ws_B = 0;
    DevMem la_kt, la_vt;  // relu(K)^T and V^T per channel, token-contiguous (fused linear attention)
    DevMem x32, fin32, xa16, qkv16, o16, r16, q16, hid16, glu16, la_ws, la_ws2, d_t, e1, emb, tmod, mod_all,
        lat_in, np_out;
    DevMem loop_lat[2], loop_x0[2];  // denoise loop: latent ping-pong and converted-output history
    // graphs keyed by (kind, Bl, H, W, L, pointers)
    std::map<std::tuple<int, int64_t, int64_t, int64_t, int64_t, const void *, const void *, const void *, const void *>,
             GraphEntry>
        graphs;
    // whole denoise loops, keyed by shape, buffers and schedule (a few kept)
    std::map<std::string, GraphEntry> loop_graphs;
    int64_t last_M = 0, last_B = 0, last_N = 0;
    int64_t loop_steps = 0, loop_n = 0;  // shape of the last denoise loop (its converted outputs stay in loop_x0)
    // Execution switches, read from the environment once by sana_dit_create:
    // SANA_DIT_CFG_BRANCHES=0 runs the CFG pair as one chain, SANA_DIT_NO_GRAPH=1
    // launches the forward's kernels directly instead of replaying a graph.
    bool cfg_branches = true, use_graphs = true;

    ~sana_dit() {
        for (auto & kv : graphs)
            if (kv.second.exec) (void)hipGraphExecDestroy(kv.second.exec);
        for (auto & kv : loop_graphs)
            if (kv.second.exec) (void)hipGraphExecDestroy(kv.second.exec);
        if (ev_fork) (void)hipEventDestroy(ev_fork);
        if (ev_join) (void)hipEventDestroy(ev_join);
        if (ev_head_fork) (void)hipEventDestroy(ev_head_fork);
        if (ev_head_join) (void)hipEventDestroy(ev_head_join);
        if (ev_ctx) (void)hipEventDestroy(ev_ctx);
        if (ev_loop) (void)hipEventDestroy(ev_loop);
        if (stream2) (void)hipStreamDestroy(stream2);
        if (stream) (void)hipStreamDestroy(stream);
    }
};

namespace {

void drop_loop_graphs(sana_dit * c) {
    for (auto & kv : c->loop_graphs)
        if (kv.second.exec) (void)hipGraphExecDestroy(kv.second.exec);
    c->loop_graphs.clear();
}

void drop_graphs(sana_dit * c) {
    for (auto & kv : c->graphs)
        if (kv.second.exec) (void)hipGraphExecDestroy(kv.second.exec);
    c->graphs.clear();
    drop_loop_graphs(c);
}

// A weight upload: the captured graphs go, and so does the conditioning when
// the weight is one it was computed from (caption projection, caption_norm,
// cross-attention k / v): the next forward then needs sana_dit_set_context
// again instead of running on stale cross K/V.
void weights_changed(sana_dit * c, bool conditioning) {
    drop_graphs(c);
    if (conditioning) c->ctx_ready = false;
}

bool conditioning_weight(const std::string & name) {
    return name.rfind("caption_projection.", 0) == 0 || name == "caption_norm.weight";
}

bool conditioning_block_weight(const std::string & suffix) {
    return suffix.rfind("attn2.to_k.", 0) == 0 || suffix.rfind("attn2.to_v.", 0) == 0;
}

// Host fp32 -> device fp16 [rows, ld] with zero padding; src is [rows, cols]
// (or [cols, rows] when transposed).  A value fp16 cannot hold is refused
// (SANA_ERR_FORMAT naming `tensor`) before anything is copied.
void upload_f16(DevMem & dst, const float * src, int64_t rows, int64_t cols, int64_t ld, bool transposed,
                const std::string & tensor, int64_t row_offset = 0, int64_t total_rows = -1) {
    if (total_rows < 0) total_rows = rows;
    std::vector<half_t> h((size_t)rows * ld, (half_t)0.0f);
    // rows converted on several host threads (a 28-block model is 600M values);
    // the lowest source index fp16 cannot hold is reported
    std::atomic<size_t> bad(SIZE_MAX);
    host_parallel((size_t)rows, 16, [&](size_t r0, size_t r1) {
        for (size_t r = r0; r < r1; ++r)
            for (int64_t c = 0; c < cols; ++c) {
                const size_t i = transposed ? (size_t)(c * rows + (int64_t)r) : r * (size_t)cols + (size_t)c;
                const float v = src[i];
                if (!(v <= kF16Max && v >= -kF16Max)) {
                    atomic_min(bad, i);
                    continue;
                }
                h[r * (size_t)ld + (size_t)c] = (half_t)v;
            }
    });
    if (bad.load() != SIZE_MAX) (void)to_f16_checked(src[bad.load()], tensor, bad.load());  // throws
    if (!dst.p) dst.ensure((size_t)total_rows * ld * sizeof(half_t));
    copy_to_device(dst.as<half_t>() + (size_t)row_offset * ld, h.data(), h.size() * sizeof(half_t), "upload");
}

// Host fp16 bits [rows, cols] -> device fp16 [rows, ld]: one copy straight
// from `src` (e.g. a mapped GGUF F16 payload) when ld == cols, else a padded
// staging copy.  Non-finite values are refused.
void upload_f16_bits(DevMem & dst, const uint16_t * src, int64_t rows, int64_t cols, int64_t ld,
                     const std::string & tensor, int64_t row_offset = 0, int64_t total_rows = -1) {
    if (total_rows < 0) total_rows = rows;
    check_f16_bits_finite(src, (size_t)rows * cols, tensor);
    if (!dst.p) dst.ensure((size_t)total_rows * ld * sizeof(half_t));
    half_t * d = dst.as<half_t>() + (size_t)row_offset * ld;
    if (ld == cols) {
        copy_to_device(d, src, (size_t)rows * cols * 2, "upload");
        return;
    }
    std::vector<uint16_t> h((size_t)rows * ld, 0);
    for (int64_t r = 0; r < rows; ++r) std::memcpy(&h[(size_t)r * ld], src + (size_t)r * cols, (size_t)cols * 2);
    copy_to_device(d, h.data(), h.size() * 2, "upload");
}

void upload_f32(DevMem & dst, const float * src, size_t n, size_t offset = 0, size_t total = 0) {
    if (!dst.p) dst.ensure((total ? total : n) * sizeof(float));
    copy_to_device(dst.as<float>() + offset, src, n * sizeof(float), "upload");
}

void upload_f32_transposed(DevMem & dst, const float * src, int64_t rows, int64_t cols, bool src_transposed) {
    // dst = [rows, cols] row-major where src is [rows, cols] (or [cols, rows] if src_transposed)
    std::vector<float> h((size_t)rows * cols);
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c) h[(size_t)r * cols + c] = src_transposed ? src[c * rows + r] : src[r * cols + c];
    upload_f32(dst, h.data(), h.size());
}

void expect_shape(const char * name, const int64_t * shape, int ndim, std::vector<int64_t> want) {
    bool ok = ndim == (int)want.size();
    for (int i = 0; ok && i < ndim; ++i) ok = shape[i] == want[i];
    if (!ok) {
        std::string got, exp;
        for (int i = 0; i < ndim; ++i) got += (i ? "," : "") + std::to_string(shape[i]);
        for (size_t i = 0; i < want.size(); ++i) exp += (i ? "," : "") + std::to_string(want[i]);
        throw_err(SANA_ERR_SHAPE, std::string(name) + ": shape [" + got + "] expected [" + exp + "]");
    }
}

// ---------------------------------------------------------------- forward pieces
// The fused q | k | v projection of the linear-attention path (kGemmQKV):
// relu(q) token-major into qkv16 (ld 3C), relu(K)^T and V^T into la_kt / la_vt.
void gemm_qkv_split(sana_dit * c, BlockDev & w, int64_t B, int64_t N, const half_t * xa16, half_t * qkv16,
                    half_t * kt16, half_t * vt16, int co, hipStream_t s) {
    sana::GemmParams p;
    p.co = co;
    p.A = xa16;
    p.lda = c->Cp;
    p.W = w.w_qkv.as<half_t>();
    p.ldw = c->Cp;
    p.M = (int)(B * N);
    p.N = (int)(3 * c->C);
    p.K = (int)c->Cp;
    p.bias = w.has_qkv_bias ? w.b_qkv.as<float>() : nullptr;
    p.mode = sana::kGemmQKV;
    p.out16 = qkv16;
    p.ldo16 = 3 * c->C;
    p.kt16 = kt16;
    p.vt16 = vt16;
    p.qkv_c = (int)c->C;
    p.qkv_n = (int)N;
    launch_check(sana::gemm(p, s), "gemm_qkv");
}

// Whether the self attention runs as kGemmQKV + one fused linear-attention kernel.
// The fused linear attention rebuilds each head's state in every workgroup
// that shares the head, which stops paying off on long sequences: at 16384
// tokens per image the chunked path (chunk states, then reduction and apply;
// then three kernels) made the 4096 px forward 2 ms faster (57.9 against
// 59.9 ms), at 4096 tokens they tie.
constexpr int64_t kLaFusedMaxTokens = 8192;

bool fused_linear_attention(const sana_dit * c, int64_t N) {
    return sana::linear_attention_fused_ok((int)N, (int)c->Ds) && c->C % 8 == 0 && N <= kLaFusedMaxTokens;
}

// Whether the q | k | v projection writes the kGemmQKV layouts: head_dim 32,
// for the fused kernel up to kLaFusedMaxTokens and the chunked path from
// relu(K)^T / V^T beyond (at 16384 tokens per branch 55 us against 80 us for
// the token-major three-kernel path, when both were three kernels).
bool qkv_split_layout(const sana_dit * c, int64_t N) {
    return sana::linear_attention_fused_ok((int)N, (int)c->Ds) && c->C % 8 == 0;
}

void gemm_store(sana_dit * c, const half_t * A, int64_t lda, const half_t * W, int64_t ldw, int64_t M, int64_t N,
                int64_t K, const float * bias, int act, half_t * o16, int64_t ldo16, float * o32, int64_t ldo32,
                hipStream_t s, int co = 1) {
    sana::GemmParams p;
    p.co = co;
    p.A = A;
    p.lda = lda;
    p.W = W;
    p.ldw = ldw;
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    p.bias = bias;
    p.mode = sana::kGemmStore;
    p.act = act;
    p.out16 = o16;
    p.ldo16 = ldo16;
    p.out32 = o32;
    p.ldo32 = ldo32;
    (void)c;
    launch_check(sana::gemm(p, s), "gemm");
}

void gemm_resid(const half_t * A, int64_t lda, const half_t * W, int64_t ldw, int64_t M, int64_t N, int64_t K,
                const float * bias, const float * gate_a, const float * gate_t, int64_t gate_stride, int64_t rpb,
                float * x, int64_t ldx, half_t * o16, int64_t ldo16, hipStream_t s, int co = 1) {
    sana::GemmParams p;
    p.co = co;
    p.A = A;
    p.lda = lda;
    p.W = W;
    p.ldw = ldw;
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    p.bias = bias;
    p.mode = sana::kGemmResidual;
    p.gate_a = gate_a;
    p.gate_t = gate_t;
    p.gate_stride = gate_stride;
    p.rows_per_batch = (int)rpb;
    p.out32 = x;
    p.ldo32 = ldx;
    p.out16 = o16;
    p.ldo16 = ldo16;
    launch_check(sana::gemm(p, s), "gemm_residual");
}

void ensure_context_buffers(sana_dit * c, int64_t B, int64_t L) {
    const int64_t Lp = round_up(L, 32);
    if (B * L > c->ctx_B * c->ctx_L || Lp > c->ctx_Lp || B != c->ctx_B) {
        drop_graphs(c);
        c->cap32.ensure((size_t)B * L * c->Ccap * 4);
        c->cap16.ensure((size_t)B * L * c->Ccap_p * 2);
        c->caph16.ensure((size_t)B * L * c->Cp * 2);
        c->capf32.ensure((size_t)B * L * c->C * 4);
        c->ctx32.ensure((size_t)B * L * c->C * 4);
        c->ctx16.ensure((size_t)B * L * c->Cp * 2);
        c->kc.ensure((size_t)B * L * c->L_ * c->C * 2);
        c->vt.ensure((size_t)c->L_ * B * c->C * Lp * 2);  // zero: key padding must read as 0
        c->bias.ensure((size_t)B * L * 4);
        c->ctx_Lp = Lp;
    }
    c->ctx_B = B;
    c->ctx_L = L;
}

// Caption projection (optional): the normalized fp16 context rows.
void enqueue_context_rows(sana_dit * c, const float * caption, bool projected, int64_t B, int64_t L, hipStream_t s) {
    const int64_t R = B * L, C = c->C;
    if (!projected) {
        launch_check(sana::to_f16_padded(caption, (int)R, (int)c->Ccap, c->cap16.as<half_t>(), c->Ccap_p, s), "to_f16");
        gemm_store(c, c->cap16.as<half_t>(), c->Ccap_p, c->w_cap1.as<half_t>(), c->Ccap_p, R, C, c->Ccap_p,
                   c->b_cap1.as<float>(), sana::kActGelu, c->caph16.as<half_t>(), c->Cp, nullptr, 0, s);
        gemm_store(c, c->caph16.as<half_t>(), c->Cp, c->w_cap2.as<half_t>(), c->Cp, R, C, c->Cp, c->b_cap2.as<float>(),
                   sana::kActNone, nullptr, 0, c->capf32.as<float>(), C, s);
        launch_check(sana::rms_norm_f16(c->capf32.as<float>(), C, c->cap_norm.as<float>(), c->ctx16.as<half_t>(),
                                        c->Cp, c->ctx32.as<float>(), (int)R, (int)C, 1e-5f, s),
                     "rms_norm");
    } else {
        launch_check(sana::to_f16_padded(caption, (int)R, (int)C, c->ctx16.as<half_t>(), c->Cp, s), "to_f16");
    }
}

// Cross K of all blocks: [B*L, layers*C].
void enqueue_context_k(sana_dit * c, int64_t B, int64_t L, hipStream_t s) {
    const int64_t R = B * L, C = c->C;
    gemm_store(c, c->ctx16.as<half_t>(), c->Cp, c->w_k_all.as<half_t>(), c->Cp, R, c->L_ * C, c->Cp,
               c->b_k_all.as<float>(), sana::kActNone, c->kc.as<half_t>(), c->L_ * C, nullptr, 0, s);
}

// Cross V^T of all blocks: rows (blk, channel), columns (b, key).
void enqueue_context_vt(sana_dit * c, int64_t B, int64_t L, hipStream_t s) {
    const int64_t R = B * L, C = c->C;
    sana::GemmParams p;
    p.A = c->w_v_all.as<half_t>();
    p.lda = c->Cp;
    p.W = c->ctx16.as<half_t>();
    p.ldw = c->Cp;
    p.M = (int)(c->L_ * C);
    p.N = (int)R;
    p.K = (int)c->Cp;
    p.bias = c->b_v_all.as<float>();
    p.mode = sana::kGemmVT;
    p.out16 = c->vt.as<half_t>();
    p.vt_rows = (int)C;
    p.vt_cols = (int)L;
    p.vt_batch = (int)B;
    p.vt_ld = c->ctx_Lp;
    launch_check(sana::gemm(p, s), "gemm_vt");
}

// Caption projection (optional) + cross K/V of all blocks, enqueued on s.
void enqueue_context(sana_dit * c, const float * caption, bool projected, int64_t B, int64_t L, hipStream_t s) {
    enqueue_context_rows(c, caption, projected, B, L, s);
    enqueue_context_k(c, B, L, s);
    enqueue_context_vt(c, B, L, s);
}

void ensure_forward_buffers(sana_dit * c, int64_t B, int64_t N) {
    const int64_t M = B * N;
    if (M > c->ws_M || B > c->ws_B) {
        drop_graphs(c);
        const int64_t C = c->C;
        c->x32.ensure((size_t)M * C * 4);
        c->fin32.ensure((size_t)M * C * 4);
        c->xa16.ensure((size_t)M * c->Cp * 2);
        c->qkv16.ensure((size_t)M * 3 * C * 2);
        c->la_kt.ensure((size_t)M * C * 2);
        c->la_vt.ensure((size_t)M * C * 2);
        c->o16.ensure((size_t)M * c->Cp * 2);
        c->r16.ensure((size_t)M * c->Cp * 2);
        c->q16.ensure((size_t)M * C * 2);
        c->hid16.ensure((size_t)M * c->E * 2);
        c->glu16.ensure((size_t)M * c->Fp * 2);
        c->la_ws.ensure(sana::linattn_workspace_floats((int)B, (int)N, (int)c->Hs, (int)c->Ds) * 4);
        c->la_ws2.ensure(sana::linattn_workspace_floats(1, (int)N, (int)c->Hs, (int)c->Ds) * 4);
        c->d_t.ensure((size_t)B * 4);
        c->e1.ensure((size_t)B * C * 4);
        c->emb.ensure((size_t)B * C * 4);
        c->tmod.ensure((size_t)B * 6 * C * 4);
        c->mod_all.ensure((size_t)c->L_ * B * 6 * C * 4);
        c->lat_in.ensure((size_t)B * c->Cl * N * 4);
        c->np_out.ensure((size_t)B * c->Cl * N * 4);
        c->ws_M = M;
        c->ws_B = B;
    }
}

// Per-block adaLN modulation of every block (t_mod + table), for B batch rows.
void enqueue_mod(sana_dit * c, int64_t B, hipStream_t s) {
    launch_check(sana::mod_combine(c->tmod.as<float>(), c->sst_all.as<float>(), (int)c->L_, (int)B, (int)(6 * c->C),
                                   c->mod_all.as<float>(), s),
                 "mod_combine");
}

void enqueue_time(sana_dit * c, int64_t B, hipStream_t s) {
    const int64_t C = c->C;
    // the sinusoid is computed inside linear_1, and the per-block modulation
    // tables are added in the time projection's epilogue
    launch_check(sana::gemv_sinusoid_f32(c->d_t.as<float>(), c->freq.as<float>(), c->w_t1.as<float>(),
                                         c->b_t1.as<float>(), c->e1.as<float>(), (int)B, 256, (int)C, s),
                 "time linear_1");
    launch_check(sana::gemv_f32(c->e1.as<float>(), c->w_t2.as<float>(), c->b_t2.as<float>(), c->emb.as<float>(),
                                (int)B, (int)C, (int)C, 1, s),
                 "time linear_2");
    launch_check(sana::gemv_comb_f32(c->emb.as<float>(), c->w_tp.as<float>(), c->b_tp.as<float>(),
                                     c->tmod.as<float>(), c->sst_all.as<float>(), (int)c->L_, c->mod_all.as<float>(),
                                     (int)B, (int)C, (int)(6 * C), 1, s),
                 "time projection");
}

// Stage hook: called after each stage of a block (0 self, 1 cross, 2 ff).
typedef void (*StageHook)(void *, int);

// One block on batch rows [b0, b0 + B) of a Btot-row batch (the whole batch
// by default); co is the number of such launches running concurrently on
// other streams (tile choice).
// extra workgroups of each block LN launch that warm the cache, dispatched
// before the rows (1024 px forward: 5.67 ms without the warm-up, 5.58 / 5.52 /
// 5.50 ms with 128 / 256 / 512 workgroups; 256 dispatched after the rows 5.53)
constexpr int kWarmWorkgroups = 512;

void enqueue_block(sana_dit * c, int64_t i, int64_t B, int64_t N, const float * xbias, hipStream_t s,
                   StageHook hook = nullptr, void * hook_ctx = nullptr, int64_t b0 = 0, int64_t Btot = -1,
                   int co = 1) {
    BlockDev & w = *c->blocks[i];
    if (Btot < 0) Btot = B;
    const int64_t C = c->C, M = B * N, side = (int64_t)std::llround(std::sqrt((double)N)), r0 = b0 * N;
    const int64_t Lc = c->ctx_L;
    float * x32 = c->x32.as<float>() + r0 * C;
    half_t * xa16 = c->xa16.as<half_t>() + r0 * c->Cp;
    half_t * qkv16 = c->qkv16.as<half_t>() + r0 * 3 * C;
    half_t * o16 = c->o16.as<half_t>() + r0 * c->Cp;
    half_t * r16 = c->r16.as<half_t>() + r0 * c->Cp;
    half_t * q16 = c->q16.as<half_t>() + r0 * C;
    half_t * hid16 = c->hid16.as<half_t>() + r0 * c->E;
    half_t * glu16 = c->glu16.as<half_t>() + r0 * c->Fp;
    // modulation rows of this block: [Btot][6C] = shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp
    const float * mod = c->mod_all.as<float>() + ((size_t)i * Btot + b0) * 6 * C;
    // The GEMM weights come from HBM on every forward (the 28 blocks' 1 GB
    // exceeds the 256 MB last-level cache), and a GEMM waits on its first
    // k-tiles the longer for it.  The two LN launches carry extra workgroups
    // that pull weights into that cache ahead of use: LN1 this block's cross
    // and point weights, LN2 the next block's q|k|v and out weights.  CFG
    // branches each read their share.  The inverted-FFN weights are left cold:
    // warming them measured no gain.
    sana::CacheWarm warm1, warm2;
    {
        const int64_t parts = Btot > B ? Btot : 1, part = Btot > B ? b0 : 0;
        auto add = [&](sana::CacheWarm & cw, const DevMem & m) {
            const int64_t n16 = (int64_t)(m.bytes / 16), per = (n16 + parts - 1) / parts;
            const int64_t lo = std::min(n16, per * part), hi = std::min(n16, lo + per);
            cw.p[cw.n] = static_cast<const char *>(m.p) + lo * 16;
            cw.bytes[cw.n] = (hi - lo) * 16;
            ++cw.n;
        };
        warm1.workgroups = warm2.workgroups = kWarmWorkgroups;
        add(warm1, w.w_cq);
        add(warm1, w.w_co);
        add(warm1, w.w_pt);
        if (i + 1 < c->L_) {
            add(warm2, c->blocks[i + 1]->w_qkv);
            add(warm2, c->blocks[i + 1]->w_out);
        }
    }
    // self attention: LN + modulate(shift_msa, scale_msa)
    launch_check(sana::ln_modulate(x32, C, xa16, c->Cp, (int)M, (int)C, (int)N, 1e-6f,
                                   w.has_ln1 ? w.ln1_g.as<float>() : nullptr, w.has_ln1 ? w.ln1_b.as<float>() : nullptr,
                                   mod, nullptr, 6 * C, 0, C, s, &warm1),
                 "ln_modulate");
    float * la_ws = (b0 > 0 && B == 1) ? c->la_ws2.as<float>() : c->la_ws.as<float>();
    if (qkv_split_layout(c, N)) {
        half_t * kt16 = c->la_kt.as<half_t>() + b0 * C * N;
        half_t * vt16 = c->la_vt.as<half_t>() + b0 * C * N;
        gemm_qkv_split(c, w, B, N, xa16, qkv16, kt16, vt16, co, s);
        if (fused_linear_attention(c, N))
            launch_check(sana::linear_attention_fused(qkv16, 3 * C, kt16, vt16, o16, c->Cp, (int)B, (int)N,
                                                      (int)c->Hs, (int)c->Ds, s, co),
                         "linear_attention_fused");
        else
            launch_check(sana::linear_attention_chunked(qkv16, 3 * C, kt16, vt16, o16, c->Cp, (int)B, (int)N,
                                                        (int)c->Hs, (int)c->Ds, la_ws, s),
                         "linear_attention_chunked");
    } else {
        gemm_store(c, xa16, c->Cp, w.w_qkv.as<half_t>(), c->Cp, M, 3 * C, c->Cp,
                   w.has_qkv_bias ? w.b_qkv.as<float>() : nullptr, sana::kActNone, qkv16, 3 * C, nullptr, 0, s, co);
        launch_check(sana::linear_attention(qkv16, qkv16 + C, qkv16 + 2 * C, 3 * C, o16, c->Cp, (int)B, (int)N,
                                            (int)c->Hs, (int)c->Ds, la_ws, s),
                     "linear_attention");
    }
    // x += gate_msa * (o Wo^T + bo); r16 = fp16(x) for the cross-attention query
    gemm_resid(o16, c->Cp, w.w_out.as<half_t>(), c->Cp, M, C, c->Cp, w.b_out.as<float>(), mod + 2 * C, nullptr, 6 * C,
               N, x32, C, r16, c->Cp, s, co);
    if (hook) hook(hook_ctx, 0);
    // cross attention
    gemm_store(c, r16, c->Cp, w.w_cq.as<half_t>(), c->Cp, M, C, c->Cp, w.b_cq.as<float>(), sana::kActNone, q16, C,
               nullptr, 0, s, co);
    const half_t * kc = c->kc.as<half_t>() + (size_t)b0 * Lc * c->L_ * C + i * C;
    const half_t * vt = c->vt.as<half_t>() + ((size_t)i * Btot + b0) * C * c->ctx_Lp;
    launch_check(sana::cross_attention(q16, C, kc, c->L_ * C, vt, c->ctx_Lp, xbias ? xbias + b0 * Lc : nullptr, o16,
                                       c->Cp, (int)B, (int)N, (int)Lc, (int)c->Hc, (int)c->Dc, s),
                 "cross_attention");
    gemm_resid(o16, c->Cp, w.w_co.as<half_t>(), c->Cp, M, C, c->Cp, w.b_co.as<float>(), nullptr, nullptr, 0, N, x32, C,
               nullptr, 0, s, co);
    if (hook) hook(hook_ctx, 1);
    // Mix-FFN
    launch_check(sana::ln_modulate(x32, C, xa16, c->Cp, (int)M, (int)C, (int)N, 1e-6f,
                                   w.has_ln2 ? w.ln2_g.as<float>() : nullptr, w.has_ln2 ? w.ln2_b.as<float>() : nullptr,
                                   mod, nullptr, 6 * C, 3 * C, 4 * C, s, warm2.n ? &warm2 : nullptr),
                 "ln_modulate");
    gemm_store(c, xa16, c->Cp, w.w_inv.as<half_t>(), c->Cp, M, c->E, c->Cp, w.b_inv.as<float>(), sana::kActSilu,
               hid16, c->E, nullptr, 0, s, co);
    launch_check(sana::dwconv_glu(hid16, c->E, w.w_dw.as<float>(), w.b_dw.as<float>(), glu16, c->Fp, (int)B,
                                  (int)side, (int)side, (int)c->F, s),
                 "dwconv_glu");
    gemm_resid(glu16, c->Fp, w.w_pt.as<half_t>(), c->Fp, M, C, c->Fp, nullptr, mod + 5 * C, nullptr, 6 * C, N, x32, C,
               nullptr, 0, s, co);
    if (hook) hook(hook_ctx, 2);
}


void enqueue_patch_embed(sana_dit * c, const float * latent, int64_t Bl, int64_t N, hipStream_t s) {
    launch_check(sana::patch_embed(latent, (int)Bl, (int)(2 * Bl), (int)c->Cl, (int)N, c->w_patch_t.as<float>(),
                                   c->b_patch.as<float>(), c->x32.as<float>(), (int)c->C, s),
                 "patch_embed");
}

// Start `s2` after the work queued so far on s, and `s` after what is then queued on s2.
void fork_to(hipEvent_t ev, hipStream_t s, hipStream_t s2) {
    hip_check(hipEventRecord(ev, s), "hipEventRecord");
    hip_check(hipStreamWaitEvent(s2, ev, 0), "hipStreamWaitEvent");
}
void join_from(hipEvent_t ev, hipStream_t s, hipStream_t s2) {
    hip_check(hipEventRecord(ev, s2), "hipEventRecord");
    hip_check(hipStreamWaitEvent(s, ev, 0), "hipStreamWaitEvent");
}

void enqueue_body(sana_dit * c, int64_t Bl, int64_t Hh, int64_t Ww, const float * xbias, float * out,
                  hipStream_t s);

// The forward: patch and time embeddings, then the blocks and the final layer.
// (Running the patch embedding on the second stream beside the time embedding
// measured no faster.)
void enqueue_forward(sana_dit * c, const float * latent, int64_t Bl, int64_t Hh, int64_t Ww, const float * xbias,
                     float * out, hipStream_t s) {
    enqueue_patch_embed(c, latent, Bl, Hh * Ww, s);
    enqueue_time(c, 2 * Bl, s);
    enqueue_body(c, Bl, Hh, Ww, xbias, out, s);
}

// The step: the caption projection and cross K/V on s, and beside them on the
// second stream the forward's head (patch and time embeddings), which needs
// neither; the blocks start when both are done (step 5.564 -> 5.518 ms in one
// process; the head's ~60 us of small kernels hide behind the context GEMMs).
void enqueue_step(sana_dit * c, const float * caption, int64_t L, const float * latent, int64_t Bl, int64_t Hh,
                  int64_t Ww, const float * xbias, float * out, hipStream_t s) {
    fork_to(c->ev_head_fork, s, c->stream2);
    enqueue_patch_embed(c, latent, Bl, Hh * Ww, c->stream2);
    enqueue_time(c, 2 * Bl, c->stream2);
    enqueue_context_rows(c, caption, false, 2 * Bl, L, s);
    // cross K on s and cross V^T on the second stream (after the head)
    fork_to(c->ev_ctx, s, c->stream2);
    enqueue_context_k(c, 2 * Bl, L, s);
    enqueue_context_vt(c, 2 * Bl, L, c->stream2);
    join_from(c->ev_head_join, s, c->stream2);
    enqueue_body(c, Bl, Hh, Ww, xbias, out, s);
}

// Blocks (the CFG pair as two concurrent chains) and the final layer.
void enqueue_body(sana_dit * c, int64_t Bl, int64_t Hh, int64_t Ww, const float * xbias, float * out,
                  hipStream_t s) {
    const int64_t B = 2 * Bl, N = Hh * Ww;
    // The CFG pair runs its two batch rows as two concurrent chains (graph
    // branches): each kernel then covers half the rows, and the two chains fill
    // each other's launch gaps and tails and share the weights through the caches.
    if (B == 2 && c->cfg_branches) {
        // batch row 0 on s, row 1 on stream2, forked after the time embedding
        // and joined before the final layer
        hip_check(hipEventRecord(c->ev_fork, s), "hipEventRecord");
        hip_check(hipStreamWaitEvent(c->stream2, c->ev_fork, 0), "hipStreamWaitEvent");
        for (int64_t i = 0; i < c->L_; ++i) {
            enqueue_block(c, i, 1, N, xbias, s, nullptr, nullptr, 0, 2, 2);
            enqueue_block(c, i, 1, N, xbias, c->stream2, nullptr, nullptr, 1, 2, 2);
        }
        hip_check(hipEventRecord(c->ev_join, c->stream2), "hipEventRecord");
        hip_check(hipStreamWaitEvent(s, c->ev_join, 0), "hipStreamWaitEvent");
    } else {
        for (int64_t i = 0; i < c->L_; ++i) enqueue_block(c, i, B, N, xbias, s);
    }
    launch_check(sana::final_layer(c->x32.as<float>(), c->emb.as<float>(), c->sst_final.as<float>(),
                                   c->w_proj.as<float>(), c->b_proj.as<float>(), c->fin32.as<float>(), out, (int)B,
                                   (int)N, (int)c->C,
                                   (int)c->Cl, 1e-6f, s),
                 "final_layer");
}

// Tensors every block needs (load_block_weights, src/transformer.cpp:214-308).
const char * const kBlockRequired[] = {
    "scale_shift_table", "attn1.to_q.weight", "attn1.to_k.weight", "attn1.to_v.weight", "attn1.to_out.0.weight",
    "attn1.to_out.0.bias", "attn2.to_q.weight", "attn2.to_q.bias", "attn2.to_k.weight", "attn2.to_k.bias",
    "attn2.to_v.weight", "attn2.to_v.bias", "attn2.to_out.0.weight", "attn2.to_out.0.bias",
    "ff.conv_inverted.weight", "ff.conv_inverted.bias", "ff.conv_depth.weight", "ff.conv_depth.bias",
    "ff.conv_point.weight",
};
const char * const kTopRequired[] = {
    "patch_embed.proj.weight", "patch_embed.proj.bias", "time_embed.emb.timestep_embedder.linear_1.weight",
    "time_embed.emb.timestep_embedder.linear_1.bias", "time_embed.emb.timestep_embedder.linear_2.weight",
    "time_embed.emb.timestep_embedder.linear_2.bias", "time_embed.linear.weight", "time_embed.linear.bias",
    "caption_norm.weight", "scale_shift_table", "proj_out.weight", "proj_out.bias",
};
const char * const kCaptionRequired[] = {
    "caption_projection.linear_1.weight", "caption_projection.linear_1.bias", "caption_projection.linear_2.weight",
    "caption_projection.linear_2.bias", "caption_norm.weight",
};

std::string block_key(int64_t blk, const char * suffix) { return "blk" + std::to_string(blk) + "." + suffix; }

void require(sana_dit * c, const std::string & key, const std::string & shown) {
    if (!c->have.count(key)) throw_err(SANA_ERR_STATE, "weight not uploaded: " + shown);
}

void check_block(sana_dit * c, int64_t blk) {
    for (const char * sfx : kBlockRequired)
        require(c, block_key(blk, sfx), "transformer_blocks." + std::to_string(blk) + "." + sfx);
}

void check_context_weights(sana_dit * c, bool caption) {
    if (caption)
        for (const char * n : kCaptionRequired) require(c, n, n);
    for (int64_t i = 0; i < c->L_; ++i)
        for (const char * sfx : {"attn2.to_k.weight", "attn2.to_k.bias", "attn2.to_v.weight", "attn2.to_v.bias"})
            require(c, block_key(i, sfx), "transformer_blocks." + std::to_string(i) + "." + sfx);
}

void check_ready(sana_dit * c) {
    for (const char * n : kTopRequired) require(c, n, n);
    for (const char * n : kCaptionRequired) require(c, n, n);
    for (int64_t i = 0; i < c->L_; ++i) check_block(c, i);
}

void set_t(sana_dit * c, int64_t B, float t, hipStream_t s) {
    hipLaunchKernelGGL(fill_kernel, dim3((unsigned)((B + 63) / 64)), dim3(64), 0, s, c->d_t.as<float>(), (int)B, t);
    hip_check(hipGetLastError(), "fill");
}


// Capture `body` on the context stream into an executable graph.
template <class Body>
hipGraphExec_t capture_graph(sana_dit * c, Body body) {
    hipGraph_t g = nullptr;
    hip_check(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    try {
        body(c->stream);
    } catch (...) {
        (void)hipStreamEndCapture(c->stream, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
    }
    hip_check(hipStreamEndCapture(c->stream, &g), "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    hipError_t r = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    hip_check(r, "hipGraphInstantiate");
    return exec;
}

template <class T>
void key_append(std::string & k, const T & v) {
    k.append(reinterpret_cast<const char *>(&v), sizeof(T));
}

// Run `body` on stream s through a cached HIP graph (captured on the context
// stream on first use for this key).
template <class Body>
void run_graph(sana_dit * c,
               const std::tuple<int, int64_t, int64_t, int64_t, int64_t, const void *, const void *, const void *,
                                const void *> & key,
               hipStream_t s, Body body) {
    if (!c->use_graphs) {
        body(s);
        return;
    }
    auto it = c->graphs.find(key);
    if (it == c->graphs.end()) {
        GraphEntry e;
        e.exec = capture_graph(c, body);
        it = c->graphs.emplace(key, e).first;
    }
    hip_check(hipGraphLaunch(it->second.exec, s), "hipGraphLaunch");
}

struct BlockSuffix {
    const char * name;
    int kind;
};

}  // namespace

namespace {

// Where a linear weight goes among the fp16 GEMM operands: rows [row_off,
// row_off + rows) of a [total, ld] buffer, from a [rows, cols] weight (cols <
// ld are zero padding); conv1x1 weights arrive as [rows, cols, 1, 1].
struct OperandSlot {
    DevMem * dst = nullptr;
    int64_t rows = 0, cols = 0, ld = 0, row_off = 0, total = 0;
    bool conv1x1 = false;
};

bool block_operand(sana_dit * c, int64_t blk, const std::string & s, OperandSlot & o) {
    BlockDev & w = *c->blocks[blk];
    const int64_t C = c->C, E = c->E, F = c->F, Cp = c->Cp;
    auto set = [&](DevMem & d, int64_t rows, int64_t cols, int64_t ld, int64_t off, int64_t total, bool conv) {
        o.dst = &d;
        o.rows = rows;
        o.cols = cols;
        o.ld = ld;
        o.row_off = off;
        o.total = total;
        o.conv1x1 = conv;
        return true;
    };
    if (s == "attn1.to_q.weight") return set(w.w_qkv, C, C, Cp, 0, 3 * C, false);
    if (s == "attn1.to_k.weight") return set(w.w_qkv, C, C, Cp, C, 3 * C, false);
    if (s == "attn1.to_v.weight") return set(w.w_qkv, C, C, Cp, 2 * C, 3 * C, false);
    if (s == "attn1.to_out.0.weight") return set(w.w_out, C, C, Cp, 0, C, false);
    if (s == "attn2.to_q.weight") return set(w.w_cq, C, C, Cp, 0, C, false);
    if (s == "attn2.to_k.weight") return set(c->w_k_all, C, C, Cp, blk * C, c->L_ * C, false);
    if (s == "attn2.to_v.weight") return set(c->w_v_all, C, C, Cp, blk * C, c->L_ * C, false);
    if (s == "attn2.to_out.0.weight") return set(w.w_co, C, C, Cp, 0, C, false);
    if (s == "ff.conv_inverted.weight") return set(w.w_inv, E, C, Cp, 0, E, true);
    if (s == "ff.conv_point.weight") return set(w.w_pt, C, F, c->Fp, 0, C, true);
    return false;
}

bool top_operand(sana_dit * c, const std::string & n, OperandSlot & o) {
    const int64_t C = c->C;
    o = OperandSlot{};
    if (n == "caption_projection.linear_1.weight") {
        o.dst = &c->w_cap1;
        o.rows = C;
        o.cols = c->Ccap;
        o.ld = c->Ccap_p;
    } else if (n == "caption_projection.linear_2.weight") {
        o.dst = &c->w_cap2;
        o.rows = C;
        o.cols = C;
        o.ld = c->Cp;
    } else {
        return false;
    }
    o.total = C;
    return true;
}

std::string block_tensor_name(int64_t blk, const std::string & s) {
    return "transformer_blocks." + std::to_string(blk) + "." + s;
}

}  // namespace

// Scratch of sana_hip_linear_attention_noalloc: the chunk partial states, the
// fp16 hi/lo state pair and the partial maxima of the three-kernel linear
// attention (what the allocating entry point takes as its workspace).  Each GPU
// the library runs on holds its own copy of the array until the process ends.
// The kernels overwrite every element they later read, so nothing is cleared.
constexpr size_t kLaScratchFloats = (size_t)4 << 20;  // 16 MiB
static __device__ __align__(256) float scratch[kLaScratchFloats];

namespace {
constexpr int kScratchDevices = 64;
std::mutex scratch_mu;
float * scratch_addr[kScratchDevices] = {};

// Device address of `scratch` on the current device `dev`, looked up on the
// first call for that device (the array's name is only a host-side stand-in).
// The address is kept for the life of the process: a hipDeviceReset, which
// reloads the code object and its static array, is not supported in between.
float * device_scratch(int dev) {
    if (dev < 0 || dev >= kScratchDevices) throw_err(SANA_ERR_INVALID_ARGUMENT, "scratch: device index out of range");
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_addr[dev]) {
        void * p = nullptr;
        hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (!p) throw_err(SANA_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
        scratch_addr[dev] = static_cast<float *>(p);
    }
    return scratch_addr[dev];
}

// ---------------------------------------------------------------------------
// Packed weight image: every device weight buffer of a context in its device
// layout (fp16 GEMM operands K-padded and fused, stacked cross K/V, tap-major
// depthwise taps, fp32 vectors), so a later load is one mapped read and one
// copy per buffer, with no conversion or packing.
//   header | uploaded tensor names ('\n'-joined) | 3 flag bytes per block
//   (has_ln1, has_ln2, has_qkv_bias) | buffer table | payloads (4 KiB aligned)
// Each table entry holds the buffer's bytes, file offset and checksum.
constexpr char kPackMagic[8] = {'S', 'A', 'N', 'A', 'P', 'K', '0', '1'};
constexpr uint32_t kPackVersion = 1;
constexpr uint64_t kPackAlign = 4096;

struct PackHeader {
    char magic[8];
    uint32_t version, nbuf;
    int64_t dims[10];       // layers, hidden, ffn, caption_dim, latent_channels, self_heads, cross_heads, Cp, Fp, Ccap_p
    uint64_t key;           // caller's key of the source weights (0: none)
    uint64_t names_bytes, flags_bytes, table_offset, file_bytes;
};
struct PackEntry {
    uint64_t bytes, offset, checksum;
};

// The buffers in file order with the bytes each must hold; `optional` ones
// (q|k|v bias, LayerNorm affine) may be absent (0 bytes).
struct PackBuf {
    DevMem * m;
    uint64_t bytes;
    bool optional;
};
constexpr size_t kPackTop = 21, kPackPerBlock = 17;  // entries before the blocks, entries per block
// per-block entry indices of the flagged optional buffers
constexpr size_t kPackQkvBias = 1, kPackLn1 = 13, kPackLn2 = 15;

std::vector<PackBuf> pack_buffers(sana_dit * c) {
    const uint64_t L = c->L_, C = c->C, E = c->E, Cp = c->Cp, Fp = c->Fp, Cl = c->Cl;
    std::vector<PackBuf> v = {
        {&c->w_k_all, L * C * Cp * 2, false}, {&c->b_k_all, L * C * 4, false},  {&c->w_v_all, L * C * Cp * 2, false},
        {&c->b_v_all, L * C * 4, false},      {&c->sst_all, L * 6 * C * 4, false},
        {&c->w_cap1, C * (uint64_t)c->Ccap_p * 2, false}, {&c->b_cap1, C * 4, false},
        {&c->w_cap2, C * Cp * 2, false},      {&c->b_cap2, C * 4, false},       {&c->cap_norm, C * 4, false},
        {&c->w_patch_t, Cl * C * 4, false},   {&c->b_patch, C * 4, false},      {&c->w_t1, C * 256 * 4, false},
        {&c->b_t1, C * 4, false},             {&c->w_t2, C * C * 4, false},     {&c->b_t2, C * 4, false},
        {&c->w_tp, 6 * C * C * 4, false},     {&c->b_tp, 6 * C * 4, false},     {&c->sst_final, 2 * C * 4, false},
        {&c->w_proj, C * Cl * 4, false},      {&c->b_proj, Cl * 4, false},
    };
    if (v.size() != kPackTop) throw_err(SANA_ERR_STATE, "packed image layout");
    for (auto & bp : c->blocks) {
        BlockDev & w = *bp;
        const PackBuf blk[] = {
            {&w.w_qkv, 3 * C * Cp * 2, false}, {&w.b_qkv, 3 * C * 4, true}, {&w.w_out, C * Cp * 2, false},
            {&w.b_out, C * 4, false},          {&w.w_cq, C * Cp * 2, false},  {&w.b_cq, C * 4, false},
            {&w.w_co, C * Cp * 2, false},      {&w.b_co, C * 4, false},       {&w.w_inv, E * Cp * 2, false},
            {&w.b_inv, E * 4, false},          {&w.w_dw, 9 * E * 4, false},   {&w.b_dw, E * 4, false},
            {&w.w_pt, C * Fp * 2, false},      {&w.ln1_g, C * 4, true},       {&w.ln1_b, C * 4, true},
            {&w.ln2_g, C * 4, true},           {&w.ln2_b, C * 4, true},
        };
        static_assert(sizeof(blk) / sizeof(blk[0]) == kPackPerBlock, "block entry count");
        v.insert(v.end(), std::begin(blk), std::end(blk));
    }
    return v;
}

void pack_dims(const sana_dit * c, int64_t * d) {
    const int64_t v[10] = {c->L_, c->C, c->E, c->Ccap, c->Cl, c->Hs, c->Hc, c->Cp, c->Fp, c->Ccap_p};
    std::copy(v, v + 10, d);
}

// 64-bit FNV-1a over the 8-byte words of fixed 4 MiB chunks, the chunk values
// folded in order (the same result on any number of threads).
uint64_t pack_checksum(const unsigned char * p, uint64_t n) {
    constexpr uint64_t kChunk = 4u << 20, kBasis = 14695981039346656037ULL, kPrime = 1099511628211ULL;
    const uint64_t nch = (n + kChunk - 1) / kChunk;
    std::vector<uint64_t> hs((size_t)nch);
    host_parallel((size_t)nch, 1, [&](size_t c0, size_t c1) {
        for (size_t ci = c0; ci < c1; ++ci) {
            const uint64_t lo = ci * kChunk, hi = std::min(n, lo + kChunk);
            uint64_t h = kBasis, i = lo;
            for (; i + 8 <= hi; i += 8) {
                uint64_t w;
                std::memcpy(&w, p + i, 8);
                h = (h ^ w) * kPrime;
            }
            for (; i < hi; ++i) h = (h ^ p[i]) * kPrime;
            hs[ci] = h;
        }
    });
    uint64_t h = kBasis ^ n;
    for (uint64_t x : hs) h = (h ^ x) * kPrime;
    return h;
}

// Read-only mapping of a whole file, unmapped on scope exit.
struct FileMap {
    const unsigned char * p = nullptr;
    size_t n = 0;
    explicit FileMap(const std::string & path) {
        const int fd = open(path.c_str(), O_RDONLY);
        if (fd < 0) throw_err(SANA_ERR_IO, "cannot open packed weights: " + path);
        struct stat st;
        if (fstat(fd, &st) != 0 || st.st_size <= 0) {
            close(fd);
            throw_err(SANA_ERR_FORMAT, "packed weights file is empty: " + path);
        }
        n = (size_t)st.st_size;
        void * m = mmap(nullptr, n, PROT_READ, MAP_PRIVATE, fd, 0);
        close(fd);
        if (m == MAP_FAILED) throw_err(SANA_ERR_IO, "cannot map packed weights: " + path);
        p = static_cast<const unsigned char *>(m);
    }
    ~FileMap() {
        if (p) munmap(const_cast<unsigned char *>(p), n);
    }
    FileMap(const FileMap &) = delete;
    FileMap & operator=(const FileMap &) = delete;
};
}  // namespace

extern "C" {

const char * sana_dit_last_error(void) { return g_last_error.c_str(); }

int sana_dit_create(const sana_dit_config * cfg, sana_dit ** out) {
    if (!cfg || !out) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    if (cfg->layers <= 0 || cfg->hidden <= 0 || cfg->ffn <= 0 || cfg->ffn % 2 || cfg->caption_dim <= 0 ||
        cfg->latent_channels <= 0 || cfg->self_heads <= 0 || cfg->cross_heads <= 0)
        return set_err(SANA_ERR_INVALID_ARGUMENT, "config dimensions must be positive (ffn even)");
    if (cfg->hidden % cfg->self_heads != 0)
        return set_err(SANA_ERR_INVALID_ARGUMENT, "self attention hidden size must be divisible by self_num_heads");
    if (cfg->hidden % cfg->cross_heads != 0)
        return set_err(SANA_ERR_INVALID_ARGUMENT, "cross attention hidden size must be divisible by cross_num_heads");
    if (cfg->hidden > 2048) return set_err(SANA_ERR_INVALID_ARGUMENT, "hidden > 2048 not supported");
    if (cfg->latent_channels > 32) return set_err(SANA_ERR_INVALID_ARGUMENT, "latent_channels > 32 not supported");
    if (cfg->hidden / cfg->self_heads > 100) return set_err(SANA_ERR_INVALID_ARGUMENT, "self head_dim > 100");
    if (cfg->hidden / cfg->cross_heads > 256) return set_err(SANA_ERR_INVALID_ARGUMENT, "cross head_dim > 256");
    auto c = std::make_unique<sana_dit>();
    int rc = guarded([&] {
        c->cfg = *cfg;
        c->C = cfg->hidden;
        c->E = cfg->ffn;
        c->F = cfg->ffn / 2;
        c->Ccap = cfg->caption_dim;
        c->Cl = cfg->latent_channels;
        c->L_ = cfg->layers;
        c->Hs = cfg->self_heads;
        c->Hc = cfg->cross_heads;
        c->Ds = c->C / c->Hs;
        c->Dc = c->C / c->Hc;
        c->Cp = round_up(c->C, 64);
        c->Fp = round_up(c->F, 64);
        c->Ccap_p = round_up(c->Ccap, 64);
        const char * eb = std::getenv("SANA_DIT_CFG_BRANCHES");
        c->cfg_branches = !(eb && eb[0] == '0');
        const char * eg = std::getenv("SANA_DIT_NO_GRAPH");
        c->use_graphs = !(eg && eg[0] == '1');
        hip_check(hipSetDevice(cfg->device), "hipSetDevice");
        hip_check(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "hipStreamCreate");
        hip_check(hipStreamCreateWithFlags(&c->stream2, hipStreamNonBlocking), "hipStreamCreate");
        hip_check(hipEventCreateWithFlags(&c->ev_fork, hipEventDisableTiming), "hipEventCreate");
        hip_check(hipEventCreateWithFlags(&c->ev_join, hipEventDisableTiming), "hipEventCreate");
        hip_check(hipEventCreateWithFlags(&c->ev_head_fork, hipEventDisableTiming), "hipEventCreate");
        hip_check(hipEventCreateWithFlags(&c->ev_head_join, hipEventDisableTiming), "hipEventCreate");
        hip_check(hipEventCreateWithFlags(&c->ev_ctx, hipEventDisableTiming), "hipEventCreate");
        hip_check(hipEventCreateWithFlags(&c->ev_loop, hipEventDisableTiming), "hipEventCreate");
        for (int64_t i = 0; i < c->L_; ++i) c->blocks.emplace_back(new BlockDev());
        // sinusoid frequencies exactly as the reference computes them in fp32
        // (src/transformer.cpp:89,97-99)
        std::vector<float> f(128);
        const float ls = -std::log(10000.0f) / 128.0f;
        for (int i = 0; i < 128; ++i) f[i] = std::exp(static_cast<float>(i) * ls);
        upload_f32(c->freq, f.data(), 128);
        const int64_t C = c->C;
        c->w_k_all.ensure((size_t)c->L_ * C * c->Cp * 2);
        c->w_v_all.ensure((size_t)c->L_ * C * c->Cp * 2);
        c->b_k_all.ensure((size_t)c->L_ * C * 4);
        c->b_v_all.ensure((size_t)c->L_ * C * 4);
        c->sst_all.ensure((size_t)c->L_ * 6 * C * 4);
    });
    if (rc != SANA_OK) return rc;
    *out = c.release();
    return SANA_OK;
}

void sana_dit_destroy(sana_dit * c) { delete c; }

int sana_dit_set_weight(sana_dit * c, const char * name, const float * data, const int64_t * shape, int ndim,
                        int transposed) {
    if (!c || !name || !data || !shape) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    return guarded([&] {
        const std::string n = name;
        const int64_t C = c->C, Cl = c->Cl, Ccap = c->Ccap;
        const bool tr = transposed != 0;
        if (n == "patch_embed.proj.weight") {
            expect_shape(name, shape, ndim, {C, Cl, 1, 1});
            upload_f32_transposed(c->w_patch_t, data, Cl, C, true);  // -> [Cl, C]
        } else if (n == "patch_embed.proj.bias") {
            expect_shape(name, shape, ndim, {C});
            upload_f32(c->b_patch, data, C);
        } else if (n == "time_embed.emb.timestep_embedder.linear_1.weight") {
            expect_shape(name, shape, ndim, tr ? std::vector<int64_t>{256, C} : std::vector<int64_t>{C, 256});
            upload_f32_transposed(c->w_t1, data, C, 256, tr);
        } else if (n == "time_embed.emb.timestep_embedder.linear_1.bias") {
            expect_shape(name, shape, ndim, {C});
            upload_f32(c->b_t1, data, C);
        } else if (n == "time_embed.emb.timestep_embedder.linear_2.weight") {
            expect_shape(name, shape, ndim, {C, C});
            upload_f32_transposed(c->w_t2, data, C, C, tr);
        } else if (n == "time_embed.emb.timestep_embedder.linear_2.bias") {
            expect_shape(name, shape, ndim, {C});
            upload_f32(c->b_t2, data, C);
        } else if (n == "time_embed.linear.weight") {
            expect_shape(name, shape, ndim, tr ? std::vector<int64_t>{C, 6 * C} : std::vector<int64_t>{6 * C, C});
            upload_f32_transposed(c->w_tp, data, 6 * C, C, tr);
        } else if (n == "time_embed.linear.bias") {
            expect_shape(name, shape, ndim, {6 * C});
            upload_f32(c->b_tp, data, 6 * C);
        } else if (n == "caption_norm.weight") {
            expect_shape(name, shape, ndim, {C});
            upload_f32(c->cap_norm, data, C);
        } else if (n == "scale_shift_table") {
            expect_shape(name, shape, ndim, {2, C});
            upload_f32(c->sst_final, data, 2 * C);
        } else if (n == "proj_out.weight") {
            expect_shape(name, shape, ndim, tr ? std::vector<int64_t>{C, Cl} : std::vector<int64_t>{Cl, C});
            upload_f32_transposed(c->w_proj, data, C, Cl, !tr);  // -> [C, Cl]
        } else if (n == "proj_out.bias") {
            expect_shape(name, shape, ndim, {Cl});
            upload_f32(c->b_proj, data, Cl);
        } else if (n == "caption_projection.linear_1.weight") {
            expect_shape(name, shape, ndim, tr ? std::vector<int64_t>{Ccap, C} : std::vector<int64_t>{C, Ccap});
            upload_f16(c->w_cap1, data, C, Ccap, c->Ccap_p, tr, n);
        } else if (n == "caption_projection.linear_1.bias") {
            expect_shape(name, shape, ndim, {C});
            upload_f32(c->b_cap1, data, C);
        } else if (n == "caption_projection.linear_2.weight") {
            expect_shape(name, shape, ndim, {C, C});
            upload_f16(c->w_cap2, data, C, C, c->Cp, tr, n);
        } else if (n == "caption_projection.linear_2.bias") {
            expect_shape(name, shape, ndim, {C});
            upload_f32(c->b_cap2, data, C);
        } else {
            throw_err(SANA_ERR_INVALID_ARGUMENT, "unknown weight name: " + n);
        }
        c->have[n] = 1;
        weights_changed(c, conditioning_weight(n));
    });
}

int sana_dit_set_block_weight(sana_dit * c, int64_t blk, const char * suffix, const float * data, const int64_t * shape,
                              int ndim, int transposed) {
    if (!c || !suffix || !data || !shape) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    if (blk < 0 || blk >= c->L_) return set_err(SANA_ERR_INVALID_ARGUMENT, "block index out of range");
    return guarded([&] {
        const std::string s = suffix;
        BlockDev & w = *c->blocks[blk];
        const int64_t C = c->C, E = c->E;
        const bool tr = transposed != 0;
        OperandSlot o;
        if (block_operand(c, blk, s, o)) {
            if (o.conv1x1) {
                expect_shape(suffix, shape, ndim, {o.rows, o.cols, 1, 1});
                upload_f16(*o.dst, data, o.rows, o.cols, o.ld, false, block_tensor_name(blk, s), o.row_off, o.total);
            } else {
                expect_shape(suffix, shape, ndim,
                             tr ? std::vector<int64_t>{o.cols, o.rows} : std::vector<int64_t>{o.rows, o.cols});
                upload_f16(*o.dst, data, o.rows, o.cols, o.ld, tr, block_tensor_name(blk, s), o.row_off, o.total);
            }
        } else if (s == "scale_shift_table") {
            expect_shape(suffix, shape, ndim, {6, C});
            upload_f32(c->sst_all, data, 6 * C, (size_t)blk * 6 * C, (size_t)c->L_ * 6 * C);
        } else if (s == "attn1.to_q.bias" || s == "attn1.to_k.bias" || s == "attn1.to_v.bias") {
            // not in any checkpoint (the reference loader injects zeros, src/transformer.cpp:361-362);
            // accepted for weights built in memory
            expect_shape(suffix, shape, ndim, {C});
            const int64_t part = s == "attn1.to_q.bias" ? 0 : (s == "attn1.to_k.bias" ? 1 : 2);
            upload_f32(w.b_qkv, data, C, (size_t)part * C, (size_t)3 * C);
            w.has_qkv_bias = true;
        } else if (s == "attn1.to_out.0.bias") {
            expect_shape(suffix, shape, ndim, {C});
            upload_f32(w.b_out, data, C);
        } else if (s == "attn2.to_q.bias") {
            expect_shape(suffix, shape, ndim, {C});
            upload_f32(w.b_cq, data, C);
        } else if (s == "attn2.to_k.bias") {
            expect_shape(suffix, shape, ndim, {C});
            upload_f32(c->b_k_all, data, C, blk * C, c->L_ * C);
        } else if (s == "attn2.to_v.bias") {
            expect_shape(suffix, shape, ndim, {C});
            upload_f32(c->b_v_all, data, C, blk * C, c->L_ * C);
        } else if (s == "attn2.to_out.0.bias") {
            expect_shape(suffix, shape, ndim, {C});
            upload_f32(w.b_co, data, C);
        } else if (s == "ff.conv_inverted.bias") {
            expect_shape(suffix, shape, ndim, {E});
            upload_f32(w.b_inv, data, E);
        } else if (s == "ff.conv_depth.weight") {
            expect_shape(suffix, shape, ndim, {E, 1, 3, 3});
            std::vector<float> t((size_t)9 * E);
            for (int64_t e = 0; e < E; ++e)
                for (int k = 0; k < 9; ++k) t[(size_t)k * E + e] = data[e * 9 + k];
            upload_f32(w.w_dw, t.data(), t.size());
        } else if (s == "ff.conv_depth.bias") {
            expect_shape(suffix, shape, ndim, {E});
            upload_f32(w.b_dw, data, E);
        } else {
            throw_err(SANA_ERR_INVALID_ARGUMENT, "unknown block weight suffix: " + s);
        }
        c->have["blk" + std::to_string(blk) + "." + s] = 1;
        weights_changed(c, conditioning_block_weight(s));
    });
}

int sana_dit_set_weight_f16(sana_dit * c, const char * name, const uint16_t * data, const int64_t * shape, int ndim) {
    if (!c || !name || !data || !shape) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    return guarded([&] {
        const std::string n = name;
        OperandSlot o;
        if (!top_operand(c, n, o)) throw_err(SANA_ERR_INVALID_ARGUMENT, "not a 16-bit operand weight: " + n);
        expect_shape(name, shape, ndim, {o.rows, o.cols});
        upload_f16_bits(*o.dst, data, o.rows, o.cols, o.ld, n, o.row_off, o.total);
        c->have[n] = 1;
        weights_changed(c, conditioning_weight(n));
    });
}

int sana_dit_set_block_weight_f16(sana_dit * c, int64_t blk, const char * suffix, const uint16_t * data,
                                  const int64_t * shape, int ndim) {
    if (!c || !suffix || !data || !shape) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    if (blk < 0 || blk >= c->L_) return set_err(SANA_ERR_INVALID_ARGUMENT, "block index out of range");
    return guarded([&] {
        const std::string s = suffix;
        OperandSlot o;
        if (!block_operand(c, blk, s, o)) throw_err(SANA_ERR_INVALID_ARGUMENT, "not a 16-bit operand weight: " + s);
        if (o.conv1x1)
            expect_shape(suffix, shape, ndim, {o.rows, o.cols, 1, 1});
        else
            expect_shape(suffix, shape, ndim, {o.rows, o.cols});
        upload_f16_bits(*o.dst, data, o.rows, o.cols, o.ld, block_tensor_name(blk, s), o.row_off, o.total);
        c->have["blk" + std::to_string(blk) + "." + s] = 1;
        weights_changed(c, conditioning_block_weight(s));
    });
}

int sana_dit_set_block_norm(sana_dit * c, int64_t blk, int which, const float * gamma, const float * beta) {
    if (!c) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    if (blk < 0 || blk >= c->L_ || (which != 0 && which != 1))
        return set_err(SANA_ERR_INVALID_ARGUMENT, "bad block or norm index");
    return guarded([&] {
        BlockDev & w = *c->blocks[blk];
        DevMem & g = which == 0 ? w.ln1_g : w.ln2_g;
        DevMem & b = which == 0 ? w.ln1_b : w.ln2_b;
        bool & has = which == 0 ? w.has_ln1 : w.has_ln2;
        if (!gamma && !beta) {
            has = false;
        } else {
            std::vector<float> one(c->C, 1.0f), zero(c->C, 0.0f);
            upload_f32(g, gamma ? gamma : one.data(), c->C);
            upload_f32(b, beta ? beta : zero.data(), c->C);
            has = true;
        }
        drop_graphs(c);
    });
}

int sana_dit_check_weights(sana_dit * c) {
    if (!c) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    return guarded([&] { check_ready(c); });
}

int sana_dit_save_packed(sana_dit * c, const char * path, uint64_t key) {
    if (!c || !path) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    return guarded([&] {
        check_ready(c);
        const std::vector<PackBuf> bufs = pack_buffers(c);
        PackHeader hd{};
        std::memcpy(hd.magic, kPackMagic, 8);
        hd.version = kPackVersion;
        hd.nbuf = (uint32_t)bufs.size();
        pack_dims(c, hd.dims);
        hd.key = key;
        std::string names;
        for (const auto & kv : c->have) names += kv.first + "\n";
        std::vector<uint8_t> flags;
        for (auto & bp : c->blocks) {
            flags.push_back(bp->has_ln1);
            flags.push_back(bp->has_ln2);
            flags.push_back(bp->has_qkv_bias);
        }
        hd.names_bytes = names.size();
        hd.flags_bytes = flags.size();
        hd.table_offset = sizeof(PackHeader) + names.size() + flags.size();
        std::vector<PackEntry> tab(bufs.size());
        uint64_t off = hd.table_offset + tab.size() * sizeof(PackEntry);
        for (size_t i = 0; i < bufs.size(); ++i) {
            const PackBuf & b = bufs[i];
            const uint64_t have = b.m->p ? b.bytes : 0;
            if (b.m->p && b.m->bytes < b.bytes)
                throw_err(SANA_ERR_STATE, "device weight buffer smaller than its layout (buffer " + std::to_string(i) + ")");
            if (!have && !b.optional)
                throw_err(SANA_ERR_STATE, "device weight buffer missing (buffer " + std::to_string(i) + ")");
            off = (off + kPackAlign - 1) / kPackAlign * kPackAlign;
            tab[i].bytes = have;
            tab[i].offset = off;
            off += have;
        }
        hd.file_bytes = off;
        // written to a temporary name and renamed, so a reader never maps a partial image
        const std::string tmp = std::string(path) + ".tmp" + std::to_string((long long)getpid());
        FILE * f = std::fopen(tmp.c_str(), "wb");
        if (!f) throw_err(SANA_ERR_IO, "cannot write packed weights: " + tmp);
        bool ok = true;
        std::vector<unsigned char> host;
        try {
            hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
            for (size_t i = 0; i < bufs.size() && ok; ++i) {
                if (!tab[i].bytes) continue;
                host.resize(tab[i].bytes);
                hip_check(hipMemcpy(host.data(), bufs[i].m->p, tab[i].bytes, hipMemcpyDeviceToHost), "download weights");
                tab[i].checksum = pack_checksum(host.data(), tab[i].bytes);
                ok = std::fseek(f, (long)tab[i].offset, SEEK_SET) == 0 &&
                     std::fwrite(host.data(), 1, tab[i].bytes, f) == tab[i].bytes;
            }
            ok = ok && std::fseek(f, 0, SEEK_SET) == 0 && std::fwrite(&hd, sizeof(hd), 1, f) == 1 &&
                 std::fwrite(names.data(), 1, names.size(), f) == names.size() &&
                 std::fwrite(flags.data(), 1, flags.size(), f) == flags.size() &&
                 std::fwrite(tab.data(), sizeof(PackEntry), tab.size(), f) == tab.size();
            // the full length even when the image ends in absent (zero-byte) buffers
            ok = ok && std::fflush(f) == 0 && ftruncate(fileno(f), (off_t)hd.file_bytes) == 0;
        } catch (...) {
            std::fclose(f);
            std::remove(tmp.c_str());
            throw;
        }
        ok = (std::fclose(f) == 0) && ok;
        if (!ok || std::rename(tmp.c_str(), path) != 0) {
            std::remove(tmp.c_str());
            throw_err(SANA_ERR_IO, std::string("cannot write packed weights: ") + path);
        }
    });
}

int sana_dit_load_packed(sana_dit * c, const char * path, uint64_t key) {
    if (!c || !path) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    return guarded([&] {
        const FileMap fm(path);
        const std::vector<PackBuf> bufs = pack_buffers(c);
        auto bad = [&](const std::string & why) { throw_err(SANA_ERR_FORMAT, std::string(path) + ": " + why); };
        if (fm.n < sizeof(PackHeader)) bad("truncated packed weights");
        PackHeader hd;
        std::memcpy(&hd, fm.p, sizeof(hd));
        if (std::memcmp(hd.magic, kPackMagic, 8) != 0) bad("not a packed weight image");
        if (hd.version != kPackVersion) bad("packed weight image version " + std::to_string(hd.version) + " is not supported");
        int64_t dims[10];
        pack_dims(c, dims);
        if (std::memcmp(dims, hd.dims, sizeof(dims)) != 0) bad("packed weights are for other model dimensions");
        if (hd.key != key) bad("packed weights were written from other source weights (key mismatch)");
        if (hd.nbuf != bufs.size() || hd.file_bytes != fm.n || hd.flags_bytes != 3 * c->blocks.size() ||
            hd.names_bytes > fm.n || hd.table_offset != sizeof(PackHeader) + hd.names_bytes + hd.flags_bytes ||
            hd.table_offset + (uint64_t)hd.nbuf * sizeof(PackEntry) > fm.n)
            bad("packed weight image is truncated or inconsistent");
        std::vector<PackEntry> tab(hd.nbuf);
        std::memcpy(tab.data(), fm.p + hd.table_offset, tab.size() * sizeof(PackEntry));
        const uint8_t * flags = fm.p + sizeof(PackHeader) + hd.names_bytes;
        for (size_t i = 0; i < bufs.size(); ++i) {
            const PackEntry & e = tab[i];
            const bool absent_ok = bufs[i].optional && e.bytes == 0;
            if (!absent_ok && e.bytes != bufs[i].bytes)
                bad("buffer " + std::to_string(i) + " holds " + std::to_string(e.bytes) + " bytes, the layout needs " +
                    std::to_string(bufs[i].bytes));
            if (e.offset % kPackAlign || e.offset > fm.n || e.bytes > fm.n - e.offset)
                bad("buffer " + std::to_string(i) + " lies outside the file");
        }
        for (size_t b = 0; b < c->blocks.size(); ++b) {
            // a flag set needs its buffers
            const size_t base = kPackTop + b * kPackPerBlock;
            const bool ln1 = flags[3 * b] != 0, ln2 = flags[3 * b + 1] != 0, qb = flags[3 * b + 2] != 0;
            if ((ln1 && (!tab[base + kPackLn1].bytes || !tab[base + kPackLn1 + 1].bytes)) ||
                (ln2 && (!tab[base + kPackLn2].bytes || !tab[base + kPackLn2 + 1].bytes)) ||
                (qb && !tab[base + kPackQkvBias].bytes))
                bad("block " + std::to_string(b) + " flags a buffer the image lacks");
        }
        // every checksum before any upload, so a bad image changes nothing
        for (size_t i = 0; i < bufs.size(); ++i)
            if (tab[i].bytes && pack_checksum(fm.p + tab[i].offset, tab[i].bytes) != tab[i].checksum)
                bad("checksum mismatch in buffer " + std::to_string(i));
        for (size_t i = 0; i < bufs.size(); ++i) {
            if (!tab[i].bytes) continue;
            DevMem & m = *bufs[i].m;
            if (m.p && m.bytes < tab[i].bytes) {
                hip_check(hipFree(m.p), "hipFree");
                m.p = nullptr;
                m.bytes = 0;
            }
            if (!m.p) m.ensure(tab[i].bytes, false);
            copy_to_device(m.p, fm.p + tab[i].offset, tab[i].bytes, "upload packed weights");
        }
        for (size_t b = 0; b < c->blocks.size(); ++b) {
            c->blocks[b]->has_ln1 = flags[3 * b] != 0;
            c->blocks[b]->has_ln2 = flags[3 * b + 1] != 0;
            c->blocks[b]->has_qkv_bias = flags[3 * b + 2] != 0;
        }
        const char * nm = reinterpret_cast<const char *>(fm.p + sizeof(PackHeader));
        std::string cur;
        for (uint64_t i = 0; i < hd.names_bytes; ++i) {
            if (nm[i] == '\n') {
                if (!cur.empty()) c->have[cur] = 1;
                cur.clear();
            } else {
                cur += nm[i];
            }
        }
        weights_changed(c, true);
        check_ready(c);
    });
}

int sana_dit_set_context(sana_dit * c, const float * data, int64_t B, int64_t L, int64_t dim, int projected,
                         const float * bias) {
    if (!c || !data) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    if (B <= 0 || L <= 0 || L > 512) return set_err(SANA_ERR_INVALID_ARGUMENT, "context batch/length out of range");
    if (dim != (projected ? c->C : c->Ccap))
        return set_err(SANA_ERR_SHAPE, "context feature width %lld does not match %s", (long long)dim,
                       projected ? "hidden" : "caption_dim");
    return guarded([&] {
        check_context_weights(c, projected == 0);
        ensure_context_buffers(c, B, L);
        const size_t n = (size_t)B * L * dim;
        DevMem & dst = projected ? c->ctx32 : c->cap32;
        hip_check(hipMemcpyAsync(dst.p, data, n * 4, hipMemcpyHostToDevice, c->stream), "upload context");
        c->ctx_bias = bias != nullptr;
        if (bias)
            hip_check(hipMemcpyAsync(c->bias.p, bias, (size_t)B * L * 4, hipMemcpyHostToDevice, c->stream),
                      "upload bias");
        enqueue_context(c, dst.as<float>(), projected != 0, B, L, c->stream);
        hip_check(hipStreamSynchronize(c->stream), "context");
        c->ctx_ready = true;
    });
}

int sana_dit_get_context(sana_dit * c, float * out) {
    if (!c || !out) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    if (!c->ctx_ready) return set_err(SANA_ERR_STATE, "no context set");
    return guarded([&] {
        // the context may have been computed on the context's stream or a caller's
        hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
        hip_check(hipMemcpy(out, c->ctx32.p, (size_t)c->ctx_B * c->ctx_L * c->C * 4, hipMemcpyDeviceToHost),
                  "download context");
    });
}

static int check_forward_args(sana_dit * c, int64_t Bl, int64_t Hh, int64_t Ww) {
    if (Bl <= 0 || Hh <= 0 || Ww <= 0) return set_err(SANA_ERR_INVALID_ARGUMENT, "latent dims must be positive");
    if (Hh * Ww > 65535) return set_err(SANA_ERR_INVALID_ARGUMENT, "grid too large");
    // Any H x W whose token count is a perfect square, as infer_square_side
    // (src/transformer.cpp:18-24): the patch embedding and the final layer only
    // see the flattened NCHW pixel index y * W + x, and the depthwise conv of
    // every block runs on the side x side grid of the tokens
    // (src/transformer.cpp:765-767), whatever H and W are.
    const int64_t N = Hh * Ww, side = (int64_t)std::llround(std::sqrt((double)N));
    if (side * side != N) return set_err(SANA_ERR_INVALID_ARGUMENT, "token count must form a square grid");
    (void)c;
    return SANA_OK;
}

int sana_dit_forward_device(sana_dit * c, const float * d_latent, int64_t Bl, int64_t Hh, int64_t Ww, float t,
                            float * d_out, void * stream) {
    if (!c || !d_latent || !d_out) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    int rc = check_forward_args(c, Bl, Hh, Ww);
    if (rc) return rc;
    if (!c->ctx_ready) return set_err(SANA_ERR_STATE, "no context set");
    if (c->ctx_B != 2 * Bl)
        return set_err(SANA_ERR_INVALID_ARGUMENT, "context batch size must equal 2 * latent batch size for CFG");
    return guarded([&] {
        hipStream_t s = stream ? static_cast<hipStream_t>(stream) : c->stream;
        const int64_t B = 2 * Bl, N = Hh * Ww;
        ensure_forward_buffers(c, B, N);
        c->last_M = B * N;
        c->last_B = B;
        c->last_N = N;
        set_t(c, B, t, s);
        run_graph(c, std::make_tuple(1, Bl, Hh, Ww, c->ctx_L, (const void *)d_latent, (const void *)d_out,
                                     (const void *)nullptr, (const void *)(intptr_t)c->ctx_bias),
                  s, [&](hipStream_t gs) {
                      enqueue_forward(c, d_latent, Bl, Hh, Ww, c->ctx_bias ? c->bias.as<float>() : nullptr, d_out, gs);
                  });
    });
}

int sana_dit_forward(sana_dit * c, const float * latent, int64_t Bl, int64_t Hh, int64_t Ww, float t,
                     float * noise_pred) {
    if (!c || !latent || !noise_pred) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    int rc = check_forward_args(c, Bl, Hh, Ww);
    if (rc) return rc;
    return guarded([&] {
        const int64_t B = 2 * Bl, N = Hh * Ww;
        ensure_forward_buffers(c, B, N);
        hip_check(hipMemcpyAsync(c->lat_in.p, latent, (size_t)Bl * c->Cl * N * 4, hipMemcpyHostToDevice, c->stream),
                  "upload latent");
        int r = sana_dit_forward_device(c, c->lat_in.as<float>(), Bl, Hh, Ww, t, c->np_out.as<float>(), c->stream);
        if (r != SANA_OK) throw_err(r, g_last_error);
        hip_check(hipMemcpyAsync(noise_pred, c->np_out.p, (size_t)B * c->Cl * N * 4, hipMemcpyDeviceToHost, c->stream),
                  "download");
        hip_check(hipStreamSynchronize(c->stream), "forward");
    });
}

int sana_dit_step_device(sana_dit * c, const float * d_caption, int64_t L, const float * d_bias,
                         const float * d_latent, int64_t Bl, int64_t Hh, int64_t Ww, float t, float * d_out,
                         void * stream) {
    if (!c || !d_caption || !d_latent || !d_out) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    int rc = check_forward_args(c, Bl, Hh, Ww);
    if (rc) return rc;
    if (L <= 0 || L > 512) return set_err(SANA_ERR_INVALID_ARGUMENT, "caption length out of range");
    return guarded([&] {
        check_ready(c);
        hipStream_t s = stream ? static_cast<hipStream_t>(stream) : c->stream;
        const int64_t B = 2 * Bl, N = Hh * Ww;
        ensure_context_buffers(c, B, L);
        ensure_forward_buffers(c, B, N);
        c->last_M = B * N;
        c->last_B = B;
        c->last_N = N;
        set_t(c, B, t, s);
        run_graph(c, std::make_tuple(2, Bl, Hh, Ww, L, (const void *)d_caption, (const void *)d_bias,
                                     (const void *)d_latent, (const void *)d_out),
                  s, [&](hipStream_t gs) { enqueue_step(c, d_caption, L, d_latent, Bl, Hh, Ww, d_bias, d_out, gs); });
        // keep the context state consistent for later sana_dit_forward* calls
        c->ctx_bias = d_bias != nullptr;
        if (d_bias)
            hip_check(hipMemcpyAsync(c->bias.p, d_bias, (size_t)B * L * 4, hipMemcpyDeviceToDevice, s), "bias");
        c->ctx_ready = true;
    });
}

int sana_dit_block_forward(sana_dit * c, int64_t blk, const float * x, const float * t_mod, int64_t B, int64_t N,
                           float * a_self, float * a_cross, float * a_ff) {
    if (!c || !x || !t_mod) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    if (blk < 0 || blk >= c->L_) return set_err(SANA_ERR_INVALID_ARGUMENT, "block index out of range");
    if (!c->ctx_ready) return set_err(SANA_ERR_STATE, "no context set");
    if (B != c->ctx_B) return set_err(SANA_ERR_INVALID_ARGUMENT, "input and context batch size must match");
    const int64_t side = (int64_t)std::llround(std::sqrt((double)N));
    if (N <= 0 || side * side != N) return set_err(SANA_ERR_INVALID_ARGUMENT, "token count must form a square grid");
    return guarded([&] {
        check_block(c, blk);
        ensure_forward_buffers(c, B, N);
        const size_t n = (size_t)B * N * c->C;
        hip_check(hipMemcpyAsync(c->x32.p, x, n * 4, hipMemcpyHostToDevice, c->stream), "upload x");
        hip_check(hipMemcpyAsync(c->tmod.p, t_mod, (size_t)B * 6 * c->C * 4, hipMemcpyHostToDevice, c->stream),
                  "upload t_mod");
        enqueue_mod(c, B, c->stream);
        struct Hook {
            sana_dit * c;
            size_t n;
            float * outs[3];
        } h{c, n, {a_self, a_cross, a_ff}};
        enqueue_block(c, blk, B, N, c->ctx_bias ? c->bias.as<float>() : nullptr, c->stream, [](void * p, int stage) {
            Hook * hk = static_cast<Hook *>(p);
            if (hk->outs[stage])
                hip_check(hipMemcpyAsync(hk->outs[stage], hk->c->x32.p, hk->n * 4, hipMemcpyDeviceToHost, hk->c->stream),
                          "download stage");
        }, &h);
        hip_check(hipStreamSynchronize(c->stream), "block_forward");
    });
}

int sana_dit_run_blocks(sana_dit * c, int64_t begin, int64_t end, const float * x, const float * t_mod, int64_t B,
                        int64_t N, float * out) {
    if (!c || !x || !t_mod || !out) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    if (begin < 0 || begin > end || end > c->L_) return set_err(SANA_ERR_INVALID_ARGUMENT, "invalid model block range");
    if (!c->ctx_ready) return set_err(SANA_ERR_STATE, "no context set");
    if (B != c->ctx_B) return set_err(SANA_ERR_INVALID_ARGUMENT, "input and context batch size must match");
    const int64_t side = (int64_t)std::llround(std::sqrt((double)N));
    if (N <= 0 || side * side != N) return set_err(SANA_ERR_INVALID_ARGUMENT, "token count must form a square grid");
    return guarded([&] {
        for (int64_t i = begin; i < end; ++i) check_block(c, i);
        ensure_forward_buffers(c, B, N);
        const size_t n = (size_t)B * N * c->C;
        hip_check(hipMemcpyAsync(c->x32.p, x, n * 4, hipMemcpyHostToDevice, c->stream), "upload x");
        hip_check(hipMemcpyAsync(c->tmod.p, t_mod, (size_t)B * 6 * c->C * 4, hipMemcpyHostToDevice, c->stream),
                  "upload t_mod");
        enqueue_mod(c, B, c->stream);
        for (int64_t i = begin; i < end; ++i)
            enqueue_block(c, i, B, N, c->ctx_bias ? c->bias.as<float>() : nullptr, c->stream);
        hip_check(hipMemcpyAsync(out, c->x32.p, n * 4, hipMemcpyDeviceToHost, c->stream), "download x");
        hip_check(hipStreamSynchronize(c->stream), "run_blocks");
    });
}

namespace {

float flow_lambda(float sigma) {  // log(alpha) - log(sigma) with alpha = 1 - sigma
    return std::log(1.0f - sigma) - std::log(sigma);
}

// The whole loop on `s`: step i runs the forward at timesteps[i] on latent
// buffer i % 2 and writes buffer (i + 1) % 2; the converted outputs of the two
// latest steps alternate in loop_x0.  With graphs on, the whole loop (latent
// copy, and per step the timestep fill, the forward and the CFG + solver
// update) is one graph, captured once per shape, buffers and schedule.
// Returns the buffer holding the result.
float * enqueue_loop(sana_dit * c, const float * d_latent, int64_t Bl, int64_t Hh, int64_t Ww, const float * ts,
                     const float * sg, int64_t steps, float guidance, hipStream_t s) {
    const int64_t n = Bl * c->Cl * Hh * Ww;
    const int64_t B = 2 * Bl, N = Hh * Ww;
    for (int k = 0; k < 2; ++k) {
        c->loop_lat[k].ensure((size_t)n * 4, false);
        c->loop_x0[k].ensure((size_t)n * 4, false);
    }
    c->last_M = B * N;
    c->last_B = B;
    c->last_N = N;
    const float * xbias = c->ctx_bias ? c->bias.as<float>() : nullptr;
    auto body = [&](hipStream_t gs) {
        hip_check(hipMemcpyAsync(c->loop_lat[0].p, d_latent, (size_t)n * 4, hipMemcpyDeviceToDevice, gs), "latent");
        for (int64_t i = 0; i < steps; ++i) {
            float * cur = c->loop_lat[i & 1].as<float>();
            float * nxt = c->loop_lat[(i + 1) & 1].as<float>();
            set_t(c, B, ts[i], gs);
            enqueue_forward(c, cur, Bl, Hh, Ww, xbias, c->np_out.as<float>(), gs);
            // step_sana_scheduler (src/scheduler.cpp:272-318) with solver_order 2, midpoint,
            // lower_order_final: first order at the first and at the last step.
            const bool first = i == 0 || i == steps - 1;
            const float st_v = sg[i + 1], s0_v = sg[i];
            const float alpha_t = 1.0f - st_v;
            const float h = flow_lambda(st_v) - flow_lambda(s0_v);
            const float ca = st_v / s0_v, cb = -alpha_t * (std::exp(-h) - 1.0f);
            float cc = 0.0f, inv_r0 = 0.0f;
            if (!first) {
                const float h0 = flow_lambda(s0_v) - flow_lambda(sg[i - 1]);
                inv_r0 = 1.0f / (h0 / h);
                cc = -0.5f * alpha_t * (std::exp(-h) - 1.0f);
            }
            hipLaunchKernelGGL(cfg_dpm_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, gs,
                               c->np_out.as<float>(), cur, c->loop_x0[(i + 1) & 1].as<float>(), nxt,
                               c->loop_x0[i & 1].as<float>(), (int)n, guidance, s0_v, ca, cb, cc, inv_r0,
                               first ? 0 : 1);
            hip_check(hipGetLastError(), "cfg_dpm");
        }
    };
    if (!c->use_graphs) {
        body(s);
    } else {
        std::string key;
        for (int64_t v : {Bl, Hh, Ww, c->ctx_L, (int64_t)c->ctx_bias, steps}) key_append(key, v);
        for (const void * p : {(const void *)d_latent, (const void *)c->loop_lat[0].p, (const void *)c->loop_lat[1].p,
                               (const void *)c->loop_x0[0].p, (const void *)c->loop_x0[1].p,
                               (const void *)c->np_out.p})
            key_append(key, p);
        key_append(key, guidance);
        for (int64_t i = 0; i < steps; ++i) key_append(key, ts[i]);
        for (int64_t i = 0; i <= steps; ++i) key_append(key, sg[i]);
        auto it = c->loop_graphs.find(key);
        if (it == c->loop_graphs.end()) {
            if (c->loop_graphs.size() >= 4) drop_loop_graphs(c);
            GraphEntry e;
            e.exec = capture_graph(c, body);
            it = c->loop_graphs.emplace(key, e).first;
        }
        hip_check(hipGraphLaunch(it->second.exec, s), "hipGraphLaunch");
    }
    hip_check(hipEventRecord(c->ev_loop, s), "hipEventRecord");
    c->loop_steps = steps;
    c->loop_n = n;
    return c->loop_lat[steps & 1].as<float>();
}

int check_loop_args(sana_dit * c, int64_t Bl, int64_t Hh, int64_t Ww, const float * ts, const float * sg,
                    int64_t steps) {
    int rc = check_forward_args(c, Bl, Hh, Ww);
    if (rc) return rc;
    if (!ts || !sg || steps <= 0) return set_err(SANA_ERR_INVALID_ARGUMENT, "schedule must have at least one step");
    if (!c->ctx_ready) return set_err(SANA_ERR_STATE, "no context set");
    if (c->ctx_B != 2 * Bl)
        return set_err(SANA_ERR_INVALID_ARGUMENT, "context batch size must equal 2 * latent batch size for CFG");
    for (int64_t i = 0; i < steps; ++i)
        if (!(sg[i] > 0.0f && sg[i] < 1.0f)) return set_err(SANA_ERR_INVALID_ARGUMENT, "sigmas must lie in (0, 1)");
    if (sg[steps] != 0.0f) return set_err(SANA_ERR_INVALID_ARGUMENT, "final sigma must be 0");
    return SANA_OK;
}

}  // namespace

int sana_dit_denoise_loop_device(sana_dit * c, const float * d_latent, int64_t Bl, int64_t Hh, int64_t Ww,
                                 const float * timesteps, const float * sigmas, int64_t steps, float guidance,
                                 float * d_final, void * stream) {
    if (!c || !d_latent || !d_final) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    int rc = check_loop_args(c, Bl, Hh, Ww, timesteps, sigmas, steps);
    if (rc) return rc;
    return guarded([&] {
        hipStream_t s = stream ? static_cast<hipStream_t>(stream) : c->stream;
        ensure_forward_buffers(c, 2 * Bl, Hh * Ww);
        float * res = enqueue_loop(c, d_latent, Bl, Hh, Ww, timesteps, sigmas, steps, guidance, s);
        hip_check(hipMemcpyAsync(d_final, res, (size_t)Bl * c->Cl * Hh * Ww * 4, hipMemcpyDeviceToDevice, s), "final");
    });
}

int sana_dit_denoise_loop(sana_dit * c, const float * latent, int64_t Bl, int64_t Hh, int64_t Ww,
                          const float * timesteps, const float * sigmas, int64_t steps, float guidance,
                          float * final_latent) {
    if (!c || !latent || !final_latent) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    int rc = check_loop_args(c, Bl, Hh, Ww, timesteps, sigmas, steps);
    if (rc) return rc;
    return guarded([&] {
        const int64_t n = Bl * c->Cl * Hh * Ww;
        ensure_forward_buffers(c, 2 * Bl, Hh * Ww);
        hip_check(hipMemcpyAsync(c->lat_in.p, latent, (size_t)n * 4, hipMemcpyHostToDevice, c->stream), "latent");
        float * res = enqueue_loop(c, c->lat_in.as<float>(), Bl, Hh, Ww, timesteps, sigmas, steps, guidance, c->stream);
        hip_check(hipMemcpyAsync(final_latent, res, (size_t)n * 4, hipMemcpyDeviceToHost, c->stream), "final");
        hip_check(hipStreamSynchronize(c->stream), "denoise_loop");
    });
}

int sana_dit_loop_model_outputs(sana_dit * c, float * x0_prev, float * x0_last) {
    if (!c || !x0_last) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    if (c->loop_steps <= 0) return set_err(SANA_ERR_STATE, "no denoise loop has run");
    return guarded([&] {
        const int64_t st = c->loop_steps;
        const size_t bytes = (size_t)c->loop_n * 4;
        // the loop may have been queued on a caller's stream
        hip_check(hipStreamWaitEvent(c->stream, c->ev_loop, 0), "hipStreamWaitEvent");
        // step i writes its converted output to loop_x0[i & 1] (cfg_dpm_kernel's x0_out)
        hip_check(hipMemcpyAsync(x0_last, c->loop_x0[(st - 1) & 1].p, bytes, hipMemcpyDeviceToHost, c->stream),
                  "x0");
        if (x0_prev && st >= 2)
            hip_check(hipMemcpyAsync(x0_prev, c->loop_x0[st & 1].p, bytes, hipMemcpyDeviceToHost, c->stream), "x0");
        hip_check(hipStreamSynchronize(c->stream), "loop_model_outputs");
    });
}

int sana_dit_time_embed(sana_dit * c, const float * t, int64_t B, float * embedded, float * t_mod) {
    if (!c || !t) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    if (B <= 0) return set_err(SANA_ERR_INVALID_ARGUMENT, "batch must be positive");
    return guarded([&] {
        for (const char * n : kTopRequired) require(c, n, n);
        for (int64_t i = 0; i < c->L_; ++i) require(c, block_key(i, "scale_shift_table"), "block scale_shift_table");
        ensure_forward_buffers(c, B, 1);
        hip_check(hipMemcpyAsync(c->d_t.p, t, (size_t)B * 4, hipMemcpyHostToDevice, c->stream), "upload t");
        enqueue_time(c, B, c->stream);
        if (embedded)
            hip_check(hipMemcpyAsync(embedded, c->emb.p, (size_t)B * c->C * 4, hipMemcpyDeviceToHost, c->stream), "dl");
        if (t_mod)
            hip_check(hipMemcpyAsync(t_mod, c->tmod.p, (size_t)B * 6 * c->C * 4, hipMemcpyDeviceToHost, c->stream),
                      "dl");
        hip_check(hipStreamSynchronize(c->stream), "time_embed");
    });
}

int sana_dit_time_kernel(sana_dit * c, int which, int iters, float * avg_ms, double * flops, double * bytes,
                         char * name, size_t name_cap) {
    if (!c || !avg_ms || iters <= 0) return set_err(SANA_ERR_INVALID_ARGUMENT, "bad argument");
    if (c->last_M <= 0) return set_err(SANA_ERR_STATE, "run a forward first");
    if (which < 0 || which > 9) return set_err(SANA_ERR_INVALID_ARGUMENT, "which must be 0..9");
    if (!c->ctx_ready) return set_err(SANA_ERR_STATE, "no context set");
    return guarded([&] {
        // The shape and launch of the last forward: one batch row per launch
        // (co = 2) when the CFG pair ran as two branches, else the whole batch.
        const int64_t N = c->last_N, C = c->C, E = c->E, F = c->F, Lc = c->ctx_L, Btot = c->last_B;
        const bool branches = Btot == 2 && c->cfg_branches;
        const int64_t B = branches ? 1 : Btot, M = B * N, side = (int64_t)std::llround(std::sqrt((double)N));
        const int co = branches ? 2 : 1;
        hipStream_t s = c->stream;
        const float * xbias = c->ctx_bias ? c->bias.as<float>() : nullptr;
        // Launch i runs block i mod layers, as the forward cycles through the
        // blocks, so the weights come from HBM; outputs go to the forward's own
        // buffers (they are overwritten).
        auto run = [&](int i) {
            const int64_t blk = i % c->L_;
            BlockDev & w = *c->blocks[blk];
            const float * mod = c->mod_all.as<float>() + (size_t)blk * Btot * 6 * C;
            half_t * kt16 = c->la_kt.as<half_t>();
            half_t * vt16 = c->la_vt.as<half_t>();
            switch (which) {
                case 0:
                    if (qkv_split_layout(c, N))
                        gemm_qkv_split(c, w, B, N, c->xa16.as<half_t>(), c->qkv16.as<half_t>(), kt16, vt16, co, s);
                    else
                        gemm_store(c, c->xa16.as<half_t>(), c->Cp, w.w_qkv.as<half_t>(), c->Cp, M, 3 * C, c->Cp,
                                   nullptr, sana::kActNone, c->qkv16.as<half_t>(), 3 * C, nullptr, 0, s, co);
                    break;
                case 1:
                    gemm_resid(c->o16.as<half_t>(), c->Cp, w.w_out.as<half_t>(), c->Cp, M, C, c->Cp,
                               w.b_out.as<float>(), mod + 2 * C, nullptr, 6 * C, N, c->x32.as<float>(), C,
                               c->r16.as<half_t>(), c->Cp, s, co);
                    break;
                case 2:
                    gemm_store(c, c->r16.as<half_t>(), c->Cp, w.w_cq.as<half_t>(), c->Cp, M, C, c->Cp,
                               w.b_cq.as<float>(), sana::kActNone, c->q16.as<half_t>(), C, nullptr, 0, s, co);
                    break;
                case 3:
                    gemm_resid(c->o16.as<half_t>(), c->Cp, w.w_co.as<half_t>(), c->Cp, M, C, c->Cp,
                               w.b_co.as<float>(), nullptr, nullptr, 0, N, c->x32.as<float>(), C, nullptr, 0, s, co);
                    break;
                case 4:
                    gemm_store(c, c->xa16.as<half_t>(), c->Cp, w.w_inv.as<half_t>(), c->Cp, M, E, c->Cp,
                               w.b_inv.as<float>(), sana::kActSilu, c->hid16.as<half_t>(), E, nullptr, 0, s, co);
                    break;
                case 5:
                    gemm_resid(c->glu16.as<half_t>(), c->Fp, w.w_pt.as<half_t>(), c->Fp, M, C, c->Fp, nullptr,
                               mod + 5 * C, nullptr, 6 * C, N, c->x32.as<float>(), C, nullptr, 0, s, co);
                    break;
                case 6:
                    launch_check(sana::ln_modulate(c->x32.as<float>(), C, c->xa16.as<half_t>(), c->Cp, (int)M, (int)C,
                                                   (int)N, 1e-6f, w.has_ln1 ? w.ln1_g.as<float>() : nullptr,
                                                   w.has_ln1 ? w.ln1_b.as<float>() : nullptr, mod, nullptr, 6 * C, 0,
                                                   C, s),
                                 "ln_modulate");
                    break;
                case 7:
                    if (fused_linear_attention(c, N))
                        launch_check(sana::linear_attention_fused(c->qkv16.as<half_t>(), 3 * C, kt16, vt16,
                                                                  c->o16.as<half_t>(), c->Cp, (int)B, (int)N,
                                                                  (int)c->Hs, (int)c->Ds, s, co),
                                     "linear_attention_fused");
                    else if (qkv_split_layout(c, N))
                        launch_check(sana::linear_attention_chunked(c->qkv16.as<half_t>(), 3 * C, kt16, vt16,
                                                                    c->o16.as<half_t>(), c->Cp, (int)B, (int)N,
                                                                    (int)c->Hs, (int)c->Ds, c->la_ws.as<float>(), s),
                                     "linear_attention_chunked");
                    else
                        launch_check(sana::linear_attention(c->qkv16.as<half_t>(), c->qkv16.as<half_t>() + C,
                                                            c->qkv16.as<half_t>() + 2 * C, 3 * C, c->o16.as<half_t>(),
                                                            c->Cp, (int)B, (int)N, (int)c->Hs, (int)c->Ds,
                                                            c->la_ws.as<float>(), s),
                                     "linear_attention");
                    break;
                case 8: {
                    const half_t * kc = c->kc.as<half_t>() + blk * C;
                    const half_t * vt = c->vt.as<half_t>() + (size_t)blk * Btot * C * c->ctx_Lp;
                    launch_check(sana::cross_attention(c->q16.as<half_t>(), C, kc, c->L_ * C, vt, c->ctx_Lp, xbias,
                                                       c->o16.as<half_t>(), c->Cp, (int)B, (int)N, (int)Lc, (int)c->Hc,
                                                       (int)c->Dc, s),
                                 "cross_attention");
                    break;
                }
                default:
                    launch_check(sana::dwconv_glu(c->hid16.as<half_t>(), E, w.w_dw.as<float>(), w.b_dw.as<float>(),
                                                  c->glu16.as<half_t>(), c->Fp, (int)B, (int)side, (int)side, (int)F,
                                                  s),
                                 "dwconv_glu");
            }
        };
        // algorithmic work per launch: flops of the contractions; bytes of the
        // interface tensors at their stored precision (weights included for the
        // GEMMs, no re-reads)
        const double m = (double)M, h2 = 2.0, f4 = 4.0;
        double fl = 0.0, by = 0.0;
        switch (which) {
            case 0: fl = 2 * m * 3 * C * C; by = h2 * (m * C + 3.0 * C * C + m * 3 * C); break;
            case 1: fl = 2 * m * C * C; by = h2 * (m * C + (double)C * C + m * C) + f4 * 2 * m * C; break;
            case 2: fl = 2 * m * C * C; by = h2 * (m * C + (double)C * C + m * C); break;
            case 3: fl = 2 * m * C * C; by = h2 * (m * C + (double)C * C) + f4 * 2 * m * C; break;
            case 4: fl = 2 * m * E * C; by = h2 * (m * C + (double)E * C + m * E); break;
            case 5: fl = 2 * m * C * F; by = h2 * (m * F + (double)C * F) + f4 * 2 * m * C; break;
            case 6: fl = 0.0; by = f4 * m * C + h2 * m * C; break;
            case 7: fl = 2.0 * 2 * B * N * c->Hs * (c->Ds + 1) * c->Ds; by = h2 * 4 * m * C; break;
            case 8: fl = 2.0 * 2 * B * N * Lc * C; by = h2 * (2 * m * C + 2.0 * B * Lc * C); break;
            default: fl = 2.0 * m * E * 9; by = h2 * (m * E + m * F); break;
        }
        run(c->L_ - 1);  // warm
        hipEvent_t e0, e1;
        hip_check(hipEventCreate(&e0), "event");
        hip_check(hipEventCreate(&e1), "event");
        hip_check(hipEventRecord(e0, s), "record");
        for (int i = 0; i < iters; ++i) run(i);
        hip_check(hipEventRecord(e1, s), "record");
        hip_check(hipEventSynchronize(e1), "sync");
        float ms = 0.0f;
        hip_check(hipEventElapsedTime(&ms, e0, e1), "elapsed");
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        *avg_ms = ms / iters;
        if (flops) *flops = fl;
        if (bytes) *bytes = by;
        if (name && name_cap) {
            const std::string nm = sana::last_kernel();
            const size_t n = std::min(nm.size(), name_cap - 1);
            std::memcpy(name, nm.data(), n);
            name[n] = '\0';
        }
    });
}

// ---------------------------------------------------------------- kernel-level launchers
int sana_hip_gemm(const void * A, int64_t lda, const void * W, int64_t ldw, int64_t M, int64_t N, int64_t K,
                  const float * bias, int act, void * out16, int64_t ldo16, float * out32, int64_t ldo32,
                  void * stream) {
    if (act < 0 || act > 3) return set_err(SANA_ERR_INVALID_ARGUMENT, "act must be 0..3");
    return guarded([&] {
        gemm_store(nullptr, static_cast<const half_t *>(A), lda, static_cast<const half_t *>(W), ldw, M, N, K, bias, act,
                   static_cast<half_t *>(out16), ldo16, out32, ldo32, static_cast<hipStream_t>(stream));
    });
}

int sana_hip_gemm_residual(const void * A, int64_t lda, const void * W, int64_t ldw, int64_t M, int64_t N, int64_t K,
                           const float * bias, const float * gate_a, const float * gate_t, int64_t gate_stride,
                           int64_t rpb, float * x, int64_t ldx, void * out16, int64_t ldo16, void * stream) {
    return guarded([&] {
        gemm_resid(static_cast<const half_t *>(A), lda, static_cast<const half_t *>(W), ldw, M, N, K, bias, gate_a,
                   gate_t, gate_stride, rpb, x, ldx, static_cast<half_t *>(out16), ldo16,
                   static_cast<hipStream_t>(stream));
    });
}

int sana_hip_ln_modulate(const float * x, int64_t ldx, void * out16, int64_t ldo, int64_t M, int64_t C, int64_t rpb,
                         float eps, const float * gamma, const float * beta, const float * mod_a, const float * mod_t,
                         int64_t mod_stride, int64_t shift_off, int64_t scale_off, void * stream) {
    return guarded([&] {
        launch_check(sana::ln_modulate(x, ldx, static_cast<half_t *>(out16), ldo, (int)M, (int)C, (int)rpb, eps, gamma,
                                       beta, mod_a, mod_t, mod_stride, shift_off, scale_off,
                                       static_cast<hipStream_t>(stream)),
                     "ln_modulate");
    });
}

size_t sana_hip_linear_attention_workspace(int64_t B, int64_t N, int64_t H, int64_t D) {
    return sana::linattn_workspace_floats((int)B, (int)N, (int)H, (int)D) * sizeof(float);
}

int sana_hip_linear_attention(const void * q, const void * k, const void * v, int64_t ld, void * out, int64_t ldo,
                              int64_t B, int64_t N, int64_t H, int64_t D, float * ws, void * stream) {
    return guarded([&] {
        launch_check(sana::linear_attention(static_cast<const half_t *>(q), static_cast<const half_t *>(k),
                                            static_cast<const half_t *>(v), ld, static_cast<half_t *>(out), ldo,
                                            (int)B, (int)N, (int)H, (int)D, ws, static_cast<hipStream_t>(stream)),
                     "linear_attention");
    });
}

int sana_hip_linear_attention_noalloc(const void * q, const void * k, const void * v, int64_t ld, void * out,
                                      int64_t ldo, int64_t B, int64_t N, int64_t H, int64_t D, void * stream) {
    return guarded([&] {
        if (B <= 0 || N <= 0 || H <= 0 || D <= 0 || D > 112 || B * H > 65535 || N > (1 << 30))
            throw_err(SANA_ERR_INVALID_ARGUMENT, "linear_attention_noalloc: B, H >= 1 with B * H <= 65535, "
                                                 "N in [1, 2^30], D in [1, 112]");
        const size_t need = sana::linattn_workspace_floats((int)B, (int)N, (int)H, (int)D);
        if (need > kLaScratchFloats)
            throw_err(SANA_ERR_INVALID_ARGUMENT,
                      "linear_attention_noalloc: needs " + std::to_string(need * sizeof(float)) +
                          " bytes of scratch, above the static " + std::to_string(kLaScratchFloats * sizeof(float)) +
                          " (use sana_hip_linear_attention with a workspace)");
        int dev = 0;
        hip_check(hipGetDevice(&dev), "hipGetDevice");
        float * ws = device_scratch(dev);
        launch_check(sana::linear_attention(static_cast<const half_t *>(q), static_cast<const half_t *>(k),
                                            static_cast<const half_t *>(v), ld, static_cast<half_t *>(out), ldo,
                                            (int)B, (int)N, (int)H, (int)D, ws, static_cast<hipStream_t>(stream)),
                     "linear_attention_noalloc");
    });
}

int sana_hip_cross_attention(const void * q, int64_t ldq, const void * k, int64_t ldk, const void * vt, int64_t ldvt,
                             const float * bias, void * out, int64_t ldo, int64_t B, int64_t N, int64_t L, int64_t H,
                             int64_t D, void * stream) {
    return guarded([&] {
        launch_check(sana::cross_attention(static_cast<const half_t *>(q), ldq, static_cast<const half_t *>(k), ldk,
                                           static_cast<const half_t *>(vt), ldvt, bias, static_cast<half_t *>(out), ldo,
                                           (int)B, (int)N, (int)L, (int)H, (int)D, static_cast<hipStream_t>(stream)),
                     "cross_attention");
    });
}

int sana_hip_dwconv_glu(const void * x, int64_t ldx, const float * wt, const float * bias, void * out, int64_t ldo,
                        int64_t B, int64_t Hh, int64_t Ww, int64_t F, void * stream) {
    return guarded([&] {
        launch_check(sana::dwconv_glu(static_cast<const half_t *>(x), ldx, wt, bias, static_cast<half_t *>(out), ldo,
                                      (int)B, (int)Hh, (int)Ww, (int)F, static_cast<hipStream_t>(stream)),
                     "dwconv_glu");
    });
}

int sana_hip_hbm_peak(const void * src, void * dst, int64_t bytes, float * sink, int64_t * sink_floats,
                      void * stream) {
    return guarded([&] {
        if (sink_floats) *sink_floats = (int64_t)sana::hbm_peak_workgroups() * 256;
        if (!src && !dst && !sink && bytes == 0) return;
        if (!src || bytes < 16 || bytes % 16 || (!dst && !sink))
            throw SanaError{SANA_ERR_INVALID_ARGUMENT, "hbm_peak: src, bytes (a positive multiple of 16) and dst or "
                                                       "sink required"};
        launch_check(sana::hbm_peak(src, dst, bytes, sink, static_cast<hipStream_t>(stream)), "hbm_peak");
    });
}

int sana_hip_mfma_peak(int64_t workgroups, int64_t iters, int zero_operands, float * sink, void * stream,
                       double * flops) {
    return guarded([&] {
        if (workgroups <= 0 || workgroups > 65536 || iters <= 0 || iters > (1 << 24) || !sink || !flops)
            throw SanaError{SANA_ERR_INVALID_ARGUMENT, "mfma_peak: workgroups in [1, 65536], iters in [1, 2^24], "
                                                       "sink and flops required"};
        launch_check(sana::mfma_peak((int)workgroups, (int)iters, zero_operands != 0, sink,
                                     static_cast<hipStream_t>(stream)),
                     "mfma_peak");
        *flops = sana::mfma_peak_flops((int)workgroups, (int)iters);
    });
}

}  // extern "C"
