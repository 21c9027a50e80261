// DC-AE VAE decoder (the stage after the denoising loop, src/vae.cpp:243-325,
// src/vae_ops.cpp) on one MI355X, and its C ABI.
//
// Layout: activations are NHWC ("token-major", [B * H * W, C]) on the device.
//   residual   fp32 [P, C], P = B * H * W (the reference's NCHW hidden tensor);
//   conv input fp16 with a one-pixel zero border, [B][(H + 2) * (W + 2)][C],
//              so every 3x3 tap of an output pixel is one contiguous channel
//              run and the implicit-GEMM conv (gemm.hip, conv modes) needs no
//              bounds checks;
//   1x1 input  fp16 [P, C].
// Every 1x1 and 3x3 convolution is an MFMA GEMM (3x3: K = 9 taps x C,
// tap-major weights; the nearest-2x upsample is folded into the A addressing);
// the RMSNorm + residual, the conv_in shortcut, the depthwise 5x5 and the grouped
// 1x1 of the multiscale attention are the kernels below; the ReLU linear
// attention and the depthwise 3x3 + GLU of GLUMBConv are the DiT's kernels.
//
// Multiscale attention heads.  The reference treats each 3 * 32 consecutive
// channels of concat(q, k, v) (and of its multiscale branch) as one head's
// q | k | v (src/vae_ops.cpp:705-713).  The upload permutes those 32-channel
// groups so that head h's q, k and v sit at h * 32 in three contiguous
// [q | k | v] sections; the depthwise 5x5 and grouped 1x1 act per channel and
// per group, so the same permutation of their weights keeps them exact.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/sana_dit.h"
#include "gguf.h"
#include "hip_common.h"
#include "host_util.h"
#include "kernels.h"

using sana::half_t;
using namespace sana_host;

namespace {

constexpr int kVaeHead = 32;  // head dim and grouped-conv group size

// ---------------------------------------------------------------------------
// kernels

// Scaled latent (x / scaling_factor, NCHW fp32) -> the bordered NHWC fp16
// conv_in input [B][(h + 2) * (w + 2)][64] (channels past Cl and the border
// zero), and the channel-repeat shortcut of run_vae_decoder_input
// (src/vae.cpp:233-240): x32[p][c] = scaled[c / rep] at pixel p (0 without
// the shortcut).
__global__ void vae_prep_kernel(const float * __restrict__ lat, int B, int Cl, int h, int w, float inv_sf,
                                f16 * __restrict__ pad, int ldp, float * __restrict__ x32, int Ctop, int rep,
                                int shortcut) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t npad = (int64_t)B * (h + 2) * (w + 2) * ldp;
    if (i < npad) {
        const int c = (int)(i % ldp);
        const int64_t q = i / ldp;
        const int xx = (int)(q % (w + 2)) - 1, yy = (int)((q / (w + 2)) % (h + 2)) - 1;
        const int b = (int)(q / ((int64_t)(w + 2) * (h + 2)));
        float v = 0.0f;
        if (c < Cl && yy >= 0 && yy < h && xx >= 0 && xx < w) v = lat[(((int64_t)b * Cl + c) * h + yy) * w + xx] * inv_sf;
        pad[i] = (f16)v;
    }
    const int64_t nx = (int64_t)B * h * w * Ctop;
    if (i < nx) {
        const int oc = (int)(i % Ctop);
        const int64_t p = i / Ctop;
        const int xx = (int)(p % w), yy = (int)((p / w) % h), b = (int)(p / ((int64_t)w * h));
        x32[i] = shortcut ? lat[(((int64_t)b * Cl + oc / rep) * h + yy) * w + xx] * inv_sf : 0.0f;
    }
}

// Zero the one-pixel border of a [B][(H + 2) * (W + 2)][ld] fp16 buffer.
__global__ void vae_zero_border_kernel(f16 * __restrict__ buf, int B, int H, int W, int ld) {
    const int per = 2 * (W + 2) + 2 * H;  // border pixels per image
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t n = (int64_t)B * per * (ld / 8);
    if (i >= n) return;
    const int c8 = (int)(i % (ld / 8));
    const int64_t q = i / (ld / 8);
    const int b = (int)(q / per), k = (int)(q % per);
    int y, x;
    if (k < W + 2) {
        y = 0;
        x = k;
    } else if (k < 2 * (W + 2)) {
        y = H + 1;
        x = k - (W + 2);
    } else {
        const int r = k - 2 * (W + 2);
        y = 1 + r / 2;
        x = (r & 1) ? W + 1 : 0;
    }
    f16x8 z;
#pragma unroll
    for (int e = 0; e < 8; ++e) z[e] = (f16)0.0f;
    *reinterpret_cast<f16x8 *>(buf + (((int64_t)b * (H + 2) + y) * (W + 2) + x) * ld + c8 * 8) = z;
}

// Per-pixel RMSNorm over channels (rms_norm_4d_channelwise,
// src/vae_ops.cpp:476-560): v = x / sqrt(mean(x^2) + eps) * w + b, then the
// block's residual (+ res, src/vae_ops.cpp:581,605,804) and the decoder's
// final ReLU (src/vae.cpp:320).  One wave per pixel; fp32 out and/or fp16 out
// (plain, or into the interior of a bordered H x W grid when pad != 0).
template <int NC4>  // float4 chunks per lane, C <= 256 * NC4
__global__ __launch_bounds__(256) void vae_rmsnorm_kernel(const float * __restrict__ x, int C, int P,
                                                          const float * __restrict__ w,
                                                          const float * __restrict__ bias,
                                                          const float * __restrict__ res, int relu, float eps,
                                                          float * __restrict__ out32, f16 * __restrict__ out16,
                                                          int pad, int H, int W) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= P) return;
    const int n4 = C >> 2;
    const float4 * xr = reinterpret_cast<const float4 *>(x + (int64_t)row * C);
    float4 v[NC4];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < NC4; ++i) {
        const int c4 = lane + 64 * i;
        if (c4 < n4) {
            v[i] = xr[c4];
            ss += (v[i].x * v[i].x + v[i].y * v[i].y) + (v[i].z * v[i].z + v[i].w * v[i].w);
        } else {
            v[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
    const float inv = 1.0f / sqrtf(wave_sum(ss) * (1.0f / (float)C) + eps);
    int64_t orow = row;
    if (pad) {
        const int hw = H * W, img = row / hw, rem = row - img * hw, yy = rem / W, xx = rem - yy * W;
        orow = ((int64_t)img * (H + 2) + yy + 1) * (W + 2) + xx + 1;
    }
#pragma unroll
    for (int i = 0; i < NC4; ++i) {
        const int c4 = lane + 64 * i;
        if (c4 >= n4) continue;
        const float4 g = reinterpret_cast<const float4 *>(w)[c4];
        const float4 bb = bias ? reinterpret_cast<const float4 *>(bias)[c4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float o[4] = {v[i].x * inv * g.x + bb.x, v[i].y * inv * g.y + bb.y, v[i].z * inv * g.z + bb.z,
                      v[i].w * inv * g.w + bb.w};
        if (res) {
            const float4 r = reinterpret_cast<const float4 *>(res + (int64_t)row * C)[c4];
            o[0] += r.x; o[1] += r.y; o[2] += r.z; o[3] += r.w;
        }
        if (relu) {
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = fmaxf(o[e], 0.0f);
        }
        if (out32) reinterpret_cast<float4 *>(out32 + (int64_t)row * C)[c4] = make_float4(o[0], o[1], o[2], o[3]);
        if (out16) {
            f16x4 h;
#pragma unroll
            for (int e = 0; e < 4; ++e) h[e] = (f16)o[e];
            *reinterpret_cast<f16x4 *>(out16 + orow * C + 4 * c4) = h;
        }
    }
}

// Depthwise 5x5, zero padding, no bias (the multiscale proj_in,
// depthwise_conv5x5_process_plane src/common_ops.cpp:628-649): taps in (ky, kx)
// order.  Token-major fp16 in/out [P][C], tap-major fp32 weights [25][C]; one
// thread per (pixel, 8 channels).
__global__ __launch_bounds__(256) void vae_dw5x5_kernel(const f16 * __restrict__ in, const float * __restrict__ w,
                                                        f16 * __restrict__ out, int B, int H, int W, int C) {
    const int G = C / 8;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)B * H * W * G) return;
    const int g = (int)(i % G);
    const int64_t p = i / G;
    const int xx = (int)(p % W), yy = (int)((p / W) % H), b = (int)(p / ((int64_t)W * H));
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
    for (int ky = 0; ky < 5; ++ky) {
        const int iy = yy + ky - 2;
        if (iy < 0 || iy >= H) continue;
        for (int kx = 0; kx < 5; ++kx) {
            const int ix = xx + kx - 2;
            if (ix < 0 || ix >= W) continue;
            const f16x8 v = *reinterpret_cast<const f16x8 *>(in + (((int64_t)b * H + iy) * W + ix) * C + g * 8);
            const float4 * wp = reinterpret_cast<const float4 *>(w + (ky * 5 + kx) * C + g * 8);
            const float4 w0 = wp[0], w1 = wp[1];
            const float wk[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] += (float)v[e] * wk[e];
        }
    }
    f16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = (f16)acc[e];
    *reinterpret_cast<f16x8 *>(out + p * C + g * 8) = o;
}

// Grouped 1x1 conv with groups of 32 channels (the multiscale proj_out,
// grouped_conv2d_1x1 src/vae_ops.cpp:243-300): out[p][32 g + o] =
// sum_i w[g][o][i] in[p][32 g + i].  A workgroup: 32 pixels x one group, the
// group's 32 x 32 weights in LDS; a thread: 4 outputs of one pixel.
__global__ __launch_bounds__(256) void vae_grouped32_kernel(const f16 * __restrict__ in, const float * __restrict__ w,
                                                            f16 * __restrict__ out, int P, int C) {
    __shared__ float ws[32][33];
    const int g = blockIdx.y;
    const int tid = threadIdx.x;
    for (int e = tid; e < 32 * 32; e += 256) ws[e >> 5][e & 31] = w[(int64_t)g * 1024 + e];
    __syncthreads();
    const int pix = blockIdx.x * 32 + (tid >> 3), o0 = (tid & 7) * 4;
    if (pix >= P) return;
    const f16 * src = in + (int64_t)pix * C + g * 32;
    float x[32];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const f16x8 v = *reinterpret_cast<const f16x8 *>(src + q * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[q * 8 + e] = (float)v[e];
    }
    f16x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < 32; ++i) a += ws[o0 + j][i] * x[i];
        o[j] = (f16)a;
    }
    *reinterpret_cast<f16x4 *>(out + (int64_t)pix * C + g * 32 + o0) = o;
}

// NHWC [B * H * W][C] -> NCHW [B][C][H][W] (the conv_out image, C = 3, or the
// conv_in stage output).
__global__ void vae_to_nchw_kernel(const float * __restrict__ in, float * __restrict__ img, int B, int C, int H,
                                   int W) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t hw = (int64_t)H * W;
    if (i >= (int64_t)B * C * hw) return;
    const int64_t s = i % hw;
    const int c = (int)((i / hw) % C), b = (int)(i / (C * hw));
    img[i] = in[((int64_t)b * hw + s) * C + c];
}

unsigned blocks_for(int64_t n, int per = 256) { return (unsigned)((n + per - 1) / per); }

// ---------------------------------------------------------------------------
// device model

struct ResDev {
    DevMem w1, b1, w2, nw, nb;
};
struct AttnDev {
    DevMem wqkv, dw5, grp, wout, anw, anb;     // multiscale attention
    DevMem winv, binv, wdw, bdw, wpt, gnw, gnb;  // GLUMBConv
};
struct LevelDev {
    int64_t C = 0;
    bool attn = false;
    DevMem up_w, up_b;  // upsample conv from level + 1 (absent at the top level)
    ResDev res[3];
    AttnDev att[3];
};

}  // namespace

struct sana_vae {
    int device = 0;
    int64_t Cl = 32, L = 0, head = kVaeHead, expand = 4;
    float scaling = 0.41407f;
    std::vector<std::unique_ptr<LevelDev>> lv;
    DevMem cin_w, cin_b, nout_w, nout_b, cout_w, cout_b;
    std::map<std::string, bool> loaded;
    std::vector<std::string> required;
    // workspace
    DevMem lat16, x32, xs32, t32, pad0, pad1, a16, qkv16, dw16, ms16, mrg16, hid16, glu16, la_ws, o32, img;
    hipStream_t stream = nullptr;
};

namespace {

void upload(DevMem & d, const void * src, size_t bytes) {
    d.ensure(bytes, false);
    copy_to_device(d.p, src, bytes, "hipMemcpy weights");
}

void upload_f32(DevMem & d, const float * src, size_t n) { upload(d, src, n * 4); }

// fp32 -> fp16 GEMM operand; a value fp16 cannot hold fails with
// SANA_ERR_FORMAT naming the tensor.
void upload_f16(DevMem & d, const float * v, size_t n, const std::string & tensor) {
    std::vector<_Float16> h(n);
    for (size_t i = 0; i < n; ++i) h[i] = to_f16_checked(v[i], tensor, i);
    upload(d, h.data(), h.size() * 2);
}

// [Cout, Cin, 3, 3] -> tap-major fp16 [Cout][9][cin_pad] (zero past Cin).
void upload_conv3(DevMem & d, const float * w, int64_t Cout, int64_t Cin, int64_t cin_pad, const std::string & tensor) {
    std::vector<_Float16> t((size_t)Cout * 9 * cin_pad, (_Float16)0.0f);
    for (int64_t o = 0; o < Cout; ++o)
        for (int64_t c = 0; c < Cin; ++c)
            for (int k = 0; k < 9; ++k) {
                const size_t i = ((size_t)o * Cin + c) * 9 + k;
                t[((size_t)o * 9 + k) * cin_pad + c] = to_f16_checked(w[i], tensor, i);
            }
    upload(d, t.data(), t.size() * 2);
}

// Physical position of channel `lc` of concat(q, k, v) (3C channels, heads of
// 32): logical group j = lc / 32 is head j / 3's q, k or v (j % 3); it moves
// to section j % 3, head slot j / 3.
int64_t qkv_perm(int64_t lc, int64_t heads) {
    const int64_t j = lc / kVaeHead;
    return ((j % 3) * heads + j / 3) * kVaeHead + lc % kVaeHead;
}

void expect(const char * name, const int64_t * shape, int ndim, std::vector<int64_t> want) {
    bool ok = ndim == (int)want.size();
    for (int i = 0; ok && i < ndim; ++i) ok = shape[i] == want[i];
    if (!ok) {
        std::string got, exp;
        for (int i = 0; i < ndim; ++i) got += (i ? "," : "") + std::to_string(shape[i]);
        for (size_t i = 0; i < want.size(); ++i) exp += (i ? "," : "") + std::to_string(want[i]);
        throw_err(SANA_ERR_SHAPE, std::string("vae weight ") + name + " has shape [" + got + "], expected [" + exp + "]");
    }
}

void set_weight(sana_vae * v, const std::string & n, const float * d, const int64_t * sh, int nd) {
    const int64_t L = v->L, top = v->lv[L - 1]->C, C0 = v->lv[0]->C;
    auto need = [&](std::vector<int64_t> s) { expect(n.c_str(), sh, nd, std::move(s)); };
    if (n == "decoder.conv_in.weight") {
        need({top, v->Cl, 3, 3});
        upload_conv3(v->cin_w, d, top, v->Cl, round_up(v->Cl, 64), n);
    } else if (n == "decoder.conv_in.bias") {
        need({top});
        upload_f32(v->cin_b, d, top);
    } else if (n == "decoder.norm_out.weight") {
        need({C0});
        upload_f32(v->nout_w, d, C0);
    } else if (n == "decoder.norm_out.bias") {
        need({C0});
        upload_f32(v->nout_b, d, C0);
    } else if (n == "decoder.conv_out.weight") {
        need({3, C0, 3, 3});
        upload_conv3(v->cout_w, d, 3, C0, C0, n);
    } else if (n == "decoder.conv_out.bias") {
        need({3});
        upload_f32(v->cout_b, d, 3);
    } else {
        const std::string pre = "decoder.up_blocks.";
        if (n.compare(0, pre.size(), pre) != 0) throw_err(SANA_ERR_INVALID_ARGUMENT, "unknown vae weight " + n);
        size_t pos = pre.size();
        const size_t dot = n.find('.', pos);
        if (dot == std::string::npos) throw_err(SANA_ERR_INVALID_ARGUMENT, "unknown vae weight " + n);
        const int64_t li = std::stoll(n.substr(pos, dot - pos));
        if (li < 0 || li >= L) throw_err(SANA_ERR_INVALID_ARGUMENT, "vae up block index out of range: " + n);
        const size_t dot2 = n.find('.', dot + 1);
        const int64_t layer = std::stoll(n.substr(dot + 1, dot2 - dot - 1));
        const std::string rest = n.substr(dot2 + 1);
        LevelDev & lvd = *v->lv[li];
        const int64_t C = lvd.C, base = li + 1 < L ? 1 : 0;
        if (base == 1 && layer == 0) {
            const int64_t Cp = v->lv[li + 1]->C;
            if (rest == "conv.weight") {
                need({C, Cp, 3, 3});
                upload_conv3(lvd.up_w, d, C, Cp, Cp, n);
            } else if (rest == "conv.bias") {
                need({C});
                upload_f32(lvd.up_b, d, C);
            } else {
                throw_err(SANA_ERR_INVALID_ARGUMENT, "unknown vae weight " + n);
            }
        } else {
            const int64_t k = layer - base;
            if (k < 0 || k > 2) throw_err(SANA_ERR_INVALID_ARGUMENT, "vae layer index out of range: " + n);
            if (!lvd.attn) {
                ResDev & r = lvd.res[k];
                if (rest == "conv1.weight") { need({C, C, 3, 3}); upload_conv3(r.w1, d, C, C, C, n); }
                else if (rest == "conv1.bias") { need({C}); upload_f32(r.b1, d, C); }
                else if (rest == "conv2.weight") { need({C, C, 3, 3}); upload_conv3(r.w2, d, C, C, C, n); }
                else if (rest == "norm.weight") { need({C}); upload_f32(r.nw, d, C); }
                else if (rest == "norm.bias") { need({C}); upload_f32(r.nb, d, C); }
                else throw_err(SANA_ERR_INVALID_ARGUMENT, "unknown vae weight " + n);
            } else {
                AttnDev & a = lvd.att[k];
                const int64_t heads = C / kVaeHead, Hd = v->expand * C;
                if (rest == "attn.to_q.weight" || rest == "attn.to_k.weight" || rest == "attn.to_v.weight") {
                    need({C, C});
                    const int64_t t = rest == "attn.to_q.weight" ? 0 : (rest == "attn.to_k.weight" ? 1 : 2);
                    // rows of q, k, v go to their permuted places in the fused [3C, C] weight
                    std::vector<_Float16> all;
                    if (a.wqkv.p) {
                        all.resize((size_t)3 * C * C);
                        hip_check(hipMemcpy(all.data(), a.wqkv.p, all.size() * 2, hipMemcpyDeviceToHost), "hipMemcpy");
                    } else {
                        all.assign((size_t)3 * C * C, (_Float16)0.0f);
                    }
                    for (int64_t o = 0; o < C; ++o) {
                        const int64_t ph = qkv_perm(t * C + o, heads);
                        for (int64_t i = 0; i < C; ++i) all[(size_t)ph * C + i] = to_f16_checked(d[o * C + i], n, (size_t)(o * C + i));
                    }
                    upload(a.wqkv, all.data(), all.size() * 2);
                } else if (rest == "attn.to_qkv_multiscale.0.proj_in.weight") {
                    need({3 * C, 1, 5, 5});
                    std::vector<float> t((size_t)25 * 3 * C);
                    for (int64_t c = 0; c < 3 * C; ++c)
                        for (int kk = 0; kk < 25; ++kk) t[(size_t)kk * 3 * C + qkv_perm(c, heads)] = d[c * 25 + kk];
                    upload_f32(a.dw5, t.data(), t.size());
                } else if (rest == "attn.to_qkv_multiscale.0.proj_out.weight") {
                    need({3 * C, kVaeHead, 1, 1});
                    std::vector<float> t((size_t)3 * C * kVaeHead);
                    for (int64_t oc = 0; oc < 3 * C; ++oc) {
                        const int64_t po = qkv_perm(oc, heads);
                        for (int64_t i = 0; i < kVaeHead; ++i) t[(size_t)po * kVaeHead + i] = d[oc * kVaeHead + i];
                    }
                    upload_f32(a.grp, t.data(), t.size());
                } else if (rest == "attn.to_out.weight") {
                    need({C, 2 * C});
                    upload_f16(a.wout, d, (size_t)(2 * C * C), n);
                } else if (rest == "attn.norm_out.weight") { need({C}); upload_f32(a.anw, d, C); }
                else if (rest == "attn.norm_out.bias") { need({C}); upload_f32(a.anb, d, C); }
                else if (rest == "conv_out.conv_inverted.weight") {
                    need({2 * Hd, C, 1, 1});
                    upload_f16(a.winv, d, (size_t)(2 * Hd * C), n);
                } else if (rest == "conv_out.conv_inverted.bias") { need({2 * Hd}); upload_f32(a.binv, d, 2 * Hd); }
                else if (rest == "conv_out.conv_depth.weight") {
                    need({2 * Hd, 1, 3, 3});
                    std::vector<float> t((size_t)9 * 2 * Hd);
                    for (int64_t c = 0; c < 2 * Hd; ++c)
                        for (int kk = 0; kk < 9; ++kk) t[(size_t)kk * 2 * Hd + c] = d[c * 9 + kk];
                    upload_f32(a.wdw, t.data(), t.size());
                } else if (rest == "conv_out.conv_depth.bias") { need({2 * Hd}); upload_f32(a.bdw, d, 2 * Hd); }
                else if (rest == "conv_out.conv_point.weight") {
                    need({C, Hd, 1, 1});
                    upload_f16(a.wpt, d, (size_t)(C * Hd), n);
                } else if (rest == "conv_out.norm.weight") { need({C}); upload_f32(a.gnw, d, C); }
                else if (rest == "conv_out.norm.bias") { need({C}); upload_f32(a.gnb, d, C); }
                else throw_err(SANA_ERR_INVALID_ARGUMENT, "unknown vae weight " + n);
            }
        }
    }
    v->loaded[n] = true;
}

std::vector<std::string> required_names(const sana_vae * v) {
    std::vector<std::string> r = {"decoder.conv_in.weight",  "decoder.conv_in.bias",  "decoder.norm_out.weight",
                                  "decoder.norm_out.bias",   "decoder.conv_out.weight", "decoder.conv_out.bias"};
    for (int64_t i = 0; i < v->L; ++i) {
        const std::string p = "decoder.up_blocks." + std::to_string(i) + ".";
        int64_t base = 0;
        if (i + 1 < v->L) {
            r.push_back(p + "0.conv.weight");
            r.push_back(p + "0.conv.bias");
            base = 1;
        }
        for (int64_t l = base; l < base + 3; ++l) {
            const std::string q = p + std::to_string(l) + ".";
            if (!v->lv[i]->attn) {
                for (const char * s : {"conv1.weight", "conv1.bias", "conv2.weight", "norm.weight", "norm.bias"})
                    r.push_back(q + s);
            } else {
                for (const char * s : {"attn.to_q.weight", "attn.to_k.weight", "attn.to_v.weight",
                                       "attn.to_qkv_multiscale.0.proj_in.weight",
                                       "attn.to_qkv_multiscale.0.proj_out.weight", "attn.to_out.weight",
                                       "attn.norm_out.weight", "attn.norm_out.bias", "conv_out.conv_inverted.weight",
                                       "conv_out.conv_inverted.bias", "conv_out.conv_depth.weight",
                                       "conv_out.conv_depth.bias", "conv_out.conv_point.weight",
                                       "conv_out.norm.weight", "conv_out.norm.bias"})
                    r.push_back(q + s);
            }
        }
    }
    return r;
}

// ---------------------------------------------------------------------------
// decode

void gemm_plain(const half_t * A, int64_t lda, const DevMem & W, int64_t M, int64_t N, int64_t K, const float * bias,
                int act, half_t * out16, int64_t ldo16, float * out32, int64_t ldo32, hipStream_t s) {
    sana::GemmParams p;
    p.A = A;
    p.lda = lda;
    p.W = W.as<half_t>();
    p.ldw = K;
    p.M = (int)M;
    p.N = (int)N;
    p.K = (int)K;
    p.bias = bias;
    p.act = act;
    p.out16 = out16;
    p.ldo16 = ldo16;
    p.out32 = out32;
    p.ldo32 = ldo32;
    launch_check(sana::gemm(p, s), "vae gemm");
}

// 3x3 conv as an implicit GEMM over the bordered input (conv = 1) or its
// nearest-2x upsample (conv = 2).  Residual mode: x += acc + bias.
void gemm_conv(int conv, const half_t * A, int64_t cin, const DevMem & W, int64_t B, int64_t H, int64_t Wd,
               int64_t N, const float * bias, int act, bool residual, float * x32, half_t * out16, bool pad16,
               float * out32, hipStream_t s, const float * up_src = nullptr, int64_t up_c = 0) {
    sana::GemmParams p;
    p.conv = conv;
    p.conv_h = (int)H;
    p.conv_w = (int)Wd;
    p.A = A;
    p.lda = cin;
    p.W = W.as<half_t>();
    p.ldw = 9 * cin;
    p.M = (int)(B * H * Wd);
    p.N = (int)N;
    p.K = (int)(9 * cin);
    p.bias = bias;
    p.act = act;
    p.out16 = out16;
    p.ldo16 = N;
    p.out16_pad = pad16 ? 1 : 0;
    if (residual) {
        p.mode = sana::kGemmResidual;
        p.out32 = x32;
        p.ldo32 = N;
        if (up_src) {
            p.up_src = up_src;
            p.up_c = (int)up_c;
            p.up_rep = (int)(N * 4 / up_c);
        }

    } else {
        p.out32 = out32;
        p.ldo32 = N;
    }
    launch_check(sana::gemm(p, s), "vae conv gemm");
}

void rmsnorm(const float * x, int64_t C, int64_t P, const DevMem & w, const DevMem * b, const float * res, bool relu,
             float * out32, half_t * out16, bool pad, int64_t H, int64_t W, hipStream_t s) {
    const dim3 g((unsigned)((P + 3) / 4)), t(256);
    f16 * o16 = reinterpret_cast<f16 *>(out16);
    const float * bp = b ? b->as<float>() : nullptr;
#define SANA_VAE_RMS(n4) \
    hipLaunchKernelGGL((vae_rmsnorm_kernel<n4>), g, t, 0, s, x, (int)C, (int)P, w.as<float>(), bp, res, relu ? 1 : 0, \
                       1e-5f, out32, o16, pad ? 1 : 0, (int)H, (int)W)
    if (C <= 256) SANA_VAE_RMS(1);
    else if (C <= 512) SANA_VAE_RMS(2);
    else SANA_VAE_RMS(4);
#undef SANA_VAE_RMS
    launch_check(hipGetLastError(), "vae rmsnorm");
}

void zero_border(const DevMem & buf, int64_t B, int64_t H, int64_t W, int64_t ld, hipStream_t s) {
    const int64_t n = B * (2 * (W + 2) + 2 * H) * (ld / 8);
    hipLaunchKernelGGL(vae_zero_border_kernel, dim3(blocks_for(n)), dim3(256), 0, s, buf.as<f16>(), (int)B, (int)H,
                       (int)W, (int)ld);
    launch_check(hipGetLastError(), "vae zero border");
}

void ensure_workspace(sana_vae * v, int64_t B, int64_t h, int64_t w) {
    size_t mx_pc = 0, mx_pad = 0, mx_att = 0, mx_la = 0;
    int64_t H = h, W = w;
    for (int64_t i = v->L - 1; i >= 0; --i) {
        if (i + 1 < v->L) {
            H *= 2;
            W *= 2;
        }
        const int64_t C = v->lv[i]->C, P = B * H * W;
        mx_pc = std::max(mx_pc, (size_t)(P * C));
        mx_pad = std::max(mx_pad, (size_t)(B * (H + 2) * (W + 2) * C));
        if (v->lv[i]->attn) {
            mx_att = std::max(mx_att, (size_t)(P * C));
            mx_la = std::max(mx_la, sana::linattn_workspace_floats((int)B, (int)(H * W), (int)(C / kVaeHead), kVaeHead));
        }
    }
    const int64_t top = v->lv[v->L - 1]->C;
    mx_pc = std::max(mx_pc, (size_t)(B * h * w * top));
    v->lat16.ensure((size_t)B * (h + 2) * (w + 2) * round_up(v->Cl, 64) * 2, false);
    v->x32.ensure(mx_pc * 4, false);
    v->xs32.ensure(mx_pc * 4, false);
    v->t32.ensure(mx_pc * 4, false);
    v->pad0.ensure(mx_pad * 2, false);
    v->pad1.ensure(mx_pad * 2, false);
    v->a16.ensure(mx_pc * 2, false);
    if (mx_att) {
        v->qkv16.ensure(mx_att * 3 * 2, false);
        v->dw16.ensure(mx_att * 3 * 2, false);
        v->ms16.ensure(mx_att * 3 * 2, false);
        v->mrg16.ensure(mx_att * 2 * 2, false);
        v->hid16.ensure(mx_att * 2 * v->expand * 2, false);
        v->glu16.ensure(mx_att * v->expand * 2, false);
        v->la_ws.ensure(mx_la * 4 + 16, false);
    }
    v->o32.ensure((size_t)(B * H * W * 3) * 4, false);
}

void check_ready(const sana_vae * v) {
    for (const std::string & n : v->required)
        if (!v->loaded.count(n)) throw_err(SANA_ERR_STATE, "vae weight not set: " + n);
}

// run_vae_decode (src/vae.cpp:243-325) on device pointers.
void decode(sana_vae * v, const float * lat, int64_t B, int64_t h, int64_t w, float * img, hipStream_t s) {
    check_ready(v);
    if (B <= 0 || h <= 0 || w <= 0) throw_err(SANA_ERR_INVALID_ARGUMENT, "vae decode: empty latent");
    ensure_workspace(v, B, h, w);
    const int64_t L = v->L, top = v->lv[L - 1]->C, clp = round_up(v->Cl, 64);
    const int64_t rep = top / v->Cl;
    // latent / scaling_factor -> bordered fp16 conv_in input and the channel-repeat shortcut in x32
    {
        const int64_t n = std::max<int64_t>(B * (h + 2) * (w + 2) * clp, B * h * w * top);
        hipLaunchKernelGGL(vae_prep_kernel, dim3(blocks_for(n)), dim3(256), 0, s, lat, (int)B, (int)v->Cl, (int)h,
                           (int)w, 1.0f / v->scaling, v->lat16.as<f16>(), (int)clp, v->x32.as<float>(), (int)top,
                           (int)rep, 1);
        launch_check(hipGetLastError(), "vae prep");
    }
    DevMem * cur = &v->pad0;   // bordered fp16 input of the next 3x3 conv
    DevMem * oth = &v->pad1;
    int64_t H = h, W = w, C = top;
    const bool top_attn = v->lv[L - 1]->attn;
    if (!top_attn) zero_border(*cur, B, H, W, C, s);
    // conv_in + shortcut (x32 already holds the shortcut): x32 += conv + bias
    gemm_conv(1, v->lat16.as<half_t>(), clp, v->cin_w, B, H, W, top, v->cin_b.as<float>(), sana::kActNone, true,
              v->x32.as<float>(), top_attn ? v->a16.as<half_t>() : cur->as<half_t>(), !top_attn, nullptr, s);
    for (int64_t li = L - 1; li >= 0; --li) {
        LevelDev & lvd = *v->lv[li];
        if (li + 1 < L) {
            // upsample block: xs32 = shortcut(x32) + conv(upsample(cur)) + bias, the
            // shortcut gathered from the low-resolution residual in the epilogue
            const int64_t Co = lvd.C, H2 = 2 * H, W2 = 2 * W;
            if (!lvd.attn) zero_border(*oth, B, H2, W2, Co, s);
            gemm_conv(2, cur->as<half_t>(), C, lvd.up_w, B, H2, W2, Co, lvd.up_b.as<float>(), sana::kActNone, true,
                      v->xs32.as<float>(), lvd.attn ? v->a16.as<half_t>() : oth->as<half_t>(), !lvd.attn, nullptr, s,
                      v->x32.as<float>(), C);
            std::swap(v->x32.p, v->xs32.p);
            std::swap(v->x32.bytes, v->xs32.bytes);
            std::swap(cur, oth);
            H = H2;
            W = W2;
            C = Co;
            if (!lvd.attn) zero_border(*oth, B, H, W, C, s);
        } else if (!lvd.attn) {
            zero_border(*oth, B, H, W, C, s);
        }
        const int64_t P = B * H * W;
        float * x = v->x32.as<float>();
        // the level's last layer hands a bordered fp16 copy to the next upsample conv
        const bool next_up = li > 0;
        if (next_up) zero_border(lvd.attn ? *cur : *cur, B, H, W, C, s);
        for (int k = 0; k < 3; ++k) {
            const bool last = k == 2;
            if (!lvd.attn) {
                ResDev & r = lvd.res[k];
                gemm_conv(1, cur->as<half_t>(), C, r.w1, B, H, W, C, r.b1.as<float>(), sana::kActSilu, false, nullptr,
                          oth->as<half_t>(), true, nullptr, s);
                // RMSNorm + residual as its own streaming pass: folded into conv2's
                // epilogue it ran slower (938 us against 448 + 402 us at 1024²), the
                // epilogue's memory phase being exposed
                gemm_conv(1, oth->as<half_t>(), C, r.w2, B, H, W, C, nullptr, sana::kActNone, false, nullptr, nullptr,
                          false, v->t32.as<float>(), s);
                // next: conv1 of the next ResBlock, the next upsample, or (level 0, last) the final norm
                rmsnorm(v->t32.as<float>(), C, P, r.nw, &r.nb, x, false, x, cur->as<half_t>(), true, H, W, s);
            } else {
                AttnDev & a = lvd.att[k];
                const int64_t heads = C / kVaeHead;
                half_t * qkv = v->qkv16.as<half_t>();
                gemm_plain(v->a16.as<half_t>(), C, a.wqkv, P, 3 * C, C, nullptr, sana::kActNone, qkv, 3 * C, nullptr,
                           0, s);
                {
                    const int64_t n = P * (3 * C / 8);
                    hipLaunchKernelGGL(vae_dw5x5_kernel, dim3(blocks_for(n)), dim3(256), 0, s,
                                       reinterpret_cast<const f16 *>(qkv), a.dw5.as<float>(), v->dw16.as<f16>(), (int)B,
                                       (int)H, (int)W, (int)(3 * C));
                    launch_check(hipGetLastError(), "vae dw5x5");
                    hipLaunchKernelGGL(vae_grouped32_kernel, dim3(blocks_for(P, 32), (unsigned)(3 * heads)), dim3(256),
                                       0, s, v->dw16.as<f16>(), a.grp.as<float>(), v->ms16.as<f16>(), (int)P,
                                       (int)(3 * C));
                    launch_check(hipGetLastError(), "vae grouped 1x1");
                }
                half_t * mrg = v->mrg16.as<half_t>();
                const half_t * ms = v->ms16.as<half_t>();
                launch_check(sana::linear_attention(qkv, qkv + C, qkv + 2 * C, 3 * C, mrg, 2 * C, (int)B,
                                                    (int)(H * W), (int)heads, kVaeHead, v->la_ws.as<float>(), s),
                             "vae linear attention");
                launch_check(sana::linear_attention(ms, ms + C, ms + 2 * C, 3 * C, mrg + C, 2 * C, (int)B,
                                                    (int)(H * W), (int)heads, kVaeHead, v->la_ws.as<float>(), s),
                             "vae linear attention");
                gemm_plain(mrg, 2 * C, a.wout, P, C, 2 * C, nullptr, sana::kActNone, nullptr, 0, v->t32.as<float>(), C,
                           s);
                rmsnorm(v->t32.as<float>(), C, P, a.anw, &a.anb, x, false, x, v->a16.as<half_t>(), false, H, W, s);
                // GLUMBConv: inverted 1x1 (+ bias, SiLU), depthwise 3x3 + GLU, point 1x1
                const int64_t Hd = v->expand * C;
                gemm_plain(v->a16.as<half_t>(), C, a.winv, P, 2 * Hd, C, a.binv.as<float>(), sana::kActSilu,
                           v->hid16.as<half_t>(), 2 * Hd, nullptr, 0, s);
                launch_check(sana::dwconv_glu(v->hid16.as<half_t>(), 2 * Hd, a.wdw.as<float>(), a.bdw.as<float>(),
                                              v->glu16.as<half_t>(), Hd, (int)B, (int)H, (int)W, (int)Hd, s),
                             "vae dwconv glu");
                gemm_plain(v->glu16.as<half_t>(), Hd, a.wpt, P, C, Hd, nullptr, sana::kActNone, nullptr, 0,
                           v->t32.as<float>(), C, s);
                const bool to_pad = last && next_up;
                rmsnorm(v->t32.as<float>(), C, P, a.gnw, &a.gnb, x, false, x,
                        to_pad ? cur->as<half_t>() : v->a16.as<half_t>(), to_pad, H, W, s);
            }
        }
    }
    // norm_out + ReLU -> bordered fp16, conv_out -> [P][3] -> NCHW image
    const int64_t P = B * H * W;
    zero_border(*cur, B, H, W, C, s);
    rmsnorm(v->x32.as<float>(), C, P, v->nout_w, &v->nout_b, nullptr, true, nullptr, cur->as<half_t>(), true, H, W, s);
    gemm_conv(1, cur->as<half_t>(), C, v->cout_w, B, H, W, 3, v->cout_b.as<float>(), sana::kActNone, false, nullptr,
              nullptr, false, v->o32.as<float>(), s);
    hipLaunchKernelGGL(vae_to_nchw_kernel, dim3(blocks_for(B * 3 * H * W)), dim3(256), 0, s, v->o32.as<float>(), img,
                       (int)B, 3, (int)H, (int)W);
    launch_check(hipGetLastError(), "vae to nchw");
}

// run_vae_decoder_input (src/vae.cpp:211-241) on device pointers: conv_in of
// the unscaled latent (+ shortcut) -> out NCHW [B, top, h, w].
void decoder_input(sana_vae * v, const float * lat, int64_t B, int64_t h, int64_t w, bool shortcut, float * out,
                   hipStream_t s) {
    for (const char * n : {"decoder.conv_in.weight", "decoder.conv_in.bias"})
        if (!v->loaded.count(n)) throw_err(SANA_ERR_STATE, std::string("vae weight not set: ") + n);
    if (B <= 0 || h <= 0 || w <= 0) throw_err(SANA_ERR_INVALID_ARGUMENT, "vae decoder input: empty latent");
    const int64_t top = v->lv[v->L - 1]->C, clp = round_up(v->Cl, 64), rep = top / v->Cl;
    v->lat16.ensure((size_t)(B * (h + 2) * (w + 2) * clp) * 2, false);
    v->x32.ensure((size_t)(B * h * w * top) * 4, false);
    const int64_t n = std::max<int64_t>(B * (h + 2) * (w + 2) * clp, B * h * w * top);
    hipLaunchKernelGGL(vae_prep_kernel, dim3(blocks_for(n)), dim3(256), 0, s, lat, (int)B, (int)v->Cl, (int)h, (int)w,
                       1.0f, v->lat16.as<f16>(), (int)clp, v->x32.as<float>(), (int)top, (int)rep, shortcut ? 1 : 0);
    launch_check(hipGetLastError(), "vae prep");
    gemm_conv(1, v->lat16.as<half_t>(), clp, v->cin_w, B, h, w, top, v->cin_b.as<float>(), sana::kActNone, true,
              v->x32.as<float>(), nullptr, false, nullptr, s);
    hipLaunchKernelGGL(vae_to_nchw_kernel, dim3(blocks_for(B * top * h * w)), dim3(256), 0, s, v->x32.as<float>(), out,
                       (int)B, (int)top, (int)h, (int)w);
    launch_check(hipGetLastError(), "vae to nchw");
}

void validate_config(const sana_vae_config * c) {
    if (c->levels < 1 || c->levels > SANA_VAE_MAX_LEVELS)
        throw_err(SANA_ERR_INVALID_ARGUMENT, "vae levels must be in [1, 8]");
    if (c->latent_channels <= 0 || c->latent_channels > 64)
        throw_err(SANA_ERR_INVALID_ARGUMENT, "vae latent channels must be in [1, 64]");
    if (c->head_dim != kVaeHead) throw_err(SANA_ERR_INVALID_ARGUMENT, "vae attention head dim must be 32");
    if (c->expand <= 0) throw_err(SANA_ERR_INVALID_ARGUMENT, "vae GLUMBConv expansion must be positive");
    if (!(c->scaling_factor > 0.0f)) throw_err(SANA_ERR_INVALID_ARGUMENT, "vae scaling_factor must be positive");
    for (int64_t i = 0; i < c->levels; ++i) {
        const int64_t C = c->channels[i];
        if (C <= 0 || C % 64 || C > 1024)
            throw_err(SANA_ERR_INVALID_ARGUMENT, "vae level channels must be multiples of 64 up to 1024");
        if (i + 1 < c->levels && (C * 4) % c->channels[i + 1])
            throw_err(SANA_ERR_INVALID_ARGUMENT, "VAE upsample shortcut channel ratio is invalid");
    }
    if (c->channels[c->levels - 1] % c->latent_channels)
        throw_err(SANA_ERR_INVALID_ARGUMENT, "vae decoder conv_in output channels must be divisible by latent channels");
}

const float * gguf_payload(const sana::gguf::MappedFile & f, const sana::gguf::TensorInfo & t,
                           std::vector<float> & tmp) {
    using namespace sana::gguf;
    if (t.type != kF32 && t.type != kF16 && t.type != kBF16)
        throw_err(SANA_ERR_FORMAT, "unsupported gguf tensor type for " + t.name);
    try {
        return payload_f32(f, t, tmp);
    } catch (const std::runtime_error & e) {
        throw_err(SANA_ERR_FORMAT, e.what());
    }
    return nullptr;
}

}  // namespace

extern "C" {

int sana_vae_create(const sana_vae_config * cfg, sana_vae ** out) {
    if (!cfg || !out) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    return guarded([&] {
        validate_config(cfg);
        int ndev = 0;
        hip_check(hipGetDeviceCount(&ndev), "hipGetDeviceCount");
        if (cfg->device < 0 || cfg->device >= ndev) throw_err(SANA_ERR_INVALID_ARGUMENT, "no such device");
        hip_check(hipSetDevice(cfg->device), "hipSetDevice");
        auto * v = new sana_vae();
        v->device = cfg->device;
        v->Cl = cfg->latent_channels;
        v->L = cfg->levels;
        v->expand = cfg->expand;
        v->scaling = cfg->scaling_factor;
        for (int64_t i = 0; i < v->L; ++i) {
            v->lv.push_back(std::make_unique<LevelDev>());
            v->lv[i]->C = cfg->channels[i];
            v->lv[i]->attn = cfg->attention[i] != 0;
        }
        v->required = required_names(v);
        *out = v;
    });
}

int sana_vae_destroy(sana_vae * v) {
    if (!v) return SANA_OK;
    (void)hipSetDevice(v->device);
    (void)hipDeviceSynchronize();
    delete v;
    return SANA_OK;
}

int sana_vae_set_weight(sana_vae * v, const char * name, const float * data, const int64_t * shape, int ndim) {
    if (!v || !name || !data || !shape) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    return guarded([&] {
        hip_check(hipSetDevice(v->device), "hipSetDevice");
        set_weight(v, name, data, shape, ndim);
    });
}

int sana_vae_check_weights(sana_vae * v) {
    if (!v) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    return guarded([&] { check_ready(v); });
}

int sana_vae_load_gguf(sana_vae * v, const char * path) {
    if (!v || !path) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    return guarded([&] {
        using namespace sana::gguf;
        hip_check(hipSetDevice(v->device), "hipSetDevice");
        Index idx;
        try {
            idx = read_index(path);
        } catch (const std::exception & e) {
            throw_err(SANA_ERR_IO, e.what());
        }
        MappedFile f(path);
        std::map<std::string, const TensorInfo *> by;
        for (const auto & t : idx.tensors) by[t.name] = &t;
        std::vector<float> tmp;
        for (const std::string & n : v->required) {
            auto it = by.find(n);
            if (it == by.end()) throw_err(SANA_ERR_INVALID_ARGUMENT, "weight name not found in weight index: " + n);
            const TensorInfo & t = *it->second;
            set_weight(v, n, gguf_payload(f, t, tmp), t.shape.data(), (int)t.shape.size());
        }
    });
}

int sana_vae_decode_device(sana_vae * v, const float * latent, int64_t B, int64_t H, int64_t W, float * image,
                           void * stream) {
    if (!v || !latent || !image) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    return guarded([&] {
        hip_check(hipSetDevice(v->device), "hipSetDevice");
        decode(v, latent, B, H, W, image, static_cast<hipStream_t>(stream));
    });
}

int sana_vae_decoder_input(sana_vae * v, const float * latent, int64_t B, int64_t H, int64_t W, int in_shortcut,
                           float * out) {
    if (!v || !latent || !out) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    return guarded([&] {
        hip_check(hipSetDevice(v->device), "hipSetDevice");
        if (B <= 0 || H <= 0 || W <= 0) throw_err(SANA_ERR_INVALID_ARGUMENT, "vae decoder input: empty latent");
        const int64_t top = v->lv[v->L - 1]->C;
        const size_t nl = (size_t)(B * v->Cl * H * W), no = (size_t)(B * top * H * W);
        DevMem dl, dout;
        dl.ensure(nl * 4, false);
        dout.ensure(no * 4, false);
        hip_check(hipMemcpy(dl.p, latent, nl * 4, hipMemcpyHostToDevice), "hipMemcpy latent");
        decoder_input(v, dl.as<float>(), B, H, W, in_shortcut != 0, dout.as<float>(), nullptr);
        hip_check(hipMemcpy(out, dout.p, no * 4, hipMemcpyDeviceToHost), "hipMemcpy decoder input");
    });
}

int sana_vae_decode(sana_vae * v, const float * latent, int64_t B, int64_t H, int64_t W, float * image) {
    if (!v || !latent || !image) return set_err(SANA_ERR_INVALID_ARGUMENT, "null argument");
    return guarded([&] {
        hip_check(hipSetDevice(v->device), "hipSetDevice");
        if (B <= 0 || H <= 0 || W <= 0) throw_err(SANA_ERR_INVALID_ARGUMENT, "vae decode: empty latent");
        const int64_t up = (int64_t)1 << (v->L - 1);
        const size_t nl = (size_t)(B * v->Cl * H * W), ni = (size_t)(B * 3 * H * up * W * up);
        DevMem dl, di;
        dl.ensure(nl * 4, false);
        di.ensure(ni * 4, false);
        hip_check(hipMemcpy(dl.p, latent, nl * 4, hipMemcpyHostToDevice), "hipMemcpy latent");
        decode(v, dl.as<float>(), B, H, W, di.as<float>(), nullptr);
        hip_check(hipMemcpy(image, di.p, ni * 4, hipMemcpyDeviceToHost), "hipMemcpy image");
    });
}

}  // extern "C"
