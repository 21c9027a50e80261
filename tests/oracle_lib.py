"""ctypes binding of oracle/liboracle.so -- the CPU parity oracle.

Test infrastructure: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use this module, and only as the checker.
"""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "oracle", "liboracle.so")

_f = ctypes.POINTER(ctypes.c_float)
_sz = ctypes.c_size_t
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        L.oracle_last_error.restype = ctypes.c_char_p
        L.oracle_model_create.restype = ctypes.c_void_p
        L.oracle_model_create.argtypes = [_sz] * 7
        L.oracle_model_destroy.argtypes = [ctypes.c_void_p]
        L.oracle_digest.restype = ctypes.c_uint64
        L.oracle_digest.argtypes = [_f, _sz]
        _lib = L
    return _lib


def fp(a):
    """Pointer to a C-contiguous float32 array (None -> NULL)."""
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_f)


def check(rc):
    if rc != 0:
        raise ValueError(lib().oracle_last_error().decode())


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def randn(shape, seed):
    out = np.empty(shape, dtype=np.float32)
    check(lib().oracle_randn(fp(out), _sz(out.size), ctypes.c_uint64(seed)))
    return out


def digest(a):
    a = f32(a)
    return int(lib().oracle_digest(fp(a), _sz(a.size)))


def linear(x, w, b=None):
    """x [..., K] . w[N, K]^T + b."""
    x = f32(x)
    w = f32(w)
    M = x.size // x.shape[-1]
    K = x.shape[-1]
    N = w.shape[0]
    out = np.empty(x.shape[:-1] + (N,), np.float32)
    check(lib().oracle_linear(fp(x), fp(w), fp(None if b is None else f32(b)), fp(out), _sz(M), _sz(K), _sz(N)))
    return out


def layer_norm(x, eps, gamma=None, beta=None):
    x = f32(x)
    out = np.empty_like(x)
    C = x.shape[-1]
    check(lib().oracle_layer_norm(fp(x), fp(None if gamma is None else f32(gamma)),
                                  fp(None if beta is None else f32(beta)), fp(out),
                                  _sz(x.size // C), _sz(C), ctypes.c_float(eps)))
    return out


def rms_norm(x, eps, weight=None):
    x = f32(x)
    out = np.empty_like(x)
    C = x.shape[-1]
    check(lib().oracle_rms_norm(fp(x), fp(None if weight is None else f32(weight)), fp(out),
                                _sz(x.size // C), _sz(C), ctypes.c_float(eps)))
    return out


def modulate(x, shift, scale):
    """x [B,N,C], shift/scale [B,C]."""
    x = f32(x)
    B, N, C = x.shape
    out = np.empty_like(x)
    check(lib().oracle_modulate(fp(x), fp(f32(shift)), fp(f32(scale)), fp(out), _sz(B), _sz(N), _sz(C)))
    return out


def linear_attention(q, k, v, heads):
    q, k, v = f32(q), f32(k), f32(v)
    B, N, C = q.shape
    out = np.empty_like(q)
    check(lib().oracle_linear_attention(fp(q), fp(k), fp(v), fp(out), _sz(B), _sz(N), _sz(k.shape[1]),
                                        _sz(heads), _sz(C // heads)))
    return out


def attention(q, k, v, heads, bias=None):
    """q [B,Nq,C], k/v [B,L,C], bias [B,L] or None."""
    q, k, v = f32(q), f32(k), f32(v)
    B, Nq, C = q.shape
    L = k.shape[1]
    out = np.empty_like(q)
    check(lib().oracle_attention(fp(q), fp(k), fp(v), fp(None if bias is None else f32(bias)), fp(out),
                                 _sz(B), _sz(Nq), _sz(L), _sz(heads), _sz(C // heads)))
    return out


def depthwise3x3(x, w, b=None):
    """x token-major grid [B,H,W,C], w [C,3,3]."""
    x = f32(x)
    B, H, W, C = x.shape
    out = np.empty_like(x)
    check(lib().oracle_depthwise3x3(fp(x), fp(f32(w)), fp(None if b is None else f32(b)), fp(out),
                                    _sz(B), _sz(H), _sz(W), _sz(C)))
    return out


def glumb_conv(x, side_h, side_w, inv_w, inv_b, dw_w, dw_b, pt_w):
    x = f32(x)
    B, N, Cin = x.shape
    E = inv_w.shape[0]
    Cout = pt_w.shape[0]
    out = np.empty((B, N, Cout), np.float32)
    check(lib().oracle_glumb_conv(fp(x), fp(f32(inv_w)), fp(None if inv_b is None else f32(inv_b)),
                                  fp(f32(dw_w)), fp(None if dw_b is None else f32(dw_b)), fp(f32(pt_w)), fp(out),
                                  _sz(B), _sz(side_h), _sz(side_w), _sz(Cin), _sz(E), _sz(Cout)))
    return out


def caption_projection(x, w1, b1, w2, b2, norm_w):
    x = f32(x)
    C = w2.shape[0]
    rows = x.size // x.shape[-1]
    out = np.empty(x.shape[:-1] + (C,), np.float32)
    check(lib().oracle_caption_projection(fp(x), fp(f32(w1)), fp(f32(b1)), fp(f32(w2)), fp(f32(b2)),
                                          fp(f32(norm_w)), fp(out), _sz(rows), _sz(x.shape[-1]), _sz(C)))
    return out


def timestep_embedding(t, dim=256):
    t = f32(t)
    out = np.empty((t.size, dim), np.float32)
    check(lib().oracle_timestep_embedding(fp(t), fp(out), _sz(t.size), _sz(dim)))
    return out


def scheduler_timesteps(steps):
    ts = np.empty(steps, np.float32)
    sg = np.empty(steps + 1, np.float32)
    check(lib().oracle_scheduler_timesteps(_sz(steps), fp(ts), fp(sg)))
    return ts, sg


class BlockWeights(ctypes.Structure):
    _fields_ = [(n, _f) for n in (
        "scale_shift_table", "attn_norm_gamma", "attn_norm_beta", "q_w", "q_b", "k_w", "k_b", "v_w", "v_b",
        "out_w", "out_b", "cq_w", "cq_b", "ck_w", "ck_b", "cv_w", "cv_b", "co_w", "co_b",
        "mlp_norm_gamma", "mlp_norm_beta", "inv_w", "inv_b", "dw_w", "dw_b", "pt_w")] + [
        ("hidden", _sz), ("ffn", _sz), ("self_heads", _sz), ("cross_heads", _sz)]


def block_forward(weights, x, context, t_mod, bias=None):
    """weights: dict of the 26 SanaBlockWeights tensors (PyTorch order) + heads."""
    keep = {}
    st = BlockWeights()
    for name, _ in BlockWeights._fields_[:26]:
        arr = f32(weights[name])
        keep[name] = arr
        setattr(st, name, fp(arr))
    st.hidden = keep["scale_shift_table"].shape[1]
    st.ffn = keep["inv_w"].shape[0]
    st.self_heads = weights["self_heads"]
    st.cross_heads = weights["cross_heads"]
    x, context, t_mod = f32(x), f32(context), f32(t_mod)
    B, N, C = x.shape
    outs = [np.empty_like(x) for _ in range(3)]
    check(lib().oracle_block_forward(ctypes.byref(st), fp(x), fp(context), fp(t_mod),
                                     fp(None if bias is None else f32(bias)), _sz(B), _sz(N),
                                     _sz(context.shape[1]), *[fp(o) for o in outs]))
    return outs


class Model:
    """Whole-model oracle with synthetic or supplied weights (GGUF names)."""

    def __init__(self, layers=28, hidden=1152, ffn=5760, caption=2304, latent=32, self_heads=36, cross_heads=16,
                 generate=True):
        self.dims = dict(layers=layers, hidden=hidden, ffn=ffn, caption=caption, latent=latent,
                         self_heads=self_heads, cross_heads=cross_heads)
        self.h = lib().oracle_model_create(layers, hidden, ffn, caption, latent, self_heads, cross_heads)
        if generate:
            check(lib().oracle_model_generate(ctypes.c_void_p(self.h)))

    def __del__(self):
        if getattr(self, "h", None):
            lib().oracle_model_destroy(ctypes.c_void_p(self.h))
            self.h = None

    def set(self, name, arr):
        arr = f32(arr)
        check(lib().oracle_model_set(ctypes.c_void_p(self.h), name.encode(), fp(arr), _sz(arr.size)))

    def get(self, name, shape):
        out = np.empty(shape, np.float32)
        check(lib().oracle_model_get(ctypes.c_void_p(self.h), name.encode(), fp(out), _sz(out.size)))
        return out

    def project_caption(self, caption):
        caption = f32(caption)
        B, L, _ = caption.shape
        out = np.empty((B, L, self.dims["hidden"]), np.float32)
        check(lib().oracle_model_project_caption(ctypes.c_void_p(self.h), fp(caption), _sz(B), _sz(L), fp(out)))
        return out

    def time(self, t):
        t = f32(np.atleast_1d(t))
        C = self.dims["hidden"]
        emb = np.empty((t.size, C), np.float32)
        tmod = np.empty((t.size, 6 * C), np.float32)
        check(lib().oracle_model_time(ctypes.c_void_p(self.h), fp(t), _sz(t.size), fp(emb), fp(tmod)))
        return emb, tmod

    def patch_embed(self, latent):
        latent = f32(latent)
        B, _, H, W = latent.shape
        out = np.empty((B, H * W, self.dims["hidden"]), np.float32)
        check(lib().oracle_model_patch_embed(ctypes.c_void_p(self.h), fp(latent), _sz(B), _sz(H), _sz(W), fp(out)))
        return out

    def block(self, i, x, context, t_mod, bias=None):
        x, context, t_mod = f32(x), f32(context), f32(t_mod)
        B, N, _ = x.shape
        outs = [np.empty_like(x) for _ in range(3)]
        check(lib().oracle_model_block(ctypes.c_void_p(self.h), _sz(i), fp(x), fp(context), fp(t_mod),
                                       fp(None if bias is None else f32(bias)), _sz(B), _sz(N),
                                       _sz(context.shape[1]), *[fp(o) for o in outs]))
        return outs

    def forward(self, latent, context, t, bias=None):
        latent, context = f32(latent), f32(context)
        Bl, Cl, H, W = latent.shape
        out = np.empty((2 * Bl, Cl, H, W), np.float32)
        check(lib().oracle_model_forward(ctypes.c_void_p(self.h), fp(latent), _sz(Bl), _sz(H), _sz(W), fp(context),
                                         _sz(context.shape[1]), fp(None if bias is None else f32(bias)),
                                         ctypes.c_float(t), fp(out)))
        return out

    def loop(self, latent, caption, steps, guidance, bias=None):
        latent, caption = f32(latent), f32(caption)
        Bl, Cl, H, W = latent.shape
        out = np.empty_like(latent)
        check(lib().oracle_model_loop(ctypes.c_void_p(self.h), fp(latent), _sz(Bl), _sz(H), _sz(W), fp(caption),
                                      _sz(caption.shape[1]), fp(None if bias is None else f32(bias)), _sz(steps),
                                      ctypes.c_float(guidance), fp(out)))
        return out


def mask_bias(L=300, uncond_real=1, cond_real=40):
    """The additive padding mask of the Gemma encoder (src/gemma_encoder.cpp:177-184)."""
    b = np.full((2, L), -10000.0, np.float32)
    b[0, :uncond_real] = 0.0
    b[1, :cond_real] = 0.0
    return b


# ---------------------------------------------------------------- VAE decoder
SMALL_VAE = dict(latent=32, channels=(64, 64, 128, 128), attn=(False, False, True, True), head_dim=32, expand=4)
FULL_VAE = dict(latent=32, channels=(128, 256, 512, 512, 1024, 1024), attn=(False, False, False, True, True, True),
                head_dim=32, expand=4)


def vae_manifest(cfg):
    """GGUF name -> PyTorch-order shape of the synthetic decoder (oracle/vae_spec.h)."""
    ch, attn, L = cfg["channels"], cfg["attn"], len(cfg["channels"])
    m = {"decoder.conv_in.weight": (ch[-1], cfg["latent"], 3, 3), "decoder.conv_in.bias": (ch[-1],),
         "decoder.norm_out.weight": (ch[0],), "decoder.norm_out.bias": (ch[0],),
         "decoder.conv_out.weight": (3, ch[0], 3, 3), "decoder.conv_out.bias": (3,)}
    for i in range(L):
        p, C, base = f"decoder.up_blocks.{i}.", ch[i], 0
        if i + 1 < L:
            m[p + "0.conv.weight"] = (C, ch[i + 1], 3, 3)
            m[p + "0.conv.bias"] = (C,)
            base = 1
        for l in range(base, base + 3):
            q = f"{p}{l}."
            if not attn[i]:
                m.update({q + "conv1.weight": (C, C, 3, 3), q + "conv1.bias": (C,), q + "conv2.weight": (C, C, 3, 3),
                          q + "norm.weight": (C,), q + "norm.bias": (C,)})
            else:
                Hd = cfg["expand"] * C
                m.update({q + "attn.to_q.weight": (C, C), q + "attn.to_k.weight": (C, C),
                          q + "attn.to_v.weight": (C, C),
                          q + "attn.to_qkv_multiscale.0.proj_in.weight": (3 * C, 1, 5, 5),
                          q + "attn.to_qkv_multiscale.0.proj_out.weight": (3 * C, cfg["head_dim"], 1, 1),
                          q + "attn.to_out.weight": (C, 2 * C), q + "attn.norm_out.weight": (C,),
                          q + "attn.norm_out.bias": (C,),
                          q + "conv_out.conv_inverted.weight": (2 * Hd, C, 1, 1),
                          q + "conv_out.conv_inverted.bias": (2 * Hd,),
                          q + "conv_out.conv_depth.weight": (2 * Hd, 1, 3, 3),
                          q + "conv_out.conv_depth.bias": (2 * Hd,),
                          q + "conv_out.conv_point.weight": (C, Hd, 1, 1), q + "conv_out.norm.weight": (C,),
                          q + "conv_out.norm.bias": (C,)})
    return m


class Vae:
    """Whole-decoder oracle with the synthetic weights (or supplied ones)."""

    def __init__(self, full=False, generate=True, cfg=None):
        L = lib()
        L.oracle_vae_create.restype = ctypes.c_void_p
        L.oracle_vae_create.argtypes = [ctypes.c_int]
        L.oracle_vae_create_config.restype = ctypes.c_void_p
        L.oracle_vae_create_config.argtypes = [_sz, _sz, ctypes.POINTER(_sz), ctypes.POINTER(ctypes.c_int)]
        L.oracle_vae_destroy.argtypes = [ctypes.c_void_p]
        if cfg is not None:
            self.cfg = dict(SMALL_VAE, **cfg)
            n = len(self.cfg["channels"])
            ch = (_sz * n)(*self.cfg["channels"])
            at = (ctypes.c_int * n)(*[1 if a else 0 for a in self.cfg["attn"]])
            self.h = L.oracle_vae_create_config(self.cfg["latent"], n, ch, at)
        else:
            self.cfg = FULL_VAE if full else SMALL_VAE
            self.h = L.oracle_vae_create(1 if full else 0)
        if generate:
            check(L.oracle_vae_generate(ctypes.c_void_p(self.h)))

    def __del__(self):
        if getattr(self, "h", None):
            lib().oracle_vae_destroy(ctypes.c_void_p(self.h))
            self.h = None

    def get(self, name, shape=None):
        shape = shape or vae_manifest(self.cfg)[name]
        out = np.empty(shape, np.float32)
        check(lib().oracle_vae_get(ctypes.c_void_p(self.h), name.encode(), fp(out), _sz(out.size)))
        return out

    def set(self, name, arr):
        arr = f32(arr)
        check(lib().oracle_vae_set(ctypes.c_void_p(self.h), name.encode(), fp(arr), _sz(arr.size)))

    def upscale(self):
        return 2 ** (len(self.cfg["channels"]) - 1)

    def decoder_input(self, latent):
        latent = f32(latent)
        B, _, H, W = latent.shape
        out = np.empty((B, self.cfg["channels"][-1], H, W), np.float32)
        check(lib().oracle_vae_decoder_input(ctypes.c_void_p(self.h), fp(latent), _sz(B), _sz(H), _sz(W), fp(out)))
        return out

    def layer(self, kind, level, layer, x):
        x = f32(x)
        B, C, H, W = x.shape
        out = np.empty_like(x)
        fn = {"res": lib().oracle_vae_res_block, "attn": lib().oracle_vae_attention,
              "glumb": lib().oracle_vae_glumb}[kind]
        check(fn(ctypes.c_void_p(self.h), _sz(level), _sz(layer), fp(x), fp(out), _sz(B), _sz(H), _sz(W)))
        return out

    def decode(self, latent):
        latent = f32(latent)
        B, _, H, W = latent.shape
        s = self.upscale()
        out = np.empty((B, 3, H * s, W * s), np.float32)
        check(lib().oracle_vae_decode(ctypes.c_void_p(self.h), fp(latent), _sz(B), _sz(H), _sz(W), fp(out)))
        return out


def vae_conv3x3(x, w, b=None, order=-1):
    """order -1: as the reference dispatches by size; 0: im2col order; 1: tap order."""
    x, w = f32(x), f32(w)
    B, Cin, H, W = x.shape
    out = np.empty((B, w.shape[0], H, W), np.float32)
    check(lib().oracle_vae_conv3x3(fp(x), fp(w), fp(None if b is None else f32(b)), fp(out), _sz(B), _sz(Cin),
                                   _sz(w.shape[0]), _sz(H), _sz(W), ctypes.c_int(order)))
    return out


def vae_rms_norm(x, w, b=None, eps=1e-5):
    x = f32(x)
    B, C, H, W = x.shape
    out = np.empty_like(x)
    check(lib().oracle_vae_rms_norm(fp(x), fp(f32(w)), fp(None if b is None else f32(b)), fp(out), _sz(B), _sz(C),
                                    _sz(H * W), ctypes.c_float(eps)))
    return out


def vae_dw5x5(x, w, b=None):
    x = f32(x)
    B, C, H, W = x.shape
    out = np.empty_like(x)
    check(lib().oracle_vae_dw5x5(fp(x), fp(f32(w)), fp(None if b is None else f32(b)), fp(out), _sz(B), _sz(C),
                                 _sz(H), _sz(W)))
    return out


def vae_grouped_conv1x1(x, w, groups):
    x, w = f32(x), f32(w)
    B, Cin, H, W = x.shape
    out = np.empty((B, w.shape[0], H, W), np.float32)
    check(lib().oracle_vae_grouped_conv1x1(fp(x), fp(w), fp(out), _sz(B), _sz(Cin), _sz(w.shape[0]), _sz(groups),
                                           _sz(H * W)))
    return out


def vae_upsample(x, w, b, shortcut=True):
    x, w = f32(x), f32(w)
    B, Cin, H, W = x.shape
    out = np.empty((B, w.shape[0], 2 * H, 2 * W), np.float32)
    check(lib().oracle_vae_upsample(fp(x), fp(w), fp(f32(b)), fp(out), _sz(B), _sz(Cin), _sz(w.shape[0]), _sz(H),
                                    _sz(W), ctypes.c_int(1 if shortcut else 0)))
    return out
