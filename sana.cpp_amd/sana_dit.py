"""ctypes binding of libsana_dit.so (the C ABI declared in include/sana_dit.h).

This is the Python-side stub a caller binds; tests and bench.py use it.  It
never falls back to anything: if the library is missing or a call fails, it
raises.

Callers that also pass torch tensors must import torch before the first call
here loads the library: torch carries its own HIP runtime, which finds no GPU
when the system ROCm runtime that libsana_dit.so links was loaded first.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsana_dit.so")

SANA_OK = 0
SANA_ERR_INVALID_ARGUMENT = -1
SANA_ERR_SHAPE = -2
SANA_ERR_IO = -3
SANA_ERR_FORMAT = -4
SANA_ERR_HIP = -5
SANA_ERR_OUT_OF_MEMORY = -6
SANA_ERR_STATE = -7

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_fp = ctypes.POINTER(ctypes.c_float)


class Config(ctypes.Structure):
    _fields_ = [("layers", _i64), ("hidden", _i64), ("ffn", _i64), ("caption_dim", _i64),
                ("latent_channels", _i64), ("self_heads", _i64), ("cross_heads", _i64), ("device", ctypes.c_int)]


SANA_VAE_MAX_LEVELS = 8


class VaeConfig(ctypes.Structure):
    _fields_ = [("latent_channels", _i64), ("levels", _i64), ("channels", _i64 * SANA_VAE_MAX_LEVELS),
                ("attention", ctypes.c_int32 * SANA_VAE_MAX_LEVELS), ("head_dim", _i64), ("expand", _i64),
                ("scaling_factor", ctypes.c_float), ("device", ctypes.c_int)]


class GemmaConfig(ctypes.Structure):
    _fields_ = [("vocab", _i64), ("hidden", _i64), ("layers", _i64), ("heads", _i64), ("kv_heads", _i64),
                ("head_dim", _i64), ("ffn", _i64), ("sliding_window", _i64), ("rms_eps", ctypes.c_float),
                ("rope_theta", ctypes.c_float), ("attn_softcap", ctypes.c_float), ("query_scale", ctypes.c_float),
                ("device", ctypes.c_int)]


# name -> (restype, argtypes); exactly the entry points of include/sana_dit.h
PROTOTYPES = {
    "sana_dit_last_error": (ctypes.c_char_p, []),
    "sana_dit_create": (ctypes.c_int, [ctypes.POINTER(Config), ctypes.POINTER(_vp)]),
    "sana_dit_destroy": (None, [_vp]),
    "sana_dit_set_weight": (ctypes.c_int, [_vp, ctypes.c_char_p, _vp, ctypes.POINTER(_i64), ctypes.c_int,
                                           ctypes.c_int]),
    "sana_dit_set_block_weight": (ctypes.c_int, [_vp, _i64, ctypes.c_char_p, _vp, ctypes.POINTER(_i64),
                                                 ctypes.c_int, ctypes.c_int]),
    "sana_dit_set_block_norm": (ctypes.c_int, [_vp, _i64, ctypes.c_int, _vp, _vp]),
    "sana_dit_set_weight_f16": (ctypes.c_int, [_vp, ctypes.c_char_p, _vp, ctypes.POINTER(_i64), ctypes.c_int]),
    "sana_dit_set_block_weight_f16": (ctypes.c_int, [_vp, _i64, ctypes.c_char_p, _vp, ctypes.POINTER(_i64),
                                                     ctypes.c_int]),
    "sana_dit_check_weights": (ctypes.c_int, [_vp]),
    "sana_dit_load_gguf": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p]),
    "sana_dit_save_packed": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_uint64]),
    "sana_dit_load_packed": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_uint64]),
    "sana_dit_load_gguf_cached": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p,
                                                 ctypes.c_char_p, ctypes.POINTER(ctypes.c_int)]),
    "sana_dit_set_context": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, ctypes.c_int, _vp]),
    "sana_dit_get_context": (ctypes.c_int, [_vp, _vp]),
    "sana_dit_forward": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, ctypes.c_float, _vp]),
    "sana_dit_forward_device": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, ctypes.c_float, _vp, _vp]),
    "sana_dit_step_device": (ctypes.c_int, [_vp, _vp, _i64, _vp, _vp, _i64, _i64, _i64, ctypes.c_float, _vp, _vp]),
    "sana_dit_block_forward": (ctypes.c_int, [_vp, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _vp]),
    "sana_dit_run_blocks": (ctypes.c_int, [_vp, _i64, _i64, _vp, _vp, _i64, _i64, _vp]),
    "sana_dit_denoise_loop": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, ctypes.c_float, _vp]),
    "sana_dit_denoise_loop_device": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, ctypes.c_float, _vp,
                                                    _vp]),
    "sana_dit_loop_model_outputs": (ctypes.c_int, [_vp, _vp, _vp]),
    "sana_dit_time_embed": (ctypes.c_int, [_vp, _vp, _i64, _vp, _vp]),
    "sana_hip_hbm_peak": (ctypes.c_int, [_vp, _vp, _i64, _vp, ctypes.POINTER(_i64), _vp]),
    "sana_dit_time_kernel": (ctypes.c_int, [_vp, ctypes.c_int, ctypes.c_int, _fp, ctypes.POINTER(ctypes.c_double),
                                            ctypes.POINTER(ctypes.c_double), ctypes.c_char_p, ctypes.c_size_t]),
    "sana_randn_torch_cpu": (ctypes.c_int, [_vp, _i64, ctypes.c_uint64]),
    "sana_gguf_num_tensors": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_i64)]),
    "sana_gguf_tensor_info": (ctypes.c_int, [ctypes.c_char_p, _i64, ctypes.c_char_p, ctypes.c_size_t,
                                             ctypes.POINTER(_i64), ctypes.POINTER(ctypes.c_int),
                                             ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_uint64)]),
    "sana_hip_gemm": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, ctypes.c_int, _vp, _i64, _vp,
                                     _i64, _vp]),
    "sana_hip_gemm_residual": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i64,
                                              _vp, _i64, _vp, _i64, _vp]),
    "sana_hip_ln_modulate": (ctypes.c_int, [_vp, _i64, _vp, _i64, _i64, _i64, _i64, ctypes.c_float, _vp, _vp, _vp,
                                            _vp, _i64, _i64, _i64, _vp]),
    "sana_hip_linear_attention": (ctypes.c_int, [_vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp]),
    "sana_hip_linear_attention_noalloc": (ctypes.c_int, [_vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _vp]),
    "sana_hip_linear_attention_workspace": (ctypes.c_size_t, [_i64, _i64, _i64, _i64]),
    "sana_hip_cross_attention": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64,
                                                _i64, _i64, _vp]),
    "sana_hip_dwconv_glu": (ctypes.c_int, [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp]),
    "sana_hip_mfma_peak": (ctypes.c_int, [_i64, _i64, ctypes.c_int, _vp, _vp, ctypes.POINTER(ctypes.c_double)]),
    "sana_vae_create": (ctypes.c_int, [ctypes.POINTER(VaeConfig), ctypes.POINTER(_vp)]),
    "sana_vae_destroy": (ctypes.c_int, [_vp]),
    "sana_vae_set_weight": (ctypes.c_int, [_vp, ctypes.c_char_p, _vp, ctypes.POINTER(_i64), ctypes.c_int]),
    "sana_vae_check_weights": (ctypes.c_int, [_vp]),
    "sana_vae_load_gguf": (ctypes.c_int, [_vp, ctypes.c_char_p]),
    "sana_vae_decode": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, _vp]),
    "sana_vae_decoder_input": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, ctypes.c_int, _vp]),
    "sana_gemma_create": (ctypes.c_int, [ctypes.POINTER(GemmaConfig), ctypes.POINTER(_vp)]),
    "sana_gemma_destroy": (ctypes.c_int, [_vp]),
    "sana_gemma_set_weight": (ctypes.c_int, [_vp, ctypes.c_char_p, _vp, ctypes.POINTER(_i64), ctypes.c_int]),
    "sana_gemma_check_weights": (ctypes.c_int, [_vp]),
    "sana_gemma_load_gguf": (ctypes.c_int, [_vp, ctypes.c_char_p]),
    "sana_gemma_encode": (ctypes.c_int, [_vp, _vp, _i64, _vp]),
    "sana_gemma_encode_pair": (ctypes.c_int, [_vp, _vp, _i64, _vp, _i64, _vp, _vp]),
    "sana_vae_decode_device": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    "sana_op_gemm_f32": (ctypes.c_int, [_vp, _i64, _i64, _vp, _i64, _i64, ctypes.c_int, _vp, ctypes.c_int, _vp, _i64,
                                        _i64, _i64, _i64, _i64, _i64, ctypes.c_int, _vp]),
    "sana_op_unary_f32": (ctypes.c_int, [_vp, _vp, _i64, ctypes.c_int, _vp]),
    "sana_op_softmax_f32": (ctypes.c_int, [_vp, _vp, _i64, _i64, ctypes.c_float, _vp, _i64, _vp]),
    "sana_op_rms_norm_f32": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, ctypes.c_float, _vp]),
    "sana_op_dwconv_f32": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp]),
    "sana_op_glu_f32": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, _vp]),
    "sana_op_linear_attention_f32": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp]),
    "sana_op_heads_f32": (ctypes.c_int, [_vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_int, _vp]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class SanaError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def check(rc):
    if rc != SANA_OK:
        raise SanaError(rc, lib().sana_dit_last_error().decode())


def ptr(x):
    """Address of a numpy array, a torch tensor, an int or None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    if isinstance(x, np.ndarray):
        assert x.flags["C_CONTIGUOUS"]
        return x.ctypes.data
    return x.data_ptr()  # torch tensor


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class Dit:
    """One device context (weights, workspace, graphs) of the DiT."""

    def __init__(self, layers=28, hidden=1152, ffn=5760, caption_dim=2304, latent_channels=32, self_heads=36,
                 cross_heads=16, device=0):
        cfg = Config(layers, hidden, ffn, caption_dim, latent_channels, self_heads, cross_heads, device)
        self.cfg = cfg
        h = _vp()
        check(lib().sana_dit_create(ctypes.byref(cfg), ctypes.byref(h)))
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            lib().sana_dit_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def set_weight(self, name, arr, transposed=False):
        arr = _f32(arr)
        shape = (_i64 * arr.ndim)(*arr.shape)
        if name.startswith("transformer_blocks."):
            _, idx, suffix = name.split(".", 2)
            check(lib().sana_dit_set_block_weight(self.h, int(idx), suffix.encode(), ptr(arr), shape, arr.ndim,
                                                  int(transposed)))
        else:
            check(lib().sana_dit_set_weight(self.h, name.encode(), ptr(arr), shape, arr.ndim, int(transposed)))

    def set_weight_f16(self, name, arr):
        """A linear weight as fp16 (numpy float16, PyTorch-order shape): its
        bits go to the device's fp16 operand buffer unchanged."""
        arr = np.ascontiguousarray(arr, dtype=np.float16)
        shape = (_i64 * arr.ndim)(*arr.shape)
        if name.startswith("transformer_blocks."):
            _, idx, suffix = name.split(".", 2)
            check(lib().sana_dit_set_block_weight_f16(self.h, int(idx), suffix.encode(), ptr(arr), shape, arr.ndim))
        else:
            check(lib().sana_dit_set_weight_f16(self.h, name.encode(), ptr(arr), shape, arr.ndim))

    def set_block_norm(self, block, which, gamma=None, beta=None):
        g = None if gamma is None else _f32(gamma)
        b = None if beta is None else _f32(beta)
        check(lib().sana_dit_set_block_norm(self.h, block, which, ptr(g), ptr(b)))

    def check_weights(self):
        check(lib().sana_dit_check_weights(self.h))

    def load_gguf(self, model, caption, denoiser):
        check(lib().sana_dit_load_gguf(self.h, model.encode(), caption.encode(), denoiser.encode()))

    def save_packed(self, path, key=0):
        check(lib().sana_dit_save_packed(self.h, path.encode(), key))

    def load_packed(self, path, key=0):
        check(lib().sana_dit_load_packed(self.h, path.encode(), key))

    def load_gguf_cached(self, model, caption, denoiser, cache):
        """Returns True when the packed cache was used."""
        used = ctypes.c_int(0)
        check(lib().sana_dit_load_gguf_cached(self.h, model.encode(), caption.encode(), denoiser.encode(),
                                              cache.encode(), ctypes.byref(used)))
        return bool(used.value)

    def set_context(self, data, projected, bias=None):
        data = _f32(data)
        B, L, dim = data.shape
        b = None if bias is None else _f32(bias)
        check(lib().sana_dit_set_context(self.h, ptr(data), B, L, dim, int(projected), ptr(b)))

    def get_context(self, shape):
        out = np.empty(shape, np.float32)
        check(lib().sana_dit_get_context(self.h, ptr(out)))
        return out

    def forward(self, latent, t):
        latent = _f32(latent)
        Bl, Cl, H, W = latent.shape
        out = np.empty((2 * Bl, Cl, H, W), np.float32)
        check(lib().sana_dit_forward(self.h, ptr(latent), Bl, H, W, float(t), ptr(out)))
        return out

    def forward_device(self, d_latent, shape, t, d_out, stream=None):
        Bl, Cl, H, W = shape
        check(lib().sana_dit_forward_device(self.h, ptr(d_latent), Bl, H, W, float(t), ptr(d_out), stream))

    def step_device(self, d_caption, L, d_bias, d_latent, shape, t, d_out, stream=None):
        Bl, Cl, H, W = shape
        check(lib().sana_dit_step_device(self.h, ptr(d_caption), L, ptr(d_bias), ptr(d_latent), Bl, H, W, float(t),
                                         ptr(d_out), stream))

    def block_forward(self, block, x, t_mod):
        x = _f32(x)
        t_mod = _f32(t_mod)
        B, N, C = x.shape
        outs = [np.empty_like(x) for _ in range(3)]
        check(lib().sana_dit_block_forward(self.h, block, ptr(x), ptr(t_mod), B, N, *[ptr(o) for o in outs]))
        return outs

    def run_blocks(self, begin, end, x, t_mod):
        x = _f32(x)
        t_mod = _f32(t_mod)
        B, N, C = x.shape
        out = np.empty_like(x)
        check(lib().sana_dit_run_blocks(self.h, begin, end, ptr(x), ptr(t_mod), B, N, ptr(out)))
        return out

    def denoise_loop(self, latent, timesteps, sigmas, guidance):
        latent = _f32(latent)
        ts, sg = _f32(timesteps), _f32(sigmas)
        Bl, Cl, H, W = latent.shape
        out = np.empty_like(latent)
        check(lib().sana_dit_denoise_loop(self.h, ptr(latent), Bl, H, W, ptr(ts), ptr(sg), ts.size, float(guidance),
                                          ptr(out)))
        return out

    def denoise_loop_device(self, d_latent, shape, timesteps, sigmas, guidance, d_out, stream=None):
        ts, sg = _f32(timesteps), _f32(sigmas)
        Bl, Cl, H, W = shape
        check(lib().sana_dit_denoise_loop_device(self.h, ptr(d_latent), Bl, H, W, ptr(ts), ptr(sg), ts.size,
                                                 float(guidance), ptr(d_out), stream))

    def time_embed(self, t):
        t = _f32(np.atleast_1d(t))
        C = self.cfg.hidden
        emb = np.empty((t.size, C), np.float32)
        tmod = np.empty((t.size, 6 * C), np.float32)
        check(lib().sana_dit_time_embed(self.h, ptr(t), t.size, ptr(emb), ptr(tmod)))
        return emb, tmod

    # kernel classes of sana_dit_time_kernel, in its `which` order
    KERNELS = ("qkv", "attn_out", "cross_q", "cross_out", "ffn_inverted", "ffn_point", "ln_modulate",
               "linear_attention", "cross_attention", "dwconv_glu")

    def time_kernel(self, which, iters):
        """(avg ms, flops, bytes, kernel name) of one block kernel launched as the
        last forward launched it."""
        ms = ctypes.c_float()
        fl, by = ctypes.c_double(), ctypes.c_double()
        name = ctypes.create_string_buffer(256)
        check(lib().sana_dit_time_kernel(self.h, which, iters, ctypes.byref(ms), ctypes.byref(fl), ctypes.byref(by),
                                         name, 256))
        return ms.value, fl.value, by.value, name.value.decode()


def gguf_index(path):
    """[(name, shape, ggml_type, absolute_offset)] of a GGUF file (CPU only)."""
    n = _i64()
    check(lib().sana_gguf_num_tensors(path.encode(), ctypes.byref(n)))
    out = []
    for i in range(n.value):
        name = ctypes.create_string_buffer(1024)
        shape = (_i64 * 4)()
        nd, ty, off = ctypes.c_int(), ctypes.c_int(), ctypes.c_uint64()
        check(lib().sana_gguf_tensor_info(path.encode(), i, name, 1024, shape, ctypes.byref(nd), ctypes.byref(ty),
                                          ctypes.byref(off)))
        out.append((name.value.decode(), tuple(shape[:nd.value]), ty.value, off.value))
    return out


def randn(shape, seed):
    """torch.randn(shape) on the CPU generator seeded with `seed` (float32)."""
    out = np.empty(shape, np.float32)
    check(lib().sana_randn_torch_cpu(ptr(out), out.size, seed))
    return out


def seeded_weights(layers=28, hidden=1152, ffn=5760, caption_dim=2304, latent_channels=32, scale=0.02):
    """The seeded synthetic weights the reference CPU baseline builds: tensor i
    of the byte-wise sorted names of the three weight files is scale *
    randn(shape, 1000 + i), except caption_norm.weight, which is all ones.
    Yields (name, float32 array) in that order."""
    m = manifest(layers, hidden, ffn, caption_dim, latent_channels)
    for i, name in enumerate(sorted(m)):
        if name == "caption_norm.weight":
            yield name, np.ones(m[name], np.float32)
        else:
            w = randn(m[name], 1000 + i)
            w *= np.float32(scale)
            yield name, w


def manifest(layers=28, hidden=1152, ffn=5760, caption_dim=2304, latent_channels=32, time_freq=256):
    """{GGUF tensor name: PyTorch-order shape} of the three weight files the
    loader reads (src/transformer.cpp:171-190 caption, :214-308 per block,
    :473-484 denoiser)."""
    C, E = hidden, ffn
    shapes = {}
    for i in range(layers):
        p = f"transformer_blocks.{i}."
        shapes.update({
            p + "scale_shift_table": (6, C), p + "attn1.to_q.weight": (C, C), p + "attn1.to_k.weight": (C, C),
            p + "attn1.to_v.weight": (C, C), p + "attn1.to_out.0.weight": (C, C), p + "attn1.to_out.0.bias": (C,),
            p + "attn2.to_q.weight": (C, C), p + "attn2.to_q.bias": (C,), p + "attn2.to_k.weight": (C, C),
            p + "attn2.to_k.bias": (C,), p + "attn2.to_v.weight": (C, C), p + "attn2.to_v.bias": (C,),
            p + "attn2.to_out.0.weight": (C, C), p + "attn2.to_out.0.bias": (C,),
            p + "ff.conv_inverted.weight": (E, C, 1, 1), p + "ff.conv_inverted.bias": (E,),
            p + "ff.conv_depth.weight": (E, 1, 3, 3), p + "ff.conv_depth.bias": (E,),
            p + "ff.conv_point.weight": (C, E // 2, 1, 1)})
    shapes.update({
        "caption_projection.linear_1.weight": (C, caption_dim), "caption_projection.linear_1.bias": (C,),
        "caption_projection.linear_2.weight": (C, C), "caption_projection.linear_2.bias": (C,),
        "patch_embed.proj.weight": (C, latent_channels, 1, 1), "patch_embed.proj.bias": (C,),
        "time_embed.emb.timestep_embedder.linear_1.weight": (C, time_freq),
        "time_embed.emb.timestep_embedder.linear_1.bias": (C,),
        "time_embed.emb.timestep_embedder.linear_2.weight": (C, C),
        "time_embed.emb.timestep_embedder.linear_2.bias": (C,),
        "time_embed.linear.weight": (6 * C, C), "time_embed.linear.bias": (6 * C,),
        "caption_norm.weight": (C,), "scale_shift_table": (2, C), "proj_out.weight": (latent_channels, C),
        "proj_out.bias": (latent_channels,)})
    return shapes


def vae_manifest(channels, attention, latent_channels=32, head_dim=32, expand=4):
    """{GGUF tensor name: PyTorch-order shape} of the DC-AE decoder weights the
    loader reads (src/vae.cpp:10-118): conv_in / norm_out / conv_out, then per
    up block an upsample conv (all but the innermost block) and three ResBlocks
    or three EfficientViT layers (multiscale attention + GLUMBConv)."""
    L, top, out = len(channels), channels[-1], channels[0]
    shapes = {"decoder.conv_in.weight": (top, latent_channels, 3, 3), "decoder.conv_in.bias": (top,),
              "decoder.norm_out.weight": (out,), "decoder.norm_out.bias": (out,),
              "decoder.conv_out.weight": (3, out, 3, 3), "decoder.conv_out.bias": (3,)}
    for i, C in enumerate(channels):
        p = f"decoder.up_blocks.{i}."
        base = 0
        if i + 1 < L:
            shapes.update({p + "0.conv.weight": (C, channels[i + 1], 3, 3), p + "0.conv.bias": (C,)})
            base = 1
        for l in range(base, base + 3):
            q = f"{p}{l}."
            if not attention[i]:
                shapes.update({q + "conv1.weight": (C, C, 3, 3), q + "conv1.bias": (C,),
                               q + "conv2.weight": (C, C, 3, 3), q + "norm.weight": (C,), q + "norm.bias": (C,)})
            else:
                E = expand * C
                shapes.update({
                    q + "attn.to_q.weight": (C, C), q + "attn.to_k.weight": (C, C), q + "attn.to_v.weight": (C, C),
                    q + "attn.to_qkv_multiscale.0.proj_in.weight": (3 * C, 1, 5, 5),
                    q + "attn.to_qkv_multiscale.0.proj_out.weight": (3 * C, head_dim, 1, 1),
                    q + "attn.to_out.weight": (C, 2 * C), q + "attn.norm_out.weight": (C,),
                    q + "attn.norm_out.bias": (C,), q + "conv_out.conv_inverted.weight": (2 * E, C, 1, 1),
                    q + "conv_out.conv_inverted.bias": (2 * E,), q + "conv_out.conv_depth.weight": (2 * E, 1, 3, 3),
                    q + "conv_out.conv_depth.bias": (2 * E,), q + "conv_out.conv_point.weight": (C, E, 1, 1),
                    q + "conv_out.norm.weight": (C,), q + "conv_out.norm.bias": (C,)})
    return shapes


class Vae:
    """One device context of the DC-AE VAE decoder (weights and workspace).

    channels / attention are per level as the reference's decoder.up_blocks.{i}
    (level 0 = output resolution)."""

    def __init__(self, channels, attention, latent_channels=32, head_dim=32, expand=4, scaling_factor=0.41407,
                 device=0):
        n = len(channels)
        cfg = VaeConfig()
        cfg.latent_channels, cfg.levels, cfg.head_dim, cfg.expand = latent_channels, n, head_dim, expand
        cfg.scaling_factor, cfg.device = scaling_factor, device
        for i in range(n):
            cfg.channels[i] = channels[i]
            cfg.attention[i] = 1 if attention[i] else 0
        self.cfg, self.levels, self.latent_channels = cfg, n, latent_channels
        h = _vp()
        check(lib().sana_vae_create(ctypes.byref(cfg), ctypes.byref(h)))
        self.h = h
        self._destroy = lib().sana_vae_destroy  # still callable during interpreter shutdown

    def close(self):
        if getattr(self, "h", None):
            self._destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def set_weight(self, name, arr):
        arr = _f32(arr)
        shape = (_i64 * arr.ndim)(*arr.shape)
        check(lib().sana_vae_set_weight(self.h, name.encode(), ptr(arr), shape, arr.ndim))

    def check_weights(self):
        check(lib().sana_vae_check_weights(self.h))

    def load_gguf(self, path):
        check(lib().sana_vae_load_gguf(self.h, str(path).encode()))

    def decode(self, latent):
        latent = _f32(latent)
        B, _, H, W = latent.shape
        s = 2 ** (self.levels - 1)
        out = np.empty((B, 3, H * s, W * s), np.float32)
        check(lib().sana_vae_decode(self.h, ptr(latent), B, H, W, ptr(out)))
        return out

    def decoder_input(self, latent, in_shortcut=True):
        """conv_in (+ channel-repeat shortcut) of an unscaled latent: [B, C_top, H, W]."""
        latent = _f32(latent)
        B, _, H, W = latent.shape
        out = np.empty((B, self.cfg.channels[self.levels - 1], H, W), np.float32)
        check(lib().sana_vae_decoder_input(self.h, ptr(latent), B, H, W, int(in_shortcut), ptr(out)))
        return out

    def decode_device(self, latent, shape, image, stream):
        B, _, H, W = shape
        check(lib().sana_vae_decode_device(self.h, ptr(latent), B, H, W, ptr(image), stream))


GEMMA2_2B = dict(vocab=256000, hidden=2304, layers=26, heads=8, kv_heads=4, head_dim=256, ffn=9216,
                 sliding_window=4096, rms_eps=1e-6, rope_theta=10000.0, softcap=50.0, query_scale=1.0 / 16.0)


def gemma_manifest(vocab, hidden, layers, heads, kv_heads, head_dim, ffn, **_):
    """{GGUF tensor name: PyTorch-order shape} of a Gemma-2 encoder as llama.cpp names it."""
    Dq, Dkv = heads * head_dim, kv_heads * head_dim
    m = {"token_embd.weight": (vocab, hidden), "output_norm.weight": (hidden,)}
    for l in range(layers):
        p = f"blk.{l}."
        m.update({p + "attn_norm.weight": (hidden,), p + "attn_q.weight": (Dq, hidden),
                  p + "attn_k.weight": (Dkv, hidden), p + "attn_v.weight": (Dkv, hidden),
                  p + "attn_output.weight": (hidden, Dq), p + "post_attention_norm.weight": (hidden,),
                  p + "ffn_norm.weight": (hidden,), p + "ffn_gate.weight": (ffn, hidden),
                  p + "ffn_up.weight": (ffn, hidden), p + "ffn_down.weight": (hidden, ffn),
                  p + "post_ffw_norm.weight": (hidden,)})
    return m


class Gemma:
    """One device context of the Gemma-2 text encoder.  cfg keys as GEMMA2_2B."""

    def __init__(self, cfg, device=0):
        c = GemmaConfig()
        c.vocab, c.hidden, c.layers, c.heads = cfg["vocab"], cfg["hidden"], cfg["layers"], cfg["heads"]
        c.kv_heads, c.head_dim, c.ffn = cfg["kv_heads"], cfg["head_dim"], cfg["ffn"]
        c.sliding_window, c.rms_eps, c.rope_theta = cfg["sliding_window"], cfg["rms_eps"], cfg["rope_theta"]
        c.attn_softcap, c.query_scale, c.device = cfg["softcap"], cfg["query_scale"], device
        self.cfg = dict(cfg)
        h = _vp()
        check(lib().sana_gemma_create(ctypes.byref(c), ctypes.byref(h)))
        self.h = h
        self._destroy = lib().sana_gemma_destroy

    def close(self):
        if getattr(self, "h", None):
            self._destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def set_weight(self, name, arr):
        arr = _f32(arr)
        shape = (_i64 * arr.ndim)(*arr.shape)
        check(lib().sana_gemma_set_weight(self.h, name.encode(), ptr(arr), shape, arr.ndim))

    def check_weights(self):
        check(lib().sana_gemma_check_weights(self.h))

    def load_gguf(self, path):
        check(lib().sana_gemma_load_gguf(self.h, str(path).encode()))

    def encode(self, tokens):
        tokens = np.ascontiguousarray(tokens, np.int32)
        out = np.empty((tokens.size, self.cfg["hidden"]), np.float32)
        check(lib().sana_gemma_encode(self.h, ptr(tokens), tokens.size, ptr(out)))
        return out

    def encode_pair(self, tokens_a, tokens_b):
        """Both sequences in one pass; equals (encode(a), encode(b))."""
        a = np.ascontiguousarray(tokens_a, np.int32)
        b = np.ascontiguousarray(tokens_b, np.int32)
        oa = np.empty((a.size, self.cfg["hidden"]), np.float32)
        ob = np.empty((b.size, self.cfg["hidden"]), np.float32)
        check(lib().sana_gemma_encode_pair(self.h, ptr(a), a.size, ptr(b), b.size, ptr(oa), ptr(ob)))
        return oa, ob
