"""Weight uploads into the fp16 GEMM operands (C ABI, GPU context).

The reference keeps every weight in fp32 (src/weights_io.cpp:340-355); here
the linear weights run as fp16 operands, so an upload must refuse what fp16
cannot hold rather than store inf or NaN: |w| > 65504, inf and NaN fail with
SANA_ERR_FORMAT naming the tensor, in the DiT, the VAE and the Gemma encoder,
through the fp32 entry points and through sana_dit_load_gguf.

The raw-fp16 entry points (sana_dit_set_weight_f16 /
sana_dit_set_block_weight_f16, which sana_dit_load_gguf uses for F16
payloads) must leave the device in exactly the state the fp32 path leaves it
in for the same fp16-representable values: the forwards are compared bit for
bit.
"""
import os
import sys

import numpy as np
import pytest

import oracle_lib as O
import sana_dit
from gguf_writer import GGML_BF16, GGML_F16, GGML_F32, write_gguf

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle"))
import gemma_oracle as G  # noqa: E402

pytestmark = pytest.mark.gpu

SMALL = dict(layers=2, hidden=128, ffn=256, caption_dim=96, latent_channels=8, self_heads=4, cross_heads=2)
OPERANDS = ("attn1.to_q.weight", "attn1.to_k.weight", "attn1.to_v.weight", "attn1.to_out.0.weight",
            "attn2.to_q.weight", "attn2.to_k.weight", "attn2.to_v.weight", "attn2.to_out.0.weight",
            "ff.conv_inverted.weight", "ff.conv_point.weight")
TOP_OPERANDS = ("caption_projection.linear_1.weight", "caption_projection.linear_2.weight")


def small_weights(seed=3):
    rng = np.random.default_rng(seed)
    out = {}
    for n, shape in sana_dit.manifest(2, 128, 256, 96, 8).items():
        out[n] = (np.ones(shape, np.float32) if n == "caption_norm.weight"
                  else rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02))
    return out


def is_operand(name):
    return name in TOP_OPERANDS or any(name.endswith("." + s) for s in OPERANDS)


def expect_format_error(fn, tensor):
    with pytest.raises(sana_dit.SanaError) as e:
        fn()
    print("refused:", e.value)
    assert e.value.code == sana_dit.SANA_ERR_FORMAT
    assert tensor in str(e.value)


@pytest.mark.parametrize("bad", [1e5, -7e4, np.inf, np.nan])
def test_dit_upload_refuses_values_outside_fp16(bad):
    d = sana_dit.Dit(**SMALL)
    try:
        w = small_weights()
        for name in ("transformer_blocks.1.attn1.to_out.0.weight", "transformer_blocks.0.ff.conv_point.weight",
                     "caption_projection.linear_1.weight"):
            a = w[name].copy()
            a.reshape(-1)[a.size // 3] = bad
            expect_format_error(lambda: d.set_weight(name, a), name)
        # the largest finite fp16 magnitude is accepted
        a = w["transformer_blocks.0.attn2.to_q.weight"].copy()
        a[0, 0], a[1, 1] = 65504.0, -65504.0
        d.set_weight("transformer_blocks.0.attn2.to_q.weight", a)
    finally:
        d.close()


def test_f16_entry_points_match_fp32_path_bit_for_bit():
    """Operand weights given as fp16 bits vs the same values as fp32: identical forwards."""
    w = small_weights()
    latent = O.randn((1, 8, 8, 8), 42)
    caption = O.randn((2, 16, 96), 43)
    outs = []
    for use_f16 in (False, True):
        d = sana_dit.Dit(**SMALL)
        try:
            for n, a in w.items():
                if is_operand(n):
                    h = a.astype(np.float16)
                    if use_f16:
                        d.set_weight_f16(n, h)
                    else:
                        d.set_weight(n, h.astype(np.float32))
                else:
                    d.set_weight(n, a)
            d.check_weights()
            d.set_context(caption, projected=False)
            outs.append(d.forward(latent, 999.0))
        finally:
            d.close()
    assert np.isfinite(outs[0]).all()
    assert np.array_equal(outs[0], outs[1])


def test_f16_entry_points_refuse_bad_input():
    d = sana_dit.Dit(**SMALL)
    try:
        h = np.zeros((128, 128), np.float16)
        h[3, 4] = np.inf
        expect_format_error(lambda: d.set_weight_f16("transformer_blocks.0.attn1.to_q.weight", h),
                            "transformer_blocks.0.attn1.to_q.weight")
        h[3, 4] = np.nan
        expect_format_error(lambda: d.set_weight_f16("caption_projection.linear_2.weight", h),
                            "caption_projection.linear_2.weight")
        # tensors that stay fp32 on the device have no fp16 entry
        for name, shape in (("transformer_blocks.0.ff.conv_depth.weight", (256, 1, 3, 3)),
                            ("time_embed.linear.weight", (768, 128))):
            with pytest.raises(sana_dit.SanaError) as e:
                d.set_weight_f16(name, np.zeros(shape, np.float16))
            assert e.value.code == sana_dit.SANA_ERR_INVALID_ARGUMENT
        with pytest.raises(sana_dit.SanaError) as e:
            d.set_weight_f16("transformer_blocks.0.attn1.to_q.weight", np.zeros((128, 64), np.float16))
        assert e.value.code == sana_dit.SANA_ERR_SHAPE
    finally:
        d.close()


@pytest.mark.parametrize("ggml_type", [GGML_F32, GGML_BF16])
def test_load_gguf_refuses_out_of_range_weight(tmp_path, ggml_type):
    """A GGUF whose linear weight holds 1e5 (F32, or BF16, whose exponent range holds it)."""
    w = small_weights()
    bad = "transformer_blocks.1.ff.conv_inverted.weight"
    w[bad].reshape(-1)[17] = 1.0e5
    path = str(tmp_path / "bad.gguf")
    write_gguf(path, w, ggml_type=ggml_type)
    d = sana_dit.Dit(**SMALL)
    try:
        expect_format_error(lambda: d.load_gguf(path, path, path), bad)
    finally:
        d.close()


def test_load_gguf_f16_is_the_fp16_bits(tmp_path):
    """sana_dit_load_gguf on an F16 file and the fp32 path on the widened values: identical forwards."""
    w = small_weights()
    path = str(tmp_path / "w16.gguf")
    write_gguf(path, w, ggml_type=GGML_F16)
    latent = O.randn((1, 8, 8, 8), 42)
    caption = O.randn((2, 16, 96), 43)
    outs = []
    for from_file in (True, False):
        d = sana_dit.Dit(**SMALL)
        try:
            if from_file:
                d.load_gguf(path, path, path)
            else:
                for n, a in w.items():
                    d.set_weight(n, a.astype(np.float16).astype(np.float32))
            d.check_weights()
            d.set_context(caption, projected=False)
            outs.append(d.forward(latent, 999.0))
        finally:
            d.close()
    assert np.array_equal(outs[0], outs[1])


def test_vae_upload_refuses_values_outside_fp16():
    cfg = O.SMALL_VAE
    v = sana_dit.Vae(cfg["channels"], cfg["attn"])
    try:
        man = O.vae_manifest(cfg)
        for name in ("decoder.conv_in.weight", "decoder.up_blocks.3.1.attn.to_k.weight",
                     "decoder.up_blocks.3.1.conv_out.conv_point.weight"):
            a = np.zeros(man[name], np.float32)
            a.reshape(-1)[5] = 2e5
            expect_format_error(lambda: v.set_weight(name, a), name)
    finally:
        v.close()


def test_gemma_upload_refuses_values_outside_fp16():
    cfg = dict(vocab=300, hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, ffn=512, sliding_window=8,
               rms_eps=1e-6, rope_theta=10000.0, softcap=50.0, query_scale=1 / 8)
    g = sana_dit.Gemma(cfg)
    try:
        w = G.random_weights(cfg, seed=5, scale=0.05)
        for name in ("token_embd.weight", "blk.1.attn_k.weight", "blk.0.ffn_up.weight"):
            a = w[name].copy()
            a.reshape(-1)[9] = -np.inf if name.endswith("up.weight") else 3e5
            expect_format_error(lambda: g.set_weight(name, a), name)
    finally:
        g.close()
