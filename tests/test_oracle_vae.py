"""Pins the VAE-decoder part of the oracle (oracle/oracle.cpp, the DC-AE ops of
src/vae.cpp and src/vae_ops.cpp).

* Bit-exact against the reference's own CPU code (tests/golden/vae_*.npz,
  written by tests/golden/make_golden.py from oracle/_ref/ref_harness): the
  whole run_vae_decode of the small synthetic decoder, its conv_in stage, both
  summation orders of the 3x3 conv, and the digests of every synthetic weight.
* Independently of the reference, each op against its closed form in fp64
  numpy (3x3 conv, 1x1 and grouped 1x1 conv, depthwise 5x5, channel RMSNorm,
  nearest-2x upsample with the pixel-shuffled shortcut, and the padded-V
  linear attention of the multiscale block), so a transposed index, a dropped
  term or a wrong head grouping fails here.
"""
import hashlib
import os

import numpy as np
import pytest

import oracle_lib as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


@pytest.fixture(scope="module")
def small():
    return O.Vae(full=False)


def test_small_decode_bit_exact(small):
    fx = golden("vae_small")
    lat = O.randn((1, 32, 8, 8), 42)
    assert sha(lat) == str(fx["latent__sha256"])
    assert sha(small.decoder_input(lat)) == str(fx["decoder_input__sha256"])
    img = small.decode(lat)
    assert img.shape == (1, 3, 64, 64)
    assert sha(img) == str(fx["image__sha256"]), np.abs(img - fx["image"]).max()


def test_conv3x3_both_orders_bit_exact():
    fx = golden("vae_conv")
    for order, name in ((0, "im2col"), (1, "tap")):
        got = O.vae_conv3x3(fx["x"], fx["w"], fx["bias"], order)
        assert sha(got) == str(fx[name + "__sha256"]), name
    # the orders differ in the last bits, so the check above tells them apart
    assert str(fx["im2col__sha256"]) != str(fx["tap__sha256"])


@pytest.mark.parametrize("which", ["small", "full"])
def test_weight_digests(which):
    fx = golden("vae_weights")
    vae = O.Vae(full=(which == "full"))
    names = [str(n) for n in fx[which + "_names"]]
    shapes = O.vae_manifest(vae.cfg)
    assert sorted(shapes) == names
    for n, h in zip(names, fx[which + "_fnv1a"]):
        assert O.digest(vae.get(n, shapes[n])) == int(h), n


# ---------------------------------------------------------------- closed forms
def conv3x3_np(x, w, b):
    B, C, H, W = x.shape
    xp = np.zeros((B, C, H + 2, W + 2))
    xp[:, :, 1:-1, 1:-1] = x
    out = np.zeros((B, w.shape[0], H, W))
    for ky in range(3):
        for kx in range(3):
            out += np.einsum("oc,bchw->bohw", w[:, :, ky, kx].astype(np.float64), xp[:, :, ky:ky + H, kx:kx + W])
    return out + (0 if b is None else b[None, :, None, None])


def test_conv3x3_closed_form():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2, 5, 7, 6)).astype(np.float32)
    w = rng.standard_normal((4, 5, 3, 3)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    ref = conv3x3_np(x, w, b)
    for order in (0, 1):
        assert rel(O.vae_conv3x3(x, w, b, order), ref) < 1e-6
    assert rel(O.vae_conv3x3(x, w, None, 0), conv3x3_np(x, w, None)) < 1e-6


def test_dw5x5_and_grouped_closed_form():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((1, 6, 9, 8)).astype(np.float32)
    w = rng.standard_normal((6, 1, 5, 5)).astype(np.float32)
    xp = np.zeros((1, 6, 13, 12))
    xp[:, :, 2:-2, 2:-2] = x
    ref = np.zeros((1, 6, 9, 8))
    for ky in range(5):
        for kx in range(5):
            ref += w[None, :, 0, ky, kx, None, None] * xp[:, :, ky:ky + 9, kx:kx + 8]
    assert rel(O.vae_dw5x5(x, w), ref) < 1e-6
    g = rng.standard_normal((6, 2, 1, 1)).astype(np.float32)   # 3 groups of 2 -> 2
    got = O.vae_grouped_conv1x1(x, g, 3)
    ref = np.concatenate([np.einsum("oi,bihw->bohw", g[2 * k:2 * k + 2, :, 0, 0].astype(np.float64),
                                    x[:, 2 * k:2 * k + 2]) for k in range(3)], axis=1)
    assert rel(got, ref) < 1e-6


def test_rms_norm_closed_form():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((2, 7, 3, 5)).astype(np.float32)
    w = rng.standard_normal(7).astype(np.float32)
    b = rng.standard_normal(7).astype(np.float32)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(axis=1, keepdims=True) + 1e-5) * w[None, :, None, None] + b[None, :, None, None]
    assert rel(O.vae_rms_norm(x, w, b), ref) < 1e-6


def test_upsample_shortcut_closed_form():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((1, 8, 3, 4)).astype(np.float32)
    w = rng.standard_normal((4, 8, 3, 3)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    up = np.repeat(np.repeat(x, 2, axis=2), 2, axis=3)
    ref = conv3x3_np(up, w, b)
    rep = 4 * 4 // 8
    for oc in range(4):
        for q in range(4):
            ref[0, oc, q // 2::2, q % 2::2] += x[0, (oc * 4 + q) // rep]
    assert rel(O.vae_upsample(x, w, b, True), ref) < 1e-6
    assert rel(O.vae_upsample(x, w, b, False), conv3x3_np(up, w, b)) < 1e-6


def test_multiscale_attention_closed_form(small):
    """One EfficientViT attention of the small decoder (level 2, C = 128, 4
    heads of 32 + 4 multiscale heads) in fp64 numpy: q|k|v 1x1 convs, the
    depthwise 5x5 + grouped 1x1 branch, heads = groups of 96 consecutive
    channels, padded-V ReLU linear attention, to_out, RMSNorm, + input."""
    rng = np.random.default_rng(4)
    C, H, W, D = 128, 6, 5, 32
    x = rng.standard_normal((1, C, H, W)).astype(np.float32)
    q = "decoder.up_blocks.2.1."
    gw = lambda n: small.get(q + n).astype(np.float64)
    xd = x.astype(np.float64)[0].reshape(C, -1)
    qkv = np.concatenate([gw(f"attn.to_{t}.weight") @ xd for t in "qkv"], axis=0)        # [3C, S]
    pin = gw("attn.to_qkv_multiscale.0.proj_in.weight")[:, 0]                            # [3C, 5, 5]
    qp = np.zeros((3 * C, H + 4, W + 4))
    qp[:, 2:-2, 2:-2] = qkv.reshape(3 * C, H, W)
    dw = np.zeros((3 * C, H, W))
    for ky in range(5):
        for kx in range(5):
            dw += pin[:, ky, kx, None, None] * qp[:, ky:ky + H, kx:kx + W]
    pout = gw("attn.to_qkv_multiscale.0.proj_out.weight")[:, :, 0, 0]                   # [3C, 32]
    dw = dw.reshape(3 * C, -1)
    ms = np.concatenate([pout[g * D:(g + 1) * D] @ dw[g * D:(g + 1) * D] for g in range(3 * C // D)], axis=0)
    heads = []
    for src in (qkv, ms):
        for h in range(C // D):
            blk = src[h * 3 * D:(h + 1) * 3 * D]
            qq, kk, vv = np.maximum(blk[:D], 0), np.maximum(blk[D:2 * D], 0), blk[2 * D:]
            vp = np.concatenate([vv, np.ones((1, vv.shape[1]))], axis=0)
            hid = (vp @ kk.T) @ qq
            heads.append(hid[:D] / (hid[D] + 1e-15))
    merged = np.concatenate(heads, axis=0)
    o = gw("attn.to_out.weight") @ merged
    nrm = o / np.sqrt((o ** 2).mean(axis=0, keepdims=True) + 1e-5)
    ref = nrm * gw("attn.norm_out.weight")[:, None] + gw("attn.norm_out.bias")[:, None] + xd
    got = small.layer("attn", 2, 1, x)
    assert rel(got[0].reshape(C, -1), ref) < 1e-5
