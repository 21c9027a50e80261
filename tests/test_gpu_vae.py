"""DC-AE VAE decoder on the GPU (sana_vae_* C ABI) against the oracle and the
reference's own output.

The oracle's decode is bit-exact with the reference's run_vae_decode
(tests/test_oracle_vae.py); here the HIP path (fp16 operands, fp32
accumulation and residuals) is held to a relative L2 of 2e-3 on the decoded
image, the per-forward bar of the DiT.  Decoder shapes go from one level of
each layer type up to the small 4-level decoder and the full Sana 1.0 decoder
(latent 32x32 -> 1024x1024, against the reference's fixture).
"""
import os

import numpy as np
import pytest

import oracle_lib as O
from conftest import rel_l2, spread_subsample

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 2e-3

CONFIGS = {
    "evit1": dict(channels=(128,), attn=(True,)),
    "res1": dict(channels=(64,), attn=(False,)),
    "up2": dict(channels=(64, 128), attn=(False, True)),
    "small": dict(channels=(64, 64, 128, 128), attn=(False, False, True, True)),
}


def build(cfg, full=False):
    import sana_dit
    ora = O.Vae(full=True) if full else O.Vae(cfg=cfg)
    dev = sana_dit.Vae(ora.cfg["channels"], ora.cfg["attn"])
    for name, shape in O.vae_manifest(ora.cfg).items():
        dev.set_weight(name, ora.get(name, shape))
    dev.check_weights()
    return ora, dev


@pytest.mark.parametrize("name,shape", [("evit1", (1, 32, 8, 8)), ("res1", (1, 32, 8, 8)), ("up2", (1, 32, 6, 10)),
                                        ("up2", (2, 32, 4, 4)), ("small", (1, 32, 8, 8))])
def test_decode_vs_oracle(name, shape):
    ora, dev = build(CONFIGS[name])
    try:
        lat = O.randn(shape, 42)
        print(f"{name} {shape}: oracle decode on the host ...", flush=True)
        ref = ora.decode(lat)
        got = dev.decode(lat)
        err = rel_l2(got, ref)
        print(f"{name} {shape}: image rel_l2 {err:.3e}")
        assert got.shape == ref.shape
        assert np.isfinite(got).all()
        assert err < TOL
        again = dev.decode(lat)
        assert np.array_equal(got, again)
    finally:
        dev.close()


def test_small_decode_vs_reference_fixture():
    fx = np.load(os.path.join(GOLDEN, "vae_small.npz"), allow_pickle=False)
    ora, dev = build(CONFIGS["small"])
    try:
        got = dev.decode(fx["latent"])
        err = rel_l2(got, fx["image"])
        print(f"small vs reference image: rel_l2 {err:.3e}")
        assert err < TOL
    finally:
        dev.close()


def test_batch_matches_single():
    ora, dev = build(CONFIGS["up2"])
    try:
        lat = O.randn((2, 32, 4, 6), 7)
        both = dev.decode(lat)
        one = np.concatenate([dev.decode(lat[i:i + 1]) for i in range(2)])
        assert rel_l2(both, one) < 1e-6
    finally:
        dev.close()


def test_rejects_bad_input():
    import sana_dit
    with pytest.raises(sana_dit.SanaError):
        sana_dit.Vae((96,), (False,))            # channels not a multiple of 64
    with pytest.raises(sana_dit.SanaError):
        sana_dit.Vae((64, 192), (False, False))  # upsample shortcut ratio 4*64 % 192 != 0
    dev = sana_dit.Vae((64,), (False,))
    try:
        with pytest.raises(sana_dit.SanaError) as e:
            dev.decode(O.randn((1, 32, 4, 4), 1))  # no weights
        assert e.value.code == sana_dit.SANA_ERR_STATE
        with pytest.raises(sana_dit.SanaError) as e:
            dev.set_weight("decoder.conv_in.weight", np.zeros((64, 32, 1, 1), np.float32))
        assert e.value.code == sana_dit.SANA_ERR_SHAPE
    finally:
        dev.close()


def test_full_decoder_vs_reference():
    """Sana 1.0 DC-AE f32c32 decoder, latent 32x32 -> 1024x1024 RGB: the
    fixture keeps a strided subsample of the reference's image, 65536 values
    spread over every row and column, and its L2 norm."""
    path = os.path.join(GOLDEN, "vae_full.npz")
    if not os.path.exists(path):
        pytest.skip("vae_full golden not generated")
    fx = np.load(path, allow_pickle=False)
    import sana_dit
    print("generating the full synthetic decoder on the host ...", flush=True)
    ora = O.Vae(full=True)
    dev = sana_dit.Vae(ora.cfg["channels"], ora.cfg["attn"])
    try:
        for name, shape in O.vae_manifest(ora.cfg).items():
            dev.set_weight(name, ora.get(name, shape))
        lat = O.randn((1, 32, 32, 32), 42)
        got = dev.decode(lat)
        assert got.shape == (1, 3, 1024, 1024)
        stride = int(fx["image__stride"])
        err = rel_l2(got.reshape(-1)[::stride], fx["image__sub"])
        norm_err = abs(np.linalg.norm(got.astype(np.float64)) / float(fx["image__l2"]) - 1.0)
        print(f"full decoder: image subsample rel_l2 {err:.3e}, L2 norm rel diff {norm_err:.3e}")
        assert np.isfinite(got).all()
        assert err < TOL
        assert norm_err < TOL
        sp = spread_subsample(got, fx, "image")
        if sp is not None:
            serr = rel_l2(*sp)
            print(f"full decoder: spread subsample ({sp[1].size} values) rel_l2 {serr:.3e}")
            assert serr < TOL
    finally:
        dev.close()


def test_decoder_input_stage():
    """run_vae_decoder_input: conv_in of the (already scaled) latent, with and
    without the channel-repeat shortcut; needs only the conv_in tensors."""
    import sana_dit
    ora = O.Vae(cfg=CONFIGS["up2"])
    dev = sana_dit.Vae(ora.cfg["channels"], ora.cfg["attn"])
    try:
        for name in ("decoder.conv_in.weight", "decoder.conv_in.bias"):
            dev.set_weight(name, ora.get(name))
        lat = O.randn((2, 32, 5, 7), 3)
        scaled = lat * (np.float32(1.0) / np.float32(0.41407))
        ref = ora.decoder_input(lat)                     # scales, conv_in, + shortcut
        got = dev.decoder_input(scaled)
        assert got.shape == (2, 128, 5, 7)
        assert rel_l2(got, ref) < TOL
        rep = 128 // 32
        short = np.repeat(scaled, rep, axis=1)           # channel oc reads latent channel oc // rep
        assert rel_l2(dev.decoder_input(scaled, in_shortcut=False), ref - short) < TOL
    finally:
        dev.close()
