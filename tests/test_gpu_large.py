"""Parity at the long-sequence shapes: one DiT block at 64x64 = 4096 image
tokens (the linear-attention + Mix-FFN microbenchmark shape, batch 2, both
self-attention head layouts) and at 128x128 = 16384 tokens (one block of the
4096 px forward), against the oracle; and the whole 28-block forward at
4096 px on the device (finite, deterministic).  Tolerance: relative L2 <= 2e-3
per stage output."""
import numpy as np
import pytest

import oracle_lib as O
from conftest import rel_l2
from test_gpu_block import upload_all

pytestmark = pytest.mark.gpu

TOL = 2e-3


@pytest.fixture(scope="module", params=[16, 36], ids=["self16x72", "self36x32"])
def one_block(request):
    import sana_dit
    heads = request.param
    m = O.Model(layers=1, self_heads=heads, cross_heads=16)
    d = sana_dit.Dit(layers=1, self_heads=heads, cross_heads=16)
    upload_all(d, m, 1)
    emb, tmod = m.time(np.array([500.0, 500.0], np.float32))
    ctx = O.randn((2, 300, 1152), 43)
    yield heads, m, d, tmod, ctx
    d.close()


def _check_block(m, d, x, tmod, ctx, label):
    print(f"{label}: oracle block on the host ...", flush=True)
    ref = m.block(0, x, ctx, tmod)
    d.set_context(ctx, projected=True)
    got = d.block_forward(0, x, tmod)
    for name, g, r in zip(("after_self", "after_cross", "after_ff"), got, ref):
        err = rel_l2(g, r)
        print(f"{label} {name}: rel_l2 {err:.3e}")
        assert err < TOL, (name, err)
    branch = rel_l2(got[2] - got[1], ref[2] - ref[1])
    print(f"{label} ffn branch: rel_l2 {branch:.3e}")
    assert branch < 1e-2


def test_block_4096_tokens(one_block):
    heads, m, d, tmod, ctx = one_block
    x = O.randn((2, 4096, 1152), 7) * np.float32(0.5)
    _check_block(m, d, x, tmod, ctx, f"N=4096 heads={heads}")


def test_block_16384_tokens(one_block):
    heads, m, d, tmod, ctx = one_block
    if heads != 36:
        pytest.skip("production head layout only at 16384 tokens")
    x = O.randn((2, 16384, 1152), 8) * np.float32(0.5)
    _check_block(m, d, x, tmod, ctx, "N=16384 heads=36")


def test_block_10000_tokens_short_last_chunk(one_block):
    # 100 x 100 tokens: the chunked linear attention (above 8192 tokens per
    # image) splits 10000 tokens into 15 chunks of 640 and a short last chunk
    # of 400, which the 16384-token case (16 full chunks) never exercises
    heads, m, d, tmod, ctx = one_block
    if heads != 36:
        pytest.skip("production head layout only on the chunked path")
    x = O.randn((2, 10000, 1152), 10) * np.float32(0.5)
    _check_block(m, d, x, tmod, ctx, "N=10000 heads=36")


def test_block_4096_tokens_large_state(one_block):
    # scale_msa + 31 multiplies the self-attention q, k and v by 32, so the
    # linear-attention state reaches ~1.5e5 at 4096 tokens, past fp16's range
    # (65504): the state's power-of-two scaling must keep the block exact
    heads, m, d, tmod, ctx = one_block
    C = 1152
    tm = tmod.copy()
    tm[:, C:2 * C] += 31.0
    x = O.randn((2, 4096, C), 8) * np.float32(0.5)
    _check_block(m, d, x, tm, ctx, f"N=4096 heads={heads} amplified")


def test_block_16384_tokens_large_state(one_block):
    # the same amplification through the chunked linear attention (chunk
    # partial states, fixed-order reduction, scaled fp16 hi/lo apply)
    heads, m, d, tmod, ctx = one_block
    if heads != 36:
        pytest.skip("production head layout only at 16384 tokens")
    C = 1152
    tm = tmod.copy()
    tm[:, C:2 * C] += 31.0
    x = O.randn((2, 16384, C), 9) * np.float32(0.5)
    _check_block(m, d, x, tm, ctx, "N=16384 heads=36 amplified")


def test_forward_4096px_finite_and_deterministic():
    import sana_dit
    print("generating the seeded 28-block weights on the host ...", flush=True)
    m = O.Model(layers=28, self_heads=36, cross_heads=16)
    d = sana_dit.Dit(layers=28, self_heads=36, cross_heads=16)
    try:
        for name, shape in sana_dit.manifest(28).items():
            d.set_weight(name, m.get(name, shape))
        d.check_weights()
        latent = O.randn((1, 32, 128, 128), 42)
        d.set_context(O.randn((2, 300, 2304), 43), projected=False)
        a = d.forward(latent, 999.0)
        b = d.forward(latent, 999.0)
        assert a.shape == (2, 32, 128, 128)
        assert np.isfinite(a).all()
        assert np.array_equal(a, b)
        print(f"4096 px noise_pred: mean {a.mean():.4f} std {a.std():.4f}")
    finally:
        d.close()
