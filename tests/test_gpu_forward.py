"""Full-model parity of the HIP path against the reference's own CPU outputs.

The golden fixtures (tests/golden/*.npz) hold the outputs of the reference's
src/*.cpp compiled from source (tests/golden/make_golden.py) on the seeded
synthetic Sana-0.6B model of oracle/model_spec.h; the oracle regenerates the
identical weights bit for bit (tests/test_oracle_golden.py pins that), and
they are uploaded here through the C ABI.

Tolerances (relative L2): 2e-3 per forward, 1e-2 on the final latent of the
20-step DPM-Solver++ loop.
"""
import os

import numpy as np
import pytest

import oracle_lib as O
from conftest import rel_l2, spread_subsample

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL_FORWARD = 2e-3
TOL_LOOP = 1e-2


def golden(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


@pytest.fixture(scope="module")
def full_model():
    import sana_dit
    print("generating the seeded 28-block weights on the host ...", flush=True)
    m = O.Model(layers=28, self_heads=36, cross_heads=16)
    d = sana_dit.Dit(layers=28, self_heads=36, cross_heads=16)
    for name, shape in sana_dit.manifest(28).items():
        d.set_weight(name, m.get(name, shape))
    d.check_weights()
    yield m, d
    d.close()


@pytest.mark.parametrize("case,masked", [("cfg2", False), ("cfg2_mask", True)])
def test_forward_1024px_vs_reference(full_model, case, masked):
    m, d = full_model
    fx = golden(case)
    latent = O.randn((1, 32, 32, 32), 42)
    caption = O.randn((2, 300, 2304), 43)
    bias = O.mask_bias(300, 1, 40) if masked else None
    d.set_context(caption, projected=False, bias=bias)
    ctx = d.get_context((2, 300, 1152))
    stride = int(fx["context__stride"])
    ctx_err = rel_l2(ctx.reshape(-1)[::stride], fx["context__sub"])
    got = d.forward(latent, 999.0)
    err = rel_l2(got, fx["noise_pred"])
    guided = got[:1] + np.float32(4.5) * (got[1:] - got[:1])
    gerr = rel_l2(guided, fx["guided"])
    print(f"{case}: context rel_l2 {ctx_err:.2e}, noise_pred rel_l2 {err:.2e}, guided rel_l2 {gerr:.2e}")
    assert ctx_err < 1e-3
    assert err < TOL_FORWARD
    assert gerr < TOL_FORWARD


def test_forward_nonsquare_vs_reference(full_model):
    """A 4x16 latent (64 tokens) against the reference's own forward of it:
    the reference runs each block's depthwise conv on the 8x8 token grid
    (src/transformer.cpp:765-767), and so does the device path."""
    m, d = full_model
    fx = golden("nonsquare")
    latent = O.randn((1, 32, 4, 16), 42)
    d.set_context(O.randn((2, 300, 2304), 43), projected=False)
    got = d.forward(latent, 999.0)
    err = rel_l2(got, fx["noise_pred"])
    print(f"nonsquare 4x16: noise_pred rel_l2 {err:.2e}")
    assert err < TOL_FORWARD


def test_forward_4096px_vs_reference(full_model):
    """4096 px (latent 128x128, 16384 image tokens): the reference's CPU forward
    is too large to store whole, so the fixture keeps, of noise_pred and
    guided, a strided subsample, 65536 values spread over every row and column
    of the grid, and their L2 norms."""
    path = os.path.join(GOLDEN, "cfg5.npz")
    if not os.path.exists(path):
        pytest.skip("cfg5 golden not generated")
    m, d = full_model
    fx = golden("cfg5")
    latent = O.randn((1, 32, 128, 128), 42)
    caption = O.randn((2, 300, 2304), 43)
    d.set_context(caption, projected=False)
    got = d.forward(latent, 999.0)
    guided = got[:1] + np.float32(4.5) * (got[1:] - got[:1])
    res = {}
    for name, arr in (("noise_pred", got), ("guided", guided)):
        stride = int(fx[name + "__stride"])
        res[name] = rel_l2(arr.reshape(-1)[::stride], fx[name + "__sub"])
        norm_err = abs(np.linalg.norm(arr.astype(np.float64)) / float(fx[name + "__l2"]) - 1.0)
        print(f"cfg5 {name}: subsample rel_l2 {res[name]:.2e}, L2 norm rel diff {norm_err:.2e}")
        assert res[name] < TOL_FORWARD
        assert norm_err < TOL_FORWARD
        sp = spread_subsample(arr, fx, name)
        if sp is not None:
            serr = rel_l2(*sp)
            print(f"cfg5 {name}: spread subsample ({sp[1].size} values) rel_l2 {serr:.2e}")
            assert serr < TOL_FORWARD


@pytest.mark.parametrize("masked", [False, True], ids=["nomask", "mask"])
def test_step_device_matches_context_then_forward(full_model, masked):
    """sana_dit_step_device (caption projection, cross K/V and forward in one
    graph, the forward's head beside the context GEMMs) gives the noise
    prediction of sana_dit_set_context + sana_dit_forward bit for bit."""
    import torch
    m, d = full_model
    latent = O.randn((1, 32, 32, 32), 42)
    caption = O.randn((2, 300, 2304), 43)
    bias = O.mask_bias(300, 1, 40) if masked else None
    d.set_context(caption, projected=False, bias=bias)
    ref = d.forward(latent, 999.0)
    dev = torch.device("cuda:0")
    d_cap = torch.from_numpy(caption).to(dev)
    d_lat = torch.from_numpy(latent).to(dev)
    d_bias = torch.from_numpy(np.ascontiguousarray(bias, np.float32)).to(dev) if masked else None
    out = torch.empty((2, 32, 32, 32), device=dev)
    for _ in range(2):  # the second call replays the captured graph
        out.fill_(float("nan"))
        d.step_device(d_cap, 300, d_bias, d_lat, (1, 32, 32, 32), 999.0, out)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert np.array_equal(got, ref)


def test_forward_deterministic(full_model):
    m, d = full_model
    latent = O.randn((1, 32, 32, 32), 42)
    caption = O.randn((2, 300, 2304), 43)
    d.set_context(caption, projected=False)
    a = d.forward(latent, 999.0)
    b = d.forward(latent, 999.0)
    assert np.array_equal(a, b)


def test_denoise_loop_1024px_vs_reference(full_model):
    path = os.path.join(GOLDEN, "cfg3.npz")
    if not os.path.exists(path):
        pytest.skip("cfg3 golden not generated")
    m, d = full_model
    fx = golden("cfg3")
    latent = O.randn((1, 32, 32, 32), 42)
    caption = O.randn((2, 300, 2304), 43)
    d.set_context(caption, projected=False)
    ts, sg = O.scheduler_timesteps(20)
    fin = d.denoise_loop(latent, ts, sg, 4.5)
    err = rel_l2(fin, fx["final_latent"])
    print(f"cfg3: final latent rel_l2 {err:.2e}")
    assert err < TOL_LOOP


SMALL = dict(layers=2, hidden=128, ffn=256, caption=96, latent=8, self_heads=4, cross_heads=2)


@pytest.fixture(scope="module")
def small_model():
    import sana_dit
    m = O.Model(**SMALL)
    d = sana_dit.Dit(layers=2, hidden=128, ffn=256, caption_dim=96, latent_channels=8, self_heads=4, cross_heads=2)
    for name, shape in sana_dit.manifest(2, 128, 256, 96, 8).items():
        d.set_weight(name, m.get(name, shape))
    d.check_weights()
    yield m, d
    d.close()


def test_small_loop_vs_oracle(small_model):
    m, d = small_model
    latent = O.randn((1, 8, 8, 8), 42)
    caption = O.randn((2, 16, 96), 43)
    ref = m.loop(latent, caption, 6, 4.5)
    d.set_context(caption, projected=False)
    ts, sg = O.scheduler_timesteps(6)
    got = d.denoise_loop(latent, ts, sg, 4.5)
    assert np.isfinite(ref).all(), "oracle loop not finite"
    assert np.isfinite(got).all(), "device loop not finite"
    err = rel_l2(got, ref)
    print(f"small loop rel_l2 {err:.2e}")
    assert err < TOL_LOOP


def test_small_run_blocks_vs_oracle(small_model):
    m, d = small_model
    rng = np.random.default_rng(7)
    x = rng.standard_normal((2, 64, 128)).astype(np.float32)
    ctx = rng.standard_normal((2, 16, 128)).astype(np.float32)
    emb, tmod = m.time(np.array([500.0, 500.0], np.float32))
    ref = x
    for i in range(2):
        ref = m.block(i, ref, ctx, tmod)[2]
    d.set_context(ctx, projected=True)
    got = d.run_blocks(0, 2, x, tmod)
    assert rel_l2(got, ref) < TOL_FORWARD


def test_small_forward_masked_vs_oracle(small_model):
    m, d = small_model
    latent = O.randn((1, 8, 8, 8), 5)
    caption = O.randn((2, 16, 96), 6)
    bias = np.full((2, 16), -10000.0, np.float32)
    bias[0, :3] = 0.0
    bias[1, :11] = 0.0
    ctx = m.project_caption(caption)
    ref = m.forward(latent, ctx, 733.0, bias)
    d.set_context(caption, projected=False, bias=bias)
    got = d.forward(latent, 733.0)
    assert rel_l2(got, ref) < TOL_FORWARD


def test_small_forward_batch2_vs_oracle(small_model):
    """A latent batch of 2 (context batch 4): the single-chain forward, patch
    embed reading latent row b % 2, uncond rows first."""
    m, d = small_model
    latent = O.randn((2, 8, 8, 8), 11)
    caption = O.randn((4, 16, 96), 12)
    ctx = m.project_caption(caption)
    ref = m.forward(latent, ctx, 610.0)
    d.set_context(caption, projected=False)
    got = d.forward(latent, 610.0)
    err = rel_l2(got, ref)
    print(f"small forward, latent batch 2: rel_l2 {err:.2e}")
    assert err < TOL_FORWARD


def test_small_forward_nonsquare_latent(small_model):
    """A 4x16 latent (64 tokens): the reference accepts any H x W whose token
    count is a perfect square and runs each block's depthwise conv on the
    side x side token grid (src/transformer.cpp:18-24, 765-767).  The device
    forward matches the oracle there, equals the 8x8 view of the same data bit
    for bit (patch embedding and final layer see only the flattened index), and
    a 4x8 latent (32 tokens) is refused with the reference's message."""
    import sana_dit
    m, d = small_model
    latent = O.randn((1, 8, 4, 16), 21)
    caption = O.randn((2, 16, 96), 22)
    ref = m.forward(latent, m.project_caption(caption), 420.0)
    d.set_context(caption, projected=False)
    got = d.forward(latent, 420.0)
    assert got.shape == (2, 8, 4, 16)
    err = rel_l2(got, ref)
    print(f"small forward, 4x16 latent: rel_l2 {err:.2e}")
    assert err < TOL_FORWARD
    sq = d.forward(latent.reshape(1, 8, 8, 8), 420.0)
    assert np.array_equal(got.reshape(sq.shape), sq)
    ts, sg = O.scheduler_timesteps(3)
    loop_ns = d.denoise_loop(latent, ts, sg, 4.5)
    loop_sq = d.denoise_loop(latent.reshape(1, 8, 8, 8), ts, sg, 4.5)
    assert np.array_equal(loop_ns.reshape(loop_sq.shape), loop_sq)
    with pytest.raises(sana_dit.SanaError, match="token count must form a square grid"):
        d.forward(O.randn((1, 8, 4, 8), 23), 420.0)


def test_conditioning_dropped_by_its_weights():
    """Uploading a weight the conditioning was computed from (cross-attention
    k / v, caption projection, caption_norm) drops it: the next forward fails
    with SANA_ERR_STATE until sana_dit_set_context runs again; other weights
    keep it."""
    import sana_dit
    m = O.Model(**SMALL)
    d = sana_dit.Dit(layers=2, hidden=128, ffn=256, caption_dim=96, latent_channels=8, self_heads=4, cross_heads=2)
    try:
        man = sana_dit.manifest(2, 128, 256, 96, 8)
        for name, shape in man.items():
            d.set_weight(name, m.get(name, shape))
        latent = O.randn((1, 8, 8, 8), 51)
        caption = O.randn((2, 16, 96), 52)
        d.set_context(caption, projected=False)
        ref = d.forward(latent, 999.0)
        for name in ("transformer_blocks.0.ff.conv_point.weight", "transformer_blocks.1.attn1.to_q.weight",
                     "scale_shift_table"):
            d.set_weight(name, m.get(name, man[name]))
            assert np.array_equal(d.forward(latent, 999.0), ref), name
        for name in ("transformer_blocks.1.attn2.to_k.weight", "transformer_blocks.0.attn2.to_v.bias",
                     "caption_projection.linear_2.weight", "caption_norm.weight"):
            d.set_weight(name, m.get(name, man[name]))
            with pytest.raises(sana_dit.SanaError) as e:
                d.forward(latent, 999.0)
            assert e.value.code == sana_dit.SANA_ERR_STATE, name
            d.set_context(caption, projected=False)
            assert np.array_equal(d.forward(latent, 999.0), ref), name
    finally:
        d.close()


def test_small_loop_batch2_vs_oracle(small_model):
    """The fused device loop on a latent batch of 2: CFG combines rows b and
    b + 2 of the noise prediction."""
    m, d = small_model
    latent = O.randn((2, 8, 8, 8), 13)
    caption = O.randn((4, 16, 96), 14)
    ref = m.loop(latent, caption, 5, 4.5)
    d.set_context(caption, projected=False)
    ts, sg = O.scheduler_timesteps(5)
    got = d.denoise_loop(latent, ts, sg, 4.5)
    err = rel_l2(got, ref)
    print(f"small loop, latent batch 2: rel_l2 {err:.2e}")
    assert err < TOL_LOOP


def test_small_forward_one_chain_no_graph_vs_oracle(monkeypatch):
    """SANA_DIT_CFG_BRANCHES=0 (the CFG pair as one chain) and
    SANA_DIT_NO_GRAPH=1 (direct launches), both read at context creation."""
    import sana_dit
    monkeypatch.setenv("SANA_DIT_CFG_BRANCHES", "0")
    monkeypatch.setenv("SANA_DIT_NO_GRAPH", "1")
    m = O.Model(**SMALL)
    d = sana_dit.Dit(layers=2, hidden=128, ffn=256, caption_dim=96, latent_channels=8, self_heads=4, cross_heads=2)
    try:
        for name, shape in sana_dit.manifest(2, 128, 256, 96, 8).items():
            d.set_weight(name, m.get(name, shape))
        latent = O.randn((1, 8, 8, 8), 15)
        caption = O.randn((2, 16, 96), 16)
        ref = m.forward(latent, m.project_caption(caption), 999.0)
        d.set_context(caption, projected=False)
        got = d.forward(latent, 999.0)
        again = d.forward(latent, 999.0)
        err = rel_l2(got, ref)
        print(f"small forward, one chain, no graph: rel_l2 {err:.2e}")
        assert err < TOL_FORWARD
        assert np.array_equal(got, again)
    finally:
        d.close()


def test_small_loop_graph_replays_match_direct_launches(small_model, monkeypatch):
    """The denoise loop as one cached graph: replayed with a forward and a loop
    of another schedule between the replays, every result equals the loop
    launched kernel by kernel (SANA_DIT_NO_GRAPH=1, read at context creation)."""
    import sana_dit
    m, d = small_model
    latent = O.randn((1, 8, 8, 8), 21)
    caption = O.randn((2, 16, 96), 22)
    ts6, sg6 = O.scheduler_timesteps(6)
    ts4, sg4 = O.scheduler_timesteps(4)
    d.set_context(caption, projected=False)
    first = d.denoise_loop(latent, ts6, sg6, 4.5)
    d.forward(O.randn((1, 8, 8, 8), 23), 500.0)
    other = d.denoise_loop(latent, ts4, sg4, 4.5)
    replays = [d.denoise_loop(latent, ts6, sg6, 4.5) for _ in range(2)]
    monkeypatch.setenv("SANA_DIT_NO_GRAPH", "1")
    e = sana_dit.Dit(layers=2, hidden=128, ffn=256, caption_dim=96, latent_channels=8, self_heads=4, cross_heads=2)
    try:
        for name, shape in sana_dit.manifest(2, 128, 256, 96, 8).items():
            e.set_weight(name, m.get(name, shape))
        e.set_context(caption, projected=False)
        direct6 = e.denoise_loop(latent, ts6, sg6, 4.5)
        direct4 = e.denoise_loop(latent, ts4, sg4, 4.5)
    finally:
        e.close()
    assert np.isfinite(direct6).all() and np.isfinite(direct4).all()
    assert np.array_equal(first, direct6)
    assert np.array_equal(other, direct4)
    for r in replays:
        assert np.array_equal(r, direct6)
