"""Pins the CPU oracle against the reference's own known-answer tests.

Every expected value below is one that the reference's C++ tests assert
(tests/test_tensor.cpp, tests/test_transformer.cpp, tests/test_scheduler_main.cpp),
with the same inputs restated here as data; tolerances are the reference's.
Linear weights: the reference tests pass them as [in, out]; the oracle takes
PyTorch order [out, in], so they are transposed here.

Beyond those, independent checks that a plausible mistake would fail:
torch.randn for the seeded generator, fp64 closed forms and brute force for
the attention kernels, and the textbook softmax.
"""
import numpy as np
import pytest

import oracle_lib as O


def a32(x):
    return np.asarray(x, np.float32)


# ---------------------------------------------------------------- tensor ops (tests/test_tensor.cpp)

def test_layer_norm_eps0():  # test_tensor.cpp:92-115
    x = a32([[[1, 3], [2, 4]]])
    assert np.array_equal(O.layer_norm(x, 0.0), a32([[[-1, 1], [-1, 1]]]))
    got = O.layer_norm(x, 0.0, gamma=a32([2, 3]), beta=a32([1, -1]))
    assert np.array_equal(got, a32([[[-1, 2], [-1, 2]]]))


def test_rms_norm():  # test_tensor.cpp:117-130
    got = O.rms_norm(a32([[[3, 4], [0, 5]]]), 0.0, a32([2, 3]))
    np.testing.assert_allclose(got.reshape(-1), [1.6970563, 3.3941126, 0.0, 4.2426405], atol=1e-5)


def test_modulate():  # test_tensor.cpp:132-148
    got = O.modulate(a32([[[1, 2], [3, 4]]]), a32([[10, 20]]), a32([[0.5, -0.5]]))
    assert np.array_equal(got.reshape(-1), a32([11.5, 21, 14.5, 22]))


def test_conv1x1_as_linear():  # test_tensor.cpp:180-212 (1x1 conv = per-pixel linear)
    x_nchw = a32([[[[1, 2], [3, 4]], [[10, 20], [30, 40]]]])
    w = a32([[1, 0], [0, 1], [1, 1]])
    b = a32([0, 0, -1])
    tok = x_nchw.reshape(2, 4).T.copy()
    out = O.linear(tok, w, b).T.reshape(3, 2, 2)
    assert out[0, 0, 0] == 1 and out[0, 1, 1] == 4 and out[1, 0, 0] == 10 and out[1, 1, 1] == 40
    assert np.array_equal(out[2].reshape(-1), a32([10, 21, 32, 43]))


def test_depthwise3x3():  # test_tensor.cpp:214-242
    x = a32([[[[1, 10], [2, 20]], [[3, 30], [4, 40]]]])       # token-major [B, H, W, C]
    w = np.zeros((2, 3, 3), np.float32)
    w[0, 1, 1] = 1
    w[1, 1, 1] = 2
    got = O.depthwise3x3(x, w, a32([0.5, -1]))
    assert np.array_equal(got[0, :, :, 0].reshape(-1), a32([1.5, 2.5, 3.5, 4.5]))
    assert np.array_equal(got[0, :, :, 1].reshape(-1), a32([19, 39, 59, 79]))


def test_depthwise3x3_neighbours_brute_force():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2, 5, 4, 3)).astype(np.float32)
    w = rng.standard_normal((3, 3, 3)).astype(np.float32)
    b = rng.standard_normal(3).astype(np.float32)
    xp = np.pad(x.astype(np.float64), ((0, 0), (1, 1), (1, 1), (0, 0)))
    ref = np.zeros(x.shape)
    for ky in range(3):
        for kx in range(3):
            ref += xp[:, ky:ky + 5, kx:kx + 4, :] * w[:, ky, kx]
    ref += b
    np.testing.assert_allclose(O.depthwise3x3(x, w, b), ref, rtol=1e-5, atol=1e-5)


def test_glumb_conv_closed_form():  # test_tensor.cpp:273-313
    x = a32([[[1, 2]]])                      # [B, N=1, C=2]
    inv_w = np.zeros((4, 2), np.float32)
    inv_w[0, 0] = inv_w[1, 1] = inv_w[2, 0] = inv_w[3, 1] = 1
    dw = np.zeros((4, 3, 3), np.float32)
    dw[:, 1, 1] = 1
    pt = a32([[1, 0], [0, 1]])
    got = O.glumb_conv(x, 1, 1, inv_w, np.zeros(4, np.float32), dw, np.zeros(4, np.float32), pt)
    s1 = np.float32(1) / (np.float32(1) + np.exp(np.float32(-1)))
    s2 = np.float32(2) / (np.float32(1) + np.exp(np.float32(-2)))
    e0 = s1 * (s1 / (np.float32(1) + np.exp(-s1)))
    e1 = s2 * (s2 / (np.float32(1) + np.exp(-s2)))
    np.testing.assert_allclose(got.reshape(-1), [e0, e1], atol=1e-6)


# ---------------------------------------------------------------- transformer ops (tests/test_transformer.cpp)

def test_linear_2d():  # test_transformer.cpp:77-100 (weight given [in, out])
    w_in_out = a32([[7, 8], [9, 10], [11, 12]])
    got = O.linear(a32([[1, 2, 3], [4, 5, 6]]), w_in_out.T.copy(), a32([1, -2]))
    assert np.array_equal(got, a32([[59, 62], [140, 152]]))


Q = a32([[[1, 0], [0, 1]]])   # [B=1, N=2, C=2], one head of dim 2
K = a32([[[1, 2], [3, 4]]])
V = a32([[[10, 20], [30, 40]]])


def test_attention_4d():  # test_transformer.cpp:229-234
    got = O.attention(Q, K, V, 1)
    np.testing.assert_allclose(got.reshape(-1), [26.088594, 36.088594, 26.088594, 36.088594], atol=1e-5)


def test_linear_attention_4d():  # test_transformer.cpp:236-241
    got = O.linear_attention(Q, K, V, 1)
    np.testing.assert_allclose(got.reshape(-1), [25.0, 35.0, 23.333334, 33.333332], atol=1e-5)


def test_project_caption_context():  # test_transformer.cpp:243-292
    x = a32([[[1, 2, 3, 4], [5, 6, 7, 8]]])
    w1 = np.zeros((4, 2), np.float32)   # [in, out]
    w1[0, 0] = w1[1, 1] = 1
    w2 = np.eye(2, dtype=np.float32)
    got = O.caption_projection(x, w1.T.copy(), np.zeros(2, np.float32), w2, np.zeros(2, np.float32), a32([1, 2]))
    np.testing.assert_allclose(got.reshape(-1), [0.5590534, 2.5980382, 0.9053573, 2.1728575], atol=1e-5)


EYE = np.eye(2, dtype=np.float32)
Z2 = np.zeros(2, np.float32)
BLOCK_IN = a32([[[1, 0], [0, 1]]])


def test_attention_block_identity():  # test_transformer.cpp:310-344
    got = O.lib().oracle_attention_block
    out = np.empty_like(BLOCK_IN)
    args = [O.fp(BLOCK_IN)] + [O.fp(EYE), O.fp(Z2)] * 4 + [O.fp(out)]
    O.check(got(*args, O._sz(1), O._sz(2), O._sz(2), O._sz(1)))
    np.testing.assert_allclose(out.reshape(-1), [1, 0, 0, 1], atol=1e-5)


def test_cross_attention_block():  # test_transformer.cpp:346-371
    ctx = a32([[[2, 0], [0, 3]]])
    out = np.empty_like(BLOCK_IN)
    args = [O.fp(BLOCK_IN), O.fp(ctx), None] + [O.fp(EYE), O.fp(Z2)] * 4 + [O.fp(out)]
    O.check(O.lib().oracle_cross_attention_block(*args, O._sz(1), O._sz(2), O._sz(2), O._sz(2), O._sz(1)))
    np.testing.assert_allclose(out.reshape(-1), [1.6088594, 0.5867110, 0.2140836, 2.6788745], atol=1e-5)


def _kat_block(proj_w):
    """The SanaBlockWeights of test_transformer.cpp:395-431 (hidden 2, 1 head)."""
    inv_w = np.zeros((4, 2), np.float32)
    inv_w[0, 0] = inv_w[1, 1] = inv_w[2, 0] = inv_w[3, 1] = 1
    dw = np.zeros((4, 3, 3), np.float32)
    dw[:, 1, 1] = 1
    w = {"scale_shift_table": np.zeros((6, 2), np.float32), "attn_norm_gamma": np.ones(2, np.float32),
         "attn_norm_beta": Z2, "mlp_norm_gamma": np.ones(2, np.float32), "mlp_norm_beta": Z2,
         "inv_w": inv_w, "inv_b": np.zeros(4, np.float32), "dw_w": dw, "dw_b": np.zeros(4, np.float32),
         "pt_w": EYE, "self_heads": 1, "cross_heads": 1}
    for n in ("q", "k", "v", "out", "cq", "ck", "cv", "co"):
        w[n + "_w"] = proj_w
        w[n + "_b"] = Z2
    return w


KAT_X = a32([[[1, 0]]])
KAT_CTX = a32([[[2, 0], [0, 3]]])
KAT_TMOD = np.zeros((1, 12), np.float32)
KAT_TMOD[0, [4, 5, 10, 11]] = 1


def test_block_forward():  # test_transformer.cpp:373-440
    out = O.block_forward(_kat_block(EYE), KAT_X, KAT_CTX, KAT_TMOD)[2]
    np.testing.assert_allclose(out.reshape(-1), [4.3467007, -0.9475632], atol=1e-5)


def test_block_forward_residual_only():  # test_transformer.cpp:442-484
    out = O.block_forward(_kat_block(np.zeros((2, 2), np.float32)), KAT_X, KAT_CTX, KAT_TMOD)[2]
    np.testing.assert_allclose(out.reshape(-1), [1.3607715, 0.0313307], atol=1e-5)


# ---------------------------------------------------------------- scheduler (tests/test_scheduler_main.cpp)

def test_scheduler_timesteps():  # test_scheduler_main.cpp:27-41
    ts, sg = O.scheduler_timesteps(4)
    np.testing.assert_allclose(ts, [999, 899, 749, 499], atol=1e-3)
    np.testing.assert_allclose(sg, [0.99966644, 0.89963979, 0.74962479, 0.49966654, 0.0], atol=1e-6)


def _sched(fn, *arrays_and_scalars):
    import ctypes
    out = np.empty(1, np.float32)
    arrays = [a for a in arrays_and_scalars if isinstance(a, list)]
    fn_args = [O.fp(a32(a)) for a in arrays]
    scal = [ctypes.c_float(v) for v in arrays_and_scalars if not isinstance(v, list)]
    O.check(fn(*fn_args, O._sz(1), *scal, O.fp(out)))
    return float(out[0])


def test_scheduler_updates():  # test_scheduler_main.cpp:80-115
    L = O.lib()
    conv = _sched(L.oracle_sched_convert, [2.0], [4.0], 0.8)
    assert abs(conv - 2.4) < 1e-6
    first = _sched(L.oracle_sched_first_order, [conv], [4.0], 0.5, 0.8)
    assert abs(first - 3.4) < 1e-5
    # previous_model_outputs = [2.4, 2.0]: m0 = back() = 2.0, m1 = 2.4
    second = _sched(L.oracle_sched_second_order, [3.4], [2.0], [2.4], 0.2, 0.5, 0.8)
    assert abs(second - 2.44) < 1e-5


# ---------------------------------------------------------------- independent pins

def test_randn_matches_torch():
    """Same mt19937 stream, 24-bit uniforms and Box-Muller pairing as torch.randn
    on CPU; torch evaluates log/cos/sin with its own vector math, so values agree
    to a few ulp rather than bit for bit (bit-exactness against the reference's
    randn_torch_cpu is pinned by the weight digests of the golden fixtures)."""
    torch = pytest.importorskip("torch")
    for seed, n in ((42, 16), (43, 1000), (7, 37), (1000, 4608)):
        g = torch.Generator().manual_seed(seed)
        ref = torch.randn(n, generator=g).numpy()
        got = O.randn((n,), seed)
        assert np.abs(got - ref).max() < 1e-5, (seed, n)
        assert got[0] == pytest.approx(ref[0], abs=1e-6)


def test_linear_attention_brute_force():
    rng = np.random.default_rng(3)
    B, N, H, D = 2, 9, 3, 4
    q, k, v = (rng.standard_normal((B, N, H * D)).astype(np.float32) for _ in range(3))
    got = O.linear_attention(q, k, v, H)
    r = lambda a: np.maximum(a.astype(np.float64), 0).reshape(B, N, H, D)
    fq, fk, vv = r(q), r(k), v.astype(np.float64).reshape(B, N, H, D)
    w = np.einsum("bthd,bshd->bhts", fq, fk)                      # O(N^2) form
    ref = np.einsum("bhts,bshd->bthd", w, vv) / (w.sum(-1).transpose(0, 2, 1)[..., None] + 1e-15)
    np.testing.assert_allclose(got, ref.reshape(B, N, H * D), rtol=1e-4, atol=1e-5)
    # a non-positive query row gives exactly 0 (numerator 0, denominator eps)
    q2 = q.copy()
    q2[0, 4, :D] = -1.0
    assert np.all(O.linear_attention(q2, k, v, H)[0, 4, :D] == 0.0)


def test_attention_textbook_and_mask():
    rng = np.random.default_rng(4)
    B, N, L, H, D = 2, 5, 7, 2, 3
    q = rng.standard_normal((B, N, H * D)).astype(np.float32)
    k = rng.standard_normal((B, L, H * D)).astype(np.float32)
    v = rng.standard_normal((B, L, H * D)).astype(np.float32)
    s = np.einsum("bnhd,blhd->bhnl", q.reshape(B, N, H, D).astype(np.float64),
                  k.reshape(B, L, H, D).astype(np.float64)) / np.sqrt(D)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ref = np.einsum("bhnl,blhd->bnhd", p, v.reshape(B, L, H, D)).reshape(B, N, H * D)
    np.testing.assert_allclose(O.attention(q, k, v, H), ref, rtol=1e-5, atol=1e-6)
    # the -10000 padding bias equals dropping the padded keys
    bias = np.zeros((B, L), np.float32)
    bias[:, 4:] = -10000.0
    masked = O.attention(q, k, v, H, bias)
    sliced = O.attention(q, np.ascontiguousarray(k[:, :4]), np.ascontiguousarray(v[:, :4]), H)
    np.testing.assert_allclose(masked, sliced, rtol=1e-6, atol=1e-7)


def test_timestep_embedding_closed_form():
    t = a32([0.0, 999.0])
    got = O.timestep_embedding(t, 256)
    f = np.exp(-np.log(10000.0) * np.arange(128) / 128.0)
    ref = np.concatenate([np.cos(t[:, None] * f), np.sin(t[:, None] * f)], axis=1)
    np.testing.assert_allclose(got, ref, atol=2e-3)   # fp32 argument rounding at t = 999
    assert np.array_equal(got[0, :128], np.ones(128, np.float32))
    assert np.array_equal(got[0, 128:], np.zeros(128, np.float32))
