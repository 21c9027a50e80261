"""Packed weight images (sana_dit_save_packed / sana_dit_load_packed) and the
GGUF load through a packed cache (sana_dit_load_gguf_cached), on a GPU context.

A packed image holds the device buffers as uploaded, so a context loaded from
it must give the forward of the context it was written from bit for bit, and
an image that does not match (other dimensions, other key, a flipped byte, a
short file) must be refused with nothing uploaded.
"""
import os

import numpy as np
import pytest

import oracle_lib as O
import sana_dit
from gguf_writer import GGML_F16, GGML_F32, write_gguf

pytestmark = pytest.mark.gpu

SMALL = dict(layers=2, hidden=128, ffn=256, caption_dim=96, latent_channels=8, self_heads=4, cross_heads=2)


def small_weights(seed=5):
    rng = np.random.default_rng(seed)
    out = {}
    for n, shape in sana_dit.manifest(2, 128, 256, 96, 8).items():
        out[n] = (np.ones(shape, np.float32) if n == "caption_norm.weight"
                  else rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02))
    return out


def make_context(w, extras=True):
    d = sana_dit.Dit(**SMALL)
    for n, a in w.items():
        d.set_weight(n, a)
    if extras:
        # the optional buffers: LayerNorm affine on block 0, q|k|v bias on block 1
        rng = np.random.default_rng(9)
        d.set_block_norm(0, 0, 1 + 0.1 * rng.standard_normal(128).astype(np.float32),
                         0.1 * rng.standard_normal(128).astype(np.float32))
        for s in ("to_q", "to_k", "to_v"):
            d.set_weight(f"transformer_blocks.1.attn1.{s}.bias", 0.05 * rng.standard_normal(128).astype(np.float32))
    d.check_weights()
    return d


def run(d):
    d.set_context(O.randn((2, 16, 96), 43), projected=False)
    return d.forward(O.randn((1, 8, 8, 8), 42), 999.0)


def expect_error(fn, code, text=None):
    with pytest.raises(sana_dit.SanaError) as e:
        fn()
    print("refused:", e.value)
    assert e.value.code == code
    if text:
        assert text in str(e.value)


def test_packed_round_trip_bit_for_bit(tmp_path):
    path = str(tmp_path / "small.sanapk")
    d = make_context(small_weights())
    try:
        ref = run(d)
        d.save_packed(path, 77)
    finally:
        d.close()
    assert os.path.getsize(path) > 0
    assert not [f for f in os.listdir(tmp_path) if ".tmp" in f]
    e = sana_dit.Dit(**SMALL)
    try:
        e.load_packed(path, 77)
        e.check_weights()
        got = run(e)
    finally:
        e.close()
    assert np.array_equal(got, ref)


def test_packed_refusals_leave_the_context_unchanged(tmp_path):
    path = str(tmp_path / "small.sanapk")
    src = make_context(small_weights())
    try:
        src.save_packed(path, 5)
    finally:
        src.close()
    raw = open(path, "rb").read()
    d = make_context(small_weights(seed=6), extras=False)
    try:
        ref = run(d)
        expect_error(lambda: d.load_packed(path, 6), sana_dit.SANA_ERR_FORMAT, "key mismatch")
        expect_error(lambda: d.load_packed(str(tmp_path / "missing.sanapk"), 5), sana_dit.SANA_ERR_IO)
        flipped = bytearray(raw)
        flipped[len(raw) - 100] ^= 0x40  # inside the last payload
        bad = str(tmp_path / "flipped.sanapk")
        open(bad, "wb").write(bytes(flipped))
        expect_error(lambda: d.load_packed(bad, 5), sana_dit.SANA_ERR_FORMAT, "checksum")
        short = str(tmp_path / "short.sanapk")
        open(short, "wb").write(raw[:len(raw) // 2])
        expect_error(lambda: d.load_packed(short, 5), sana_dit.SANA_ERR_FORMAT)
        open(short, "wb").write(raw[:40])
        expect_error(lambda: d.load_packed(short, 5), sana_dit.SANA_ERR_FORMAT)
        notpk = str(tmp_path / "text.sanapk")
        open(notpk, "wb").write(b"x" * 4096)
        expect_error(lambda: d.load_packed(notpk, 5), sana_dit.SANA_ERR_FORMAT, "not a packed")
        assert np.array_equal(run(d), ref)
    finally:
        d.close()
    other = sana_dit.Dit(**dict(SMALL, layers=1))
    try:
        expect_error(lambda: other.load_packed(path, 5), sana_dit.SANA_ERR_FORMAT, "dimensions")
    finally:
        other.close()


def test_save_packed_needs_every_weight(tmp_path):
    d = sana_dit.Dit(**SMALL)
    try:
        expect_error(lambda: d.save_packed(str(tmp_path / "x.sanapk"), 0), sana_dit.SANA_ERR_STATE)
    finally:
        d.close()
    assert not os.listdir(tmp_path)


@pytest.mark.parametrize("ggml_type", [GGML_F32, GGML_F16], ids=["f32", "f16"])
def test_load_gguf_cached(tmp_path, ggml_type):
    """First load: GGUF, cache written; second: from the cache, same forward
    bit for bit as sana_dit_load_gguf; a GGUF with a new modification time
    invalidates the cache."""
    w = small_weights()
    gg = str(tmp_path / "w.gguf")
    write_gguf(gg, w, ggml_type=ggml_type)
    cache = str(tmp_path / "w.sanapk")
    d = sana_dit.Dit(**SMALL)
    try:
        d.load_gguf(gg, gg, gg)
        ref = run(d)
    finally:
        d.close()
    used = []
    for _ in range(2):
        e = sana_dit.Dit(**SMALL)
        try:
            used.append(e.load_gguf_cached(gg, gg, gg, cache))
            assert np.array_equal(run(e), ref)
        finally:
            e.close()
        assert os.path.exists(cache)
    assert used == [False, True]
    st = os.stat(gg)
    os.utime(gg, ns=(st.st_atime_ns, st.st_mtime_ns + 10**9))
    e = sana_dit.Dit(**SMALL)
    try:
        assert e.load_gguf_cached(gg, gg, gg, cache) is False
        assert np.array_equal(run(e), ref)
        assert e.load_gguf_cached(gg, gg, gg, cache) is True
    finally:
        e.close()
