"""The C ABI library loads on a host without a GPU and exports exactly the
entry points that include/sana_dit.h declares; the Python binding binds all
of them.  No compute call is made here."""
import ctypes
import os
import re

import sana_dit

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    text = open(os.path.join(ROOT, "include", "sana_dit.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sana_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared()
    assert "sana_dit_forward" in names and "sana_hip_gemm" in names
    assert len(names) >= 20


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(sana_dit.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    assert sorted(sana_dit.PROTOTYPES) == declared()


def test_last_error_is_empty_string_initially():
    # a fresh process: other tests in this one may have left a message
    import subprocess
    import sys
    code = ("import ctypes, sys; sys.path.insert(0, %r); import sana_dit; "
            "print(repr(sana_dit.lib().sana_dit_last_error()))" % os.path.join(ROOT, "sana.cpp_amd"))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, check=True).stdout
    assert out.strip() == "b''"


def test_create_rejects_bad_config_without_gpu():
    # argument validation happens before any device call
    cfg = sana_dit.Config(28, 1152, 5760, 2304, 32, 35, 16, 0)   # 1152 % 35 != 0
    h = ctypes.c_void_p()
    rc = sana_dit.lib().sana_dit_create(ctypes.byref(cfg), ctypes.byref(h))
    assert rc == sana_dit.SANA_ERR_INVALID_ARGUMENT
    assert b"divisible" in sana_dit.lib().sana_dit_last_error()


def test_vae_create_rejects_bad_config_without_gpu():
    for channels, attn, msg in (((96,), (0,), b"multiples of 64"), ((64, 192), (0, 0), b"shortcut")):
        cfg = sana_dit.VaeConfig()
        cfg.latent_channels, cfg.levels, cfg.head_dim, cfg.expand = 32, len(channels), 32, 4
        cfg.scaling_factor, cfg.device = 0.41407, 0
        for i, c in enumerate(channels):
            cfg.channels[i], cfg.attention[i] = c, attn[i]
        h = ctypes.c_void_p()
        rc = sana_dit.lib().sana_vae_create(ctypes.byref(cfg), ctypes.byref(h))
        assert rc == sana_dit.SANA_ERR_INVALID_ARGUMENT
        assert msg in sana_dit.lib().sana_dit_last_error()


def test_vae_manifest_matches_the_reference_weight_set():
    # the oracle's manifest is pinned name by name against the reference loader
    # (tests/golden/vae_weights.npz, tests/test_oracle_vae.py)
    import oracle_lib as O
    for cfg in (O.FULL_VAE, O.SMALL_VAE):
        got = sana_dit.vae_manifest(cfg["channels"], cfg["attn"], cfg["latent"])
        assert got == {k: tuple(v) for k, v in O.vae_manifest(cfg).items()}


def test_randn_torch_cpu_entry_point():
    """sana_randn_torch_cpu (host only): the oracle's generator bit for bit --
    itself pinned to torch.randn and, through the golden weight digests, to the
    reference's randn_torch_cpu -- including a ragged tail (n % 16 != 0)."""
    import numpy as np
    import oracle_lib as O
    for shape, seed in (((16,), 1), ((1, 32, 32, 32), 42), ((2, 300, 2304), 43), ((37,), 5), ((1152, 2880), 1007)):
        assert np.array_equal(sana_dit.randn(shape, seed), O.randn(shape, seed)), (shape, seed)
    # torch.manual_seed(42); torch.randn(3): the well-known first draws
    assert np.allclose(sana_dit.randn((16,), 42)[:3], [1.9269, 1.4873, 0.9007], atol=1e-4)
    rc = sana_dit.lib().sana_randn_torch_cpu(sana_dit.ptr(np.empty(8, np.float32)), 8, 0)
    assert rc == sana_dit.SANA_ERR_INVALID_ARGUMENT


def test_seeded_weights_follow_the_reference_harness_rule():
    """sana_dit.seeded_weights: 0.02 * randn(shape, 1000 + sorted index), caption_norm ones
    (the rule of the reference CPU baseline's weights), checked on a small manifest."""
    import numpy as np
    import oracle_lib as O
    w = dict(sana_dit.seeded_weights(2, 128, 256, 96, 16))
    names = sorted(sana_dit.manifest(2, 128, 256, 96, 16))
    assert list(w) == names
    for i, n in enumerate(names):
        want = (np.ones(w[n].shape, np.float32) if n == "caption_norm.weight"
                else O.randn(w[n].shape, 1000 + i) * np.float32(0.02))
        assert np.array_equal(w[n], want), n
