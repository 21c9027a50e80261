"""The drop-in C++ API (sana.cpp_amd/host/*.h, libsana_cpp.so) through the test
program tests/cpp/dropin_test.cpp, and GGUF reading through the C ABI.

CPU: Tensor / scheduler / host-side transformer known answers and exception
types (tests/test_tensor.cpp, tests/test_scheduler_main.cpp,
tests/test_transformer.cpp of the reference), and GGUF index + loader checks
on files written by tests/gguf_writer.py.
GPU: block_forward known answers, small-model parity of every device entry
point against the oracle, the loop on GGUF-loaded weights, and the 20-step
1024 px loop on the seeded Sana-0.6B model against the reference's output.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import oracle_lib as O
import sana_dit
from conftest import rel_l2
from gguf_writer import GGML_BF16, GGML_F16, GGML_F32, write_gguf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "_build", "dropin_test")
GOLDEN = os.path.join(ROOT, "tests", "golden")

SMALL = dict(layers=2, hidden=128, ffn=256, caption=96, latent=8, self_heads=4, cross_heads=2)


def run_exe(*args, timeout=300):
    assert os.path.exists(EXE), "tests/cpp/_build/dropin_test missing: run __graft_entry__.build()"
    print("running dropin_test", *args, flush=True)
    res = subprocess.run([EXE, *args], capture_output=True, text=True, timeout=timeout)
    print(res.stdout[-4000:], res.stderr[-2000:], flush=True)
    return res


def small_gguf(path, ggml_type=GGML_F32):
    m = O.Model(**SMALL)
    names = sana_dit.manifest(2, 128, 256, 96, 8)
    write_gguf(path, {n: m.get(n, s) for n, s in names.items()}, ggml_type=ggml_type)
    return m, names


def small_vae_gguf(path, ggml_type=GGML_F32):
    v = O.Vae(full=False)
    write_gguf(path, {n: v.get(n, s) for n, s in O.vae_manifest(v.cfg).items()}, ggml_type=ggml_type)
    return v


def test_dropin_vae_loaders(tmp_path):
    """vae.h: find_vae_decoder_up_block_prefixes + load_vae_weights on a GGUF of
    the small synthetic decoder, tensors compared with the oracle's (no GPU)."""
    path = str(tmp_path / "vae_small.gguf")
    small_vae_gguf(path)
    res = run_exe("vae", path, timeout=120)
    assert res.returncode == 0 and " 0 failures" in res.stdout


REF_SRC = "/root/reference/src"


@pytest.mark.skipif(not os.path.isdir(REF_SRC), reason="the reference tree is not present on this host")
def test_option_a_sources_compile_against_reference_headers(tmp_path):
    """INTEGRATION.md Option A: host/transformer.cpp and host/vae.cpp replace the
    reference's src/transformer.cpp and src/vae.cpp inside its own build, so they
    must compile against the reference's transformer.h, vae.h, tensor.h,
    scheduler.h and weights_io.h (copied next to them, so the quoted includes
    resolve to the reference's headers), plus the three files of ours they also
    include: host/fingerprint.h, csrc/gguf.h and include/sana_dit.h."""
    import glob
    import shutil
    host = tmp_path / "sana.cpp_amd" / "host"
    host.mkdir(parents=True)
    (tmp_path / "sana.cpp_amd" / "csrc").mkdir()
    (tmp_path / "include").mkdir()
    for h in glob.glob(os.path.join(REF_SRC, "*.h")):
        shutil.copy(h, host)
    for f in ("transformer.cpp", "vae.cpp", "fingerprint.h"):
        shutil.copy(os.path.join(ROOT, "sana.cpp_amd", "host", f), host)
    shutil.copy(os.path.join(ROOT, "sana.cpp_amd", "csrc", "gguf.h"), tmp_path / "sana.cpp_amd" / "csrc")
    shutil.copy(os.path.join(ROOT, "include", "sana_dit.h"), tmp_path / "include")
    for src in ("transformer.cpp", "vae.cpp"):
        res = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-Wall", str(host / src)], capture_output=True,
                             text=True, timeout=120)
        assert res.returncode == 0, res.stderr[-3000:]


def test_dropin_host_api():
    res = run_exe("cpu", timeout=120)
    assert res.returncode == 0 and " 0 failures" in res.stdout


def test_dropin_gguf_loaders(tmp_path):
    path = str(tmp_path / "small.gguf")
    small_gguf(path)
    res = run_exe("gguf", path, timeout=120)
    assert res.returncode == 0 and " 0 failures" in res.stdout


def _gguf_index(path):
    lib = sana_dit.lib()
    n = ctypes.c_int64()
    rc = lib.sana_gguf_num_tensors(path.encode(), ctypes.byref(n))
    if rc != 0:
        return rc, None
    out = []
    for i in range(n.value):
        name = ctypes.create_string_buffer(256)
        shape = (ctypes.c_int64 * 4)()
        nd, ty, off = ctypes.c_int(), ctypes.c_int(), ctypes.c_uint64()
        assert lib.sana_gguf_tensor_info(path.encode(), i, name, 256, shape, ctypes.byref(nd), ctypes.byref(ty),
                                         ctypes.byref(off)) == 0
        out.append((name.value.decode(), tuple(shape[:nd.value]), ty.value, off.value))
    return 0, out


@pytest.mark.parametrize("ggml_type,dtype", [(GGML_F32, np.float32), (GGML_F16, np.float16)])
def test_gguf_index_round_trip(tmp_path, ggml_type, dtype):
    rng = np.random.default_rng(0)
    tensors = {"a.weight": rng.standard_normal((3, 5)).astype(np.float32),
               "blocks.0.scale_shift_table": rng.standard_normal((6, 7)).astype(np.float32),
               "c": rng.standard_normal((2, 1, 3, 3)).astype(np.float32),
               "d.bias": rng.standard_normal(9).astype(np.float32)}
    path = str(tmp_path / "t.gguf")
    write_gguf(path, tensors, alignment=64, ggml_type=ggml_type)
    rc, idx = _gguf_index(path)
    assert rc == 0
    raw = open(path, "rb").read()
    assert [e[0] for e in idx] == list(tensors)
    for (name, shape, ty, off), (ref_name, arr) in zip(idx, tensors.items()):
        assert shape == arr.shape and ty == ggml_type
        assert off % 64 == 0
        got = np.frombuffer(raw, dtype=dtype, count=arr.size, offset=off).reshape(arr.shape)
        np.testing.assert_array_equal(got, arr.astype(dtype))


def test_gguf_bf16_type_reported(tmp_path):
    path = str(tmp_path / "b.gguf")
    write_gguf(path, {"w": np.ones((4, 4), np.float32)}, ggml_type=GGML_BF16)
    rc, idx = _gguf_index(path)
    assert rc == 0 and idx[0][2] == GGML_BF16


@pytest.mark.parametrize("damage", ["magic", "truncated", "version"])
def test_gguf_malformed_files_are_errors(tmp_path, damage):
    path = str(tmp_path / "bad.gguf")
    write_gguf(path, {"w": np.ones((4, 4), np.float32)})
    raw = bytearray(open(path, "rb").read())
    if damage == "magic":
        raw[:4] = b"GGUX"
    elif damage == "version":
        raw[4:8] = (99).to_bytes(4, "little")
    else:
        raw = raw[:40]
    open(path, "wb").write(bytes(raw))
    rc, _ = _gguf_index(path)
    assert rc in (sana_dit.SANA_ERR_FORMAT, sana_dit.SANA_ERR_IO)
    assert sana_dit.lib().sana_dit_last_error()


def test_gguf_missing_file_is_io_error(tmp_path):
    rc, _ = _gguf_index(str(tmp_path / "none.gguf"))
    assert rc == sana_dit.SANA_ERR_IO


# ---------------------------------------------------------------- GPU


@pytest.mark.gpu
def test_dropin_device_paths():
    res = run_exe("gpu", timeout=110)
    assert res.returncode == 0 and " 0 failures" in res.stdout


@pytest.mark.gpu
def test_dropin_op_level_api():
    """common_ops.h / transformer_ops.h on the GPU: the reference's known answers
    (exact where the reference asserts ==), exception types, and random shapes
    against the oracle at rel-L2 1e-5 (fp32 throughout)."""
    res = run_exe("ops", timeout=110)
    assert res.returncode == 0 and " 0 failures" in res.stdout


@pytest.mark.gpu
def test_dropin_loop_on_gguf_weights(tmp_path):
    path = str(tmp_path / "small.gguf")
    small_gguf(path)
    res = run_exe("gguf", path, "run", timeout=110)
    assert res.returncode == 0 and " 0 failures" in res.stdout


@pytest.mark.gpu
def test_dropin_vae_decode(tmp_path):
    """run_vae_decode / run_vae_decoder_input of vae.h on GGUF-loaded weights
    against the oracle (rel-L2 2e-3), resident-weight reuse and re-upload."""
    path = str(tmp_path / "vae_small.gguf")
    small_vae_gguf(path)
    res = run_exe("vae", path, "run", timeout=110)
    assert res.returncode == 0 and " 0 failures" in res.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("ggml_type", [GGML_F32, GGML_F16])
def test_vae_load_gguf_abi_decode(tmp_path, ggml_type):
    """sana_vae_load_gguf, then a decode against the oracle on the same
    (for F16: the same rounded) weights."""
    path = str(tmp_path / "vae_small.gguf")
    v = small_vae_gguf(path, ggml_type)
    if ggml_type == GGML_F16:
        for n, s in O.vae_manifest(v.cfg).items():
            v.set(n, v.get(n, s).astype(np.float16).astype(np.float32))
    dev = sana_dit.Vae(v.cfg["channels"], v.cfg["attn"])
    try:
        dev.load_gguf(path)
        dev.check_weights()
        lat = O.randn((1, 32, 6, 6), 5)
        assert rel_l2(dev.decode(lat), v.decode(lat)) < 2e-3
    finally:
        dev.close()


@pytest.mark.gpu
def test_load_gguf_abi_forward(tmp_path):
    """sana_dit_load_gguf on one file holding every tensor, then a forward."""
    path = str(tmp_path / "small.gguf")
    m, _ = small_gguf(path)
    d = sana_dit.Dit(layers=2, hidden=128, ffn=256, caption_dim=96, latent_channels=8, self_heads=4, cross_heads=2)
    try:
        d.load_gguf(path, path, path)
        d.check_weights()
        latent = O.randn((1, 8, 8, 8), 42)
        caption = O.randn((2, 16, 96), 43)
        ref = m.forward(latent, m.project_caption(caption), 999.0)
        d.set_context(caption, projected=False)
        assert rel_l2(d.forward(latent, 999.0), ref) < 2e-3
    finally:
        d.close()


@pytest.mark.gpu
@pytest.mark.parametrize("ggml_type", [GGML_F16, GGML_BF16])
def test_load_gguf_abi_16bit_forward(tmp_path, ggml_type):
    """sana_dit_load_gguf on F16 and BF16 payloads: the forward matches the
    oracle run on the same weights rounded to that format."""
    path = str(tmp_path / "small16.gguf")
    m, names = small_gguf(path, ggml_type)
    for n, shape in names.items():
        w = m.get(n, shape)
        if ggml_type == GGML_F16:
            r = w.astype(np.float16).astype(np.float32)
        else:
            r = ((w.view(np.uint32) >> 16) << 16).view(np.float32)  # the writer truncates to bf16
        m.set(n, r)
    d = sana_dit.Dit(layers=2, hidden=128, ffn=256, caption_dim=96, latent_channels=8, self_heads=4, cross_heads=2)
    try:
        d.load_gguf(path, path, path)
        latent = O.randn((1, 8, 8, 8), 42)
        caption = O.randn((2, 16, 96), 43)
        ref = m.forward(latent, m.project_caption(caption), 999.0)
        d.set_context(caption, projected=False)
        err = rel_l2(d.forward(latent, 999.0), ref)
        print(f"gguf type {ggml_type}: forward rel_l2 {err:.2e}")
        assert err < 2e-3
    finally:
        d.close()


@pytest.mark.gpu
def test_dropin_full_loop_1024px_vs_reference(tmp_path):
    path = os.path.join(GOLDEN, "cfg3.npz")
    if not os.path.exists(path):
        pytest.skip("cfg3 golden not generated")
    fx = np.load(path, allow_pickle=False)
    cap, lat, out = (str(tmp_path / n) for n in ("caption.f32", "latent.f32", "out.f32"))
    O.randn((2, 300, 2304), 43).tofile(cap)
    O.randn((1, 32, 32, 32), 42).tofile(lat)
    res = run_exe("full-loop", cap, lat, "20", out, timeout=110)
    assert res.returncode == 0 and " 0 failures" in res.stdout
    got = np.fromfile(out, np.float32).reshape(1, 32, 32, 32)
    err = rel_l2(got, fx["final_latent"])
    print(f"drop-in 20-step loop: final latent rel_l2 {err:.2e}")
    assert err < 1e-2
