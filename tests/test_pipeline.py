"""The three stages of sana_infer (src/infer_main.cpp:152-181,341-398) chained
through the drop-in C++ API by tests/cpp/dropin_test.cpp `pipeline`:
encode_prompt_pair -> the seeded initial latent -> run_full_denoising_loop_with_cfg
with the encoder's attention bias -> run_vae_decode.

Small synthetic models keep the oracle chain to seconds:
- a 2-layer Gemma-2 (hidden 128) with a trained SentencePiece-BPE vocabulary;
- a 2-block DiT (hidden 128, 4 x 32 self heads, 2 x 64 cross heads) whose
  caption width is the encoder's hidden size;
- the small DC-AE decoder (latent 32, 8x upsampling).
The sequence length (300), the 20 steps, guidance 4.5 and seed 42 are
sana_infer's.

Each stage is held to its own bar while chained: the prompt-pair embeddings to
2e-3 and the bias exactly (the oracle steps of tests/test_gemma_encoder.py);
the initial latent exactly (randn_torch_cpu); the final latent against the
oracle loop run on the oracle's embeddings and bias to 1e-2; the image against
the oracle decode of the device's final latent to 2e-3.
"""
import os
import struct

import numpy as np
import pytest

import oracle_lib as O
import sana_dit
from conftest import rel_l2
from gguf_writer import GGML_F32, write_gguf
from test_gemma_encoder import CHI, G, expected_ids, run_exe, sp_model, tokenizer_metadata  # noqa: F401

DIT = dict(layers=2, hidden=128, ffn=256, caption=128, latent=32, self_heads=4, cross_heads=2)
GEMMA = dict(hidden=128, layers=2, heads=2, kv_heads=1, head_dim=64, ffn=256, sliding_window=16, rms_eps=1e-6,
             rope_theta=10000.0, softcap=50.0, query_scale=1 / 8)
L, STEPS, SEED, SIDE = 300, 20, 42, 8


def gemma_gguf(path, sp, proto):
    cfg = dict(GEMMA, vocab=len(proto.pieces))
    w = G.random_weights(cfg, seed=21, scale=0.05)
    meta = tokenizer_metadata(sp, proto)
    meta.update({"general.architecture": "gemma2", "gemma2.embedding_length": cfg["hidden"],
                 "gemma2.block_count": cfg["layers"], "gemma2.feed_forward_length": cfg["ffn"],
                 "gemma2.attention.head_count": cfg["heads"], "gemma2.attention.head_count_kv": cfg["kv_heads"],
                 "gemma2.attention.key_length": cfg["head_dim"], "gemma2.attention.value_length": cfg["head_dim"],
                 "gemma2.attention.layer_norm_rms_epsilon": float(cfg["rms_eps"]),
                 "gemma2.attention.sliding_window": cfg["sliding_window"],
                 "gemma2.attn_logit_softcapping": float(cfg["softcap"]), "gemma2.rope.freq_base": 10000.0})
    write_gguf(path, w, ggml_type=GGML_F32, metadata=meta)
    return cfg, w


def oracle_prompt_pair(sp, cfg, w, prompt, negative):
    """src/gemma_encoder.cpp:186-244 with sentencepiece ids and the oracle forward."""
    total = len(expected_ids(sp, CHI)) + L - 2
    pos = expected_ids(sp, CHI + prompt)
    neg = expected_ids(sp, negative)
    pos_emb = G.select_rows_first_and_last(G.forward(w, cfg, pos + [0] * (total - len(pos))), L)
    neg_emb = G.forward(w, cfg, neg + [0] * (L - len(neg)))
    pos_real = 1 + sum(1 for p in range(total - (L - 1), total) if p < len(pos))
    bias = np.stack([G.attention_bias(len(neg), L), G.attention_bias(pos_real, L)]).astype(np.float32)
    return np.stack([neg_emb, pos_emb]).astype(np.float32), bias


@pytest.mark.gpu
def test_sana_infer_chain_vs_oracle(sp_model, tmp_path):
    sp, proto = sp_model
    gcfg, gw = gemma_gguf(str(tmp_path / "gemma.gguf"), sp, proto)
    m = O.Model(**DIT)
    names = sana_dit.manifest(DIT["layers"], DIT["hidden"], DIT["ffn"], DIT["caption"], DIT["latent"])
    write_gguf(str(tmp_path / "dit.gguf"), {n: m.get(n, s) for n, s in names.items()}, ggml_type=GGML_F32)
    v = O.Vae(full=False)
    write_gguf(str(tmp_path / "vae.gguf"), {n: v.get(n, s) for n, s in O.vae_manifest(v.cfg).items()},
               ggml_type=GGML_F32)
    prompt, negative = "a house by the lake", ""
    cases = b"".join(struct.pack("<I", len(s.encode())) + s.encode() for s in (prompt, negative))
    cases += struct.pack("<6I", L, STEPS, SEED, SIDE, DIT["self_heads"], DIT["cross_heads"])
    (tmp_path / "cases.bin").write_bytes(cases)
    out = tmp_path / "out.f32"
    res = run_exe("pipeline", str(tmp_path / "gemma.gguf"), str(tmp_path / "dit.gguf"), str(tmp_path / "vae.gguf"),
                  str(tmp_path / "cases.bin"), str(out), timeout=110)
    assert res.returncode == 0 and " 0 failures" in res.stdout

    got = np.fromfile(out, np.float32)
    sizes = [("emb", (2, L, GEMMA["hidden"])), ("bias", (2, L)), ("lat0", (1, 32, SIDE, SIDE)),
             ("lat", (1, 32, SIDE, SIDE)), ("img", (1, 3, 8 * SIDE, 8 * SIDE))]
    parts, off = {}, 0
    for name, shape in sizes:
        n = int(np.prod(shape))
        parts[name] = got[off:off + n].reshape(shape)
        off += n
    assert off == got.size

    emb, bias = oracle_prompt_pair(sp, gcfg, gw, prompt, negative)
    assert np.array_equal(parts["bias"], bias)
    err_emb = rel_l2(parts["emb"], emb)
    assert np.array_equal(parts["lat0"], O.randn((1, 32, SIDE, SIDE), SEED))
    lat = m.loop(parts["lat0"], emb, STEPS, 4.5, bias)
    err_lat = rel_l2(parts["lat"], lat)
    img = v.decode(parts["lat"])
    err_img = rel_l2(parts["img"], img)
    print(f"sana_infer chain: embeddings {err_emb:.2e}, final latent {err_lat:.2e}, image {err_img:.2e}")
    assert np.isfinite(parts["img"]).all()
    assert err_emb < 2e-3
    assert err_lat < 1e-2
    assert err_img < 2e-3
