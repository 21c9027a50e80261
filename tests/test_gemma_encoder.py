"""The drop-in Gemma-2 prompt encoder (sana.cpp_amd/host/gemma_encoder.h)
through tests/cpp/dropin_test.cpp.

Tokenizer.  The reference tokenizes with llama.cpp's SentencePiece
tokenizer, which is not available here.  The independent implementation it
is held to is the sentencepiece library itself.  A BPE model is trained
offline on a small corpus (identity normalisation, byte fallback, two
user-defined symbols, no dummy prefix: Gemma's settings). Its vocabulary,
scores and piece types are written as GGUF tokenizer metadata, and the C++
tokenizer's ids must equal sentencepiece's (plus the BOS token) on every case
(CPU).

encode_prompt_pair (GPU).  Runs on a small synthetic Gemma-2 model with that
vocabulary. It is checked against the same steps done here: the instruction
prefix, padding, the first-and-last row selection and the padding bias of
src/gemma_encoder.cpp:186-244, with sentencepiece ids and the pinned oracle
forward (oracle/gemma_oracle.py).  Tolerance 2e-3.
"""
import glob
import os
import struct
import subprocess
import sys

import numpy as np
import pytest

from conftest import rel_l2
from gguf_writer import GGML_F32, write_gguf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "_build", "dropin_test")
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import gemma_oracle as G  # noqa: E402

spm = pytest.importorskip("sentencepiece")
from sentencepiece import sentencepiece_model_pb2  # noqa: E402

# src/gemma_encoder.cpp:18-26 (diffusers' complex_human_instruction)
CHI = ("Given a user prompt, generate an 'Enhanced prompt' that provides detailed visual descriptions suitable for "
       "image generation. Evaluate the level of detail in the user prompt:\n"
       "- If the prompt is simple, focus on adding specifics about colors, shapes, sizes, textures, and spatial "
       "relationships to create vivid and concrete scenes.\n"
       "- If the prompt is already detailed, refine and enhance the existing details slightly without "
       "overcomplicating.\n"
       "Here are examples of how to transform or refine prompts:\n"
       "- User Prompt: A cat sleeping -> Enhanced: A small, fluffy white cat curled up in a round shape, sleeping "
       "peacefully on a warm sunny windowsill, surrounded by pots of blooming red flowers.\n"
       "- User Prompt: A busy city street -> Enhanced: A bustling city street scene at dusk, featuring glowing street "
       "lamps, a diverse crowd of people in colorful clothing, and a double-decker bus passing by towering glass "
       "skyscrapers.\n"
       "Please generate only the enhanced description for the prompt below and avoid including any additional "
       "commentary or evaluations:\n"
       "User Prompt: ")

CASES = ["", "a", " leading and trailing spaces  ", "multiple   spaces\n\nand\tnewlines",
         "A red fox standing in fresh snow at sunrise, photorealistic", "ünïcødé ✓ 😀 日本語",
         "<start_of_turn>user\nhello<end_of_turn>\n<start_of_turn>model", "x<end_of_turn><end_of_turn>y",
         CHI + "a small wooden boat on a calm lake"]


def run_exe(*args, timeout=300):
    assert os.path.exists(EXE), "tests/cpp/_build/dropin_test missing: run __graft_entry__.build()"
    print("running dropin_test", *args, flush=True)
    res = subprocess.run([EXE, *args], capture_output=True, text=True, timeout=timeout)
    print(res.stdout[-3000:], res.stderr[-2000:], flush=True)
    return res


@pytest.fixture(scope="module")
def sp_model(tmp_path_factory):
    d = tmp_path_factory.mktemp("spm")
    corpus = d / "corpus.txt"
    # the prompts plus the text of the test sources: varied English and code
    # (any fixed text works: the checks compare two tokenizers on one model)
    sources = sorted(glob.glob(os.path.join(ROOT, "tests", "*.py")))
    corpus.write_text((CHI + "\n" + "\n".join(CASES[:6]) + "\n") * 3 +
                      "".join(open(f, encoding="utf-8").read() for f in sources))
    spm.SentencePieceTrainer.train(
        input=str(corpus), model_prefix=str(d / "bpe"), vocab_size=700, model_type="bpe", byte_fallback=True,
        add_dummy_prefix=False, remove_extra_whitespaces=False, normalization_rule_name="identity",
        character_coverage=1.0, user_defined_symbols=["<start_of_turn>", "<end_of_turn>"], minloglevel=2)
    proto = sentencepiece_model_pb2.ModelProto()
    proto.ParseFromString((d / "bpe.model").read_bytes())
    return spm.SentencePieceProcessor(model_file=str(d / "bpe.model")), proto


def tokenizer_metadata(sp, proto):
    return {"tokenizer.ggml.model": "llama",
            "tokenizer.ggml.tokens": [p.piece for p in proto.pieces],
            "tokenizer.ggml.scores": ("f32", [float(p.score) for p in proto.pieces]),
            "tokenizer.ggml.token_type": ("i32", [int(p.type) for p in proto.pieces]),
            "tokenizer.ggml.bos_token_id": sp.bos_id(), "tokenizer.ggml.add_bos_token": True,
            "tokenizer.ggml.add_space_prefix": False}


def expected_ids(sp, text):
    return [sp.bos_id()] + sp.encode(text)


def test_tokenizer_matches_sentencepiece(sp_model, tmp_path):
    sp, proto = sp_model
    path = str(tmp_path / "vocab.gguf")
    write_gguf(path, {"token_embd.weight": np.zeros((len(proto.pieces), 4), np.float32)},
               metadata=tokenizer_metadata(sp, proto))
    cases = bytearray()
    for text in CASES:
        b, ids = text.encode(), expected_ids(sp, text)
        cases += struct.pack("<I", len(b)) + b + struct.pack(f"<I{len(ids)}i", len(ids), *ids)
    (tmp_path / "cases.bin").write_bytes(bytes(cases))
    # the cases must exercise merges, byte fallback and the user-defined symbols
    all_ids = [i for t in CASES for i in expected_ids(sp, t)]
    assert any(proto.pieces[i].type == 6 for i in all_ids) and any(proto.pieces[i].type == 4 for i in all_ids)
    assert any(len(proto.pieces[i].piece) > 3 and proto.pieces[i].type == 1 for i in all_ids)
    res = run_exe("gemma-tok", path, str(tmp_path / "cases.bin"), timeout=120)
    assert res.returncode == 0 and " 0 failures" in res.stdout


SMALL = dict(hidden=128, layers=2, heads=2, kv_heads=1, head_dim=64, ffn=256, sliding_window=16, rms_eps=1e-6,
             rope_theta=10000.0, softcap=50.0, query_scale=1 / 8)


@pytest.mark.gpu
def test_encode_prompt_pair_vs_oracle(sp_model, tmp_path):
    sp, proto = sp_model
    cfg = dict(SMALL, vocab=len(proto.pieces))
    w = G.random_weights(cfg, seed=11, scale=0.05)
    meta = tokenizer_metadata(sp, proto)
    meta.update({"general.architecture": "gemma2", "gemma2.embedding_length": cfg["hidden"],
                 "gemma2.block_count": cfg["layers"], "gemma2.feed_forward_length": cfg["ffn"],
                 "gemma2.attention.head_count": cfg["heads"], "gemma2.attention.head_count_kv": cfg["kv_heads"],
                 "gemma2.attention.key_length": cfg["head_dim"], "gemma2.attention.value_length": cfg["head_dim"],
                 "gemma2.attention.layer_norm_rms_epsilon": float(cfg["rms_eps"]),
                 "gemma2.attention.sliding_window": cfg["sliding_window"],
                 "gemma2.attn_logit_softcapping": float(cfg["softcap"]), "gemma2.rope.freq_base": 10000.0})
    path = str(tmp_path / "gemma.gguf")
    write_gguf(path, w, ggml_type=GGML_F32, metadata=meta)
    L, prompt, negative = 300, "a small wooden boat on a calm lake", "blurry"
    cases = b"".join(struct.pack("<I", len(s.encode())) + s.encode() for s in (prompt, negative)) + struct.pack("<I", L)
    (tmp_path / "cases.bin").write_bytes(cases)
    out = tmp_path / "out.f32"
    res = run_exe("gemma", path, str(tmp_path / "cases.bin"), str(out), timeout=110)
    assert res.returncode == 0 and " 0 failures" in res.stdout
    got = np.fromfile(out, np.float32)
    emb, bias = got[:2 * L * cfg["hidden"]].reshape(2, L, cfg["hidden"]), got[2 * L * cfg["hidden"]:].reshape(2, L)
    # the reference's steps with sentencepiece ids and the oracle forward
    chi = len(expected_ids(sp, CHI))
    total = chi + L - 2
    pos = expected_ids(sp, CHI + prompt)
    neg = expected_ids(sp, negative)
    pos_full = G.forward(w, cfg, pos + [0] * (total - len(pos)))
    pos_emb = G.select_rows_first_and_last(pos_full, L)
    neg_emb = G.forward(w, cfg, neg + [0] * (L - len(neg)))
    pos_real = 1 + sum(1 for p in range(total - (L - 1), total) if p < len(pos))
    assert bias[0].tolist() == G.attention_bias(len(neg), L).tolist()
    assert bias[1].tolist() == G.attention_bias(pos_real, L).tolist()
    for b, ref in ((0, neg_emb), (1, pos_emb)):
        err = rel_l2(emb[b], ref)
        print(f"prompt pair row {b}: rel_l2 {err:.3e}")
        assert err < 2e-3
