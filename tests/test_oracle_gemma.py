"""Pins the Gemma-2 encoder oracle (oracle/gemma_oracle.py).

The reference runs Gemma-2 through llama.cpp, which is not available here,
so the oracle's restatement of the Gemma-2 forward is checked against an
independent implementation: transformers' Gemma2Model (eager attention,
fp32, CPU) with the same random weights.  Both norm conventions are checked:
GGUF stores the RMSNorm weights as 1 + w, transformers keeps w.  The
configurations cover GQA, the logit soft-cap and the sliding window of the
even layers.  The host helpers of src/gemma_encoder.cpp are pinned against
the reference's own test (tests/test_gemma_encoder.cpp).
"""
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle"))
import gemma_oracle as G  # noqa: E402

torch = pytest.importorskip("torch")
transformers = pytest.importorskip("transformers")

HF_NORMS = {"attn_norm": "input_layernorm", "post_attention_norm": "post_attention_layernorm",
            "ffn_norm": "pre_feedforward_layernorm", "post_ffw_norm": "post_feedforward_layernorm"}
HF_MATS = {"attn_q": "self_attn.q_proj", "attn_k": "self_attn.k_proj", "attn_v": "self_attn.v_proj",
           "attn_output": "self_attn.o_proj", "ffn_gate": "mlp.gate_proj", "ffn_up": "mlp.up_proj",
           "ffn_down": "mlp.down_proj"}


def hf_model(cfg, w):
    hcfg = transformers.Gemma2Config(
        vocab_size=cfg["vocab"], hidden_size=cfg["hidden"], intermediate_size=cfg["ffn"],
        num_hidden_layers=cfg["layers"], num_attention_heads=cfg["heads"], num_key_value_heads=cfg["kv_heads"],
        head_dim=cfg["head_dim"], query_pre_attn_scalar=int(round(cfg["query_scale"] ** -2)),
        attn_logit_softcapping=cfg["softcap"], sliding_window=cfg["sliding_window"], rms_norm_eps=cfg["rms_eps"],
        hidden_activation="gelu_pytorch_tanh", max_position_embeddings=1024)
    hcfg._attn_implementation = "eager"
    m = transformers.Gemma2Model(hcfg).float().eval()
    sd = {"embed_tokens.weight": w["token_embd.weight"], "norm.weight": w["output_norm.weight"] - 1}
    for l in range(cfg["layers"]):
        for g, h in HF_NORMS.items():
            sd[f"layers.{l}.{h}.weight"] = w[f"blk.{l}.{g}.weight"] - 1
        for g, h in HF_MATS.items():
            sd[f"layers.{l}.{h}.weight"] = w[f"blk.{l}.{g}.weight"]
    m.load_state_dict({k: torch.from_numpy(np.ascontiguousarray(v, np.float32)) for k, v in sd.items()}, strict=True)
    return m


CASES = {
    "gqa_sliding": dict(vocab=97, hidden=64, layers=3, heads=4, kv_heads=2, head_dim=32, ffn=96, rms_eps=1e-6,
                        rope_theta=10000.0, softcap=50.0, sliding_window=4, query_scale=32 ** -0.5),
    "mqa_softcap": dict(vocab=61, hidden=48, layers=2, heads=3, kv_heads=1, head_dim=16, ffn=80, rms_eps=1e-6,
                        rope_theta=10000.0, softcap=1.5, sliding_window=64, query_scale=16 ** -0.5),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_forward_matches_transformers(case):
    cfg = CASES[case]
    w = G.random_weights(cfg, seed=3, scale=0.2)
    tokens = np.random.default_rng(1).integers(0, cfg["vocab"], size=13)
    ref = hf_model(cfg, w)(input_ids=torch.from_numpy(tokens[None]).long()).last_hidden_state[0].detach().numpy()
    got = G.forward(w, cfg, tokens)
    err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert err < 2e-5, err


def test_soft_cap_and_window_are_exercised():
    """The cases above must depend on the soft-cap and the window: switching
    either off changes the output (so a dropped term would fail the match)."""
    cfg = CASES["gqa_sliding"]
    w = G.random_weights(cfg, seed=3, scale=0.2)
    tokens = np.random.default_rng(1).integers(0, cfg["vocab"], size=13)
    base = G.forward(w, cfg, tokens)
    for change in (dict(sliding_window=0), dict(softcap=1e6)):
        other = G.forward(w, dict(cfg, **change), tokens)
        assert np.linalg.norm(other - base) / np.linalg.norm(base) > 1e-4, change


def test_rope_closed_form():
    x = np.random.default_rng(0).standard_normal((5, 2, 8))
    r = G.rope_neox(x, 10000.0)
    # position 0 is the identity; norms of each rotated pair are preserved
    assert np.allclose(r[0], x[0])
    n = lambda a: a[..., :4] ** 2 + a[..., 4:] ** 2
    assert np.allclose(n(r), n(x))
    # pair i at position p is rotated by p * 10000^(-2i/8)
    ang = 3 * 10000.0 ** (-2 * 1 / 8)
    assert np.isclose(r[3, 0, 1], x[3, 0, 1] * np.cos(ang) - x[3, 0, 5] * np.sin(ang))


def test_select_rows_first_and_last_reference_cases():
    """tests/test_gemma_encoder.cpp:7-33 of the reference: 10 x 2 rows [2r, 2r + 1]."""
    x = np.arange(20, dtype=np.float32).reshape(10, 2)
    assert G.select_rows_first_and_last(x, 4).tolist() == [[0, 1], [14, 15], [16, 17], [18, 19]]
    assert G.select_rows_first_and_last(x, 10).tolist() == x.tolist()
    assert G.select_rows_first_and_last(x, 1).tolist() == [[0, 1]]
    for bad in (0, 11):
        with pytest.raises(ValueError):
            G.select_rows_first_and_last(x, bad)


def test_attention_bias():
    b = G.attention_bias(3, 5)
    assert b.tolist() == [0.0, 0.0, 0.0, -10000.0, -10000.0]
