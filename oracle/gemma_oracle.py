"""Gemma-2 text-encoder oracle.  TEST INFRASTRUCTURE: only tests/ may import it.

The reference encodes prompts with llama.cpp (src/gemma_encoder.cpp:95-152:
llama_decode in embeddings mode, no pooling, returning the per-token hidden
states after the final RMSNorm).  llama.cpp (release b9966) is not part of
the reference tree and is absent here, so this module restates the published
Gemma-2 decoder forward that llama.cpp's Gemma-2 graph and Hugging Face
transformers' Gemma2Model both implement.  tests/test_oracle_gemma.py pins it
against transformers' Gemma2Model (eager attention, fp32) on small random
configurations.  The steps:

  x = embed[token] * sqrt(hidden)
  per layer l:
    h = rmsnorm(x) * attn_norm
    q, k, v = h Wq^T, h Wk^T, h Wv^T                       (GQA: heads / kv_heads queries per kv head)
    q, k = rope_neox(q, pos), rope_neox(k, pos)            (theta 10000, pairs (i, i + d/2))
    s = (q * query_scale) k^T;  s = softcap * tanh(s / softcap)
    causal mask; even layers also mask keys more than sliding_window - 1 back
    o = softmax(s) v;  x = x + rmsnorm(o Wo^T) * post_attention_norm
    h = rmsnorm(x) * ffn_norm
    x = x + rmsnorm((gelu_tanh(h Wgate^T) * (h Wup^T)) Wdown^T) * post_ffw_norm
  out = rmsnorm(x) * output_norm;  rmsnorm(v) = v / sqrt(mean(v^2) + eps)

Tensor names and orientations are the GGUF ones llama.cpp reads. Each
[out, in] matrix is stored as PyTorch [out, in]. The RMSNorm weights are
stored already offset, as 1 + w: the GGUF converter adds the 1 that Gemma's
RMSNorm applies. All arithmetic here is fp64.
"""
import numpy as np

GEMMA2_2B = dict(vocab=256000, hidden=2304, layers=26, heads=8, kv_heads=4, head_dim=256, ffn=9216,
                 rms_eps=1e-6, rope_theta=10000.0, softcap=50.0, sliding_window=4096, query_scale=1.0 / 16.0)

NORMS = ("attn_norm", "post_attention_norm", "ffn_norm", "post_ffw_norm")


def manifest(cfg):
    """{GGUF tensor name: PyTorch-order shape}."""
    H, Dq, Dkv = cfg["hidden"], cfg["heads"] * cfg["head_dim"], cfg["kv_heads"] * cfg["head_dim"]
    m = {"token_embd.weight": (cfg["vocab"], H), "output_norm.weight": (H,)}
    for l in range(cfg["layers"]):
        p = f"blk.{l}."
        m.update({p + "attn_norm.weight": (H,), p + "attn_q.weight": (Dq, H), p + "attn_k.weight": (Dkv, H),
                  p + "attn_v.weight": (Dkv, H), p + "attn_output.weight": (H, Dq),
                  p + "post_attention_norm.weight": (H,), p + "ffn_norm.weight": (H,),
                  p + "ffn_gate.weight": (cfg["ffn"], H), p + "ffn_up.weight": (cfg["ffn"], H),
                  p + "ffn_down.weight": (H, cfg["ffn"]), p + "post_ffw_norm.weight": (H,)})
    return m


def random_weights(cfg, seed=0, scale=0.02):
    """Seeded synthetic weights: N(0, scale) matrices and embeddings; norm
    weights 1 + 0.1 N(0, 1) (the stored, offset form)."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in manifest(cfg).items():
        z = rng.standard_normal(shape, dtype=np.float32)
        out[name] = (1 + np.float32(0.1) * z) if len(shape) == 1 else z * np.float32(scale)
    return out


def rmsnorm(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps) * np.asarray(w, np.float64)


def rope_neox(x, theta):
    """x [T, heads, d]: rotate the pairs (i, i + d/2) by pos * theta^(-2i/d)."""
    T, _, d = x.shape
    inv = 1.0 / theta ** (np.arange(0, d, 2, dtype=np.float64) / d)
    ang = np.arange(T, dtype=np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    a, b = x[..., : d // 2], x[..., d // 2:]
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)


def gelu_tanh(x):
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def forward(w, cfg, tokens, layers=None):
    """Hidden states after the final RMSNorm, [T, hidden] fp64."""
    f = lambda n: np.asarray(w[n], np.float64)
    H, nh, nkv, d = cfg["hidden"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    eps, T = cfg["rms_eps"], len(tokens)
    x = f("token_embd.weight")[np.asarray(tokens)] * np.sqrt(float(H))
    pos = np.arange(T)
    causal = pos[None, :] > pos[:, None]
    for l in range(cfg["layers"] if layers is None else layers):
        p = f"blk.{l}."
        h = rmsnorm(x, f(p + "attn_norm.weight"), eps)
        q = rope_neox((h @ f(p + "attn_q.weight").T).reshape(T, nh, d), cfg["rope_theta"]) * cfg["query_scale"]
        k = rope_neox((h @ f(p + "attn_k.weight").T).reshape(T, nkv, d), cfg["rope_theta"])
        v = (h @ f(p + "attn_v.weight").T).reshape(T, nkv, d)
        mask = causal.copy()
        if cfg["sliding_window"] and l % 2 == 0:
            mask |= pos[None, :] <= pos[:, None] - cfg["sliding_window"]
        o = np.empty((T, nh, d))
        for hh in range(nh):
            kv = hh // (nh // nkv)
            s = q[:, hh, :] @ k[:, kv, :].T
            s = cfg["softcap"] * np.tanh(s / cfg["softcap"])
            s = np.where(mask, -np.inf, s)
            s = np.exp(s - s.max(axis=1, keepdims=True))
            o[:, hh, :] = (s / s.sum(axis=1, keepdims=True)) @ v[:, kv, :]
        x = x + rmsnorm(o.reshape(T, nh * d) @ f(p + "attn_output.weight").T, f(p + "post_attention_norm.weight"),
                        eps)
        h = rmsnorm(x, f(p + "ffn_norm.weight"), eps)
        g = gelu_tanh(h @ f(p + "ffn_gate.weight").T) * (h @ f(p + "ffn_up.weight").T)
        x = x + rmsnorm(g @ f(p + "ffn_down.weight").T, f(p + "post_ffw_norm.weight"), eps)
    return rmsnorm(x, f("output_norm.weight"), eps)


def select_rows_first_and_last(x, keep):
    """Row 0 and the last keep - 1 rows (src/gemma_encoder.cpp:53-78)."""
    x = np.asarray(x)
    if x.ndim != 2 or keep == 0 or keep > x.shape[0]:
        raise ValueError("keep must be in (0, rows] of a rank-2 array")
    return np.concatenate([x[:1], x[x.shape[0] - (keep - 1):]], axis=0)


def attention_bias(num_real, length):
    """(1 - mask) * -10000 over `length` positions (src/gemma_encoder.cpp:175-182)."""
    return np.where(np.arange(length) < num_real, 0.0, -10000.0).astype(np.float32)
