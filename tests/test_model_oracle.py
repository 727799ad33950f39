"""Pins oracle/model_ref.py, the float64 decoder the device model is checked against.

The checks (CPU, tiny models):
  * a loop restatement written independently of the oracle — one head, one token,
    one rotary pair at a time, angles computed per element in float64 — agrees
    with the vectorized oracle on dense weights (src/lowbit/model.py:353-435 is
    the behaviour both restate; tests/test_model.py:16-88 of the reference checks
    its own model the same way);
  * a KV-cache decode equals the full forward, and greedy generation equals
    repeated full forwards (tests/test_model.py:91-106);
  * quantized oracles stay close to the dense one (tests/test_model.py:109-118),
    so a mis-decoded packed weight cannot pass unnoticed.
"""
import numpy as np
import pytest

from lowbit_amd import formats as F
from lowbit_amd import model as DM
from oracle import model_ref as MR


def loop_forward(cfg, W, tokens):
    g = lambda n: np.asarray(W[n], np.float64)  # noqa: E731
    T, D, H, KV = len(tokens), cfg.head_dim, cfg.num_heads, cfg.num_kv_heads
    half = D // 2

    def norm(row, w):
        ms = sum(v * v for v in row) / len(row)
        return np.array([v / np.sqrt(ms + cfg.rms_norm_eps) for v in row]) * w

    def rot(vec, t):
        out = np.empty(D)
        for i in range(half):
            ang = t / cfg.rope_theta ** (2.0 * i / D)
            out[i] = vec[i] * np.cos(ang) - vec[i + half] * np.sin(ang)
            out[i + half] = vec[i + half] * np.cos(ang) + vec[i] * np.sin(ang)
        return out

    x = np.stack([g("model.embed_tokens.weight")[t] for t in tokens])
    for li in range(cfg.num_layers):
        p = f"model.layers.{li}."
        hs = np.stack([norm(x[t], g(p + "input_layernorm.weight")) for t in range(T)])
        proj = {}
        for nm in ("q", "k", "v"):
            w = g(p + f"self_attn.{nm}_proj.weight")
            proj[nm] = np.stack([w @ hs[t] for t in range(T)])
            if cfg.qkv_bias:
                proj[nm] += g(p + f"self_attn.{nm}_proj.bias")
        att = np.zeros((T, H * D))
        for h in range(H):
            kvh = h * KV // H
            for t in range(T):
                q = rot(proj["q"][t, h * D:(h + 1) * D], t)
                scores = np.array([q @ rot(proj["k"][u, kvh * D:(kvh + 1) * D], u) / np.sqrt(D)
                                   for u in range(t + 1)])
                e = np.exp(scores - scores.max())
                pr = e / e.sum()
                att[t, h * D:(h + 1) * D] = sum(pr[u] * proj["v"][u, kvh * D:(kvh + 1) * D] for u in range(t + 1))
        x = x + np.stack([g(p + "self_attn.o_proj.weight") @ att[t] for t in range(T)])
        hs = np.stack([norm(x[t], g(p + "post_attention_layernorm.weight")) for t in range(T)])
        gate = np.stack([g(p + "mlp.gate_proj.weight") @ hs[t] for t in range(T)])
        up = np.stack([g(p + "mlp.up_proj.weight") @ hs[t] for t in range(T)])
        mlp = gate * (1.0 / (1.0 + np.exp(-gate))) * up
        x = x + np.stack([g(p + "mlp.down_proj.weight") @ mlp[t] for t in range(T)])
    xn = np.stack([norm(x[t], g("model.norm.weight")) for t in range(T)])
    head = g("model.embed_tokens.weight") if cfg.tie_word_embeddings else g("lm_head.weight")
    return xn @ head.T


def rel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / np.abs(b).max())


VARIANTS = [{}, dict(num_kv_heads=1, tie_word_embeddings=False, qkv_bias=False, head_dim=32, num_heads=8),
            dict(num_kv_heads=4), dict(head_dim=128, num_heads=2, num_kv_heads=1)]


@pytest.mark.parametrize("over", VARIANTS)
def test_oracle_matches_loop_restatement(over):
    cfg = DM.tiny_config(num_layers=1, **over)
    W = DM.random_weights(cfg, seed=7)
    toks = [3, 1, 4, 1, 5, 9]
    ref = loop_forward(cfg, W, toks)
    out = MR.RefModel(cfg, W).forward(toks, logits="all")
    # the oracle rotates with float32-rounded tables, the loop with exact angles
    assert rel(out, ref) < 1e-6


def test_oracle_kv_decode_and_generate():
    cfg = DM.tiny_config()
    W = DM.random_weights(cfg, seed=3)
    m = MR.RefModel(cfg, W)
    toks = (np.arange(20) * 7) % cfg.vocab_size
    full = m.forward(toks, logits="all")
    c = m.new_cache(32)
    parts = [m.forward(toks[:8], c, logits="all"), m.forward(toks[8:11], c, logits="all")]
    parts += [m.forward([t], c)[None] for t in toks[11:]]
    assert c.length == 20
    assert rel(np.concatenate(parts), full) < 1e-12
    g = m.generate(toks[:5], 5)
    seq, manual = list(toks[:5]), []
    for _ in range(5):
        manual.append(int(np.argmax(m.forward(seq))))
        seq.append(manual[-1])
    assert g == manual
    with pytest.raises(ValueError):
        m.forward(list(range(13)), c)  # 20 + 13 > 32


@pytest.mark.parametrize("backend", ["w4a16", "w4a8", "mxfp4"])
def test_quantized_oracle_close_to_dense(backend):
    cfg = DM.tiny_config()
    W = DM.random_weights(cfg, seed=3)
    toks = (np.arange(24) * 5) % cfg.vocab_size
    ref = MR.RefModel(cfg, W).forward(toks, logits="all")
    qz = F.quantize_mxfp4 if backend == "mxfp4" else F.quantize_int4
    out = MR.RefModel(cfg, W, backend, qz).forward(toks, logits="all")
    assert rel(out, ref) < 0.1
    assert np.mean(out.argmax(1) == ref.argmax(1)) >= 0.9


def test_device_model_host_config():
    """tiny_config / qwen2_config / random_weights / rope_tables of the device model
    module (host code; src/lowbit/model.py:195-198, 483-513)."""
    cfg = DM.tiny_config()
    assert (cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size, cfg.num_layers, cfg.num_heads,
            cfg.num_kv_heads, cfg.head_dim, cfg.max_position) == (97, 256, 384, 2, 4, 2, 64, 256)
    assert cfg.tie_word_embeddings and cfg.qkv_bias
    q = DM.qwen2_config()
    assert (q.hidden_size, q.num_layers, q.num_heads, q.num_kv_heads, q.intermediate_size, q.vocab_size) == \
        (896, 24, 14, 2, 4864, 151936)
    W = DM.random_weights(cfg, seed=1)
    assert W["model.layers.1.self_attn.k_proj.weight"].shape == (128, 256)
    assert W["model.layers.0.self_attn.q_proj.bias"].shape == (256,)
    assert "lm_head.weight" not in W
    assert all(v.dtype == np.float32 for v in W.values())
    W2 = DM.random_weights(cfg, seed=1)
    assert all(np.array_equal(W[k], W2[k]) for k in W)
    c, s = DM.rope_tables(64, 10, 10000.0)
    assert c.dtype == np.float32 and c.shape == (10, 32)
    np.testing.assert_array_equal(c[0], 1.0)
    np.testing.assert_array_equal(s[0], 0.0)
    # position 1, pair 0 rotates by exactly one radian
    assert abs(float(s[1, 0]) - np.sin(1.0)) < 1e-7
    with pytest.raises(ValueError):
        DM.Model(cfg, W, backend="fp32")


def test_w4a8_near_tie_flips():
    """An activation 7e-8 int8 steps from a .5 tie (layer 0's o-projection input,
    token 5, column 67 of this model) rounds to 24 in the oracle; rounded to 25 it
    moves the logits by 4.4e-3. rel_with_flips finds exactly that flip for a result
    computed on the other side of the tie, and finds none for a wrong result."""
    cfg = DM.tiny_config(num_kv_heads=4, head_dim=128, num_heads=4, hidden_size=512)
    W = DM.random_weights(cfg, seed=7)
    toks = [3, 1, 4, 1, 5, 9, 2, 6, 5, 3, 5]
    m = MR.RefModel(cfg, W, "w4a8", F.quantize_int4)
    base = m.forward(toks, logits="all")
    close = [t for t in m.near_ties if t[3] < 1e-6]
    assert [t[:3] for t in close] == [("0.o", 5, 67)]
    other = MR.RefModel(cfg, W, "w4a8", F.quantize_int4, flip=[("0.o", 5, 67)]).forward(toks, logits="all")
    assert 1e-3 < MR.rel(other, base) < 1e-2
    r, flips = MR.rel_with_flips(m, toks, other)
    assert r < 1e-12 and flips == (("0.o", 5, 67),)
    assert MR.rel_with_flips(m, toks, base) == (0.0, ())
    wrong = base.copy()
    wrong[3, 7] += 0.01 * np.abs(base).max()
    r, flips = MR.rel_with_flips(m, toks, wrong)
    assert flips is None and r > 1e-3
