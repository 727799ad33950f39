"""float64 oracle of the reference's numpy decoder. TEST INFRASTRUCTURE ONLY.

Restates the forward pass of src/lowbit/model.py (Qwen2 / Llama architecture):
RMSNorm (:190-192), rotary tables and "rotate_half" rotation (:195-210), SwiGLU
(:213, 416-417), grouped-query causal attention with a KV cache (:353-378), the
layer loop, final norm and LM head (:380-435), greedy generation (:437-458). All
arithmetic is float64, except the W4A8 activation quantizer, which is defined on
float32 inputs and so sees each activation rounded to float32 first, as the
reference's activations are.

Linear layers are given as packed weights (the public int4 / MXFP4 formats) and
evaluated with this directory's own decoders and exact W4A8 accumulators
(oracle/reference.py), never with the product's GEMMs.

Parity pinning (tests/test_model_oracle.py): against a per-head, per-position
loop restatement on tiny models (dense weights), KV-cache decode equal to the
full forward, and the quantized linears against oracle/reference.py's GEMMs.
"""
from __future__ import annotations

import itertools

import numpy as np

from . import reference as R


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """x / sqrt(mean(x^2) + eps) * w over the last axis (src/lowbit/model.py:190-192)."""
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w


def rope_tables(head_dim: int, n_pos: int, theta: float):
    """float32 cos / sin [n_pos, D/2] built in float64 (src/lowbit/model.py:195-198);
    the model rotates with the float32-rounded values."""
    inv = 1.0 / theta ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim)
    ang = np.arange(n_pos, dtype=np.float64)[:, None] * inv[None]
    return np.cos(ang).astype(np.float32).astype(np.float64), np.sin(ang).astype(np.float32).astype(np.float64)


def rotate(x: np.ndarray, c: np.ndarray, s: np.ndarray) -> np.ndarray:
    """x [T, heads, D]; c, s [T, D/2]: element i pairs with i + D/2 (src/lowbit/model.py:201-210)."""
    h = x.shape[-1] // 2
    a, b = x[..., :h], x[..., h:]
    c, s = c[:, None, :], s[:, None, :]
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)


class Linear:
    """y = x . W^T (+ b) from a packed weight: kind "dense" (float64 W), "w4a16",
    "mxfp4" (float64 of the dequantized weight) or "w4a8" (per-token int8 of the
    float32-rounded input, exact int64 group sums, float64 rescale).

    W4A8 rounding ties: an activation whose scaled value x / sc lies within
    `tie_eps` int8 steps of a .5 tie can round either way under fp32 noise in the
    activation (one ulp is enough). Each such element is recorded in
    `model.near_ties` as (name, row, column, distance); elements named in
    `model.flip` as (name, row, column) are rounded the other way, which gives the
    oracle of a computation that took the other side of that tie.
    """

    def __init__(self, kind: str, w, b=None, name: str = "", model=None):
        self.kind, self.b = kind, None if b is None else np.asarray(b, np.float64)
        self.name, self.model = name, model
        if kind == "dense":
            self.w = np.asarray(w, np.float64)
        elif kind in ("w4a16", "w4a8"):
            self.qw, self.s, self.z, self.k = w.qw, w.scales, w.zeros, w.k
            self.w = R.dequant_int4(w.qw, w.scales, w.zeros)[:, :w.k]
        elif kind == "mxfp4":
            self.w = R.dequant_mxfp4(w.qw, w.e8m0)[:, :w.k]
        else:
            raise ValueError(kind)

    def _quant(self, x: np.ndarray):
        x32 = x.astype(np.float32)
        xq, xs, _ = R.quant_act_int8(x32, self.qw.shape[1] * 2)
        m = self.model
        if m is None:
            return xq, xs
        u = x32.astype(np.float64) / xs[:, None].astype(np.float64)
        d = np.abs(np.abs(u - np.floor(u)) - 0.5)
        for r, c in zip(*np.nonzero(d < m.tie_eps)):
            m.near_ties.append((self.name, int(r), int(c), float(d[r, c])))
            if (self.name, int(r), int(c)) in m.flip:
                xq = xq.copy()
                lo = np.floor(u[r, c])
                xq[r, c] = np.clip(lo + 1 if xq[r, c] == lo else lo, -127, 127)
        return xq, xs

    def __call__(self, x: np.ndarray) -> np.ndarray:
        if self.kind == "w4a8":
            xq, xs = self._quant(x)
            y = R.gemm_w4a8_ref(xq, xs, self.qw, self.s, self.z)
        else:
            y = x @ self.w.T
        return y if self.b is None else y + self.b


class Cache:
    """Per-layer float64 K and V [KV, capacity, D]; `length` positions are valid."""

    def __init__(self, cfg, capacity: int):
        shape = (cfg.num_kv_heads, capacity, cfg.head_dim)
        self.k = [np.zeros(shape) for _ in range(cfg.num_layers)]
        self.v = [np.zeros(shape) for _ in range(cfg.num_layers)]
        self.capacity, self.length = capacity, 0


class RefModel:
    """The reference Model's forward in float64 (src/lowbit/model.py:300-458).

    `quantize(w)` packs one [N, K] fp32 matrix in the backend's format (the
    public packers); q/k/v and gate/up are concatenated along N before packing,
    as the reference does (:318-326), so per-row quantization matches it.
    """

    def __init__(self, cfg, W: dict, backend: str = "dense", quantize=None, flip=(), tie_eps: float = 1e-4):
        self.cfg = cfg
        self.flip, self.tie_eps, self.near_ties = set(flip), tie_eps, []
        g = lambda n: np.asarray(W[n], np.float32)  # noqa: E731

        def lin(w, b=None, name=""):
            if backend == "dense":
                return Linear("dense", w, b, name, self)
            return Linear(backend, quantize(w), b, name, self)

        self.embed = g("model.embed_tokens.weight").astype(np.float64)
        self.layers = []
        for i in range(cfg.num_layers):
            p, a = f"model.layers.{i}.", f"model.layers.{i}.self_attn."
            wqkv = np.concatenate([g(a + "q_proj.weight"), g(a + "k_proj.weight"), g(a + "v_proj.weight")], 0)
            bqkv = (np.concatenate([g(a + "q_proj.bias"), g(a + "k_proj.bias"), g(a + "v_proj.bias")])
                    if cfg.qkv_bias else None)
            wgu = np.concatenate([g(p + "mlp.gate_proj.weight"), g(p + "mlp.up_proj.weight")], 0)
            self.layers.append(dict(ln1=g(p + "input_layernorm.weight").astype(np.float64),
                                    qkv=lin(wqkv, bqkv, f"{i}.qkv"), o=lin(g(a + "o_proj.weight"), None, f"{i}.o"),
                                    ln2=g(p + "post_attention_layernorm.weight").astype(np.float64),
                                    gate_up=lin(wgu, None, f"{i}.gate_up"),
                                    down=lin(g(p + "mlp.down_proj.weight"), None, f"{i}.down")))
        self.norm = g("model.norm.weight").astype(np.float64)
        head = (W["model.embed_tokens.weight"] if cfg.tie_word_embeddings or "lm_head.weight" not in W
                else W["lm_head.weight"])
        self.lm_head = lin(np.asarray(head, np.float32), None, "head")
        self.cos, self.sin = rope_tables(cfg.head_dim, cfg.max_position, cfg.rope_theta)

    def new_cache(self, capacity: int) -> Cache:
        return Cache(self.cfg, capacity)

    def _attention(self, q, k, v, cache: Cache, li: int, pos: int) -> np.ndarray:
        """q [T, H, D], k / v [T, KV, D] after rotation -> [T, H D] (src/lowbit/model.py:353-378)."""
        cfg = self.cfg
        T, H, D = q.shape
        KV = cfg.num_kv_heads
        cache.k[li][:, pos:pos + T] = k.transpose(1, 0, 2)
        cache.v[li][:, pos:pos + T] = v.transpose(1, 0, 2)
        S = pos + T
        out = np.empty((T, H, D))
        causal = np.arange(S)[None, :] > (pos + np.arange(T))[:, None]  # [T, S]
        for h in range(H):
            kv = h // (H // KV)
            s = q[:, h, :] @ cache.k[li][kv, :S].T / np.sqrt(D)
            s = np.where(causal, -np.inf, s)
            p = np.exp(s - s.max(axis=1, keepdims=True))
            out[:, h, :] = (p / p.sum(axis=1, keepdims=True)) @ cache.v[li][kv, :S]
        return out.reshape(T, H * D)

    def forward(self, tokens, cache: Cache | None = None, logits: str = "last") -> np.ndarray:
        """Same contract as the reference's Model.forward (src/lowbit/model.py:380-435)."""
        cfg = self.cfg
        tokens = np.asarray(tokens, np.int64).reshape(-1)
        T = len(tokens)
        own = cache is None
        cache = cache or self.new_cache(T)
        pos = cache.length
        if pos + T > cache.capacity:
            raise ValueError("KV cache full")
        H, KV, D, I = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, cfg.intermediate_size
        x = self.embed[tokens]
        c, s = self.cos[pos:pos + T], self.sin[pos:pos + T]
        for li, L in enumerate(self.layers):
            qkv = L["qkv"](rms_norm(x, L["ln1"], cfg.rms_norm_eps))
            q = rotate(qkv[:, :H * D].reshape(T, H, D), c, s)
            k = rotate(qkv[:, H * D:(H + KV) * D].reshape(T, KV, D), c, s)
            v = qkv[:, (H + KV) * D:].reshape(T, KV, D)
            x = x + L["o"](self._attention(q, k, v, cache, li, pos))
            gu = L["gate_up"](rms_norm(x, L["ln2"], cfg.rms_norm_eps))
            g = gu[:, :I]
            x = x + L["down"](g / (1.0 + np.exp(-g)) * gu[:, I:])
        if not own:
            cache.length = pos + T
        x = rms_norm(x, self.norm, cfg.rms_norm_eps)
        if logits == "none":
            return x
        if logits == "last":
            return self.lm_head(x[-1:])[0]
        return self.lm_head(x)

    def generate(self, prompt, n_new: int) -> list[int]:
        """Greedy decoding (src/lowbit/model.py:437-458)."""
        cache = self.new_cache(len(prompt) + n_new)
        logit = self.forward(list(prompt), cache)
        out = []
        for i in range(n_new):
            out.append(int(np.argmax(logit)))
            if i + 1 < n_new:
                logit = self.forward([out[-1]], cache)
        return out


def rel(a, b) -> float:
    """max |a - b| / max |b|."""
    return float(np.abs(np.asarray(a, np.float64) - b).max() / np.abs(b).max())


def rel_with_flips(ref_model: RefModel, toks, out, rows=slice(None), tol: float = 1e-5):
    """(rel error, flips) of logits `out` (rows `rows` of a forward over `toks`)
    against the oracle. When a W4A8 oracle misses by `tol` or more, it is re-run
    with each of its six closest near-ties rounded the other way, then with each
    pair of them; flips is the tuple that brought the error under `tol` (empty when
    none was needed), None when nothing did (then the smallest error is returned)."""
    ref_model.flip, ref_model.near_ties = set(), []
    r = rel(out, ref_model.forward(toks, logits="all")[rows])
    if r < tol or not ref_model.near_ties:
        return r, ()
    ties = [t[:3] for t in sorted(ref_model.near_ties, key=lambda t: t[3])[:6]]
    try:
        for fl in [(t,) for t in ties] + list(itertools.combinations(ties, 2)):
            ref_model.flip = set(fl)
            rr = rel(out, ref_model.forward(toks, logits="all")[rows])
            if rr < tol:
                return rr, fl
            r = min(r, rr)
        return r, None
    finally:
        ref_model.flip = set()
