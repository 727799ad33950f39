"""A device-resident decoder (Qwen2 / Llama architecture) on the fused GEMMs.

The reference runs this model in numpy with one ctypes GEMM per linear layer
(src/lowbit/model.py:300-470): every layer crosses the host boundary four
times. Here everything stays in HBM: token ids, activations, the KV cache, the
quantized weights (`to_device` handles) and the greedy argmax. Linear layers
call the library's GEMMs on device pointers (the decode kernels at one token,
the matrix-core kernels on t16 tiles for a prompt); the rest of a layer is the
library's decoder-layer kernels (`lbd_embed`, `lbd_rmsnorm`, `lbd_qkv_rope`,
`lbd_attention`, `lbd_swiglu`, `lbd_add`, `lbd_argmax`).

The decode position lives in device memory and the argmax writes the next token
id where the embedding lookup reads it, so one decode step is a fixed sequence
of launches: `generate` records it once as a HIP graph and replays it per token.

A one-token step (fused=True, the default) runs five launches per layer: each
linear layer is one fused GEMV (`lbd_gemv_*_fused`) whose prologue applies the
RMSNorm (q/k/v, gate/up, LM head) to its activation row and whose epilogue adds
the q/k/v bias or the residual in place, or (gate/up) writes the SwiGLU of each
gate/up output pair, so the down projection reads its activations ready-made;
the rotary embedding and the KV-cache write run inside the one-token attention,
which cuts each head's keys into slices on many compute units
(`lbd_attention_slices`) whose partial sums the o projection's prologue merges
(caches of more than 8 slices take `lbd_attention_decode_ws`, which merges in a
launch of its own); the LM head's epilogue folds the greedy argmax into a
64-bit key that `lbd_argmax_finalize` turns into the next token. Prompts (T > 1)
run the unfused sequence on the matrix-core GEMMs.

Same architecture and arithmetic as the reference model: RMSNorm in fp32, q/k/v
projections concatenated along N and gate/up rows interleaved in (gate i, up i)
pairs (quantization is per output row, so no quantized value changes), rotary embedding in the "rotate_half"
convention from float32 cos/sin tables built in float64, grouped-query causal
attention with a KV cache, SwiGLU MLP, tied or untied LM head (quantized like
the other linears). Norm weights, biases, the embedding table and the KV cache
stay fp32. Backends: "w4a16", "w4a8", "mxfp4" (the reference's "fp32" backend is
numpy sgemm and has no counterpart here).
"""
from __future__ import annotations

import ctypes as C
import time
from dataclasses import dataclass

import numpy as np

from . import formats as F
from . import kernels as K

BACKENDS = ("w4a16", "w4a8", "mxfp4")
_KIND = {"w4a16": 0, "mxfp4": 1, "w4a8": 2}
ARGMAX_SLOTS = 1024  # LBD_ARGMAX_SLOTS of include/lowbit_hip.h


# ---------------------------------------------------------------- config (src/lowbit/model.py:42-77)

@dataclass
class ModelConfig:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    tie_word_embeddings: bool = False
    qkv_bias: bool = False
    max_position: int = 4096
    name: str = "custom"


def tiny_config(**over) -> ModelConfig:
    """The reference's test model shape (src/lowbit/model.py:483-489), overridable."""
    base = dict(vocab_size=97, hidden_size=256, intermediate_size=384, num_layers=2,
                num_heads=4, num_kv_heads=2, head_dim=64, rms_norm_eps=1e-6,
                rope_theta=10000.0, tie_word_embeddings=True, qkv_bias=True,
                max_position=256, name="tiny")
    base.update(over)
    return ModelConfig(**base)


def qwen2_config(**over) -> ModelConfig:
    """a Qwen2.5-0.5B-shaped decoder (hidden 896, 24 layers, 14 / 2
    heads, MLP 4864, vocab 151936, RMSNorm + RoPE, q/k/v bias, tied embeddings)."""
    base = dict(vocab_size=151936, hidden_size=896, intermediate_size=4864, num_layers=24,
                num_heads=14, num_kv_heads=2, head_dim=64, rms_norm_eps=1e-6,
                rope_theta=1000000.0, tie_word_embeddings=True, qkv_bias=True,
                max_position=32768, name="qwen2-0.5b-shape")
    base.update(over)
    return ModelConfig(**base)


def random_weights(cfg: ModelConfig, seed: int = 0, scale: float = 0.05, float32_draws: bool = False) -> dict:
    """Random weights under the checkpoint tensor names, drawn as the reference's test
    helper draws them (src/lowbit/model.py:492-513): N(0, scale^2), embeddings x20,
    norm weights 1 + N(0, scale^2). float32_draws=True draws float32 normals directly
    (same distribution, other values, several times faster at 0.5B parameters)."""
    rng = np.random.default_rng(seed)
    if float32_draws:
        r = lambda *s: rng.standard_normal(s, dtype=np.float32) * np.float32(scale)  # noqa: E731
    else:
        r = lambda *s: (rng.standard_normal(s) * scale).astype(np.float32)  # noqa: E731
    h, i, D = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
    W = {"model.embed_tokens.weight": r(cfg.vocab_size, h) * 20,
         "model.norm.weight": 1 + r(h)}
    for li in range(cfg.num_layers):
        p = f"model.layers.{li}."
        W[p + "input_layernorm.weight"] = 1 + r(h)
        W[p + "post_attention_layernorm.weight"] = 1 + r(h)
        for nm, n in (("q", cfg.num_heads * D), ("k", cfg.num_kv_heads * D),
                      ("v", cfg.num_kv_heads * D)):
            W[p + f"self_attn.{nm}_proj.weight"] = r(n, h)
            if cfg.qkv_bias:
                W[p + f"self_attn.{nm}_proj.bias"] = r(n)
        W[p + "self_attn.o_proj.weight"] = r(h, cfg.num_heads * D)
        W[p + "mlp.gate_proj.weight"] = r(i, h)
        W[p + "mlp.up_proj.weight"] = r(i, h)
        W[p + "mlp.down_proj.weight"] = r(h, i)
    if not cfg.tie_word_embeddings:
        W["lm_head.weight"] = r(cfg.vocab_size, h)
    return W


def rope_tables(head_dim: int, n_pos: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """float32 cos / sin [n_pos, head_dim/2], angles in float64 (src/lowbit/model.py:195-198)."""
    inv = 1.0 / theta ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim)
    ang = np.arange(n_pos, dtype=np.float64)[:, None] * inv[None]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


# ---------------------------------------------------------------- device state

def _buf(nbytes: int) -> K.DeviceBuffer:
    return K.DeviceBuffer(max(16, int(nbytes)))


class KVCache:
    """Per-layer fp32 K and V [KV, capacity, D] in HBM; `length` tokens are valid."""

    def __init__(self, cfg: ModelConfig, capacity: int):
        if capacity > 16000:
            raise ValueError("KV cache capacity above 16000 positions")
        self.capacity = int(capacity)
        nb = cfg.num_kv_heads * self.capacity * cfg.head_dim * 4
        self.k = [_buf(nb) for _ in range(cfg.num_layers)]
        self.v = [_buf(nb) for _ in range(cfg.num_layers)]
        self.length = 0
        # partial sums of the one-token attention's key slices (the layers use it
        # in turn on the model's stream)
        wb = K.lib().lbd_attention_decode_work_bytes(cfg.num_heads, cfg.head_dim, self.capacity)
        self.attn_work = _buf(wb)
        # the o projection's prologue merges up to 8 slices of 4096 / head_dim keys
        # over rows of at most 2048 elements; longer caches take the merge launch
        slices = wb // (cfg.num_heads * (cfg.head_dim + 4) * 4)
        self.fused_merge = slices <= 8 and cfg.num_heads * cfg.head_dim <= 2048


@dataclass
class _Layer:
    ln1: K.DeviceBuffer
    qkv: object
    qkv_bias: K.DeviceBuffer | None
    o: object
    ln2: K.DeviceBuffer
    gate_up: object
    down: object


def _check(rc: int, what: str) -> int:
    if rc < 0:
        K._err(rc, what)
    return rc


class Model:
    """Device-resident decoder with the reference Model's constructor and calls
    (src/lowbit/model.py:300-470): `forward(tokens, cache, logits)` and greedy
    `generate(prompt, n_new, cache, timings)`."""

    def __init__(self, cfg: ModelConfig, weights: dict, backend: str = "w4a8", asym: bool = False,
                 quantize_lm_head: bool = True, int4_scale: str = "absmax", max_tokens: int = 512,
                 quantize_on_device: bool = True, fused: bool = True):
        if backend not in BACKENDS:
            raise ValueError(f"backend must be one of {BACKENDS}")
        if not quantize_lm_head:
            raise ValueError("the LM head is quantized like the other linears on the device")
        blk = F.MXBLOCK if backend == "mxfp4" else F.GROUP
        for k in (cfg.hidden_size, cfg.intermediate_size, cfg.num_heads * cfg.head_dim):
            if k % blk:
                raise ValueError(f"layer width {k} is not a multiple of the {backend} block ({blk})")
        self.cfg, self.backend, self.asym = cfg, backend, asym
        self.L = K.lib()
        s = C.c_void_p()
        _check(self.L.lb_stream_create(C.byref(s)), "stream")
        self.stream = s.value
        g = lambda n: np.ascontiguousarray(weights[n], np.float32)  # noqa: E731
        up = K.DeviceBuffer.from_array

        def lin(w):
            # the device packers write the host packers' bytes; packing on the device
            # only saves the host time (seconds per 100M weights)
            if quantize_on_device:
                if backend == "mxfp4":
                    return K.quantize_mxfp4_device(w)
                return K.quantize_int4_device(w, asym=asym, scale=int4_scale)
            wq = F.quantize_mxfp4(w) if backend == "mxfp4" else F.quantize_int4(w, asym=asym, scale=int4_scale)
            return K.to_device(wq)

        self.embed = up(g("model.embed_tokens.weight"))
        self.layers: list[_Layer] = []
        for i in range(cfg.num_layers):
            p = f"model.layers.{i}."
            a = p + "self_attn."
            wqkv = np.concatenate([g(a + "q_proj.weight"), g(a + "k_proj.weight"), g(a + "v_proj.weight")], 0)
            bqkv = (np.concatenate([g(a + "q_proj.bias"), g(a + "k_proj.bias"), g(a + "v_proj.bias")])
                    if cfg.qkv_bias else None)
            # row 2i: gate i, row 2i + 1: up i (the pairs of the glu epilogue)
            wgu = np.stack([g(p + "mlp.gate_proj.weight"), g(p + "mlp.up_proj.weight")], 1).reshape(
                2 * cfg.intermediate_size, -1)
            self.layers.append(_Layer(up(g(p + "input_layernorm.weight")), lin(wqkv),
                                      None if bqkv is None else up(bqkv), lin(g(a + "o_proj.weight")),
                                      up(g(p + "post_attention_layernorm.weight")), lin(wgu),
                                      lin(g(p + "mlp.down_proj.weight"))))
        self.norm = up(g("model.norm.weight"))
        head = (g("model.embed_tokens.weight") if cfg.tie_word_embeddings or "lm_head.weight" not in weights
                else g("lm_head.weight"))
        self.lm_head = lin(head)
        cos, sin = rope_tables(cfg.head_dim, cfg.max_position, cfg.rope_theta)
        self.cos, self.sin = up(cos), up(sin)
        self._alloc(max_tokens)
        self.tok = _buf(4 * max(max_tokens, 1))
        self.pos = _buf(4)
        self.hist: K.DeviceBuffer | None = None
        # argmax key slots of the fused LM head; lbd_argmax_finalize clears them
        self.key = _buf(8 * ARGMAX_SLOTS)
        _check(self.L.lb_memset_d(self.key.ptr, 0, 8 * ARGMAX_SLOTS), "key clear")
        # one-token steps fuse when every linear takes the small-M kernels and the
        # attention shape fits the one-token kernel
        D = cfg.head_dim
        widths = {cfg.hidden_size, cfg.intermediate_size, cfg.num_heads * D}
        prm = K._Params(-1, 0, 0, 0, 0, 0, 0)
        self.fused = bool(fused) and D in (32, 64, 128) and cfg.num_heads // cfg.num_kv_heads <= 16 and all(
            self.L.lbd_gemm_path(_KIND[backend], 1, k, C.byref(prm)) == K.ISA_GFX950 for k in widths)

    # ------------------------------------------------------------ buffers

    def _alloc(self, T: int):
        cfg = self.cfg
        h, I, D = cfg.hidden_size, cfg.intermediate_size, cfg.head_dim
        qkvw = (cfg.num_heads + 2 * cfg.num_kv_heads) * D
        self.tmax = T
        self.x, self.h, self.o = _buf(T * h * 4), _buf(T * h * 4), _buf(T * h * 4)
        self.qkv, self.att = _buf(T * qkvw * 4), _buf(T * cfg.num_heads * D * 4)
        self.gu, self.m = _buf(T * 2 * I * 4), _buf(T * I * 4)
        self.logits = _buf(cfg.vocab_size * 4)
        kmax = max(h, I, cfg.num_heads * D)
        # room for the K split of the bf16x3 prefill GEMMs (rows of 8192+ elements), so
        # the model's matrix-core GEMMs are the launches lb.gemm_* and bench.py time
        kind = 1 if self.backend == "mxfp4" else 0
        lin = [w for ly in self.layers for w in (ly.qkv, ly.o, ly.gate_up, ly.down)] + [self.lm_head]
        split = max(self.L.lbd_bf16x3_workspace_bytes_split(kind, T, w.n, w.kp) for w in lin)
        self.ws = _buf(max(self.L.lbd_w4a8_workspace_bytes(T, kmax), self.L.lbd_bf16x3_workspace_bytes(T, kmax),
                           split))

    @property
    def linear_weight_bytes(self) -> int:
        return sum(x.nbytes for L in self.layers for x in (L.qkv, L.o, L.gate_up, L.down)) + self.lm_head.nbytes

    def new_cache(self, max_len: int) -> KVCache:
        return KVCache(self.cfg, max_len)

    # ------------------------------------------------------------ one step

    def _linear(self, w, x: int, m: int, y: int):
        """y[m, n] = x[m, k] . w^T on the stream: decode kernels on the row-major
        copy, or the matrix-core kernels on the t16 copy (repacked on first use)."""
        L, prm = self.L, K._Params(-1, 0, 0, 0, 0, 0, 0)
        mfma = _check(L.lbd_gemm_path(_KIND[self.backend], m, w.kp, C.byref(prm)), "lbd_gemm_path") \
            == K.ISA_GFX950_MFMA
        s, ws = self.stream, self.ws
        if self.backend == "mxfp4":
            if mfma:
                qwt, et = w.tiles()
                rc = L.lbd_gemm_mxfp4_t16(x, m, w.kp, qwt.ptr, et.ptr, w.n, y, C.byref(prm), ws.ptr, ws.nbytes, s)
            else:
                rc = L.lbd_gemm_mxfp4(x, m, w.kp, w.qw.ptr, w.e8m0.ptr, w.n, y, C.byref(prm), s)
        else:
            zp = None if w.zeros is None else w.zeros.ptr
            if mfma and self.backend == "w4a16":
                rc = K.gemm_w4a16_tiles(w, x, m, y, prm, ws.ptr, ws.nbytes, s)
            elif mfma:
                qwt, st, zt = w.tiles()
                rc = L.lbd_gemm_w4a8_t16(x, m, w.kp, qwt.ptr, st.ptr, None if zt is None else zt.ptr, w.n, y,
                                         C.byref(prm), ws.ptr, ws.nbytes, s)
            elif self.backend == "w4a16":
                rc = L.lbd_gemm_w4a16(x, m, w.kp, w.qw.ptr, w.scales.ptr, zp, w.n, y, C.byref(prm), s)
            else:
                rc = L.lbd_gemm_w4a8(x, m, w.kp, w.qw.ptr, w.scales.ptr, zp, w.n, y, C.byref(prm), ws.ptr,
                                     ws.nbytes, s)
        _check(rc, f"{self.backend} linear")

    def _fused_linear(self, w, x: int | None, y: int, norm: int | None = None, glu: bool = False,
                      bias: int | None = None, res: int | None = None, key: int | None = None,
                      attn: tuple | None = None):
        """y[0, n] = res[n] + (act(x) . w^T)[n] + bias[n] for one token, one launch;
        act is the RMSNorm with weights `norm` (or the identity). With glu the rows
        of w are (gate, up) pairs and y[0, p] = silu(gate) * up of pair p. With
        attn = (partials, cache capacity) the activation row is the one-token
        attention merged from its key-slice partials (x unused)."""
        part, cap = attn if attn else (None, 0)
        f = K.LbdFusion(norm, self.cfg.rms_norm_eps if norm else 0.0, 0, bias, res, key, int(glu), part, cap,
                        self.cfg.head_dim if attn else 0)
        L, s = self.L, self.stream
        if self.backend == "mxfp4":
            rc = L.lbd_gemv_mxfp4_fused(x, 1, w.kp, w.qw.ptr, w.e8m0.ptr, w.n, y, C.byref(f), s)
        else:
            zp = None if w.zeros is None else w.zeros.ptr
            fn = L.lbd_gemv_w4a16_fused if self.backend == "w4a16" else L.lbd_gemv_w4a8_fused
            rc = fn(x, 1, w.kp, w.qw.ptr, w.scales.ptr, zp, w.n, y, C.byref(f), s)
        _check(rc, f"fused {self.backend} linear")

    def _step_fused(self, cache: KVCache, logits: str, argmax_hist: bool):
        """Enqueue one forward of the single token in self.tok at position *pos,
        five launches per layer."""
        cfg, L, s = self.cfg, self.L, self.stream
        h, H, KV, D = cfg.hidden_size, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
        x = self.x.ptr
        _check(L.lbd_embed(self.embed.ptr, cfg.vocab_size, h, self.tok.ptr, 1, x, s), "embed")
        for li, ly in enumerate(self.layers):
            self._fused_linear(ly.qkv, x, self.qkv.ptr, norm=ly.ln1.ptr,
                               bias=None if ly.qkv_bias is None else ly.qkv_bias.ptr)
            if cache.fused_merge:
                # key slices, merged in the o projection's prologue
                _check(L.lbd_attention_slices(self.qkv.ptr, H, KV, D, self.cos.ptr, self.sin.ptr, self.pos.ptr,
                                              cfg.max_position, cache.k[li].ptr, cache.v[li].ptr, cache.capacity,
                                              cache.attn_work.ptr, cache.attn_work.nbytes, s), "attention slices")
                self._fused_linear(ly.o, None, x, res=x, attn=(cache.attn_work.ptr, cache.capacity))
            else:
                _check(L.lbd_attention_decode_ws(self.qkv.ptr, H, KV, D, self.cos.ptr, self.sin.ptr, self.pos.ptr,
                                                 cfg.max_position, cache.k[li].ptr, cache.v[li].ptr, cache.capacity,
                                                 self.att.ptr, cache.attn_work.ptr, cache.attn_work.nbytes, s),
                       "attention decode")
                self._fused_linear(ly.o, self.att.ptr, x, res=x)
            self._fused_linear(ly.gate_up, x, self.m.ptr, norm=ly.ln2.ptr, glu=True)
            self._fused_linear(ly.down, self.m.ptr, x, res=x)
        if logits == "none":
            _check(L.lbd_rmsnorm(x, self.norm.ptr, 1, h, cfg.rms_norm_eps, self.h.ptr, s), "rmsnorm")
        elif logits == "last":
            key = self.key.ptr if argmax_hist else None
            self._fused_linear(self.lm_head, x, self.logits.ptr, norm=self.norm.ptr, key=key)
            if argmax_hist:
                hist = self.hist.ptr if self.hist is not None else None
                n = self.hist.nbytes // 4 if self.hist is not None else 0
                _check(L.lbd_argmax_finalize(self.key.ptr, self.tok.ptr, self.pos.ptr, 1, hist, n, s),
                       "argmax finalize")
        else:
            self._fused_linear(self.lm_head, x, self.all_logits.ptr, norm=self.norm.ptr)

    def _step(self, T: int, cache: KVCache, logits: str, argmax_hist: bool):
        """Enqueue one forward of the T tokens in self.tok at position *pos."""
        if T == 1 and self.fused:
            return self._step_fused(cache, logits, argmax_hist)
        cfg, L, s = self.cfg, self.L, self.stream
        h, I, H, KV, D = cfg.hidden_size, cfg.intermediate_size, cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
        qkvw = (H + 2 * KV) * D
        _check(L.lbd_embed(self.embed.ptr, cfg.vocab_size, h, self.tok.ptr, T, self.x.ptr, s), "embed")
        for li, ly in enumerate(self.layers):
            _check(L.lbd_rmsnorm(self.x.ptr, ly.ln1.ptr, T, h, cfg.rms_norm_eps, self.h.ptr, s), "rmsnorm")
            self._linear(ly.qkv, self.h.ptr, T, self.qkv.ptr)
            _check(L.lbd_qkv_rope(self.qkv.ptr, None if ly.qkv_bias is None else ly.qkv_bias.ptr, T, H, KV, D,
                                  self.cos.ptr, self.sin.ptr, self.pos.ptr, cfg.max_position,
                                  cache.k[li].ptr, cache.v[li].ptr, cache.capacity, s), "qkv rope")
            _check(L.lbd_attention(self.qkv.ptr, qkvw, cache.k[li].ptr, cache.v[li].ptr, T, H, KV, D,
                                   self.pos.ptr, cache.capacity, self.att.ptr, s), "attention")
            self._linear(ly.o, self.att.ptr, T, self.o.ptr)
            _check(L.lbd_add(self.x.ptr, self.o.ptr, T * h, s), "add")
            _check(L.lbd_rmsnorm(self.x.ptr, ly.ln2.ptr, T, h, cfg.rms_norm_eps, self.h.ptr, s), "rmsnorm")
            self._linear(ly.gate_up, self.h.ptr, T, self.gu.ptr)
            _check(L.lbd_swiglu_pairs(self.gu.ptr, T, I, self.m.ptr, s), "swiglu")
            self._linear(ly.down, self.m.ptr, T, self.o.ptr)
            _check(L.lbd_add(self.x.ptr, self.o.ptr, T * h, s), "add")
        _check(L.lbd_rmsnorm(self.x.ptr, self.norm.ptr, T, h, cfg.rms_norm_eps, self.h.ptr, s), "rmsnorm")
        if logits == "none":
            return
        if logits == "last":
            self._linear(self.lm_head, self.h.ptr + (T - 1) * h * 4, 1, self.logits.ptr)
            if argmax_hist:
                hist = self.hist.ptr if self.hist is not None else None
                n = self.hist.nbytes // 4 if self.hist is not None else 0
                _check(L.lbd_argmax(self.logits.ptr, cfg.vocab_size, self.tok.ptr, self.pos.ptr, T, hist, n, s),
                       "argmax")
        else:
            self._linear(self.lm_head, self.h.ptr, T, self.all_logits.ptr)

    def _tokens(self, tokens) -> np.ndarray:
        """int32 ids as numpy indexing reads them: negatives count from the end,
        anything outside [-vocab, vocab) raises IndexError (src/lowbit/model.py:398)."""
        t = np.asarray(tokens, np.int64).reshape(-1)
        if t.size == 0:
            raise ValueError("no tokens")
        V = self.cfg.vocab_size
        if (t.min() < -V or t.max() >= V):
            raise IndexError(f"token id out of range for a vocabulary of {V}")
        return np.ascontiguousarray(np.where(t < 0, t + V, t), np.int32)

    def _set_pos(self, p: int):
        a = np.array([p], np.int32)
        _check(self.L.lb_memcpy_h2d(self.pos.ptr, a.ctypes.data, 4), "pos upload")

    def _sync(self):
        _check(self.L.lb_stream_synchronize(self.stream), "synchronize")

    # ------------------------------------------------------------ public calls

    def forward(self, tokens, cache: KVCache | None = None, logits: str = "last") -> np.ndarray:
        """Run tokens [T] at positions cache.length.. (0 without a cache); logits="last"
        returns [V], "all" [T, V], "none" the final hidden states [T, hidden]
        (src/lowbit/model.py:380-435)."""
        cfg = self.cfg
        tokens = self._tokens(tokens)
        T = int(tokens.shape[0])
        own = cache is None
        cache = cache or self.new_cache(T)
        pos = cache.length
        if pos + T > cache.capacity:
            raise ValueError(f"KV cache full ({pos}+{T} > {cache.capacity})")
        if T > self.tmax:
            self._alloc(T)
            self.tok = _buf(4 * T)
        self._sync()
        _check(self.L.lb_memcpy_h2d(self.tok.ptr, tokens.ctypes.data, 4 * T), "token upload")
        self._set_pos(pos)
        if logits == "all":
            self.all_logits = _buf(T * cfg.vocab_size * 4)
        self._step(T, cache, logits, argmax_hist=False)
        self._sync()
        if not own:
            cache.length = pos + T
        if logits == "last":
            return self.logits.to_array((cfg.vocab_size,), np.float32)
        if logits == "all":
            return self.all_logits.to_array((T, cfg.vocab_size), np.float32)
        return self.h.to_array((T, cfg.hidden_size), np.float32)

    def generate(self, prompt, n_new: int, cache: KVCache | None = None, timings: dict | None = None,
                 graph: bool = True) -> list[int]:
        """Greedy decoding: prefill the prompt, then n_new tokens one at a time
        (src/lowbit/model.py:437-458): n_new tokens come out of one prefill and
        n_new - 1 decode forwards. The argmax runs on the device and feeds the next
        step's embedding lookup; the decode steps replay one recorded HIP graph
        (graph=False launches them one by one). timings["decode_s"] includes the
        recording of the graph."""
        prompt = self._tokens(prompt)
        T = len(prompt)
        steps = max(0, n_new - 1)
        cache = cache or self.new_cache(T + n_new)
        start = cache.length
        if start + T + steps > cache.capacity:
            raise ValueError(f"KV cache full ({start}+{T}+{steps} > {cache.capacity})")
        if T > self.tmax:
            self._alloc(T)
            self.tok = _buf(4 * T)
        # hist[p] = the token generated at position p - 1; the last one lands at start + T + steps
        self.hist = _buf(4 * (cache.capacity + 1))
        L = self.L
        self._sync()
        _check(L.lb_memcpy_h2d(self.tok.ptr, prompt.ctypes.data, 4 * T), "token upload")
        self._set_pos(start)
        t0 = time.perf_counter()
        self._step(T, cache, "last", argmax_hist=True)
        self._sync()
        t1 = time.perf_counter()
        if steps and graph:
            # every linear of a one-token step takes the decode kernels (M = 1),
            # which allocate nothing, so the step can be recorded
            s, ex = self.stream, C.c_void_p()
            _check(L.lb_stream_begin_capture(s), "begin capture")
            try:
                self._step(1, cache, "last", argmax_hist=True)
            finally:
                _check(L.lb_stream_end_capture(s, C.byref(ex)), "end capture")
            try:
                for _ in range(steps):
                    _check(L.lb_graph_launch(ex.value, s), "graph launch")
                self._sync()
            finally:
                L.lb_graph_destroy(ex.value)
        else:
            for _ in range(steps):
                self._step(1, cache, "last", argmax_hist=True)
            self._sync()
        t2 = time.perf_counter()
        cache.length = start + T + steps
        out = self.hist.to_array((cache.capacity + 1,), np.int32)[start + T:start + T + n_new]
        if timings is not None:
            timings["prefill_s"] = t1 - t0
            timings["decode_s"] = t2 - t1
            timings["decode_forwards"] = steps
        return [int(v) for v in out]
