"""A Qwen2 pipeline stage in NumPy whose projections run through the
reference's C-ABI -- the caller the reference puts in front of
libq4gemv.so (hetero/cpu_model.py:309-368), rebuilt here to drive the
MI355X library as a drop-in.

Given the same weights and a library with the reference's q4_gemv /
q4_dequant semantics, a stage produces the reference path's logits bit for
bit: the projections are the library's (bit-identical to the reference
kernel), and every NumPy expression whose evaluation order fixes the result
-- the RMSNorm, the RoPE table and rotation, the attention's einsum and
softmax, SiLU -- is evaluated as the reference evaluates it (each cites its
line).  The structure around them is this module's own: a stage holds one
parameter record per layer and runs the layer as plain functions, and the
KV cache is allocated once at a fixed capacity (it doubles if a caller goes
past it) with a storage dtype of the caller's choice -- the reference's
cache is float32 and grows in 256-position steps (hetero/cpu_model.py:207-230);
the Qwen2.5-7B decode benchmark stores float16.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence

import numpy as np

from .qlinear import QLinear, dequantize


# ---- the expressions that fix the bits --------------------------------------

def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """hetero/cpu_model.py:164-166, evaluated in the same order."""
    x = x.astype(np.float32)
    return x * (1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)) * w


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """SiLU(g) * u as hetero/cpu_model.py:169-170 and :291-292 evaluate it."""
    return g / (1.0 + np.exp(-g, dtype=np.float32)) * u


def rope_tables(head_dim: int, theta: float, n: int):
    """cos/sin [n, head_dim/2] of positions 0..n-1, built with the reference's
    float32 expressions (hetero/cpu_model.py:180-193)."""
    half = head_dim // 2
    inv = theta ** (-np.arange(0, half, dtype=np.float32) * 2.0 / head_dim)
    ang = np.arange(n, dtype=np.float32)[:, None] * inv[None, :]
    return np.cos(ang), np.sin(ang)


def rotate_half_split(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Non-traditional rotary embedding of x [B, H, L, D] at the L positions
    whose rows cos/sin [L, D/2] hold (hetero/cpu_model.py:195-204)."""
    h = x.shape[-1] // 2
    a, b = x[..., :h], x[..., h:]
    y = np.empty_like(x)
    np.subtract(a * cos, b * sin, out=y[..., :h])
    np.add(a * sin, b * cos, out=y[..., h:])
    return y


def gqa_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, causal: bool) -> np.ndarray:
    """Softmax attention of q [B, H, L, D] over k, v [B, KH, S, D], query
    head h reading kv head h // (H / KH), with the reference's einsum
    contractions and max-subtracted softmax (hetero/cpu_model.py:233-252)."""
    B, H, L, D = q.shape
    KH, S = k.shape[1], k.shape[2]
    qg = q.reshape(B, KH, H // KH, L, D)
    s = np.einsum("bkgld,bksd->bkgls", qg, k, optimize=True) * scale
    if causal and L > 1:
        visible = np.arange(S)[None, :] <= (np.arange(L)[:, None] + (S - L))
        s = np.where(visible, s, -np.inf)
    s -= s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bkgls,bksd->bkgld", p, v, optimize=True).reshape(B, H, L, D)


# ---- KV cache ----------------------------------------------------------------

class KVCache:
    """Keys and values of one layer, [1, n_kv, capacity, head_dim] in the
    storage dtype, filled up to `offset`.  update_and_fetch(k, v) appends
    L positions and returns views of every position held -- the interface the
    reference's attention calls (hetero/cpu_model.py:216-230)."""

    def __init__(self, n_kv: int, head_dim: int, capacity: int, dtype=np.float32):
        self.dtype = np.dtype(dtype)
        self.keys = np.zeros((1, n_kv, max(int(capacity), 1), head_dim), self.dtype)
        self.values = np.zeros_like(self.keys)
        self.offset = 0

    @classmethod
    def prefilled(cls, k_ctx: np.ndarray, v_ctx: np.ndarray, extra: int, dtype=np.float32) -> "KVCache":
        """A cache holding context k_ctx / v_ctx [n_kv, S, head_dim] with room
        for `extra` more positions."""
        n_kv, s, d = k_ctx.shape
        c = cls(n_kv, d, s + extra, dtype)
        c.keys[0, :, :s] = k_ctx
        c.values[0, :, :s] = v_ctx
        c.offset = s
        return c

    def update_and_fetch(self, k: np.ndarray, v: np.ndarray):
        n = k.shape[2]
        end = self.offset + n
        if end > self.keys.shape[2]:
            cap = max(end, 2 * self.keys.shape[2])
            for name in ("keys", "values"):
                old = getattr(self, name)
                new = np.zeros(old.shape[:2] + (cap, old.shape[3]), self.dtype)
                new[:, :, :self.offset] = old[:, :, :self.offset]
                setattr(self, name, new)
        self.keys[:, :, self.offset:end] = k
        self.values[:, :, self.offset:end] = v
        self.offset = end
        return self.keys[:, :, :end], self.values[:, :, :end]


# ---- the stage ---------------------------------------------------------------

@dataclass
class LayerParams:
    """One decoder layer: its seven projections and two norm weights, read
    from the reference's tensor names (hetero/cpu_model.py:263-266, :286-289,
    :298-299)."""
    q: QLinear
    k: QLinear
    v: QLinear
    o: QLinear
    gate: QLinear
    up: QLinear
    down: QLinear
    in_norm: np.ndarray
    post_norm: np.ndarray


class Stage:
    """Embedding (if owned), decoder layers [start, end), final norm and
    vocabulary head (if owned) -- the reference's NumPy Stage
    (hetero/cpu_model.py:309-368) with the shard spec as plain arguments.
    `lib` is any library with the reference's ABI (libq4gemv.so when None)."""

    def __init__(self, cfg: dict, w: Dict[str, np.ndarray], start: int = 0, end: Optional[int] = None,
                 embed: bool = True, head: bool = True, lib=None):
        if cfg.get("model_type") != "qwen2" or "quantization" not in cfg:
            raise NotImplementedError("quantised qwen2 only")
        self.cfg = cfg
        self.gs, self.bits = cfg["quantization"]["group_size"], cfg["quantization"]["bits"]
        self.eps = cfg["rms_norm_eps"]
        self.n_heads, self.n_kv = cfg["num_attention_heads"], cfg["num_key_value_heads"]
        self.head_dim = cfg["hidden_size"] // self.n_heads
        self.scale = self.head_dim ** -0.5
        self.has_embed, self.has_head = embed, head
        end = cfg["num_hidden_layers"] if end is None else end

        def proj(name):
            return QLinear(w[f"{name}.weight"], w[f"{name}.scales"], w[f"{name}.biases"], w.get(f"{name}.bias"),
                           self.gs, self.bits, lib)

        self.layers: List[LayerParams] = []
        for i in range(start, end):
            p = f"model.layers.{i}"
            a, m = f"{p}.self_attn", f"{p}.mlp"
            self.layers.append(LayerParams(
                q=proj(f"{a}.q_proj"), k=proj(f"{a}.k_proj"), v=proj(f"{a}.v_proj"), o=proj(f"{a}.o_proj"),
                gate=proj(f"{m}.gate_proj"), up=proj(f"{m}.up_proj"), down=proj(f"{m}.down_proj"),
                in_norm=np.asarray(w[f"{p}.input_layernorm.weight"]).astype(np.float32),
                post_norm=np.asarray(w[f"{p}.post_attention_layernorm.weight"]).astype(np.float32)))
        tied = bool(cfg.get("tie_word_embeddings", False))
        self.table = None
        if embed or (tied and head):
            self.table = tuple(w[f"model.embed_tokens.{t}"] for t in ("weight", "scales", "biases"))
        if head:
            self.final_norm = np.asarray(w["model.norm.weight"]).astype(np.float32)
            self.lm_head = (QLinear(*self.table, None, self.gs, self.bits, lib) if tied else proj("lm_head"))
        self._cos = self._sin = None

    # -- pieces -------------------------------------------------------------
    def embed(self, ids: np.ndarray) -> np.ndarray:
        """Dequantised embedding rows of token ids (hetero/cpu_model.py:334-338)."""
        ids = np.asarray(ids)
        flat = ids.reshape(-1)
        w, s, b = self.table
        return dequantize(w[flat], s[flat], b[flat], self.gs, self.bits).reshape(ids.shape + (-1,))

    def _rope(self, upto: int):
        if self._cos is None or self._cos.shape[0] < upto:
            self._cos, self._sin = rope_tables(self.head_dim, self.cfg["rope_theta"], max(upto, 256))
        return self._cos, self._sin

    def _attention(self, lp: LayerParams, x: np.ndarray, cache: Optional[KVCache], causal: bool) -> np.ndarray:
        B, L, _ = x.shape
        heads = lambda y, n: y.reshape(B, L, n, self.head_dim).transpose(0, 2, 1, 3)
        q, k, v = heads(lp.q(x), self.n_heads), heads(lp.k(x), self.n_kv), heads(lp.v(x), self.n_kv)
        off = 0 if cache is None else cache.offset
        cos, sin = self._rope(off + L)
        q = rotate_half_split(q, cos[off:off + L], sin[off:off + L])
        k = rotate_half_split(k, cos[off:off + L], sin[off:off + L])
        if cache is not None:
            k, v = cache.update_and_fetch(k, v)
        o = gqa_attention(q, k, v, self.scale, causal)
        return lp.o(o.transpose(0, 2, 1, 3).reshape(B, L, -1))

    def _layer(self, lp: LayerParams, x: np.ndarray, cache: Optional[KVCache], causal: bool) -> np.ndarray:
        # hetero/cpu_model.py:304-306: two residual blocks, each on the RMSNorm of the stream
        x = x + self._attention(lp, rms_norm(x, lp.in_norm, self.eps), cache, causal)
        h = rms_norm(x, lp.post_norm, self.eps)
        return x + lp.down(silu_mul(lp.gate(h), lp.up(h)))

    # -- calls ----------------------------------------------------------------
    def new_caches(self, context_k: Optional[Sequence[np.ndarray]] = None,
                   context_v: Optional[Sequence[np.ndarray]] = None, extra: int = 256,
                   dtype=np.float32) -> List[KVCache]:
        """One cache per layer: empty, or holding the given context
        [n_kv, S, head_dim] per layer, with room for `extra` positions."""
        if context_k is None:
            return [KVCache(self.n_kv, self.head_dim, extra, dtype) for _ in self.layers]
        return [KVCache.prefilled(k, v, extra, dtype) for k, v in zip(context_k, context_v)]

    def __call__(self, x, caches: Optional[List[KVCache]] = None, apply_head: bool = True,
                 last_only: bool = False) -> np.ndarray:
        """Token ids [B, L] (when the stage owns the embedding) or hidden
        states [B, L, hidden] -> hidden states, or logits when the stage owns
        the head and apply_head (hetero/cpu_model.py:357-368)."""
        h = self.embed(x) if self.has_embed else x
        h = np.asarray(h, dtype=np.float32)
        causal = h.shape[1] > 1
        for i, lp in enumerate(self.layers):
            h = self._layer(lp, h, None if caches is None else caches[i], causal)
        if not (self.has_head and apply_head):
            return h
        if last_only:
            h = h[:, -1:, :]
        return self.lm_head(rms_norm(h, self.final_norm, self.eps))


def greedy(logits) -> int:
    """The first index of the largest logit: NumpyBackend.sample at
    temperature 0 (hetero/backends.py:106-109)."""
    return int(np.asarray(logits, dtype=np.float32).reshape(-1).argmax())
