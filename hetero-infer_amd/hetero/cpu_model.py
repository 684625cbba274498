"""The NumPy Qwen2 stage of the reference, driving libq4gemv.so (the gfx950
library) through the reference's own C-ABI.

This mirrors hetero/cpu_model.py of the reference module by module -- same
names, same argument meaning, same numerics -- so that a caller that loads
<package parent>/kernel/libq4gemv.so with ctypes gets the MI355X library as a
drop-in (hetero/cpu_model.py:33-45).  Every projection goes through
q4_gemv / q4_dequant exactly as the reference makes those calls
(hetero/cpu_model.py:109-136); because libq4gemv.so reproduces the x86
kernel bit for bit, a Stage here produces the same logits as the same Stage
running on the reference kernel.

Differences from the reference, all deliberate:
  * there is no silent fp32 fallback: a missing libq4gemv.so raises (the
    reference expands weights to fp32, hetero/cpu_model.py:100-107);
  * QLinear may be given any library with the q4_gemv/q4_dequant ABI (the
    tests run the same Stage on the reference kernel compiled from source);
  * rows 2..16 of a QLinear call go through q4_gemv_batched when the library
    has it -- the result is row-for-row identical to the reference's loop
    (hetero/cpu_model.py:149-153) with the weights read once;
  * KVCache takes a storage dtype (the reference stores float32,
    hetero/cpu_model.py:221-222; the Qwen2.5-7B decode benchmark stores
    float16).
"""
from __future__ import annotations

import os
from typing import Dict, List, Optional

import numpy as np

from . import q4

HEAD_BLOCK = 512               # rows dequantised at a time on the GEMM path (cpu_model.py:26)
GEMV_ROWS_MAX = int(os.environ.get("HETERO_GEMV_ROWS", "16"))   # cpu_model.py:30
NTHREADS = int(os.environ.get("HETERO_THREADS", "0")) or (os.cpu_count() or 2)   # :60-64


def _load_kernel():
    """libq4gemv.so from <package parent>/kernel (cpu_model.py:33-45); raises if absent."""
    return q4.load()


KERNEL = None


def kernel():
    global KERNEL
    if KERNEL is None:
        KERNEL = _load_kernel()
    return KERNEL


def dequantize(w_u32: np.ndarray, scales: np.ndarray, biases: np.ndarray, group_size: int,
               bits: int, out: Optional[np.ndarray] = None) -> np.ndarray:
    """MLX layout unpack, q*scale + bias (cpu_model.py:67-81)."""
    per = 32 // bits
    mask = (1 << bits) - 1
    shifts = np.arange(per, dtype=np.uint32) * bits
    q = ((w_u32[..., None] >> shifts) & mask).reshape(w_u32.shape[0], -1).astype(np.float32)
    s = scales.astype(np.float32).repeat(group_size, axis=1)
    b = biases.astype(np.float32).repeat(group_size, axis=1)
    if out is not None:
        np.multiply(q, s, out=out)
        np.add(out, b, out=out)
        return out
    return q * s + b


class QLinear:
    """A 4-bit projection; GEMV for decode, dequant + BLAS for prompts
    (cpu_model.py:84-158)."""

    def __init__(self, w, scales, biases, bias, group_size, bits, lib=None):
        if bits != 4:
            raise NotImplementedError("libq4gemv.so handles 4-bit weights")
        self.lib = lib if lib is not None else kernel()
        self.bias = None if bias is None else np.asarray(bias, np.float32)
        self.group_size, self.bits = group_size, bits
        self.n_out, self.n_in = w.shape[0], w.shape[1] * (32 // bits)
        self.w = np.ascontiguousarray(w)
        self.scales = np.ascontiguousarray(scales, dtype=np.float16)
        self.biases = np.ascontiguousarray(biases, dtype=np.float16)
        self._batched = getattr(self.lib, "q4_gemv_batched", None)

    def _gemv(self, x: np.ndarray) -> np.ndarray:           # cpu_model.py:109-117
        xc = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(self.n_out, dtype=np.float32)
        rc = self.lib.q4_gemv(self.w.ctypes.data, self.scales.ctypes.data, self.biases.ctypes.data,
                              xc.ctypes.data, out.ctypes.data, self.n_out, self.n_in,
                              self.group_size, NTHREADS)
        if rc != 0:
            raise RuntimeError(f"q4_gemv failed with {rc}")
        return out

    def _gemv_rows(self, flat: np.ndarray) -> np.ndarray:
        """Rows 2..GEMV_ROWS_MAX: one batched call, each row == q4_gemv(row)."""
        xc = np.ascontiguousarray(flat, dtype=np.float32)
        out = np.empty((xc.shape[0], self.n_out), dtype=np.float32)
        rc = self._batched(self.w.ctypes.data, self.scales.ctypes.data, self.biases.ctypes.data,
                           xc.ctypes.data, out.ctypes.data, xc.shape[0], self.n_out, self.n_in,
                           self.group_size, NTHREADS)
        if rc != 0:
            raise RuntimeError(f"q4_gemv_batched failed with {rc}")
        return out

    def _gemm(self, flat: np.ndarray) -> np.ndarray:         # cpu_model.py:119-136
        out = np.empty((flat.shape[0], self.n_out), dtype=np.float32)
        buf = self._buf(HEAD_BLOCK)
        for lo in range(0, self.n_out, HEAD_BLOCK):
            hi = min(lo + HEAD_BLOCK, self.n_out)
            rc = self.lib.q4_dequant(self.w.ctypes.data, self.scales.ctypes.data,
                                     self.biases.ctypes.data, buf.ctypes.data, lo, hi, self.n_in,
                                     self.group_size, NTHREADS)
            if rc != 0:
                raise RuntimeError(f"q4_dequant failed with {rc}")
            out[:, lo:hi] = flat @ buf[:hi - lo].T
        return out

    def _buf(self, rows: int) -> np.ndarray:
        b = getattr(self, "_scratch", None)
        if b is None or b.shape != (rows, self.n_in):
            b = np.empty((rows, self.n_in), dtype=np.float32)
            self._scratch = b
        return b

    def __call__(self, x: np.ndarray) -> np.ndarray:         # cpu_model.py:145-158
        flat = np.asarray(x, dtype=np.float32).reshape(-1, x.shape[-1])
        if flat.shape[0] <= GEMV_ROWS_MAX:
            if flat.shape[0] > 1 and self._batched is not None:
                out = self._gemv_rows(flat)
            else:
                out = np.stack([self._gemv(flat[r]) for r in range(flat.shape[0])])
        else:
            out = self._gemm(flat)
        if self.bias is not None:
            out = out + self.bias
        return out.reshape(*x.shape[:-1], self.n_out)


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:   # cpu_model.py:164-166
    x = x.astype(np.float32)
    return x * (1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)) * w


def silu(x: np.ndarray) -> np.ndarray:                                  # cpu_model.py:169-170
    return x / (1.0 + np.exp(-x, dtype=np.float32))


class RoPE:
    """Non-traditional (half-split) rotary embedding with a cached fp32
    cos/sin table (cpu_model.py:173-204)."""

    def __init__(self, dims: int, base: float):
        self.half = dims // 2
        self.inv = base ** (-np.arange(0, self.half, dtype=np.float32) * 2.0 / dims)
        self._n = 0
        self._cos = self._sin = None

    def _table(self, upto: int):
        if self._n < upto:
            n = max(upto, 256, self._n * 2)
            ang = np.arange(n, dtype=np.float32)[:, None] * self.inv[None, :]
            self._cos, self._sin = np.cos(ang), np.sin(ang)
            self._n = n
        return self._cos, self._sin

    def __call__(self, x: np.ndarray, offset: int = 0) -> np.ndarray:
        L = x.shape[2]
        cos, sin = self._table(offset + L)
        cos, sin = cos[offset:offset + L], sin[offset:offset + L]
        x1, x2 = x[..., :self.half], x[..., self.half:]
        out = np.empty_like(x)
        np.subtract(x1 * cos, x2 * sin, out=out[..., :self.half])
        np.add(x1 * sin, x2 * cos, out=out[..., self.half:])
        return out


class KVCache:
    """Growing K/V store, STEP-position growth (cpu_model.py:207-230); `dtype`
    is the storage type (float32 in the reference)."""

    STEP = 256

    def __init__(self, dtype=np.float32):
        self.keys = self.values = None
        self.offset = 0
        self.dtype = np.dtype(dtype)

    def fill(self, k: np.ndarray, v: np.ndarray) -> None:
        """Start from a given context [B, KH, S, D] (e.g. a prefilled prompt)."""
        self.keys = self.values = None
        self.offset = 0
        self.update_and_fetch(k, v)

    def update_and_fetch(self, k, v):
        prev, L = self.offset, k.shape[2]
        if self.keys is None or prev + L > self.keys.shape[2]:
            B, H, _, D = k.shape
            grow = ((L + self.STEP - 1) // self.STEP) * self.STEP
            nk = np.zeros((B, H, prev + grow, D), self.dtype)
            nv = np.zeros((B, H, prev + grow, D), self.dtype)
            if self.keys is not None:
                nk[..., :prev, :] = self.keys[..., :prev, :]
                nv[..., :prev, :] = self.values[..., :prev, :]
            self.keys, self.values = nk, nv
        self.keys[..., prev:prev + L, :] = k
        self.values[..., prev:prev + L, :] = v
        self.offset = prev + L
        return self.keys[..., :self.offset, :], self.values[..., :self.offset, :]


def sdpa(q, k, v, scale, causal):
    """GQA attention by reshaping q to (kv-head, group) (cpu_model.py:233-252)."""
    B, H, L, D = q.shape
    KH, S = k.shape[1], k.shape[2]
    G = H // KH
    q5 = q.reshape(B, KH, G, L, D)
    s = np.einsum("bkgld,bksd->bkgls", q5, k, optimize=True) * scale
    if causal and L > 1:
        i = np.arange(L)[:, None] + (S - L)
        s = np.where(np.arange(S)[None, :] <= i, s, -np.inf)
    s -= s.max(-1, keepdims=True)
    e = np.exp(s)
    e /= e.sum(-1, keepdims=True)
    o = np.einsum("bkgls,bksd->bkgld", e, v, optimize=True)
    return o.reshape(B, H, L, D)


class Attention:                                                        # cpu_model.py:255-280
    def __init__(self, cfg, w, p, lib=None):
        dim = cfg["hidden_size"]
        self.n_heads = cfg["num_attention_heads"]
        self.n_kv = cfg["num_key_value_heads"]
        self.head_dim = dim // self.n_heads
        self.scale = self.head_dim ** -0.5
        gs, bits = cfg["quantization"]["group_size"], cfg["quantization"]["bits"]
        for proj in ("q_proj", "k_proj", "v_proj", "o_proj"):
            q = f"{p}.self_attn.{proj}"
            setattr(self, proj, QLinear(w[f"{q}.weight"], w[f"{q}.scales"], w[f"{q}.biases"],
                                        w.get(f"{q}.bias"), gs, bits, lib))
        self.rope = RoPE(self.head_dim, cfg["rope_theta"])

    def __call__(self, x, cache, causal):
        B, L, _ = x.shape
        q = self.q_proj(x).reshape(B, L, self.n_heads, -1).transpose(0, 2, 1, 3)
        k = self.k_proj(x).reshape(B, L, self.n_kv, -1).transpose(0, 2, 1, 3)
        v = self.v_proj(x).reshape(B, L, self.n_kv, -1).transpose(0, 2, 1, 3)
        offset = cache.offset if cache is not None else 0
        q = self.rope(q, offset)
        k = self.rope(k, offset)
        if cache is not None:
            k, v = cache.update_and_fetch(k, v)
        o = sdpa(q, k, v, self.scale, causal)
        return self.o_proj(o.transpose(0, 2, 1, 3).reshape(B, L, -1))


class MLP:                                                              # cpu_model.py:283-292
    def __init__(self, cfg, w, p, lib=None):
        gs, bits = cfg["quantization"]["group_size"], cfg["quantization"]["bits"]
        for proj in ("gate_proj", "up_proj", "down_proj"):
            q = f"{p}.mlp.{proj}"
            setattr(self, proj, QLinear(w[f"{q}.weight"], w[f"{q}.scales"], w[f"{q}.biases"],
                                        w.get(f"{q}.bias"), gs, bits, lib))

    def __call__(self, x):
        return self.down_proj(silu(self.gate_proj(x)) * self.up_proj(x))


class DecoderLayer:                                                     # cpu_model.py:295-306
    def __init__(self, cfg, w, idx, lib=None):
        p = f"model.layers.{idx}"
        self.eps = cfg["rms_norm_eps"]
        self.self_attn = Attention(cfg, w, p, lib)
        self.mlp = MLP(cfg, w, p, lib)
        self.in_w = w[f"{p}.input_layernorm.weight"].astype(np.float32)
        self.post_w = w[f"{p}.post_attention_layernorm.weight"].astype(np.float32)

    def __call__(self, x, cache, causal):
        x = x + self.self_attn(rms_norm(x, self.in_w, self.eps), cache, causal)
        return x + self.mlp(rms_norm(x, self.post_w, self.eps))


class Stage:
    """Embedding (if owned), layers [start, end), final norm + lm_head (if
    owned) -- cpu_model.py:309-368, with the shard spec as plain arguments."""

    def __init__(self, cfg: dict, w: Dict[str, np.ndarray], start: int = 0, end: Optional[int] = None,
                 embed: bool = True, head: bool = True, lib=None):
        if cfg.get("model_type") != "qwen2" or "quantization" not in cfg:
            raise NotImplementedError("quantised qwen2 only")
        end = cfg["num_hidden_layers"] if end is None else end
        self.cfg, self.quant = cfg, cfg["quantization"]
        self.has_embed, self.has_head = embed, head
        gs, bits = self.quant["group_size"], self.quant["bits"]
        tied = bool(cfg.get("tie_word_embeddings", False))
        if embed or (tied and head):
            self.embed_w = w["model.embed_tokens.weight"]
            self.embed_s = w["model.embed_tokens.scales"]
            self.embed_b = w["model.embed_tokens.biases"]
        self.layers = [DecoderLayer(cfg, w, i, lib) for i in range(start, end)]
        if head:
            self.norm_w = w["model.norm.weight"].astype(np.float32)
            if tied:
                self.lm_head = QLinear(self.embed_w, self.embed_s, self.embed_b, None, gs, bits, lib)
            else:
                self.lm_head = QLinear(w["lm_head.weight"], w["lm_head.scales"], w["lm_head.biases"],
                                       w.get("lm_head.bias"), gs, bits, lib)

    def embed(self, ids: np.ndarray) -> np.ndarray:                     # cpu_model.py:334-338
        flat = ids.reshape(-1)
        rows = dequantize(self.embed_w[flat], self.embed_s[flat], self.embed_b[flat],
                          self.quant["group_size"], self.quant["bits"])
        return rows.reshape(*ids.shape, -1)

    def __call__(self, x, caches=None, apply_head=True, last_only=False):
        if self.has_embed:
            x = self.embed(np.asarray(x))
        x = np.asarray(x, dtype=np.float32)
        causal = x.shape[1] > 1
        for i, layer in enumerate(self.layers):
            x = layer(x, None if caches is None else caches[i], causal)
        if self.has_head and apply_head:
            if last_only:
                x = x[:, -1:, :]
            x = self.lm_head(rms_norm(x, self.norm_w, self.cfg["rms_norm_eps"]))
        return x


def greedy(logits) -> int:
    """NumpyBackend.sample at temperature 0 (hetero/backends.py:106-109)."""
    return int(np.asarray(logits, dtype=np.float32).reshape(-1).argmax())


def qwen2_7b_config(layers: int = 28) -> dict:
    """Qwen2.5-7B architecture with MLX 4-bit group-64 quantisation."""
    return {"model_type": "qwen2", "hidden_size": 3584, "intermediate_size": 18944,
            "num_hidden_layers": layers, "num_attention_heads": 28, "num_key_value_heads": 4,
            "rms_norm_eps": 1e-6, "rope_theta": 1e6, "vocab_size": 152064,
            "tie_word_embeddings": False, "quantization": {"group_size": 64, "bits": 4}}


def synthetic_weights(cfg: dict, seed: int = 0) -> Dict[str, np.ndarray]:
    """Random-init 4-bit Qwen2 weights under the reference's tensor names
    (cpu_model.py:263-266, :286-289, :320-332)."""
    from . import synth
    gs = cfg["quantization"]["group_size"]
    h, inter, v = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
    kvd = h // cfg["num_attention_heads"] * cfg["num_key_value_heads"]
    w: Dict[str, np.ndarray] = {}

    def lin(name, n_out, n_in, bias=False):
        ww, s, b = synth.qlinear(seed, n_out, n_in, gs, tag=name)
        w[f"{name}.weight"], w[f"{name}.scales"], w[f"{name}.biases"] = ww, s, b
        if bias:
            w[f"{name}.bias"] = (synth.normal(seed, name + ".bias", n_out) * 0.02).astype(np.float32)

    lin("model.embed_tokens", v, h)
    for i in range(cfg["num_hidden_layers"]):
        p = f"model.layers.{i}"
        lin(f"{p}.self_attn.q_proj", h, h, bias=True)
        lin(f"{p}.self_attn.k_proj", kvd, h, bias=True)
        lin(f"{p}.self_attn.v_proj", kvd, h, bias=True)
        lin(f"{p}.self_attn.o_proj", h, h)
        lin(f"{p}.mlp.gate_proj", inter, h)
        lin(f"{p}.mlp.up_proj", inter, h)
        lin(f"{p}.mlp.down_proj", h, inter)
        for nrm in ("input_layernorm", "post_attention_layernorm"):
            w[f"{p}.{nrm}.weight"] = (1.0 + synth.normal(seed, f"{p}.{nrm}", h) * 0.02).astype(np.float32)
    w["model.norm.weight"] = (1.0 + synth.normal(seed, "model.norm", h) * 0.02).astype(np.float32)
    lin("lm_head", v, h)
    return w


def synthetic_kv(cfg: dict, context: int, seed: int = 0, dtype=np.float16) -> List[KVCache]:
    """One KVCache per layer pre-filled with `context` seeded N(0,1) positions."""
    from . import synth
    kh = cfg["num_key_value_heads"]
    d = cfg["hidden_size"] // cfg["num_attention_heads"]
    caches = []
    for i in range(cfg["num_hidden_layers"]):
        k = synth.normal(seed, f"kv.{i}.k", kh * context * d).astype(np.float32).reshape(1, kh, context, d)
        vv = synth.normal(seed, f"kv.{i}.v", kh * context * d).astype(np.float32).reshape(1, kh, context, d)
        c = KVCache(dtype)
        c.fill(k.astype(dtype), vv.astype(dtype))
        caches.append(c)
    return caches
