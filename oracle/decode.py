"""Decode-step oracle of the Qwen2 stage -- TEST INFRASTRUCTURE ONLY.

Only tests/, tests/golden/ and bench.py's cpu_baseline leg use this module;
the product (hetero-infer_amd/) never imports it.

It restates, for batch 1, the reference's NumPy stage
(hetero/cpu_model.py:164-368) -- one token per decode step, or a prompt
chunk of L tokens with causal attention -- with every projection going
through a library with the reference's C-ABI -- oracle/_ref, the reference
kernel/q4gemv.c compiled from source, for the fixtures.  Up to 16 rows a
projection is q4_gemv per row, above that the reference's prompt
contraction: q4_dequant of 512-row blocks, each multiplied by BLAS
(QLinear, hetero/cpu_model.py:119-158).  So its logits are
the reference path's: the GEMVs are the reference kernel's, and each NumPy
expression whose evaluation order fixes the bits is evaluated as the
reference evaluates it (cited per line).  The cache holds the context in a
storage dtype of the caller's choice (fp16 for the Qwen2.5-7B decode
workload; the reference stores float32, hetero/cpu_model.py:221-222).

Pinned by tests/test_oracle_decode.py against a float64 decode written from
the textbook definitions (explicit per-head loops, softmax, rotation angles
in float64), with planted mistakes that the comparison must catch -- for
prompts too: in exact arithmetic a causal prompt gives at its last row the
logits of decoding its tokens one by one -- and by the GEMV golden vectors
for the projections themselves.

`gemm_bf16=True` rounds both operands of the prompt contraction to bf16
(round to nearest even) before the fp32 product: the operands of the
device's matrix-core prefill GEMM, so that the tests can measure how far
that rounding alone moves the logits.
"""
from __future__ import annotations

from typing import Dict, List

import numpy as np


def _norm(x, w, eps):
    # hetero/cpu_model.py:164-166
    x = x.astype(np.float32)
    return x * (1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)) * w


def _rope(x, cos, sin):
    # hetero/cpu_model.py:199-204 (non-traditional: first and second halves)
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    out = np.empty_like(x)
    np.subtract(x1 * cos, x2 * sin, out=out[..., :half])
    np.add(x1 * sin, x2 * cos, out=out[..., half:])
    return out


def _sdpa(q, k, v, scale, causal=False):
    # hetero/cpu_model.py:233-252; the mask of :244-246 when causal and L > 1
    B, H, L, D = q.shape
    KH, S = k.shape[1], k.shape[2]
    q5 = q.reshape(B, KH, H // KH, L, D)
    s = np.einsum("bkgld,bksd->bkgls", q5, k, optimize=True) * scale
    if causal and L > 1:
        i = np.arange(L)[:, None] + (S - L)
        s = np.where(np.arange(S)[None, :] <= i, s, -np.inf)
    s -= s.max(-1, keepdims=True)
    e = np.exp(s)
    e /= e.sum(-1, keepdims=True)
    o = np.einsum("bkgls,bksd->bkgld", e, v, optimize=True)
    return o.reshape(B, H, L, D)


def bf16_round(a: np.ndarray) -> np.ndarray:
    """fp32 values rounded to the nearest bf16 (ties to even), as fp32 (finite inputs)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32)
    u = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    return u.view(np.float32)


# rows above which a projection is the prompt contraction (hetero/cpu_model.py:30)
GEMV_ROWS_MAX = 16
# rows of W dequantised per block on that path (hetero/cpu_model.py:26)
HEAD_BLOCK = 512


class DecodeOracle:
    """Greedy decoding of one sequence from a prefilled cache.

    cfg: Qwen2 config (qwen2 keys); w: host arrays under the reference's
    tensor names; ctx_k / ctx_v: per layer [n_kv, S0, head_dim] context;
    lib: ctypes library with q4_gemv; extra: decode steps the cache holds."""

    def __init__(self, cfg: dict, w: Dict[str, np.ndarray], ctx_k: List[np.ndarray], ctx_v: List[np.ndarray],
                 lib, extra: int, kv_dtype=np.float16, nthreads: int = 0, gemm_bf16: bool = False):
        self.cfg, self.w, self.lib = cfg, w, lib
        self.nthreads = nthreads
        self.gemm_bf16 = gemm_bf16
        self.gs = cfg["quantization"]["group_size"]
        self.eps = cfg["rms_norm_eps"]
        self.nh, self.nkv = cfg["num_attention_heads"], cfg["num_key_value_heads"]
        self.d = cfg["hidden_size"] // self.nh
        self.scale = self.d ** -0.5                                   # hetero/cpu_model.py:261
        self.L = cfg["num_hidden_layers"]
        if ctx_k is None:                                             # an empty cache
            ctx_k = ctx_v = [np.zeros((self.nkv, 0, self.d), kv_dtype)] * self.L
        self.s0 = ctx_k[0].shape[1]
        cap = self.s0 + extra
        self.k = [np.zeros((1, self.nkv, cap, self.d), kv_dtype) for _ in range(self.L)]
        self.v = [np.zeros((1, self.nkv, cap, self.d), kv_dtype) for _ in range(self.L)]
        for i in range(self.L):
            self.k[i][0, :, :self.s0] = ctx_k[i]
            self.v[i][0, :, :self.s0] = ctx_v[i]
        self.pos = self.s0
        # hetero/cpu_model.py:180-193: inv_freq and the angle table in float32
        half = self.d // 2
        inv = cfg["rope_theta"] ** (-np.arange(0, half, dtype=np.float32) * 2.0 / self.d)
        ang = np.arange(max(cap, 256), dtype=np.float32)[:, None] * inv[None, :]
        self.cos, self.sin = np.cos(ang), np.sin(ang)
        self._mats = {}

    def _mat(self, name):
        m = self._mats.get(name)
        if m is None:
            w = np.ascontiguousarray(self.w[f"{name}.weight"], np.uint32)
            s = np.ascontiguousarray(self.w[f"{name}.scales"], np.float16)
            b = np.ascontiguousarray(self.w[f"{name}.biases"], np.float16)
            m = self._mats[name] = (w, s, b)
        return m

    def gemv(self, name: str, x: np.ndarray) -> np.ndarray:
        """q4_gemv of matrix `name` (+ its fp32 bias, hetero/cpu_model.py:156-157)."""
        w, s, b = self._mat(name)
        xc = np.ascontiguousarray(x, np.float32).reshape(-1)
        out = np.empty(w.shape[0], np.float32)
        rc = self.lib.q4_gemv(w.ctypes.data, s.ctypes.data, b.ctypes.data, xc.ctypes.data, out.ctypes.data,
                              w.shape[0], w.shape[1] * 8, self.gs, self.nthreads)
        if rc != 0:
            raise RuntimeError(f"q4_gemv({name}) rc={rc}")
        bias = self.w.get(f"{name}.bias")
        return out if bias is None else out + np.asarray(bias, np.float32)

    def project(self, name: str, x: np.ndarray) -> np.ndarray:
        """QLinear.__call__ (hetero/cpu_model.py:139-158) of rows x [..., n_in]
        -> [L, n_out]: q4_gemv per row up to GEMV_ROWS_MAX rows, else the
        q4_dequant + BLAS contraction (:119-136); then the fp32 bias."""
        w, s, b = self._mat(name)
        n_out, n_in = w.shape[0], w.shape[1] * 8
        xs = np.ascontiguousarray(x, np.float32).reshape(-1, n_in)
        if xs.shape[0] <= GEMV_ROWS_MAX:
            out = np.empty((xs.shape[0], n_out), np.float32)
            for r in range(xs.shape[0]):
                rc = self.lib.q4_gemv(w.ctypes.data, s.ctypes.data, b.ctypes.data, xs[r].ctypes.data,
                                      out[r].ctypes.data, n_out, n_in, self.gs, self.nthreads)
                if rc != 0:
                    raise RuntimeError(f"q4_gemv({name}) rc={rc}")
        else:
            out = np.empty((xs.shape[0], n_out), np.float32)
            blk = np.empty((HEAD_BLOCK, n_in), np.float32)
            xo = bf16_round(xs) if self.gemm_bf16 else xs
            for lo in range(0, n_out, HEAD_BLOCK):
                hi = min(lo + HEAD_BLOCK, n_out)
                rc = self.lib.q4_dequant(w.ctypes.data, s.ctypes.data, b.ctypes.data, blk.ctypes.data, lo, hi, n_in,
                                         self.gs, self.nthreads)
                if rc != 0:
                    raise RuntimeError(f"q4_dequant({name}) rc={rc}")
                wb = bf16_round(blk[:hi - lo]) if self.gemm_bf16 else blk[:hi - lo]
                out[:, lo:hi] = xo @ wb.T
        bias = self.w.get(f"{name}.bias")
        return out if bias is None else out + np.asarray(bias, np.float32)

    def logits(self, token: int) -> np.ndarray:
        """Logits of the step that consumes `token` at the current position;
        the position then advances."""
        return self.prompt([token])

    def prompt(self, ids) -> np.ndarray:
        """Logits of the last of the L tokens `ids`, consumed at the current
        position onwards as one pass of the reference stage (causal
        attention when L > 1, hetero/cpu_model.py:357-368 with last_only);
        the position then advances by L.  A prompt sent in chunks
        (hetero/coordinator.py:175-182) is one call per chunk."""
        ids = [int(t) for t in np.asarray(ids).reshape(-1)]
        n = len(ids)
        if n == 0 or self.pos + n > self.k[0].shape[2]:
            raise ValueError("an empty prompt, or the oracle's cache is full")
        w, p, d = self.w, self.pos, self.d
        # embedding rows: q * s + b (hetero/cpu_model.py:67-81, :334-338)
        ew, es, eb = (w[f"model.embed_tokens.{t}"] for t in ("weight", "scales", "biases"))
        rows = []
        for t in ids:
            q = ((ew[t][:, None] >> (np.arange(8, dtype=np.uint32) * 4)) & 0xF).reshape(-1).astype(np.float32)
            rows.append(q * np.repeat(es[t].astype(np.float32), self.gs) + np.repeat(eb[t].astype(np.float32), self.gs))
        x = np.stack(rows).reshape(1, n, -1)
        cos, sin = self.cos[p:p + n], self.sin[p:p + n]
        heads = lambda y, nh: y.reshape(1, n, nh, d).transpose(0, 2, 1, 3)
        for i in range(self.L):
            pre = f"model.layers.{i}"
            a = f"{pre}.self_attn"
            h = _norm(x, w[f"{pre}.input_layernorm.weight"].astype(np.float32), self.eps)
            qh = heads(self.project(f"{a}.q_proj", h), self.nh)
            kh = heads(self.project(f"{a}.k_proj", h), self.nkv)
            vh = heads(self.project(f"{a}.v_proj", h), self.nkv)
            qh, kh = _rope(qh, cos, sin), _rope(kh, cos, sin)
            # hetero/cpu_model.py:227-230: store, then attend over every position held
            self.k[i][:, :, p:p + n] = kh
            self.v[i][:, :, p:p + n] = vh
            if n == 1:
                o = _sdpa(qh, self.k[i][:, :, :p + 1], self.v[i][:, :, :p + 1], self.scale)
            else:
                o = _sdpa(qh, self.k[i][:, :, :p + n], self.v[i][:, :, :p + n], self.scale, True)
            x = x + self.project(f"{a}.o_proj", o.transpose(0, 2, 1, 3).reshape(1, n, -1)).reshape(1, n, -1)
            m = f"{pre}.mlp"
            h = _norm(x, w[f"{pre}.post_attention_layernorm.weight"].astype(np.float32), self.eps)
            g, u = self.project(f"{m}.gate_proj", h), self.project(f"{m}.up_proj", h)
            act = g / (1.0 + np.exp(-g, dtype=np.float32)) * u         # :169-170, :291-292
            x = x + self.project(f"{m}.down_proj", act).reshape(1, n, -1)
        self.pos += n
        return self.gemv("lm_head", _norm(x[:, -1:], w["model.norm.weight"].astype(np.float32), self.eps))


def greedy(logits) -> int:
    """argmax, first index of the maximum (hetero/backends.py:106-109)."""
    return int(np.asarray(logits, np.float32).reshape(-1).argmax())
