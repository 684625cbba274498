"""Seeded synthetic inputs for the int4 GEMV path.

The reference draws its benchmark inputs from NumPy's default_rng
(kernel/autotune.py:28-34).  Here every tensor comes from a counter-based
splitmix64 stream computed with plain uint64 arithmetic, so the same seed
gives the same bits on any machine and NumPy version; the only floating-point
step is Box-Muller for the normal draws, and fixtures record the SHA-256 of
every generated input so a change there is caught rather than silently
compared against.

Distributions (MLX 4-bit layout, hetero/cpu_model.py:67-81):
  weights  q ~ U{0..15}, eight per uint32, low nibble first    [n_out, n_in/8]
  scales   fp16 |N(0, 0.02)|                                  [n_out, n_in/gs]
  biases   fp16 -8*scale + N(0, 0.002)                        [n_out, n_in/gs]
  x        fp32 N(0, 1)                                       [m, n_in]
"""
from __future__ import annotations

import hashlib
import zlib

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def stream_key(seed: int, tag: str) -> np.uint64:
    """A 64-bit stream key for (seed, tensor name)."""
    c = zlib.crc32(tag.encode())
    base = np.array([(int(seed) * 0x100000001B3 + c) & 0xFFFFFFFFFFFFFFFF], np.uint64)
    return _mix(base)[0]


def u64(seed: int, tag: str, n: int, start: int = 0) -> np.ndarray:
    """n splitmix64 outputs of stream (seed, tag), counter start..start+n-1."""
    with np.errstate(over="ignore"):
        ctr = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        return _mix(stream_key(seed, tag) + ctr * _GOLDEN)


def uniform(seed: int, tag: str, n: int) -> np.ndarray:
    """Doubles in (0, 1): 53 random bits, offset by half a step."""
    return ((u64(seed, tag, n) >> np.uint64(11)).astype(np.float64) + 0.5) * (2.0 ** -53)


def normal(seed: int, tag: str, n: int) -> np.ndarray:
    """Standard normal doubles by Box-Muller over pairs of uniforms."""
    half = (n + 1) // 2
    u = uniform(seed, tag, 2 * half)
    r = np.sqrt(-2.0 * np.log(u[:half]))
    t = 2.0 * np.pi * u[half:]
    return np.concatenate([r * np.cos(t), r * np.sin(t)])[:n]


def qweights(seed: int, n_out: int, n_in: int, tag: str = "w") -> np.ndarray:
    """Packed 4-bit weights [n_out, n_in/8] uint32, every nibble U{0..15}."""
    words = n_out * (n_in // 8)
    r = u64(seed, tag, (words + 1) // 2)
    return r.view(np.uint32)[:words].reshape(n_out, n_in // 8).copy()


def scales_biases(seed: int, n_out: int, n_groups: int, tag: str = "sb"):
    """fp16 scales |N(0,0.02)| and biases -8*scale + N(0,0.002), [n_out, n_groups]."""
    n = n_out * n_groups
    s = np.abs(normal(seed, tag + ".s", n) * 0.02).astype(np.float16)
    b = (-8.0 * s.astype(np.float64) + normal(seed, tag + ".b", n) * 0.002).astype(np.float16)
    return s.reshape(n_out, n_groups), b.reshape(n_out, n_groups)


def activations(seed: int, m: int, n_in: int, tag: str = "x") -> np.ndarray:
    """fp32 N(0, 1) activations [m, n_in]."""
    return normal(seed, tag, m * n_in).astype(np.float32).reshape(m, n_in)


def qlinear(seed: int, n_out: int, n_in: int, gs: int = 64, tag: str = ""):
    """(w, scales, biases) of one 4-bit projection."""
    w = qweights(seed, n_out, n_in, tag + "w")
    s, b = scales_biases(seed, n_out, n_in // gs, tag + "sb")
    return w, s, b


def sha256(*arrays: np.ndarray) -> str:
    h = hashlib.sha256()
    for a in arrays:
        a = np.ascontiguousarray(a)
        h.update(str(a.dtype).encode() + str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


# Qwen2.5-7B projection shapes, (name, n_in K, n_out N).
QWEN7B_SHAPES = [
    ("q_proj", 3584, 3584),
    ("k_proj", 3584, 512),
    ("v_proj", 3584, 512),
    ("o_proj", 3584, 3584),
    ("gate_proj", 3584, 18944),
    ("up_proj", 3584, 18944),
    ("down_proj", 18944, 3584),
    ("lm_head", 3584, 152064),
]


def gemv_bytes(m: int, n_out: int, n_in: int, gs: int = 64) -> int:
    """Algorithmic bytes of one call: packed W + fp16 scales and biases + fp32 x and y."""
    return n_out * n_in // 2 + 4 * n_out * (n_in // gs) + 4 * m * n_in + 4 * m * n_out
