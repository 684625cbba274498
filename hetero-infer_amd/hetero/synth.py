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


# ---- draws that NumPy and torch (CPU or GPU) reproduce bit for bit ---------
#
# A 28-layer model is 4 GB of weights: generating it with the NumPy stream
# above takes about a minute, while torch on the GPU takes well under a
# second.  The two agree bit for bit only where every floating-point step is
# one IEEE operation, so these draws avoid transcendentals: a normal-like
# value is the Irwin-Hall sum S of the four 16-bit fields of one splitmix64
# output, centred and scaled to unit variance,
#   z = float32(S - 131070) * float32(sigma * sqrt(3) / 65536)
# (one float32 multiply; S - 131070 is exact in float32), bounded by
# +-3.46 sigma.  Conversions to fp16 round to nearest even on both sides.
# The packed weights are the integer stream of qweights() unchanged.

_IH_CENTER = 2 * 65535
_U64_MASK = (1 << 64) - 1


def ih_scale(sigma: float) -> np.float32:
    return np.float32(sigma * np.sqrt(3.0) / 65536.0)


def ih_sum_np(seed: int, tag: str, n: int) -> np.ndarray:
    """S - 131070 for n draws (int64)."""
    z = u64(seed, tag, n)
    m = np.uint64(0xFFFF)
    s = (z & m) + ((z >> np.uint64(16)) & m) + ((z >> np.uint64(32)) & m) + (z >> np.uint64(48))
    return s.astype(np.int64) - _IH_CENTER


def ih_normal_np(seed: int, tag: str, n: int, sigma: float = 1.0) -> np.ndarray:
    return ih_sum_np(seed, tag, n).astype(np.float32) * ih_scale(sigma)


def qlinear_ih_np(seed: int, n_out: int, n_in: int, gs: int = 64, tag: str = "", center: float = 8.0):
    """(w, scales, biases) with the distributions of qlinear(): packed U{0..15}
    weights, fp16 scales |z * 0.02|, fp16 biases -center * scale + z' * 0.002
    (center 8 by default; -center * scale is exact in fp32 for center 8 or
    7.5)."""
    w = qweights(seed, n_out, n_in, tag + "w")
    g = n_out * (n_in // gs)
    s = np.abs(ih_normal_np(seed, tag + "sb.s", g, 0.02)).astype(np.float16)
    b = (np.float32(-center) * s.astype(np.float32) + ih_normal_np(seed, tag + "sb.b", g, 0.002)).astype(np.float16)
    return w, s.reshape(n_out, -1), b.reshape(n_out, -1)


def _signed(c: int) -> int:
    return c - (1 << 64) if c >= 1 << 63 else c


def _lsr(t, s: int):
    """Logical right shift of int64 tensor bits."""
    return (t >> s) & ((1 << (64 - s)) - 1)


def u64_torch(seed: int, tag: str, n: int, device):
    """u64() as int64 bit patterns in a torch tensor (wrapping arithmetic)."""
    import torch
    key = _signed(int(stream_key(seed, tag)))
    z = torch.arange(1, n + 1, dtype=torch.int64, device=device) * _signed(int(_GOLDEN)) + key
    z = (z ^ _lsr(z, 30)) * _signed(int(_M1))
    z = (z ^ _lsr(z, 27)) * _signed(int(_M2))
    return z ^ _lsr(z, 31)


def ih_normal_torch(seed: int, tag: str, n: int, sigma: float, device):
    import torch
    z = u64_torch(seed, tag, n, device)
    s = (z & 0xFFFF) + (_lsr(z, 16) & 0xFFFF) + (_lsr(z, 32) & 0xFFFF) + _lsr(z, 48)
    return (s - _IH_CENTER).to(torch.float32) * float(ih_scale(sigma))


def qlinear_ih_torch(seed: int, n_out: int, n_in: int, gs: int, device, tag: str = "", center: float = 8.0):
    """qlinear_ih_np on a torch device: int32 weights, int16 (fp16 bit
    pattern) scales and biases."""
    import torch
    words = n_out * (n_in // 8)
    w = u64_torch(seed, tag + "w", (words + 1) // 2, device).view(torch.int32)[:words].reshape(n_out, n_in // 8)
    g = n_out * (n_in // gs)
    s = ih_normal_torch(seed, tag + "sb.s", g, 0.02, device).abs().to(torch.float16)
    b = (s.to(torch.float32) * -float(center) + ih_normal_torch(seed, tag + "sb.b", g, 0.002, device)).to(torch.float16)
    return w.contiguous(), s.view(torch.int16).reshape(n_out, -1), b.view(torch.int16).reshape(n_out, -1)
