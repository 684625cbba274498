"""CPU oracle of the activation wire codec -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module; the product (hetero-infer_amd/) never does.

A NumPy restatement of the reference's codec, hetero/transport.py:193-225,
together with the NumPy backend's conversions either side of it,
hetero/backends.py:100-104, which the stage runner applies around every
encode/decode (hetero/engine.py:76, :97).

Pinned in tests/test_oracle_wire.py, without the reference, by:
  * fp16 rounding: an integer round-to-nearest-even on the fp32 bit pattern
    (ties, subnormals, overflow to inf) and torch's conversion;
  * int8: closed forms -- zero rows (scale 1), rows of exact multiples of a
    power-of-two scale (q = the multiple), ties at k + 1/2 (to even), the
    fp16 rounding ahead of the max, the byte layout of the payload (scales,
    then rows), and the round-trip bound |decode(encode(x)) - x| <= scale/2
    plus the last fp16 rounding.
Non-finite inputs are outside the contract: the reference's int8 bytes for
them depend on the host's float-to-int8 conversion.
"""
from __future__ import annotations

from typing import Tuple

import numpy as np


def to_wire(x) -> np.ndarray:
    """hetero/backends.py:100-101 (NumpyBackend.to_wire): fp16, round to nearest even."""
    return np.asarray(x, dtype=np.float16)


def from_wire(a) -> np.ndarray:
    """hetero/backends.py:103-104 (NumpyBackend.from_wire): fp32."""
    return np.asarray(a, dtype=np.float32)


def encode(arr, codec: str = "fp16") -> Tuple[dict, bytes]:
    """hetero/transport.py:198-211."""
    if codec == "fp16":                                        # :200-202
        h = np.asarray(arr, dtype=np.float16)
        return {"codec": "fp16", "shape": list(h.shape)}, h.tobytes()
    if codec == "int8":                                        # :203-211
        v = np.asarray(arr, dtype=np.float32)
        rows = v.reshape(-1, v.shape[-1])
        amax = np.max(np.abs(rows), axis=-1, keepdims=True)
        scale = (amax / np.float32(127.0)).astype(np.float32)  # fp32 division
        scale = np.where(scale == 0, np.float32(1.0), scale)
        q = np.rint(rows / scale)                              # fp32 division, ties to even
        q = np.clip(q, -127, 127).astype(np.int8)
        return {"codec": "int8", "shape": list(v.shape)}, scale.astype(np.float32).tobytes() + q.tobytes()
    raise ValueError(f"unknown codec {codec}")


def decode(header: dict, payload: bytes) -> np.ndarray:
    """hetero/transport.py:214-225: an fp16 array."""
    shape = tuple(header["shape"])
    if header["codec"] == "fp16":                              # :216-217
        return np.frombuffer(payload, dtype=np.float16).reshape(shape)
    if header["codec"] == "int8":                              # :218-224
        n_rows = int(np.prod(shape[:-1]))
        scales = np.frombuffer(payload[:4 * n_rows], dtype=np.float32).reshape(n_rows, 1)
        q = np.frombuffer(payload[4 * n_rows:], dtype=np.int8).reshape(n_rows, shape[-1])
        return (q.astype(np.float32) * scales).reshape(shape).astype(np.float16)
    raise ValueError(f"unknown codec {header['codec']}")


def stage_encode(x, codec: str) -> Tuple[dict, bytes]:
    """What a NumPy stage sends for its fp32 output x (hetero/engine.py:97)."""
    return encode(to_wire(x), codec)


def stage_decode(header: dict, payload: bytes) -> np.ndarray:
    """What a NumPy stage computes on from a received frame (hetero/engine.py:76)."""
    return from_wire(decode(header, payload))
