"""Pins of the wire-codec oracle (oracle/wire.py) that do not restate it:
brute-force fp16 rounding, closed forms of the int8 codec, the payload
layout and the round-trip bound (hetero/transport.py:193-225,
hetero/backends.py:100-104)."""
from __future__ import annotations

import bisect
import struct
from fractions import Fraction

import numpy as np
import pytest

from oracle import wire


# ---- fp16 rounding by its definition: the nearest fp16 value, ties to the
#      even bit pattern, |v| >= 65504 + 16 to inf (IEEE 754 binary16) ----

def _fp16_table():
    vals = []
    for bits in range(0x0000, 0x7C00):                 # +0 .. max finite
        e, m = bits >> 10, bits & 0x3FF
        v = Fraction(m, 1 << 24) if e == 0 else Fraction(1024 + m, 1 << 10) * Fraction(2) ** (e - 15)
        vals.append((v, bits))
    return [v for v, _ in vals], [b for _, b in vals]


_F16_VALS, _F16_BITS = _fp16_table()


def rne_f16_bits(f: np.float32) -> int:
    sign = 0x8000 if np.signbit(f) else 0
    a = Fraction(abs(float(f)))                        # exact: every fp32 is a double
    if a >= Fraction(65520):
        return sign | 0x7C00
    i = bisect.bisect_left(_F16_VALS, a)
    if i == len(_F16_VALS):                            # (65504, 65520): nearer the max than 2^16
        return sign | _F16_BITS[-1]
    if _F16_VALS[i] == a:
        return sign | _F16_BITS[i]
    lo, hi = i - 1, i
    dl, dh = a - _F16_VALS[lo], _F16_VALS[hi] - a
    pick = lo if dl < dh else hi if dh < dl else (lo if _F16_BITS[lo] % 2 == 0 else hi)
    return sign | _F16_BITS[pick]


def _edge_values():
    t = [0.0, -0.0, 1.0, 1 + 2 ** -11, 1 + 3 * 2 ** -11, 1 + 2 ** -12, 2 ** -24, 2 ** -25, 1.5 * 2 ** -25,
         3 * 2 ** -25, 2 ** -14, 2 ** -14 - 2 ** -25, 65504.0, 65519.99, 65519.0, 0.1, 1 / 3, 2048.5, 2049.0,
         4097.0, 1e-8]
    return np.array(t + [-v for v in t], dtype=np.float32)


def test_to_wire_is_round_to_nearest_even():
    rng = np.random.default_rng(7)
    x = np.concatenate([_edge_values(), rng.standard_normal(400).astype(np.float32),
                        (rng.standard_normal(200) * 3e4).astype(np.float32),
                        (rng.standard_normal(200) * 1e-6).astype(np.float32)])
    with np.errstate(over="ignore"):                   # |x| > 65520 rounds to inf, as it should
        got = wire.to_wire(x).view(np.uint16)
    want = np.array([rne_f16_bits(v) for v in x], dtype=np.uint16)
    assert np.array_equal(got, want)


def test_to_wire_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(8)
    x = (rng.standard_normal(20000) * np.exp(rng.uniform(-20, 12, 20000))).astype(np.float32)
    x = x[np.abs(x) < 65504]
    want = torch.from_numpy(x).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(wire.to_wire(x).view(np.uint16), want)


def test_fp16_codec_payload_and_round_trip():
    x = _edge_values().reshape(2, -1)
    h, p = wire.stage_encode(x, "fp16")
    assert h == {"codec": "fp16", "shape": [2, x.shape[1]]}
    assert len(p) == 2 * x.size
    want = np.array([rne_f16_bits(v) for v in x.reshape(-1)], dtype=np.uint16)
    assert np.array_equal(np.frombuffer(p, dtype=np.uint16), want)
    back = wire.stage_decode(h, p)
    assert back.dtype == np.float32
    assert np.array_equal(back.view(np.uint32), want.view(np.float16).astype(np.float32).view(np.uint32).reshape(2, -1))


# ---- int8 closed forms ----

def _scales_q(p: bytes, rows: int, hidden: int):
    s = np.array(struct.unpack(f"<{rows}f", p[:4 * rows]), dtype=np.float32)
    q = np.frombuffer(p[4 * rows:], dtype=np.int8).reshape(rows, hidden)
    return s, q


def test_int8_zero_row_has_scale_one():
    x = np.zeros((2, 16), np.float32)
    x[1, 3] = 2.0 ** -5
    h, p = wire.stage_encode(x, "int8")
    s, q = _scales_q(p, 2, 16)
    assert s[0] == 1.0 and not q[0].any()
    assert s[1] == np.float32(2.0 ** -5) / np.float32(127.0) and q[1, 3] == 127 and np.count_nonzero(q[1]) == 1
    assert not wire.stage_decode(h, p)[0].any()


def test_int8_exact_multiples():
    rng = np.random.default_rng(9)
    s = 2.0 ** -6
    k = rng.integers(-127, 128, size=(5, 64))
    k[:, 0] = [127, -127, 127, -127, 127]
    x = (k * s).astype(np.float32)                     # exact in fp16 and fp32
    h, p = wire.stage_encode(x, "int8")
    sc, q = _scales_q(p, 5, 64)
    assert np.all(sc == np.float32(s))                 # fl(127 s / 127) = s
    assert np.array_equal(q, k)
    assert np.array_equal(wire.stage_decode(h, p), x)


def test_int8_ties_round_to_even():
    s = 2.0 ** -4
    m = np.array([127, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, 3.5, -3.5, 0.25, -125.5], dtype=np.float64)
    x = (m * s).astype(np.float32)[None, :]
    _, p = wire.stage_encode(x, "int8")
    _, q = _scales_q(p, 1, m.size)
    assert q[0].tolist() == [127, 0, 2, 2, 0, -2, -2, 126, 4, -4, 0, -126]


def test_int8_max_is_taken_after_fp16_rounding():
    x = np.array([[1 + 2 ** -12, 0.25, -0.5]], dtype=np.float32)   # fp16: [1, 0.25, -0.5]
    _, p = wire.stage_encode(x, "int8")
    sc, q = _scales_q(p, 1, 3)
    assert sc[0] == np.float32(1.0) / np.float32(127.0)
    assert sc[0] != np.float32(1 + 2 ** -12) / np.float32(127.0)
    assert q[0, 0] == 127


def test_int8_layout_scales_then_rows():
    x = np.zeros((2, 3, 8), np.float32)
    x[0, 0, 0], x[0, 1, 1], x[0, 2, 2] = 127 * 2.0 ** -6, -127 * 2.0 ** -3, 5 * 2.0 ** -2
    x[1, :, 7] = [127 * 2.0 ** -1, 0.0, 127.0]
    h, p = wire.stage_encode(x, "int8")
    assert h == {"codec": "int8", "shape": [2, 3, 8]}
    assert len(p) == 6 * 4 + 48
    sc = struct.unpack("<6f", p[:24])
    assert (sc[0], sc[1], sc[3], sc[4], sc[5]) == (2.0 ** -6, 2.0 ** -3, 2.0 ** -1, 1.0, 1.0)
    assert sc[2] == np.float32(5 * 2.0 ** -2) / np.float32(127.0)
    q = np.frombuffer(p[24:], dtype=np.int8).reshape(6, 8)
    assert q[0, 0] == 127 and q[1, 1] == -127 and q[2, 2] == 127 and q[3, 7] == 127 and q[5, 7] == 127
    assert np.count_nonzero(q) == 5
    back = wire.stage_decode(h, p)
    assert back.shape == (2, 3, 8) and back[1, 2, 7] == 127.0 and back[0, 1, 1] == -127 * 2.0 ** -3


def test_int8_round_trip_bound():
    rng = np.random.default_rng(10)
    x = (rng.standard_normal((16, 3584)) * np.exp(rng.uniform(-3, 3, (16, 1)))).astype(np.float32)
    h, p = wire.stage_encode(x, "int8")
    sc, q = _scales_q(p, 16, 3584)
    xh = wire.to_wire(x).astype(np.float64)
    back = wire.stage_decode(h, p).astype(np.float64)
    # |q s - v| <= s/2 (plus the rounding of v / s), then one fp16 rounding
    err = np.abs(back - xh)
    bound = sc[:, None].astype(np.float64) * (0.5 + 1e-6) + np.abs(back) * 2.0 ** -11
    assert np.all(err <= bound)
    assert np.all(np.abs(q).max(axis=1) == 127)


def test_unknown_codec():
    with pytest.raises(ValueError):
        wire.encode(np.zeros((1, 8), np.float16), "bf16")
    with pytest.raises(ValueError):
        wire.decode({"codec": "bf16", "shape": [1, 8]}, b"")
