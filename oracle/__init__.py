"""CPU oracle of the int4 GEMV path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package; the product (hetero-infer_amd/) never does.

  liboq4.so                   C restatement of kernel/q4gemv.c (q4oracle.c)
  _ref/libq4gemv_ref_rR.so    the reference kernel/q4gemv.c compiled from its
                              own source (oracle/Makefile), ROWS = R
  numpy helpers               fp64 brute force and closed forms used to pin
                              the restatement where no golden vector does
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboq4.so")
REF_DIR = os.path.join(HERE, "_ref")

_VP, _I = ctypes.c_void_p, ctypes.c_int


def build() -> None:
    """make -C oracle: liboq4.so always; _ref/ when the reference is present."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def load_oracle() -> ctypes.CDLL:
    if not os.path.exists(ORACLE_SO):
        build()
    lib = ctypes.CDLL(ORACLE_SO)
    lib.oq_q4_gemv.argtypes = [_VP] * 5 + [_I] * 4
    lib.oq_q4_gemv.restype = _I
    lib.oq_q4_dequant.argtypes = [_VP] * 4 + [_I] * 4
    lib.oq_q4_dequant.restype = _I
    lib.oq_xprep.argtypes = [_VP, _I, _I, _VP, _VP, _VP]
    lib.oq_xprep.restype = None
    lib.oq_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.oq_f16_to_f32.restype = ctypes.c_float
    lib.oq_unpack.argtypes = [_VP, _VP, _I, _I, _I]
    lib.oq_unpack.restype = None
    return lib


def ref_path(rows: int = 1) -> str:
    return os.path.join(REF_DIR, f"libq4gemv_ref_r{rows}.so")


def load_ref(rows: int = 1) -> ctypes.CDLL:
    """The reference kernel compiled from source (same ABI as libq4gemv.so)."""
    lib = ctypes.CDLL(ref_path(rows))
    lib.q4_gemv.argtypes = [_VP] * 5 + [_I] * 4
    lib.q4_gemv.restype = _I
    lib.q4_dequant.argtypes = [_VP] * 4 + [_I] * 5
    lib.q4_dequant.restype = _I
    return lib


class Oracle:
    """Thin NumPy front end of liboq4.so."""

    def __init__(self):
        self.lib = load_oracle()

    def gemv(self, w, s, b, x, gs, rows_block=1):
        n_out, n_in = w.shape[0], w.shape[1] * 8
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(n_out, np.float32)
        rc = self.lib.oq_q4_gemv(w.ctypes.data, s.ctypes.data, b.ctypes.data, x.ctypes.data,
                                 out.ctypes.data, n_out, n_in, gs, rows_block)
        if rc != 0:
            raise ValueError(f"oq_q4_gemv rc={rc}")
        return out

    def gemv_rows(self, w, s, b, x2, gs):
        return np.stack([self.gemv(w, s, b, x2[m], gs) for m in range(x2.shape[0])])

    def dequant(self, w, s, b, gs, row0=0, row1=None):
        n_in = w.shape[1] * 8
        row1 = w.shape[0] if row1 is None else row1
        out = np.empty((max(row1 - row0, 0), n_in), np.float32)
        rc = self.lib.oq_q4_dequant(w.ctypes.data, s.ctypes.data, b.ctypes.data,
                                    out.ctypes.data if out.size else None, row0, row1, n_in, gs)
        if rc != 0:
            raise ValueError(f"oq_q4_dequant rc={rc}")
        return out

    def xprep(self, x, gs):
        x = np.ascontiguousarray(x, np.float32)
        n = x.shape[0]
        xq = np.empty(n, np.int16)
        xsum = np.empty(max(n // gs, 1), np.float32)
        sc = np.empty(1, np.float32)
        self.lib.oq_xprep(x.ctypes.data, n, gs, xq.ctypes.data, xsum.ctypes.data, sc.ctypes.data)
        return xq, xsum[: n // gs], float(sc[0])

    def unpack(self, w, row0=0, row1=None):
        n_in = w.shape[1] * 8
        row1 = w.shape[0] if row1 is None else row1
        out = np.empty((row1 - row0, n_in), np.uint8)
        self.lib.oq_unpack(w.ctypes.data, out.ctypes.data, row0, row1, n_in)
        return out


# ---- NumPy closed forms (independent of the C code) ----

def unpack_np(w: np.ndarray) -> np.ndarray:
    """(w >> 4j) & 0xF, low nibble first: [n_out, n_in] uint8."""
    sh = (np.arange(8, dtype=np.uint32) * 4)
    return ((w[..., None] >> sh) & 0xF).astype(np.uint8).reshape(w.shape[0], -1)


def dequant_np(w, s, b, gs) -> np.ndarray:
    """q*scale + bias in fp32 with q*scale exact (so one rounding)."""
    q = unpack_np(w).astype(np.float32)
    sf = np.repeat(s.astype(np.float32), gs, axis=1)
    bf = np.repeat(b.astype(np.float32), gs, axis=1)
    return q * sf + bf


def gemv_fp64(w, s, b, x, gs) -> np.ndarray:
    """Exact-ish fp64 brute force of W x with W the dequantised weights."""
    q = unpack_np(w).astype(np.float64)
    sf = np.repeat(s.astype(np.float64), gs, axis=1)
    bf = np.repeat(b.astype(np.float64), gs, axis=1)
    return (q * sf + bf) @ np.asarray(x, np.float64)


def normwise_rel(a, ref) -> float:
    """max|a - ref| / max|ref| (the reference's convention, tests/test_correctness.py:46-53)."""
    a = np.asarray(a, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.max(np.abs(a - ref))
    m = np.max(np.abs(ref))
    return float(d / m) if m > 0 else float(d)
