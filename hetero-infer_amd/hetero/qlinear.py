"""The 4-bit projection operator of the reference's NumPy backend, over
libq4gemv.so.

`QLinear(w, scales, biases, bias, group_size, bits)` keeps the reference's
constructor and call (hetero/cpu_model.py:84-158): MLX-layout packed weights
stay packed in host memory, a call with at most GEMV_ROWS_MAX activation
rows is a GEMV through the C-ABI, a longer prompt is the reference's
prefill contraction (512-row q4_dequant blocks, each multiplied by BLAS),
and the optional fp32 bias is added last.  The library behind it is any
object with the reference's ctypes ABI: libq4gemv.so by default, or the
reference kernel compiled from source (the tests run both).

Differences from the reference, on purpose: a missing library raises
instead of expanding the weights to fp32 (hetero/cpu_model.py:105-107), and
2..16 rows take one q4_gemv_batched call (each row bit-identical to its own
q4_gemv) where the library exports it, instead of a loop of q4_gemv calls.
"""
from __future__ import annotations

import os
from typing import Optional

import numpy as np

from . import q4

# rows above which a call is a dequant + BLAS contraction (hetero/cpu_model.py:27-30)
GEMV_ROWS_MAX = int(os.environ.get("HETERO_GEMV_ROWS", "16"))
# rows of W expanded per q4_dequant call on that path (hetero/cpu_model.py:26)
DEQUANT_BLOCK = 512
# thread hint passed through the ABI (hetero/cpu_model.py:60-64); libq4gemv.so ignores it
NTHREADS = int(os.environ.get("HETERO_THREADS", "0")) or (os.cpu_count() or 2)


def dequantize(w: np.ndarray, scales: np.ndarray, biases: np.ndarray, group_size: int,
               bits: int = 4) -> np.ndarray:
    """MLX 4-bit rows to fp32: value k of a row is nibble k % 8 (low first) of
    word k // 8, times its group's scale plus its group's bias -- one rounding,
    since q * scale is exact (hetero/cpu_model.py:67-81)."""
    if bits != 4:
        raise NotImplementedError("4-bit weights only")
    rows, words = w.shape
    nib = np.empty((rows, words, 8), np.float32)
    for j in range(8):
        nib[:, :, j] = (w >> np.uint32(4 * j)) & np.uint32(0xF)
    g = nib.reshape(rows, -1, group_size)
    return (g * scales.astype(np.float32)[:, :, None] + biases.astype(np.float32)[:, :, None]).reshape(rows, -1)


class QLinear:
    """y = x W^T (+ bias) for a 4-bit W: GEMV for decode-sized inputs,
    dequant + BLAS for prompts (the reference's QLinear, same arguments)."""

    def __init__(self, w, scales, biases, bias, group_size: int, bits: int, lib=None):
        if bits != 4:
            raise NotImplementedError("libq4gemv.so handles 4-bit weights")
        self.lib = lib if lib is not None else q4.load()
        self.group_size, self.bits = int(group_size), int(bits)
        self.w = np.ascontiguousarray(w, dtype=np.uint32)
        self.scales = np.ascontiguousarray(scales, dtype=np.float16)
        self.biases = np.ascontiguousarray(biases, dtype=np.float16)
        self.bias = None if bias is None else np.asarray(bias, dtype=np.float32)
        self.n_out, self.n_in = self.w.shape[0], self.w.shape[1] * 8
        self._wsb = (self.w.ctypes.data, self.scales.ctypes.data, self.biases.ctypes.data)
        self._block: Optional[np.ndarray] = None
        self._batched = getattr(self.lib, "q4_gemv_batched", None)

    def _check(self, rc: int, what: str):
        if rc != 0:               # the reference's caller raises on any nonzero code (cpu_model.py:115-116)
            raise RuntimeError(f"{what} failed with {rc}")

    def gemv_rows(self, xs: np.ndarray) -> np.ndarray:
        """[r, n_in] -> [r, n_out] by the library's GEMV, row by row semantics."""
        xs = np.ascontiguousarray(xs, dtype=np.float32)
        r = xs.shape[0]
        out = np.empty((r, self.n_out), dtype=np.float32)
        if r > 1 and self._batched is not None:
            self._check(self._batched(*self._wsb, xs.ctypes.data, out.ctypes.data, r, self.n_out, self.n_in,
                                      self.group_size, NTHREADS), "q4_gemv_batched")
            return out
        for i in range(r):
            self._check(self.lib.q4_gemv(*self._wsb, xs[i].ctypes.data, out[i].ctypes.data, self.n_out,
                                         self.n_in, self.group_size, NTHREADS), "q4_gemv")
        return out

    def contract(self, xs: np.ndarray) -> np.ndarray:
        """The prompt path: W expanded DEQUANT_BLOCK rows at a time by
        q4_dequant into one reused buffer, each block multiplied as
        `xs @ block.T` -- the reference's operands and BLAS call, which fix
        the result's bits (hetero/cpu_model.py:119-136)."""
        xs = np.asarray(xs, dtype=np.float32)
        out = np.empty((xs.shape[0], self.n_out), dtype=np.float32)
        if self._block is None:
            self._block = np.empty((DEQUANT_BLOCK, self.n_in), dtype=np.float32)
        blk = self._block
        for r0 in range(0, self.n_out, DEQUANT_BLOCK):
            r1 = min(self.n_out, r0 + DEQUANT_BLOCK)
            self._check(self.lib.q4_dequant(*self._wsb, blk.ctypes.data, r0, r1, self.n_in, self.group_size,
                                            NTHREADS), "q4_dequant")
            out[:, r0:r1] = xs @ blk[:r1 - r0].T
        return out

    def __call__(self, x: np.ndarray) -> np.ndarray:
        x = np.asarray(x, dtype=np.float32)
        xs = x.reshape(-1, self.n_in)
        y = self.gemv_rows(xs) if xs.shape[0] <= GEMV_ROWS_MAX else self.contract(xs)
        if self.bias is not None:
            y = y + self.bias
        return y.reshape(x.shape[:-1] + (self.n_out,))
