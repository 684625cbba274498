#!/usr/bin/env python3
"""Write the golden vectors of the int4 GEMV path from the reference kernel.

The reference kernel/q4gemv.c is compiled from its own source by
oracle/Makefile (clang, kernel/build.sh's x86 flags, one library per ROWS
value) into oracle/_ref/.  This script drives those libraries through ctypes
with the same argument types as hetero/cpu_model.py:41-44 and stores, for
seeded inputs from hetero.synth:

  golden_small.npz   small cases with inputs and outputs inline (odd row
                     counts for the ROWS tail path, gs=128, zero and constant
                     x, zero/subnormal scales, integer dots above 2^24,
                     q4_dequant row ranges, return codes)
  golden_qwen7b.npz  outputs only, for the Qwen2.5-7B shapes at M=1 (seed per
                     shape) and for 8 activation rows at two of them
  manifest.json      seeds, shapes and the SHA-256 of every input and output

Run from the repository root after `make -C oracle`:
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "hetero-infer_amd"))
from hetero import synth  # noqa: E402

OUT_DIR = os.path.dirname(os.path.abspath(__file__))
REF_DIR = os.path.join(ROOT, "oracle", "_ref")


def load_ref(rows: int):
    lib = ctypes.CDLL(os.path.join(REF_DIR, f"libq4gemv_ref_r{rows}.so"))
    lib.q4_gemv.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 4
    lib.q4_gemv.restype = ctypes.c_int
    lib.q4_dequant.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 5
    lib.q4_dequant.restype = ctypes.c_int
    return lib


def gemv(lib, w, s, b, x, n_out, n_in, gs, threads=8):
    out = np.full(n_out, np.nan, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    rc = lib.q4_gemv(w.ctypes.data, s.ctypes.data, b.ctypes.data, x.ctypes.data,
                     out.ctypes.data, n_out, n_in, gs, threads)
    return rc, out


def dequant(lib, w, s, b, row0, row1, n_in, gs, threads=4):
    out = np.full((max(row1 - row0, 0), n_in), np.nan, np.float32)
    rc = lib.q4_dequant(w.ctypes.data, s.ctypes.data, b.ctypes.data,
                        out.ctypes.data if out.size else None, row0, row1, n_in, gs, threads)
    return rc, out


def main():
    os.environ.setdefault("HETERO_KERNEL_THREADS", "8")
    libs = {r: load_ref(r) for r in (1, 2, 4, 8)}
    small, manifest = {}, {"generator": "hetero.synth (splitmix64 + Box-Muller)",
                           "reference": "kernel/q4gemv.c built by oracle/Makefile",
                           "cases": {}}

    def put(name, **arrays):
        for k, v in arrays.items():
            small[f"{name}.{k}"] = v
        manifest["cases"][name] = {k: {"shape": list(np.shape(v)), "dtype": str(np.asarray(v).dtype),
                                       "sha256": synth.sha256(np.asarray(v))}
                                   for k, v in arrays.items()}

    # --- small GEMV cases: (name, n_out, n_in, gs, seed, x-kind, scale-kind)
    cases = [
        ("g_1x64", 1, 64, 64, 101, "normal", "normal"),
        ("g_7x192", 7, 192, 64, 102, "normal", "normal"),
        ("g_13x512", 13, 512, 64, 103, "normal", "normal"),
        ("g_37x1024_gs128", 37, 1024, 128, 104, "normal", "normal"),
        ("g_64x2048", 64, 2048, 64, 105, "normal", "normal"),
        ("g_9x256_xzero", 9, 256, 64, 106, "zero", "normal"),
        ("g_9x256_xconst", 9, 256, 64, 107, "const", "normal"),
        ("g_9x256_xspike", 9, 256, 64, 108, "spike", "normal"),
        ("g_8x512_big_idot", 8, 512, 64, 109, "const", "q15"),
        ("g_11x320_subnormal", 11, 320, 64, 110, "normal", "subnormal"),
        ("g_6x384_scalezero", 6, 384, 64, 111, "normal", "zero"),
        ("g_5x768_xhuge", 5, 768, 64, 112, "huge", "normal"),
        ("g_3x4096_gs256", 3, 4096, 256, 113, "normal", "normal"),
    ]
    for name, n_out, n_in, gs, seed, xk, sk in cases:
        w, s, b = synth.qlinear(seed, n_out, n_in, gs)
        if sk == "q15":
            w[:] = np.uint32(0xFFFFFFFF)
            s[:] = np.float16(1.0)
            b[:] = np.float16(0.0)
        elif sk == "subnormal":
            s[:] = (np.abs(s.view(np.uint16)) & np.uint16(0x03FF)).view(np.float16)
            b[::2] = (b[::2].view(np.uint16) & np.uint16(0x83FF)).view(np.float16)
        elif sk == "zero":
            s[:] = np.float16(0.0)
        x = synth.activations(seed, 1, n_in)[0]
        if xk == "zero":
            x[:] = 0.0
        elif xk == "const":
            x[:] = np.float32(0.75)
        elif xk == "spike":
            x[:] = 0.0
            x[n_in // 3] = np.float32(-2.5)
            x[n_in - 1] = np.float32(1e-3)
        elif xk == "huge":
            x *= np.float32(1e30)
        outs = {}
        for r in (1, 2, 4, 8):
            rc, o = gemv(libs[r], w, s, b, x, n_out, n_in, gs)
            assert rc == 0, (name, r, rc)
            outs[f"out_rows{r}"] = o
        put(name, w=w, scales=s, biases=b, x=x, **outs)
        manifest["cases"][name]["params"] = {"n_out": n_out, "n_in": n_in, "gs": gs, "seed": seed}

    # --- return codes (must be identical in every implementation)
    w, s, b = synth.qlinear(120, 4, 256, 64)
    x = synth.activations(120, 1, 256)[0]
    rcs = {
        "gemv_gs32": gemv(libs[1], w, s, b, x, 4, 256, 32)[0],
        "gemv_nin_not_multiple": gemv(libs[1], w, s, b, x, 4, 192 + 8, 64)[0],
        "gemv_gs96": gemv(libs[1], w, s, b, x, 4, 192, 96)[0],
        "dequant_gs12": dequant(libs[1], w, s, b, 0, 2, 256, 12)[0],
        "dequant_empty": dequant(libs[1], w, s, b, 3, 3, 256, 64)[0],
        "dequant_reversed": dequant(libs[1], w, s, b, 3, 1, 256, 64)[0],
    }
    manifest["return_codes"] = {k: int(v) for k, v in rcs.items()}

    # --- q4_dequant row ranges (gs=64 and gs=32: dequant accepts gs % 8 == 0)
    for name, n_out, n_in, gs, seed, r0, r1 in [
        ("d_20x512", 20, 512, 64, 130, 0, 20),
        ("d_20x512_rows5_17", 20, 512, 64, 131, 5, 17),
        ("d_9x256_gs32", 9, 256, 32, 132, 2, 9),
    ]:
        w, s, b = synth.qlinear(seed, n_out, n_in, gs)
        rc, o = dequant(libs[1], w, s, b, r0, r1, n_in, gs)
        assert rc == 0
        put(name, w=w, scales=s, biases=b, out=o)
        manifest["cases"][name]["params"] = {"n_out": n_out, "n_in": n_in, "gs": gs,
                                             "seed": seed, "row0": r0, "row1": r1}

    np.savez_compressed(os.path.join(OUT_DIR, "golden_small.npz"), **small)

    # --- Qwen2.5-7B shapes at M=1 (seed per shape) and M=8 rows at two shapes
    big, qwen = {}, {}
    shapes = [("config0_q_proj", 3584, 3584, 0)] + [
        (name, n_in, n_out, 1000 + i) for i, (name, n_in, n_out) in enumerate(synth.QWEN7B_SHAPES)]
    for name, n_in, n_out, seed in shapes:
        w, s, b = synth.qlinear(seed, n_out, n_in, 64)
        x = synth.activations(seed, 8 if name in ("q_proj", "down_proj") else 1, n_in)
        rows = []
        for m in range(x.shape[0]):
            rc, o = gemv(libs[1], w, s, b, x[m], n_out, n_in, 64, threads=8)
            assert rc == 0
            if m == 0:
                for r in (2, 4, 8):
                    rc2, o2 = gemv(libs[r], w, s, b, x[m], n_out, n_in, 64, threads=8)
                    assert rc2 == 0 and np.array_equal(o.view(np.uint32), o2.view(np.uint32)), (name, r)
            rows.append(o)
        out = np.stack(rows)
        big[name] = out
        qwen[name] = {"seed": seed, "n_in": n_in, "n_out": n_out, "gs": 64, "m": int(x.shape[0]),
                      "sha256_w_s_b": synth.sha256(w, s, b), "sha256_x": synth.sha256(x),
                      "sha256_out": synth.sha256(out)}
        print(f"{name}: K={n_in} N={n_out} m={x.shape[0]} done", flush=True)
    np.savez_compressed(os.path.join(OUT_DIR, "golden_qwen7b.npz"), **big)
    manifest["qwen7b"] = qwen
    with open(os.path.join(OUT_DIR, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    print("wrote", OUT_DIR)


if __name__ == "__main__":
    main()
