#!/usr/bin/env python3
"""Rounding sensitivity of the decode fixture's model (tests/golden/
decode_qwen7b.json), which sets the logit tolerance of the device-resident
decode test.

The device-resident decode computes the same step as the reference path,
but its RMSNorm, softmax, exp and attention dot products round differently
from NumPy's pairwise sums, SIMD exp and BLAS.  How far that moves the
logits is a property of the model: this script perturbs the reference path
(oracle/decode.py on the reference kernel) by single roundings and records
how far its own step-0 logits move (max |diff| / max |ref|):
  * norm_fp64      every RMSNorm evaluated in float64, rounded once to float32
  * attention_fp64 the attention (scores, softmax, weighted sum) in float64
  * norm_w_ulp     layer 0's input-norm weights moved up by one ulp
and, for the drift a decode accumulates through its own KV cache, the
norm_fp64 variant run teacher-forced through all the fixture's steps of
both sequences, against the fixture's top-k logits (worst step) and whole
logit vectors (first and last step).  It adds them to decode_qwen7b.json
under "sensitivity".

Run from the repository root after make_decode_golden.py (a few minutes):
    python tests/golden/decode_sensitivity.py
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "hetero-infer_amd"))
from hetero import qwen2  # noqa: E402
import oracle  # noqa: E402
from oracle import decode as odec  # noqa: E402

META = os.path.join(os.path.dirname(os.path.abspath(__file__)), "decode_qwen7b.json")


def main():
    with open(META) as f:
        meta = json.load(f)
    cfg = meta["config"]
    w = qwen2.synthetic_weights(cfg, meta["seed"])
    ks, vs = qwen2.synthetic_context(cfg, meta["context"], meta["context_seed"])
    threads = min(16, os.cpu_count() or 1)
    os.environ.setdefault("HETERO_KERNEL_THREADS", str(threads))
    lib = oracle.load_ref(1)

    def step0():
        return odec.DecodeOracle(cfg, w, ks, vs, lib, extra=1, nthreads=threads).logits(meta["start_token"])

    base = step0()
    res = {}
    norm, sdpa = odec._norm, odec._sdpa

    def norm64(x, g, eps):
        x64 = x.astype(np.float64)
        return (x64 * (1.0 / np.sqrt((x64 * x64).mean(-1, keepdims=True) + eps)) * g).astype(np.float32)

    odec._norm = norm64
    res["norm_fp64"] = oracle.normwise_rel(step0(), base)
    odec._norm = norm
    odec._sdpa = lambda q, k, v, scale: sdpa(q.astype(np.float64), k.astype(np.float64), v.astype(np.float64),
                                             scale).astype(np.float32)
    res["attention_fp64"] = oracle.normwise_rel(step0(), base)
    odec._sdpa = sdpa
    name = "model.layers.0.input_layernorm.weight"
    g0 = w[name]
    w[name] = np.nextafter(g0, np.float32(np.inf))
    res["norm_w_ulp"] = oracle.normwise_rel(step0(), base)
    w[name] = g0
    # the norm_fp64 variant through every step, teacher-forced
    fx = np.load(META.replace(".json", ".npz"))
    full = {int(s): k for k, s in enumerate(fx["full_steps"])}
    odec._norm = norm64
    for seq in ("greedy", "forced"):
        orc = odec.DecodeOracle(cfg, w, ks, vs, lib, extra=meta["steps"], nthreads=threads)
        worst_top = 0.0
        for i, tok in enumerate(fx[f"{seq}_inputs"].tolist()):
            lg = orc.logits(tok).astype(np.float64)
            top = fx[f"{seq}_top_val"][i].astype(np.float64)
            worst_top = max(worst_top, float(np.max(np.abs(lg[fx[f"{seq}_top_idx"][i]] - top)) / fx[f"{seq}_amax"][i]))
            if i in full:
                res[f"norm_fp64_{seq}_step{i}_whole"] = oracle.normwise_rel(lg, fx[f"{seq}_full_logits"][full[i]])
        res[f"norm_fp64_{seq}_worst_top"] = worst_top
        print(seq, res, flush=True)
    odec._norm = norm
    meta["sensitivity"] = {"measure": "max |logits - reference| / max |reference|", **res}
    with open(META, "w") as f:
        json.dump(meta, f, indent=1)
    print(json.dumps(meta["sensitivity"]))


if __name__ == "__main__":
    main()
