#!/usr/bin/env python3
"""Write the golden prompt-forward fixture of the Qwen2.5-7B-architecture stage.

The workload: the model of decode_qwen7b.json (28 layers, hidden 3584,
28 query / 4 KV heads, head_dim 128, random-init 4-bit group-64 weights from
seed SEED, hetero/qwen2.py) with an empty cache, and a prompt of PROMPT
uniformly random token ids (seeded) run as one chunk -- the prefill of the
512-token prompt workload.  The reference path is oracle/decode.py
(DecodeOracle.prompt: the reference's NumPy stage for L rows, causal
attention, each projection a q4_dequant + fp32 BLAS contraction) on
oracle/_ref/libq4gemv_ref_r1.so, the reference kernel/q4gemv.c compiled from
source by oracle/Makefile.

The same oracle is run a second time with both operands of every
contraction rounded to bf16 (gemm_bf16=True): the operands of the device's
matrix-core prefill GEMM.  How far that rounding alone moves the results
is recorded, so the GPU test can state its bar from it.

Stored in prompt_qwen7b.npz (described in prompt_qwen7b.json):
  ids                [PROMPT]       the prompt's token ids
  ref_logits         [vocab]        the last position's logits, reference path
  bf16_logits        [vocab]        the same with bf16 contraction operands
  ref_top_idx / _val [TOPK]         the reference's TOPK largest logits, descending
  kv_<l>_<k|v>       [4, PROMPT, 128] fp16, layers 0 and 27: the cache the prompt wrote
and in the json the drift of the bf16 run (max |diff| / max |ref|) for the
logits and each stored cache block.

Run from the repository root after `make -C oracle` (about ten minutes on
8 cpus; about 8 GB of memory):
    python tests/golden/make_prompt_golden.py
"""
from __future__ import annotations

import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "hetero-infer_amd"))
from hetero import qwen2, synth  # noqa: E402
import oracle  # noqa: E402
from oracle.decode import DecodeOracle  # noqa: E402

OUT_DIR = os.path.dirname(os.path.abspath(__file__))
SEED, PROMPT, TOPK = 2026, 512, 64
KV_LAYERS = (0, 27)


def rel(a, b) -> float:
    return oracle.normwise_rel(a, b)


def main():
    t0 = time.time()
    cfg = qwen2.qwen2_7b_config(28)
    w = qwen2.synthetic_weights(cfg, SEED)
    ids = [int(t) for t in (synth.u64(SEED + 3, "prompt.tokens", PROMPT) % np.uint64(cfg["vocab_size"]))]
    print(f"generated in {time.time() - t0:.1f}s", flush=True)
    os.environ.setdefault("HETERO_KERNEL_THREADS", str(min(16, os.cpu_count() or 1)))
    lib = oracle.load_ref(1)
    nt = min(16, os.cpu_count() or 1)
    runs = {}
    for name, bf16 in (("ref", False), ("bf16", True)):
        t1 = time.time()
        orc = DecodeOracle(cfg, w, None, None, lib, extra=PROMPT, kv_dtype=np.float16, nthreads=nt, gemm_bf16=bf16)
        lg = orc.prompt(ids).reshape(-1)
        runs[name] = (lg, {l: (orc.k[l][0, :, :PROMPT].copy(), orc.v[l][0, :, :PROMPT].copy()) for l in KV_LAYERS})
        print(f"{name}: {time.time() - t1:.1f}s", flush=True)
    ref, bf = runs["ref"], runs["bf16"]
    order = np.lexsort((np.arange(ref[0].size), -ref[0].astype(np.float64)))[:TOPK]
    arrays = {"ids": np.array(ids, np.int64), "ref_logits": ref[0], "bf16_logits": bf[0],
              "ref_top_idx": order.astype(np.int32), "ref_top_val": ref[0][order]}
    drift = {"logits": rel(bf[0], ref[0])}
    for l in KV_LAYERS:
        for j, kv in enumerate("kv"):
            arrays[f"kv_{l}_{kv}"] = ref[1][l][j]
            drift[f"kv_{l}_{kv}"] = rel(bf[1][l][j].astype(np.float32), ref[1][l][j].astype(np.float32))
    np.savez_compressed(os.path.join(OUT_DIR, "prompt_qwen7b.npz"), **arrays)
    meta = {"workload": f"Qwen2-architecture prefill: the model of decode_qwen7b.json, an empty cache, a {PROMPT}-token "
                        "prompt of uniform random token ids in one chunk; the last position's logits",
            "reference": "oracle/decode.py DecodeOracle.prompt on kernel/q4gemv.c (ROWS=1) built by oracle/Makefile: "
                         "q4_dequant of 512-row blocks + fp32 BLAS per projection",
            "config": cfg, "seed": SEED, "prompt": PROMPT, "prompt_seed": SEED + 3, "topk": TOPK,
            "kv_layers": list(KV_LAYERS),
            "bf16_drift": {k: float(v) for k, v in drift.items()},
            "bf16_drift_meaning": "max |bf16 - ref| / max |ref| of the oracle run with both operands of every "
                                  "contraction rounded to bf16 (round to nearest even)",
            "greedy_token": int(np.argmax(ref[0])), "greedy_token_bf16": int(np.argmax(bf[0]))}
    with open(os.path.join(OUT_DIR, "prompt_qwen7b.json"), "w") as f:
        json.dump(meta, f, indent=1)
    print(f"done in {time.time() - t0:.1f}s; drift {drift}", flush=True)


if __name__ == "__main__":
    main()
