#!/usr/bin/env python3
"""Benchmark of the gfx950 int4 GEMV path on one MI355X.

Workload (one "step", the headline): the M=1 decode sweep of every
Qwen2.5-7B 4-bit projection -- 28 layers x (q, k, v, o, gate, up, down) +
lm_head, 3.99 GB of packed weights, fp16 scales/biases, fp32 x and y -- in
decode order with the projections that share x in one launch (q/k/v, and
gate+up): 4 launches per layer + lm_head = 113 launches per step, each with
its own x prologue.  Each layer has its own weights (3.9 GB resident in HBM,
far above the 256 MB Infinity Cache), so every step streams every weight
from HBM once.  The step is captured once in a HIP graph and replayed.  The
same sweep with one launch per projection (197 per step, as the reference's
caller makes one q4_gemv call per projection) is reported beside it.

Prints one JSON line:
  value         whole-step algorithmic GB/s (packed W + fp16 scales/biases +
                fp32 x and y per projection), inputs resident in HBM
  roofline      the GEMV kernel's achieved GB/s vs 8 TB/s, from HIP events on
                the launch stream over the timed replays
  per_shape     GB/s of each projection shape (events over back-to-back calls
                on distinct weights)
  small_m, prefill, wire, load
                the small-M / MLP block, M=512 prefill GEMM, activation wire
                codec and checkpoint-to-HBM legs
  decode        the 28-layer decode step (device-resident, HIP graph), its
                token agreement with the reference path's fixture, and the
                host CPU's decode rate on the reference kernel
  dropin        the NumPy stage on libq4gemv.so through the host-pointer ABI
  cpu_baseline  the reference kernel/q4gemv.c (compiled from source, tuned on
                this host) timed on a bounded sample of the same sweep
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "hetero-infer_amd"))

from hetero import sweep  # noqa: E402
from hetero.sweep import GS, HEAD_SHAPE, LAYER_SHAPES, LAYERS, gemv_bytes, make_weights  # noqa: E402,F401

HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


PMC_SUMMARY = os.path.join("profiles", "gemv_stream_qwen7b_decode_sweep_pmc.md")
CHAIN_PMC_SUMMARY = os.path.join("profiles", "gemv_chain_qwen7b_decode_sweep_trace_pmc.md")


def measured_traffic(summary=PMC_SUMMARY):
    """HBM bytes per sweep launch from a committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary
    (counter values scaled by a 256 MiB copy), or None when the summary is absent."""
    try:
        with open(os.path.join(ROOT, summary)) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def graph_us(torch, stream, body, calls, reps=5):
    """Average microseconds per call of `body` (which makes `calls` launches)
    captured in one HIP graph and replayed `reps` times on `stream`."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        body()
    with torch.cuda.stream(stream):
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * calls)


def group128_bench(torch, lib, dev, reps=5):
    """The M=1 projection sweep with group size 128 (MLX's other 4-bit
    layout): the grouped decode-order sweep (qkv, o, gate+up, down per
    layer, then lm_head) and each shape on its own, 28 distinct matrices
    per layer shape."""
    from hetero import q4
    gen = torch.Generator(device=dev)
    gen.manual_seed(4321)
    gs = 128
    layers = [[make_weights(torch, gen, n_out, n_in, dev, gs) for _, n_in, n_out in LAYER_SHAPES]
              for _ in range(LAYERS)]
    head = make_weights(torch, gen, HEAD_SHAPE[2], HEAD_SHAPE[1], dev, gs)
    xs = {k: torch.randn((1, k), device=dev, generator=gen) for k in (3584, 18944)}
    outs = {n: [torch.empty((1, n), device=dev) for _ in range(3)] for n in (512, 3584, 18944, 152064)}
    stream = torch.cuda.Stream(device=dev)
    torch.cuda.synchronize()

    def gemv(wsb):
        w, s, b = wsb
        n_out, n_in = w.shape[0], w.shape[1] * 8
        q4.check(lib, lib.q4_gemv_dev(w.data_ptr(), s.data_ptr(), b.data_ptr(), xs[n_in].data_ptr(),
                                      outs[n_out][0].data_ptr(), 1, n_out, n_in, gs, stream.cuda_stream),
                 "q4_gemv_dev")

    def multi(group):
        q4.gemv_multi_dev(group, xs[group[0][0].shape[1] * 8],
                          outs=[outs[g[0].shape[0]][i] for i, g in enumerate(group)], stream=stream, lib=lib)

    def sweep():
        for q, k, v, o, g, u, d in layers:
            multi([q, k, v])
            gemv(o)
            multi([g, u])
            gemv(d)
        gemv(head)

    n_launch = LAYERS * 4 + 1
    with torch.cuda.stream(stream):
        sweep()                                   # eager once: sizes the workspace
    torch.cuda.synchronize()
    us = graph_us(torch, stream, sweep, n_launch, reps)
    nbytes = LAYERS * sum(gemv_bytes(1, n_out, n_in, gs) for _, n_in, n_out in LAYER_SHAPES) \
        + gemv_bytes(1, HEAD_SHAPE[2], HEAD_SHAPE[1], gs)
    ms = us * n_launch * 1e-3
    res = {"gs": gs, "sweep_ms": round(ms, 4), "sweep_GB_s": round(nbytes / (ms * 1e-3) / 1e9, 1),
           "bytes_per_sweep": nbytes, "launches": n_launch, "per_shape": {}}
    for j, (name, n_in, n_out) in enumerate(LAYER_SHAPES + [HEAD_SHAPE]):
        items = [layers[l][j] for l in range(LAYERS)] if j < len(LAYER_SHAPES) else [head] * 4
        us = graph_us(torch, stream, lambda: [gemv(wsb) for wsb in items], len(items), reps)
        gbs = gemv_bytes(1, n_out, n_in, gs) / (us * 1e-6) / 1e9
        res["per_shape"][name] = {"K": n_in, "N": n_out, "us_per_call": round(us, 3), "GB_s": round(gbs, 1),
                                  "frac_peak": round(gbs / HBM_PEAK_GBS, 4)}
    del layers, head
    torch.cuda.empty_cache()
    return res


def prefill_bench(torch, lib, layers, dev, reps=3):
    """M=512 prompt over the 28 layers' projections: bf16 MFMA GEMM with the
    dequant fused into the weight-tile load.  Three launch patterns over the
    same work: one q4_gemm_bf16_dev per projection; the grouped form
    (q4_gemm_bf16_multi_dev over [q, k, v] and over [gate, up], which share
    their input, then o_proj and down_proj alone); and the prompt forward's
    form, x already in bf16 (q4_gemm_bf16in_multi_dev) and gate/up as paired
    tiles with SiLU * up in the epilogue, whose bf16 output is down's x
    (q4_gemm_bf16in_gate_up_silu_dev) -- the SiLU * mul is inside the timed
    work, its flops are not counted."""
    from hetero import q4
    m = 512
    xs = {k: torch.randn((m, k), device=dev) for k in (3584, 18944)}
    outs = {n: torch.empty((m, n), device=dev) for n in (512, 3584, 18944)}
    gouts = [torch.empty((m, n), device=dev) for n in (3584, 512, 512, 18944, 18944)]
    # the weights and x come from the default stream; the GEMMs run on a
    # non-blocking one
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=dev)
    flops = 0

    def step():
        for layer in layers:
            for w, s, b in layer:
                n_out, n_in = w.shape[0], w.shape[1] * 8
                rc = lib.q4_gemm_bf16_dev(w.data_ptr(), s.data_ptr(), b.data_ptr(), xs[n_in].data_ptr(),
                                          outs[n_out].data_ptr(), m, n_out, n_in, GS, stream.cuda_stream)
                if rc != 0:
                    raise RuntimeError(f"q4_gemm_bf16_dev rc={rc}: {q4.last_error(lib)}")

    def step_grouped():
        for layer in layers:
            q4.gemm_bf16_multi_dev(layer[0:3], xs[3584], outs=gouts[0:3], stream=stream, lib=lib)
            q4.gemm_bf16_dev(*layer[3], xs[3584], out=outs[3584], stream=stream, lib=lib)
            q4.gemm_bf16_multi_dev(layer[4:6], xs[3584], outs=gouts[3:5], stream=stream, lib=lib)
            q4.gemm_bf16_dev(*layer[6], xs[18944], out=outs[3584], stream=stream, lib=lib)

    xbs = {k: v.to(torch.bfloat16) for k, v in xs.items()}
    hb = torch.empty((m, 18944), dtype=torch.bfloat16, device=dev)

    def step_bf16():
        for layer in layers:
            q4.gemm_bf16_multi_dev(layer[0:3], xbs[3584], outs=gouts[0:3], stream=stream, lib=lib)
            q4.gemm_bf16_multi_dev([layer[3]], xbs[3584], outs=[outs[3584]], stream=stream, lib=lib)
            q4.gemm_bf16_gate_up_silu_dev(layer[4], layer[5], xbs[3584], h=hb, stream=stream, lib=lib)
            q4.gemm_bf16_multi_dev([layer[6]], hb, outs=[outs[3584]], stream=stream, lib=lib)

    def timed(fn):
        with torch.cuda.stream(stream):
            fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            fn()
        with torch.cuda.stream(stream):
            g.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(reps):
                g.replay()
            e1.record(stream)
            torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    for layer in layers:
        for w, _, _ in layer:
            flops += 2 * m * w.shape[0] * w.shape[1] * 8
    ms = timed(step)
    ms_grouped = timed(step_grouped)
    ms_bf16 = timed(step_bf16)
    tf = flops / (ms * 1e-3) / 1e12
    tf_grouped = flops / (ms_grouped * 1e-3) / 1e12
    tf_bf16 = flops / (ms_bf16 * 1e-3) / 1e12
    # error vs the reference contraction, fp32 dequant-matmul (hetero/cpu_model.py:119-136), on
    # each projection shape of layer 0: max |err| / max |ref| and norm-wise
    errs = {}
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    for (name, n_in, n_out), (w, s, b) in zip(LAYER_SHAPES, layers[0]):
        got = q4.gemm_bf16_dev(w, s, b, xs[n_in], lib=lib)
        ref = xs[n_in] @ q4.dequant_dev(w, s, b, lib=lib).t()
        d = (got - ref).double()
        errs[name] = {"max_rel": float(d.abs().max() / ref.double().abs().max()),
                      "normwise_rel": float(d.norm() / ref.double().norm())}
    torch.backends.cuda.matmul.allow_tf32 = prev
    worst = max(v["max_rel"] for v in errs.values())
    return {"workload": "M=512 prompt, 28 layers x 7 projections (K/N of the decode sweep), "
                        "group-64 dequant to bf16 fused into the weight-tile load, MFMA GEMM",
            "ms": round(ms, 3), "tflops": round(tf, 1), "frac_mfma_peak": round(tf / 2500.0, 4),
            "grouped": {"ms": round(ms_grouped, 3), "tflops": round(tf_grouped, 1),
                        "frac_mfma_peak": round(tf_grouped / 2500.0, 4),
                        "launches_per_layer": 4},
            "bf16_operands": {"ms": round(ms_bf16, 3), "tflops": round(tf_bf16, 1),
                              "frac_mfma_peak": round(tf_bf16 / 2500.0, 4), "launches_per_layer": 4,
                              "note": "x in bf16 from its producer; gate/up paired with the SiLU * up epilogue"},
            "peak_tflops_bf16_dense": 2500.0, "flops": flops,
            "max_rel_err_vs_fp32_dequant_matmul": round(worst, 6),
            "err_per_shape": {k: {kk: round(vv, 7) for kk, vv in v.items()} for k, v in errs.items()}}


def small_m_bench(torch, lib, layers, dev, ms=(1, 2, 4, 8), reps=5):
    """Small-M batched GEMV (M activation rows in flight): the q_proj shape
    (3584 -> 3584) and the MLP block (fused gate/up + SiLU*mul, then down),
    over the 28 layers' distinct weights so every call streams its weights
    from HBM; GB/s counts the weights once per call plus M rows of x and y."""
    from hetero import q4
    res = {}
    stream = torch.cuda.Stream(device=dev)
    for m in ms:
        x = torch.randn((m, 3584), device=dev)
        y = torch.empty((m, 3584), device=dev)
        h = torch.empty((m, 18944), device=dev)
        mo = torch.empty((m, 3584), device=dev)
        torch.cuda.synchronize()        # inputs from the default stream; the calls run on `stream`

        def step_q():
            for layer in layers:
                q4.gemv_dev(*layer[0], x, out=y, stream=stream, lib=lib)

        def step_mlp():
            for layer in layers:
                q4.mlp_dev(layer[4], layer[5], layer[6], x, h=h, out=mo, stream=stream, lib=lib)

        row = {}
        for name, step, nbytes in (
                ("q_proj", step_q, len(layers) * gemv_bytes(m, 3584, 3584)),
                ("mlp", step_mlp, len(layers) * (2 * gemv_bytes(m, 18944, 3584) + gemv_bytes(m, 3584, 18944)))):
            with torch.cuda.stream(stream):
                step()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                step()
            with torch.cuda.stream(stream):
                g.replay()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(reps):
                    g.replay()
                e1.record(stream)
                torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (reps * len(layers))
            gbs = nbytes / len(layers) / (us * 1e-6) / 1e9
            row[name] = {"us_per_call": round(us, 2), "GB_s": round(gbs, 1), "frac_peak": round(gbs / HBM_PEAK_GBS, 4)}
            del g
        res[f"M={m}"] = row
    return {"workload": "M rows of x (N(0,1)), q_proj 3584->3584 and the MLP block (gate/up 3584->18944 fused with "
                        "SiLU*mul, down 18944->3584), 28 layers of distinct weights, HIP graph", "rows": res}


def wire_bench(torch, lib, dev, rows_list=(1, 256, 2048), hidden=3584, reps=5):
    """Activation wire codec (include/q4wire.h): encode and decode of an fp32
    [rows][hidden] hidden state, both codecs.  Distinct input buffers (about
    600 MB in all, at most 64) are visited in turn inside one HIP graph, so
    the larger cases stream from HBM.  GB/s counts the fp32 side and the
    payload once per call."""
    from hetero import q4
    res = {}
    stream = torch.cuda.Stream(device=dev)
    for rows in rows_list:
        n = rows * hidden
        nb = int(min(64, max(2, -(-600_000_000 // (4 * n)))))
        xs = [torch.randn((rows, hidden), device=dev) for _ in range(nb)]
        outs = [torch.empty((rows, hidden), device=dev) for _ in range(nb)]
        torch.cuda.synchronize()        # inputs from the default stream; the calls run on `stream`
        row = {}
        for codec, cid in (("fp16", 0), ("int8", 1)):
            pb = int(lib.q4_wire_payload_bytes(cid, rows, hidden))
            pays = [torch.empty(pb, dtype=torch.uint8, device=dev) for _ in range(nb)]
            st = stream.cuda_stream

            def enc():
                for x, p in zip(xs, pays):
                    q4.check(lib, lib.q4_wire_encode_dev(x.data_ptr(), rows, hidden, cid, p.data_ptr(), st), "encode")

            def dec():
                for p, o in zip(pays, outs):
                    q4.check(lib, lib.q4_wire_decode_dev(p.data_ptr(), rows, hidden, cid, o.data_ptr(), st), "decode")

            for name, fn in (("encode", enc), ("decode", dec)):
                with torch.cuda.stream(stream):
                    fn()
                torch.cuda.synchronize()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=stream):
                    fn()
                with torch.cuda.stream(stream):
                    g.replay()
                    torch.cuda.synchronize()
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record(stream)
                    for _ in range(reps):
                        g.replay()
                    e1.record(stream)
                    torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / (reps * nb)
                gbs = (4 * n + pb) / (us * 1e-6) / 1e9
                row[f"{codec}_{name}"] = {"us_per_call": round(us, 3), "GB_s": round(gbs, 1),
                                          "frac_peak": round(gbs / HBM_PEAK_GBS, 4), "payload_bytes": pb}
                del g
            del pays
        res[f"rows={rows}"] = row
        del xs, outs
    return {"workload": f"fp32 hidden state [rows][{hidden}] ~ N(0,1) -> wire payload and back "
                        "(hetero/transport.py:198-225 with the NumPy backend's fp16 to_wire/from_wire), "
                        "distinct buffers per call, HIP graph", "rows": res}


def wire_cpu_baseline(rows_list=(1, 256, 2048), hidden=3584, budget_s=2.0):
    """The oracle's NumPy codec (a restatement of the reference's host
    encode/decode) on this host, per call, for the rows of wire_bench."""
    import numpy as np
    from oracle import wire
    res = {}
    rng = np.random.default_rng(0)
    for rows in rows_list:
        x = rng.standard_normal((rows, hidden)).astype(np.float32)
        row = {}
        for codec in ("fp16", "int8"):
            h, p = wire.stage_encode(x, codec)
            for name, fn in (("encode", lambda: wire.stage_encode(x, codec)),
                             ("decode", lambda: wire.stage_decode(h, p))):
                fn()
                k, t0 = 0, time.perf_counter()
                while time.perf_counter() - t0 < budget_s / (2 * len(rows_list) * 2) or k < 3:
                    fn()
                    k += 1
                row[f"{codec}_{name}"] = {"us_per_call": round((time.perf_counter() - t0) / k * 1e6, 1)}
        res[f"rows={rows}"] = row
    return {"kind": "port", "cores": 1, "sample": "oracle/wire.py (NumPy, one thread) on the same shapes",
            "rows": res}


def load_bench(torch, dev, layers=4, reps=2):
    """Checkpoint shard -> HBM (hetero/shard.py).  A synthetic MLX-layout
    checkpoint of `layers` Qwen2.5-7B decoder layers (131 MB each: U32
    weights, F16 scales/biases, F32 biases and norms, two layers per file)
    is written to a temporary directory.  It is then loaded three ways:
      * load_shard(framework="hip"): owned byte ranges through two pinned
        staging buffers, with async copies on a copy stream;
      * the reference's path, load_shard(framework="numpy") through the
        safetensors package (hetero/shard.py:131-153), then one device copy
        per tensor;
      * the same package read alone (no device), for scale.
    The files were just written, so they come from the page cache:
    host-memory -> HBM throughput, not disk."""
    import shutil
    import tempfile
    import numpy as np
    from safetensors import safe_open
    from safetensors.numpy import save_file
    from hetero import qwen2
    from hetero.shard import ShardSpec, WeightIndex
    cfg = qwen2.qwen2_7b_config(layers)
    h, inter = cfg["hidden_size"], cfg["intermediate_size"]
    kvd = h // cfg["num_attention_heads"] * cfg["num_key_value_heads"]
    rng = np.random.default_rng(0)
    d = tempfile.mkdtemp(prefix="q4ckpt", dir=os.environ.get("TMPDIR", "/tmp"))
    try:
        for f0 in range(0, layers, 2):
            t = {}
            for i in range(f0, min(layers, f0 + 2)):
                p = f"model.layers.{i}"
                for name, n_out, n_in, bias in (("self_attn.q_proj", h, h, True), ("self_attn.k_proj", kvd, h, True),
                                                ("self_attn.v_proj", kvd, h, True), ("self_attn.o_proj", h, h, False),
                                                ("mlp.gate_proj", inter, h, False), ("mlp.up_proj", inter, h, False),
                                                ("mlp.down_proj", h, inter, False)):
                    q = f"{p}.{name}"
                    t[f"{q}.weight"] = rng.integers(0, 2 ** 32, (n_out, n_in // 8), dtype=np.uint32)
                    t[f"{q}.scales"] = (rng.random((n_out, n_in // 64), dtype=np.float32) * 0.02).astype(np.float16)
                    t[f"{q}.biases"] = (rng.random((n_out, n_in // 64), dtype=np.float32) * -0.1).astype(np.float16)
                    if bias:
                        t[f"{q}.bias"] = rng.standard_normal(n_out, dtype=np.float32) * 0.02
                for nrm in ("input_layernorm", "post_attention_layernorm"):
                    t[f"{p}.{nrm}.weight"] = np.ones(h, np.float32)
            save_file(t, os.path.join(d, f"model-{f0 // 2:05d}.safetensors"), metadata={"format": "mlx"})
            del t
        with open(os.path.join(d, "config.json"), "w") as f:
            json.dump(cfg, f)
        idx = WeightIndex(d)
        spec = ShardSpec(0, layers, False, False)
        nbytes = idx.shard_bytes(spec)

        def ours():
            return idx.load_shard(spec, framework="hip", device=dev)

        def reference_path():
            out = {}
            for path in sorted({idx.entries[n][0] for n in idx.owned(spec)}):
                with safe_open(path, framework="numpy") as f:
                    for n in f.keys():
                        out[n] = torch.from_numpy(f.get_tensor(n)).to(dev)
            return out

        def host_only():
            out = {}
            for path in sorted({idx.entries[n][0] for n in idx.owned(spec)}):
                with safe_open(path, framework="numpy") as f:
                    for n in f.keys():
                        out[n] = f.get_tensor(n)
            return out

        res = {}
        for name, fn in (("load_shard_hip", ours), ("reference_numpy_then_copy", reference_path),
                         ("reference_numpy_host_only", host_only)):
            best = None
            for _ in range(reps):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                w = fn()
                torch.cuda.synchronize()
                dt = time.perf_counter() - t0
                del w
                best = dt if best is None else min(best, dt)
            res[name] = {"s": round(best, 4), "GB_s": round(nbytes / best / 1e9, 2)}
        return {"workload": f"{layers} Qwen2.5-7B decoder layers in MLX 4-bit layout, {nbytes} bytes in "
                            f"{len(os.listdir(d)) - 1} safetensors files (page cache) -> HBM", "bytes": nbytes,
                **res}
    finally:
        shutil.rmtree(d, ignore_errors=True)


DECODE_FIXTURE = os.path.join(ROOT, "tests", "golden", "decode_qwen7b.json")
PROMPT_FIXTURE = os.path.join(ROOT, "tests", "golden", "prompt_qwen7b.json")


def decode_model(torch, dev):
    """The Qwen2.5-7B-architecture decode workload of the committed fixture
    (28 layers, fp16 KV cache holding 2048 positions, seeded random-init
    4-bit weights), generated on the GPU; returns (cfg, meta, w, ks, vs)."""
    from hetero import qwen2
    with open(DECODE_FIXTURE) as f:
        meta = json.load(f)
    cfg = meta["config"]
    w = qwen2.synthetic_weights_torch(cfg, meta["seed"], dev)
    ks, vs = qwen2.synthetic_context_torch(cfg, meta["context"], meta["context_seed"], dev)
    torch.cuda.synchronize()
    return cfg, meta, w, ks, vs


def decode_bench(torch, dev, cfg, meta, w, ks, vs, steps=128):
    """Device-resident decode (one HIP graph replay per token) on the
    fixture's workload: tok/s over `steps` free-running steps, and token
    agreement with the reference path's tokens (tests/golden/decode_qwen7b.npz,
    written by the oracle on kernel/q4gemv.c), free-running and
    teacher-forced."""
    import numpy as np
    from hetero.gpu_model import GpuStage
    start = meta["start_token"]
    g = GpuStage(cfg, w, ks, vs, max_new=steps)
    g.reset(start)
    g.capture()
    g.reset(start)
    g.run(2)                                     # warm replays
    g.reset(start)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dev_tokens = g.run(steps)
    dev_s = time.perf_counter() - t0
    res = {"workload": meta["workload"] + ", one HIP graph replay per token",
           "steps": steps, "tok_s": round(steps / dev_s, 1), "ms_per_token": round(dev_s * 1e3 / steps, 3)}
    fx = np.load(DECODE_FIXTURE.replace(".json", ".npz"))
    ref = fx["greedy_tokens"].tolist()[:steps]
    n = len(ref)
    prefix = next((i for i, (a, b) in enumerate(zip(dev_tokens, ref)) if a != b), n)
    agree = {}
    for seq in ("greedy", "forced"):
        inputs = fx[f"{seq}_inputs"].tolist()[:n]
        g.reset(inputs[0])
        got = g.generate(n, tokens_in=inputs)
        agree[seq] = sum(int(a == b) for a, b in zip(got, fx[f"{seq}_tokens"].tolist()[:n]))
    margin = None
    if prefix < n:
        top = fx["greedy_top_val"][prefix]
        margin = round(float(top[0] - top[1]), 5)
    res.update({"free_running_identical_prefix": f"{prefix}/{n}",
                "reference_top2_margin_at_divergence": margin,
                "agree_teacher_forced": f"{agree['greedy']}/{n}",
                "agree_teacher_forced_random_tokens": f"{agree['forced']}/{n}",
                "reference_tokens": "tests/golden/decode_qwen7b.npz (oracle/decode.py on kernel/q4gemv.c)"})
    del g
    torch.cuda.empty_cache()
    return res


def prompt_bench(torch, dev, cfg, w, reps=3):
    """The 512-token prompt forward through the 28 layers on the device
    (GpuStage.prefill in one chunk: embedding rows, norms, the grouped bf16
    GEMMs, RoPE and the cache write, causal attention, the MLP, the final
    norm, lm_head and the greedy token of the last row), from an empty
    cache: time per prompt, prompt tokens/s, the TFLOP/s of its
    projections, and its last-position logits against the reference path's
    (tests/golden/prompt_qwen7b.npz, oracle/decode.py on kernel/q4gemv.c)."""
    import numpy as np
    import oracle
    from hetero.gpu_model import GpuStage
    with open(PROMPT_FIXTURE) as f:
        meta = json.load(f)
    fx = np.load(PROMPT_FIXTURE.replace(".json", ".npz"))
    ids = fx["ids"].tolist()
    n = len(ids)
    g = GpuStage(cfg, w, None, None, max_new=8)
    g.prefill(ids, chunk=n)                       # sizes the GEMM workspaces
    times = []
    for _ in range(reps):
        g.truncate(0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        tok = g.prefill(ids, chunk=n)             # ends with the token on the host: synchronised
        times.append(time.perf_counter() - t0)
    lg = g.logits.cpu().numpy().reshape(-1)
    ms = 1e3 * float(np.median(times))
    h, inter, nl = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"]
    kvd = cfg["num_key_value_heads"] * (h // cfg["num_attention_heads"])
    proj = nl * 2 * n * h * (h + 2 * kvd + h + 3 * inter) + 2 * h * cfg["vocab_size"]
    attn = nl * 2 * 2 * h * (n * (n + 1) // 2)    # q.k and p.v over the causal triangle, all heads
    ref = fx["ref_logits"]
    del g
    torch.cuda.empty_cache()
    return {"workload": f"{n}-token prompt (uniform random ids) through the 28-layer 4-bit Qwen2 stage in one chunk, "
                        "empty cache, last-position logits and greedy token",
            "ms": round(ms, 2), "prompt_tok_s": round(n / (ms * 1e-3), 1),
            "tflops_projections": round(proj / (ms * 1e-3) / 1e12, 1),
            "tflops_with_attention": round((proj + attn) / (ms * 1e-3) / 1e12, 1),
            "flops_projections": proj, "flops_attention": attn,
            "logits_err_vs_reference_path": round(oracle.normwise_rel(lg, ref), 6),
            "bf16_operand_drift_of_reference_path": round(meta["bf16_drift"]["logits"], 6),
            "greedy_token": tok, "reference_greedy_token": int(np.argmax(ref)),
            "reference": "tests/golden/prompt_qwen7b.npz (oracle/decode.py on kernel/q4gemv.c, fp32 BLAS)"}


def host_arrays(torch, w, ks, vs):
    """The decode model's tensors as host NumPy arrays (weights uint32,
    scales/biases float16, the rest float32; KV context float16)."""
    import numpy as np
    hw = {}
    for k, t in w.items():
        a = t.cpu().numpy()
        hw[k] = a.view(np.uint32) if k.endswith(".weight") and a.dtype == np.int32 else a
    return hw, [k.cpu().numpy() for k in ks], [v.cpu().numpy() for v in vs]


def dropin_bench(cfg, meta, hw, hks, hvs, steps=12):
    """The integration mode the reference's caller uses: the NumPy stage
    (hetero/numpy_stage.py) with every projection a host-pointer q4_gemv
    call into libq4gemv.so (x 14 KB in, y out through pinned staging; the
    weights uploaded once and kept resident).  tok/s over `steps` greedy
    steps after one warm-up step (which uploads the weights), the tokens
    checked against the reference path's, and the latency of one q4_gemv
    call on the q_proj shape."""
    import numpy as np
    from hetero import numpy_stage, q4
    lib = q4.load()
    st = numpy_stage.Stage(cfg, hw, lib=lib)
    caches = st.new_caches(hks, hvs, extra=steps + 1, dtype=np.float16)
    start = meta["start_token"]
    t0 = time.perf_counter()
    tok = numpy_stage.greedy(st(np.array([[start]]), caches, last_only=True))
    warm_s = time.perf_counter() - t0
    toks = [tok]
    t0 = time.perf_counter()
    for _ in range(steps):
        tok = numpy_stage.greedy(st(np.array([[tok]]), caches, last_only=True))
        toks.append(tok)
    dt = time.perf_counter() - t0
    ref = meta["tokens"][:len(toks)]
    # one q4_gemv call: 3584 -> 3584 (7 KB of x in, 14 KB of y out)
    qp = st.layers[0].q
    x = np.random.default_rng(0).standard_normal(qp.n_in).astype(np.float32)
    out = np.empty(qp.n_out, np.float32)
    args = (qp.w.ctypes.data, qp.scales.ctypes.data, qp.biases.ctypes.data, x.ctypes.data, out.ctypes.data,
            qp.n_out, qp.n_in, qp.group_size, 0)
    for _ in range(20):
        lib.q4_gemv(*args)
    reps = 500
    t1 = time.perf_counter()
    for _ in range(reps):
        lib.q4_gemv(*args)
    call_us = (time.perf_counter() - t1) / reps * 1e6
    lib.q4_release_all()
    return {"workload": "NumPy stage (hetero/numpy_stage.py) on libq4gemv.so through the host-pointer "
                        "q4_gemv ABI, the decode fixture's model and context",
            "tok_s": round(steps / dt, 2), "ms_per_token": round(dt * 1e3 / steps, 2),
            "first_step_s_incl_weight_upload": round(warm_s, 2),
            "agree_with_reference_tokens": f"{sum(int(a == b) for a, b in zip(toks, ref))}/{len(toks)}",
            "q4_gemv_call_us_3584x3584": round(call_us, 1)}


def host_statement():
    """The host the CPU baselines run on: CPU model, logical cpus allowed,
    physical cores among them, NUMA nodes, last-level cache, pinning."""
    allowed = sorted(os.sched_getaffinity(0))
    info = {"cpu_model": None, "logical_cpus_allowed": len(allowed), "os_cpu_count": os.cpu_count(),
            "physical_cores_allowed": None, "numa_nodes": None, "llc_bytes": None,
            "pinning": f"process affinity {allowed[0]}-{allowed[-1]}" if allowed == list(range(allowed[0], allowed[-1] + 1))
            else f"process affinity {allowed}"}
    try:
        cores, cur = set(), {}
        with open("/proc/cpuinfo") as f:
            for line in f.read().split("\n") + [""]:
                if not line.strip():
                    if cur.get("processor") is not None and int(cur["processor"]) in allowed:
                        cores.add((cur.get("physical id", "0"), cur.get("core id", cur["processor"])))
                    cur = {}
                    continue
                k, _, v = line.partition(":")
                cur[k.strip()] = v.strip()
                if k.strip() == "model name" and info["cpu_model"] is None:
                    info["cpu_model"] = v.strip()
        info["physical_cores_allowed"] = len(cores) or None
    except OSError:
        pass
    try:
        nodes = {}
        base = "/sys/devices/system/node"
        for n in sorted(os.listdir(base)):
            if n.startswith("node") and n[4:].isdigit():
                with open(os.path.join(base, n, "cpulist")) as f:
                    cl = f.read().strip()
                cpus = set()
                for part in cl.split(","):
                    if part:
                        a, _, b = part.partition("-")
                        cpus |= set(range(int(a), int(b or a) + 1))
                if cpus & set(allowed):
                    nodes[n] = cl
        info["numa_nodes"] = nodes
    except OSError:
        pass
    try:
        with open(f"/sys/devices/system/cpu/cpu{allowed[0]}/cache/index3/size") as f:
            v = f.read().strip()
        mult = {"K": 1024, "M": 1 << 20}.get(v[-1], 1)
        info["llc_bytes"] = int(v.rstrip("KM")) * mult
    except (OSError, ValueError):
        pass
    return info


def cpu_baseline(budget_s: float = 20.0):
    """The reference kernel/q4gemv.c, built from source (oracle/_ref, ROWS 1/2/4/8),
    tuned on this host by the procedure of kernel/autotune.py:49-75 (every ROWS x
    threads in {1, 2, 4, cpus, 2 cpus} within [1, 16]; 4 warm-up and 25 timed calls
    per shape) on the Qwen2.5-7B layer shapes, then timed on the M=1 sweep: passes
    over distinct layers whose weights span at least twice the last-level cache,
    the median of at least 5 repeats, extrapolated to 28 layers + lm_head."""
    import numpy as np
    import oracle
    from hetero import synth

    if not os.path.exists(oracle.ref_path(1)):
        return {"value": None, "unit": "GB/s", "cores": 0, "kind": "reference",
                "sample": "unavailable: oracle/_ref not built"}
    host = host_statement()
    cpus = host["logical_cpus_allowed"]
    threads_opts = sorted({1, 2, 4, cpus, 2 * cpus} & set(range(1, 17)))
    os.environ["HETERO_KERNEL_THREADS"] = str(max(threads_opts))   # pool size (q4gemv.c:218-223)
    layer_bytes = sum(gemv_bytes(1, n_out, n_in) for _, n_in, n_out in LAYER_SHAPES)
    llc = host["llc_bytes"] or (256 << 20)
    n_rot = max(2, -(-2 * llc // layer_bytes))
    t_gen = time.perf_counter()
    layers = [[synth.qlinear_ih_np(5000 + 10 * li + j, n_out, n_in, GS, tag="cpu.")
               for j, (_, n_in, n_out) in enumerate(LAYER_SHAPES)] for li in range(n_rot)]
    head = synth.qlinear_ih_np(5999, HEAD_SHAPE[2], HEAD_SHAPE[1], GS, tag="cpu.")
    gen_s = time.perf_counter() - t_gen
    xs = {k: synth.activations(77, 1, k)[0] for k in (3584, 18944)}
    outs = {n: np.empty(n, np.float32) for n in (512, 3584, 18944, 152064)}

    def call(lib, wsb, nt):
        w, s, b = wsb
        n_out, n_in = w.shape[0], w.shape[1] * 8
        rc = lib.q4_gemv(w.ctypes.data, s.ctypes.data, b.ctypes.data, xs[n_in].ctypes.data,
                         outs[n_out].ctypes.data, n_out, n_in, GS, nt)
        assert rc == 0

    # autotune: kernel/autotune.py:40-45 per shape (4 warm-up + 25 timed), summed over a layer's shapes
    t_start = time.perf_counter()
    tune = []
    libs = {}
    for rows in (1, 2, 4, 8):
        libs[rows] = oracle.load_ref(rows)
        for nt in threads_opts:
            tot = 0.0
            for wsb in layers[0]:
                for _ in range(4):
                    call(libs[rows], wsb, nt)
                t0 = time.perf_counter()
                for _ in range(25):
                    call(libs[rows], wsb, nt)
                tot += (time.perf_counter() - t0) / 25
            tune.append((tot, rows, nt))
    best_t, rows, nt = min(tune)
    tuning = {"rows": rows, "threads": nt, "seconds": best_t, "cpus": cpus, "arch": os.uname().machine}
    tune_s = time.perf_counter() - t_start
    lib = libs[rows]
    # timed sample: each repeat is one pass over the n_rot distinct layers
    for li in range(n_rot):
        for wsb in layers[li]:
            call(lib, wsb, nt)
    per_layer, t0 = [], time.perf_counter()
    while len(per_layer) < 5 or (time.perf_counter() - t0 < budget_s * 0.6 and len(per_layer) < 200):
        t1 = time.perf_counter()
        for li in range(n_rot):
            for wsb in layers[li]:
                call(lib, wsb, nt)
        per_layer.append((time.perf_counter() - t1) / n_rot)
    heads = []
    call(lib, head, nt)
    t0 = time.perf_counter()
    while len(heads) < 5 or (time.perf_counter() - t0 < budget_s * 0.2 and len(heads) < 100):
        t1 = time.perf_counter()
        call(lib, head, nt)
        heads.append(time.perf_counter() - t1)
    t_layer, t_head = float(np.median(per_layer)), float(np.median(heads))
    sweep_bytes = LAYERS * layer_bytes + gemv_bytes(1, HEAD_SHAPE[2], HEAD_SHAPE[1])
    t_sweep = LAYERS * t_layer + t_head
    p10, p90 = (float(np.percentile(per_layer, q)) for q in (10, 90))
    return {"value": round(sweep_bytes / t_sweep / 1e9, 3), "unit": "GB/s", "cores": nt,
            "kind": "reference", "rows": rows, "tuning_json": tuning, "host": host,
            "ms_per_sweep": round(t_sweep * 1e3, 3),
            "layer_ms_median_p10_p90": [round(t_layer * 1e3, 3), round(p10 * 1e3, 3), round(p90 * 1e3, 3)],
            "repeats": {"layer_passes": len(per_layer), "lm_head_calls": len(heads)},
            "sample": (f"kernel/q4gemv.c (clang -O3 -mavx2 -mfma -mf16c, ROWS={rows}, {nt} threads; tuned over "
                       f"ROWS 1/2/4/8 x threads {threads_opts} on the 7 layer shapes in {tune_s:.1f}s) on "
                       f"{cpus} host cpus ({host['physical_cores_allowed']} physical cores, {host['cpu_model']}): "
                       f"median of {len(per_layer)} passes over {n_rot} distinct layers "
                       f"({n_rot * layer_bytes / 1e6:.0f} MB, >= 2x the {llc / 1e6:.0f} MB last-level cache) "
                       f"and of {len(heads)} lm_head calls, extrapolated to 28 layers + lm_head: "
                       f"{t_sweep * 1e3:.1f} ms per sweep (inputs generated in {gen_s:.1f}s)")}


def cpu_decode_baseline(cfg, meta, hw, hks, hvs, rows, threads, steps=4):
    """Decode tok/s of the reference path on this host: the oracle's NumPy
    decode stage (oracle/decode.py) with every projection on the reference
    kernel/q4gemv.c built from source (tuned ROWS and threads), the fixture's
    workload, a bounded number of steps after one warm-up step; its tokens
    are checked against the fixture's."""
    import oracle
    from oracle.decode import DecodeOracle, greedy
    if not os.path.exists(oracle.ref_path(rows)):
        return None
    os.environ.setdefault("HETERO_KERNEL_THREADS", str(max(threads, 1)))
    orc = DecodeOracle(cfg, hw, hks, hvs, oracle.load_ref(rows), extra=steps + 1, nthreads=threads)
    tok = greedy(orc.logits(meta["start_token"]))
    toks = [tok]
    t0 = time.perf_counter()
    for _ in range(steps):
        tok = greedy(orc.logits(tok))
        toks.append(tok)
    dt = time.perf_counter() - t0
    ref = meta["tokens"][:len(toks)]
    return {"tok_s": round(steps / dt, 3), "ms_per_token": round(dt * 1e3 / steps, 1), "steps": steps,
            "agree_with_fixture": f"{sum(int(a == b) for a, b in zip(toks, ref))}/{len(toks)}",
            "kind": "reference", "cores": threads,
            "sample": f"oracle/decode.py on kernel/q4gemv.c ROWS={rows}, {threads} threads, {steps} timed steps"}


def chain_stamp_table(torch, chain, n_phases, dev, stream, reps=3):
    """Per-phase event times of the chained sweep (q4_chain_stamps, 100 MHz
    clock), per phase kind: medians over workgroups and layers, in
    microseconds, of each step of a phase -- the wait at the grid barrier
    before it, x loaded and staged, the int16 planes, wave 0's items, every
    wave's items and stores -- and the latency from the last workgroup's
    arrival to the first one's release.  Where the phase before does not
    write x, x is loaded and staged from the workgroup's arrival on, before
    the release; the items start at the later of release and planes.  An x
    prepared at the program's start is staged when its planes, group sums
    and scale are copied into LDS (planes then follow at once)."""
    import numpy as np
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    buf = torch.zeros((n_phases + 1) * cus * 8, dtype=torch.int64, device=dev)
    chain.stamps(buf)
    with torch.cuda.stream(stream):
        for _ in range(reps):
            chain.run(stream=stream)
    torch.cuda.synchronize()
    chain.stamps(None)
    t = buf.cpu().numpy().reshape(n_phases + 1, cus, 8).astype(np.float64) / 100.0   # us
    kinds = ["qkv", "o", "gate_up", "down"]
    rows = {}
    for p in range(1, n_phases):
        kind = "lm_head" if p == n_phases - 1 else kinds[p % 4]
        arrived, released, staged, planes, wave0 = (t[p, :, i] for i in range(1, 6))
        nxt = t[p + 1, :, 1]
        r = rows.setdefault(kind, {k: [] for k in ("barrier_wait", "release_after_last_arrival", "x_staged",
                                                   "planes", "items_wave0", "items_and_stores", "phase")})
        r["barrier_wait"].append(np.median(released - arrived))
        r["release_after_last_arrival"].append(released.min() - arrived.max())
        early = planes <= released
        ready = np.maximum(planes, released)
        r["x_staged"].append(np.median(staged - np.where(early, arrived, released)))
        r["planes"].append(np.median(planes - staged))
        r["items_wave0"].append(np.median(wave0 - ready))
        r["items_and_stores"].append(np.median(nxt - ready))
        r["phase"].append(np.median(nxt - arrived))
    return {k: {kk: round(float(np.median(vv)), 3) for kk, vv in v.items() if vv} for k, v in rows.items()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--no-graph", action="store_true", help="eager launches instead of a HIP graph")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-small-m", action="store_true")
    ap.add_argument("--no-wire", action="store_true")
    ap.add_argument("--wire-only", action="store_true", help="only the activation codec section")
    ap.add_argument("--no-load", action="store_true")
    ap.add_argument("--load-only", action="store_true", help="only the checkpoint-to-HBM section")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--decode-steps", type=int, default=128)
    ap.add_argument("--sweep-only", action="store_true",
                    help="only the grouped decode sweep (for rocprof runs)")
    ap.add_argument("--chain-only", action="store_true",
                    help="only the decode sweep as one chained program (for rocprof runs)")
    ap.add_argument("--chain-stamps", action="store_true",
                    help="with --chain-only: also the per-phase event times of the chained sweep")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the M=512 prefill leg (for counter runs)")
    ap.add_argument("--prompt-only", action="store_true",
                    help="only the 512-token prompt forward through the 28 layers (for rocprof runs)")
    ap.add_argument("--small-m-only", action="store_true",
                    help="only the small-M section (for rocprof runs)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the decode step (for rocprof runs)")
    ap.add_argument("--no-dropin", action="store_true",
                    help="skip the NumPy stage on libq4gemv.so through the host-pointer ABI")
    ap.add_argument("--dropin-only", action="store_true", help="only the host-pointer drop-in leg")
    ap.add_argument("--no-gs128", action="store_true", help="skip the group-size-128 sweep")
    ap.add_argument("--gs128-only", action="store_true", help="only the group-size-128 sweep")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run a 256 MiB device copy: the known-size reference for PMC byte counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); the int4 GEMV path "
              "shards by output rows with no collective in the kernel, so one GPU's throughput is "
              "the figure", file=sys.stderr)
        sys.exit(2)

    import torch
    from hetero import q4
    lib = q4.load()
    dev = torch.device("cuda:0")
    if args.load_only:
        print(json.dumps({"load": load_bench(torch, dev)}), flush=True)
        return
    if args.wire_only:
        res = wire_bench(torch, lib, dev)
        if not args.no_cpu_baseline:
            res["cpu_baseline"] = wire_cpu_baseline()
        print(json.dumps({"wire": res}), flush=True)
        return
    if args.decode_only:
        cfg, meta, w, ks, vs = decode_model(torch, dev)
        res = decode_bench(torch, dev, cfg, meta, w, ks, vs, steps=args.decode_steps)
        print(json.dumps({"decode": res}), flush=True)
        return
    if args.prompt_only:
        cfg, meta, w, ks, vs = decode_model(torch, dev)
        del ks, vs
        print(json.dumps({"prompt_forward": prompt_bench(torch, dev, cfg, w)}), flush=True)
        return
    if args.gs128_only:
        print(json.dumps({"group128": group128_bench(torch, lib, dev)}), flush=True)
        return
    if args.dropin_only:
        cfg, meta, w, ks, vs = decode_model(torch, dev)
        hw, hks, hvs = host_arrays(torch, w, ks, vs)
        del w, ks, vs
        torch.cuda.empty_cache()
        print(json.dumps({"dropin": dropin_bench(cfg, meta, hw, hks, hvs)}), flush=True)
        return
    t_setup = time.perf_counter()
    layers, head, xs = sweep.make_model(torch, dev, seed=1234)
    if args.prefill_only:
        print(json.dumps({"prefill": prefill_bench(torch, lib, layers, dev)}), flush=True)
        return
    if args.small_m_only:
        print(json.dumps({"small_m": small_m_bench(torch, lib, layers, dev)}), flush=True)
        return
    outs = {n: torch.empty((1, n), device=dev) for n in (512, 3584, 18944, 152064)}
    torch.cuda.synchronize()
    log(f"setup {time.perf_counter() - t_setup:.1f}s")
    stream = torch.cuda.Stream(device=dev)
    sp = stream.cuda_stream

    def gemv(wsb):
        w, s, b = wsb
        n_out, n_in = w.shape[0], w.shape[1] * 8
        rc = lib.q4_gemv_dev(w.data_ptr(), s.data_ptr(), b.data_ptr(), xs[n_in].data_ptr(),
                             outs[n_out].data_ptr(), 1, n_out, n_in, GS, sp)
        if rc != 0:
            raise RuntimeError(f"q4_gemv_dev rc={rc}: {q4.last_error(lib)}")

    def gemv_multi(group):
        k = len(group)
        n_in = group[0][0].shape[1] * 8
        arr = lambda vals: (ctypes.c_void_p * k)(*vals)
        rc = lib.q4_gemv_multi_dev(k, arr([g[0].data_ptr() for g in group]),
                                   arr([g[1].data_ptr() for g in group]),
                                   arr([g[2].data_ptr() for g in group]),
                                   arr([gouts[g[0].shape[0]][i].data_ptr() for i, g in enumerate(group)]),
                                   (ctypes.c_int * k)(*[g[0].shape[0] for g in group]),
                                   xs[n_in].data_ptr(), 1, n_in, GS, sp)
        if rc != 0:
            raise RuntimeError(f"q4_gemv_multi_dev rc={rc}: {q4.last_error(lib)}")

    gouts = {n: [torch.empty((1, n), device=dev) for _ in range(3)] for n in (512, 3584, 18944)}

    def step_calls():
        """One q4_gemv_dev call per projection, as the reference's caller makes them."""
        for layer in layers:
            for wsb in layer:
                gemv(wsb)
        gemv(head)

    def step_grouped():
        """Decode order, projections that share x in one launch: qkv, o, gate+up, down."""
        for q, k, v, o, g, u, d in layers:
            gemv_multi([q, k, v])
            gemv(o)
            gemv_multi([g, u])
            gemv(d)
        gemv(head)

    sweep_bytes = sweep.sweep_bytes()

    def timed(step, steps, warmup):
        with torch.cuda.stream(stream):
            step()                              # eager once: sizes the workspace
        torch.cuda.synchronize()
        graph = None
        if not args.no_graph:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                step()
            torch.cuda.synchronize()
        run = graph.replay if graph is not None else step
        with torch.cuda.stream(stream):
            for _ in range(warmup):
                run()
            torch.cuda.synchronize()
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            ev0.record(stream)
            for _ in range(steps):
                run()
            ev1.record(stream)
            torch.cuda.synchronize()
            wall = time.perf_counter() - t0
        return wall * 1e3 / steps, ev0.elapsed_time(ev1) / steps

    if args.chain_only:
        args.sweep_only = True
    n_launch = LAYERS * 4 + 1
    grouped_ms, grouped_ev = (float("nan"), float("nan")) if args.chain_only else \
        timed(step_grouped, args.steps, args.warmup)
    calls_ms = float("nan") if args.sweep_only else timed(step_calls, max(3, args.steps // 2), 1)[0]

    # the same sweep as one chained GEMV program (include/q4chain.h): one
    # launch, a grid barrier between phases, each phase's first weights
    # requested before its barrier.  Every phase of the sweep reads an x from
    # outside the program, as the reference's per-shape calls do, so each
    # phase's x is quantised once at the program's start (one workgroup per
    # phase) and only copied into LDS before its barrier.  It is the headline unless a barrier
    # wait timed out (then its outputs are not to be trusted and the grouped
    # launches give the figure).
    chained = None
    chain_ms = chain_ev = float("nan")
    chain_errors = -1
    chain_bad = None
    if args.chain_only or not args.sweep_only:
        # every phase its own outputs, so that after the timed replays each
        # one can be checked against the same phase run as its own launch
        phases = sweep.phases(layers, head, xs, sweep.distinct_outputs(torch, dev))
        chain = q4.Chain(phases, lib=lib)

        def step_chain():
            chain.run(stream=stream)

        chain_ms, chain_ev = timed(step_chain, args.steps, args.warmup)
        chain_errors = chain.errors()
        stamp_table = chain_stamp_table(torch, chain, len(phases), dev, stream) if args.chain_stamps else None
        chain.close()
        check = sweep.phases(layers, head, xs, sweep.distinct_outputs(torch, dev))
        with torch.cuda.stream(stream):
            sweep.run_launches(check, stream, lib=lib)
        torch.cuda.synchronize()
        chain_bad = sweep.mismatches(torch, phases, check)
        chained = {"ms_per_step": round(chain_ms, 4), "GB_s": round(sweep_bytes / (chain_ms * 1e-3) / 1e9, 1),
                   "phases": len(phases), "barrier_timeouts": chain_errors,
                   "outputs_vs_launches": {"phases_checked": len(phases),
                                           "values_checked": int(sum(o.numel() for ph in phases for o in ph[2])),
                                           "phases_differing": len(chain_bad),
                                           "first_differences": chain_bad[:5]}}
        if stamp_table is not None:
            chained["phase_events_us"] = stamp_table
        del phases, check
    use_chain = chain_errors == 0 and chain_bad == []
    if not use_chain and args.chain_only:
        raise SystemExit(f"the chained sweep reported {chain_errors} barrier timeouts and "
                         f"{len(chain_bad or [])} phases differing from their own launches")
    ms_per_step = chain_ms if use_chain else grouped_ms
    value = sweep_bytes / (ms_per_step * 1e-3) / 1e9

    if args.calibrate:
        src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    # per-shape: 28 back-to-back calls on distinct weights (lm_head: 4 calls, 307 MB each)
    per_shape = {}
    for j, (name, n_in, n_out) in enumerate([] if args.sweep_only else LAYER_SHAPES + [HEAD_SHAPE]):
        items = [layers[l][j] for l in range(LAYERS)] if j < len(LAYER_SHAPES) else [head] * 4
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for wsb in items:
                gemv(wsb)
        with torch.cuda.stream(stream):
            g.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 5
            e0.record(stream)
            for _ in range(reps):
                g.replay()
            e1.record(stream)
            torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * len(items))
        gbs = gemv_bytes(1, n_out, n_in) / (us * 1e-6) / 1e9
        per_shape[name] = {"K": n_in, "N": n_out, "us_per_call": round(us, 3),
                           "GB_s": round(gbs, 1), "frac_peak": round(gbs / HBM_PEAK_GBS, 4)}
        del g

    grouped_achieved = sweep_bytes / (grouped_ev * 1e-3) / 1e9
    if use_chain:
        achieved = sweep_bytes / (chain_ev * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4),
                    "traffic": measured_traffic(CHAIN_PMC_SUMMARY), "traffic_source": CHAIN_PMC_SUMMARY,
                    "algorithmic_bytes_per_launch": sweep_bytes,
                    "kernel": "gemv_chain_kernel: the whole sweep as one launch of 113 phases",
                    "avg_launch_us": round(chain_ev * 1e3, 3)}
        path = ("one chained GEMV program per step (include/q4chain.h): 113 phases in one persistent "
                "launch, a grid barrier between phases; each phase's x (read from outside the program) "
                "quantised once at the program's start; each phase's first weights and its prepared x "
                "loaded before its barrier")
        launches = 1
    else:
        achieved = grouped_achieved
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4),
                    "traffic": measured_traffic(), "traffic_source": PMC_SUMMARY,
                    "algorithmic_bytes_per_launch": round(sweep_bytes / n_launch),
                    "kernel": "gemv_stream_kernel<MR=1, RW, PAIR, RING, NORM=false> (x prologue "
                              "fused), averaged over the launches of the grouped sweep",
                    "avg_launch_us": round(grouped_ev * 1e3 / n_launch, 3)}
        path = "grouped launches, the projections that share x (qkv, gate+up) in one launch"
        launches = n_launch
    result = {
        "metric": "int4 GEMV HBM GB/s (% of MI355X peak) at Qwen2.5-7B shapes; decode tok/s",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4",
        "data": "synthetic (seeded uniform 4-bit weights, |N(0,0.02)| fp16 scales, "
                "-8*scale+N(0,0.002) fp16 biases, N(0,1) fp32 x)",
        "config": {"workload": "Qwen2.5-7B int4 projection sweep at M=1: 28 layers x "
                               "(q,k,v,o 3584->3584/512/512/3584, gate/up 3584->18944, "
                               "down 18944->3584) + lm_head 3584->152064, gs=64, distinct "
                               "weights per layer (3.99 GB per step), in decode order",
                   "path": path,
                   "global_batch": 1, "launches_per_step": launches,
                   "bytes_per_step": sweep_bytes, "hip_graph": not args.no_graph,
                   "parallelism": "single GPU"},
        "frac_of_peak": round(value / HBM_PEAK_GBS, 4),
        "roofline": roofline,
        "grouped_launches": None if args.chain_only else {
            "ms_per_step": round(grouped_ms, 4), "GB_s": round(sweep_bytes / (grouped_ms * 1e-3) / 1e9, 1),
            "frac_peak": round(sweep_bytes / (grouped_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "launches_per_step": n_launch,
            "kernel": "gemv_stream_kernel<MR=1, RW, PAIR, RING, NORM=false> (x prologue fused)",
            "avg_launch_us": round(grouped_ev * 1e3 / n_launch, 3),
            "achieved_per_launch_GB_s": round(grouped_achieved, 1),
            "traffic_per_launch": measured_traffic(), "traffic_source": PMC_SUMMARY},
        "per_shape": per_shape,
        "one_call_per_projection": {"ms_per_step": round(calls_ms, 4),
                                    "GB_s": round(sweep_bytes / (calls_ms * 1e-3) / 1e9, 1),
                                    "launches_per_step": LAYERS * len(LAYER_SHAPES) + 1},
        "chained": chained,
    }
    if args.sweep_only:
        args.no_prefill = args.no_cpu_baseline = args.no_decode = args.no_small_m = args.no_wire = True
        args.no_load = args.no_dropin = args.no_gs128 = True
    if not args.no_small_m:
        log("small-M ...")
        result["small_m"] = small_m_bench(torch, lib, layers, dev)
    if not args.no_prefill:
        log("prefill ...")
        result["prefill"] = prefill_bench(torch, lib, layers, dev)
    if not args.no_wire:
        log("wire codec ...")
        result["wire"] = wire_bench(torch, lib, dev)
        if not args.no_cpu_baseline:
            result["wire"]["cpu_baseline"] = wire_cpu_baseline()
    if not args.no_load:
        log("checkpoint load ...")
        result["load"] = load_bench(torch, dev)
    rows, threads = 1, 16
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        result["cpu_baseline"] = cpu_baseline(args.cpu_budget)
        rows = result["cpu_baseline"].get("rows", 1) or 1
        threads = result["cpu_baseline"].get("cores", 16) or 16
    else:
        result["cpu_baseline"] = None
    if not (args.no_decode and args.no_dropin and args.no_prefill):
        del layers, head
        torch.cuda.empty_cache()
        cfg, meta, w, ks, vs = decode_model(torch, dev)
        if not args.no_prefill:
            log("prompt forward ...")
            result["prompt_forward"] = prompt_bench(torch, dev, cfg, w)
        if not args.no_decode:
            log("decode ...")
            result["decode"] = decode_bench(torch, dev, cfg, meta, w, ks, vs, steps=args.decode_steps)
        hw = hks = hvs = None
        if not args.no_dropin or not args.no_cpu_baseline:
            hw, hks, hvs = host_arrays(torch, w, ks, vs)
        del w, ks, vs
        torch.cuda.empty_cache()
        if not args.no_dropin:
            log("drop-in (host-pointer ABI) ...")
            result["dropin"] = dropin_bench(cfg, meta, hw, hks, hvs)
        if not args.no_cpu_baseline and not args.no_decode:
            log("cpu decode baseline ...")
            result.setdefault("decode", {})["cpu_baseline"] = cpu_decode_baseline(cfg, meta, hw, hks, hvs, rows,
                                                                                 threads)
    if not args.no_gs128:
        log("group size 128 ...")
        result["group128"] = group128_bench(torch, lib, dev)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
