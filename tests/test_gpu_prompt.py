"""The device-resident prompt forward and KV-cache growth
(hetero/gpu_model.py GpuStage.prefill / _ensure) on a 2-layer
Qwen2-architecture model with random 4-bit weights.

The reference runs a prompt chunk through its stage with causal attention,
q4_gemv per row up to 16 rows and q4_dequant + fp32 BLAS above
(hetero/cpu_model.py:119-158, :233-252, :357-368; chunks from
hetero/coordinator.py:175-182).  oracle/decode.py restates that path
(DecodeOracle.prompt, pinned against a float64 textbook decode in
tests/test_oracle_decode.py).  The device runs chunks of more than 16 rows
on the bf16 matrix-core GEMM, so its logits differ from the reference
path's by the bf16 rounding of the GEMM operands.  That rounding's effect
is measured in the same test: the oracle run with both operands of its
contraction rounded to bf16 (gemm_bf16=True) drifts from the reference path
by `drift` (max |diff| / max |ref|).  The bars, per case:
  * logits against the reference path: max(2 drift, LOGIT_TOL = 1e-3), and
    the greedy token equal unless the reference's top two are within that
    error;
  * logits against the bf16 oracle: max(drift / 4, LOGIT_TOL) -- the device
    sits with the bf16 rounding, what is left is fp32 summation order
    (which can flip the bf16 rounding of single elements);
  * the keys and values the prompt wrote to the cache, layer 0 and the last
    layer: against the reference path's, within max(2 d, LOGIT_TOL) where d
    is the bf16 oracle's drift of the same rows; a cached context is not
    touched;
  * decode steps after the prompt against the bf16 oracle continuing from
    its own prompt, max(drift / 2, LOGIT_TOL): the cache positions, the
    position and the token carry over.
With no chunk above 16 rows there is no GEMM, drift is 0 and every bar is
LOGIT_TOL.

At full size -- the 28-layer Qwen2.5-7B-architecture model of the decode
fixture, an empty cache and a 512-token prompt in one chunk -- the device
runs against the committed fixture tests/golden/prompt_qwen7b.npz (written
by tests/golden/make_prompt_golden.py: the oracle on the reference kernel,
and the same with bf16 contraction operands, whose drift the fixture
records): last-position logits within max(2 drift, LOGIT_TOL) of the
reference path's and nearer the bf16 run's than that run is to the
reference, the greedy token equal unless the reference's top two are
within the error, and the keys and values of layers 0 and 27 within twice
their recorded drift.
"""
import json
import os

import numpy as np
import pytest

import oracle
from oracle.decode import DecodeOracle, greedy
from hetero import qwen2

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3
CONTEXT = 64
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
needs_ref = pytest.mark.skipif(not os.path.exists(oracle.ref_path(1)), reason="oracle/_ref not built")


def small_cfg():
    cfg = qwen2.qwen2_7b_config(layers=2)
    cfg.update(hidden_size=512, intermediate_size=1024, num_attention_heads=4,
               num_key_value_heads=2, vocab_size=1000)
    return cfg


@pytest.fixture(scope="module")
def model():
    cfg = small_cfg()
    w = qwen2.synthetic_weights(cfg, seed=11)
    ks, vs = qwen2.synthetic_context(cfg, CONTEXT, seed=12)
    return cfg, w, ks, vs


def _ids(n, seed):
    return [int(t) for t in np.random.default_rng(seed).integers(0, 1000, n)]


# (context cached before the prompt, prompt length, chunk): 40 rows in
# chunks of 24 (GEMM) and 16 (GEMV); 5 rows (GEMV) after a context; 70 rows
# in one GEMM chunk after a context (attention over 134 positions, 3 tiles)
CASES = [(False, 40, 24), (True, 5, 512), (True, 70, 512)]


@needs_ref
@pytest.mark.parametrize("ctx,n,chunk", CASES, ids=lambda v: str(v))
def test_prefill_vs_oracle(model, ctx, n, chunk):
    import torch
    from hetero.gpu_model import GpuStage
    cfg, w, ks, vs = model
    ids = _ids(n, seed=n)
    steps = 3
    kk, vv = (ks, vs) if ctx else (None, None)
    lib = oracle.load_ref(1)
    ref = DecodeOracle(cfg, w, kk, vv, lib, extra=n + steps)
    bf = DecodeOracle(cfg, w, kk, vv, lib, extra=n + steps, gemm_bf16=True)
    for lo in range(0, n, chunk):
        l_ref = ref.prompt(ids[lo:lo + chunk])
        l_bf = bf.prompt(ids[lo:lo + chunk])
    print(f"case ctx={ctx} n={n} chunk={chunk}", flush=True)
    g = GpuStage(cfg, w, kk, vv, max_new=4)
    tok = g.prefill(ids, chunk=chunk)
    torch.cuda.synchronize()
    lg = g.logits.cpu().numpy().reshape(-1)
    drift = oracle.normwise_rel(l_bf, l_ref)
    e_bf, e_ref = oracle.normwise_rel(lg, l_bf), oracle.normwise_rel(lg, l_ref)
    tol_ref = max(2 * drift, LOGIT_TOL)
    print(f"bf16 drift {drift:.2e}; device vs bf16 oracle {e_bf:.2e}, vs reference path {e_ref:.2e} "
          f"(bar {tol_ref:.2e})", flush=True)
    assert e_bf < max(drift / 4, LOGIT_TOL)
    assert e_ref < tol_ref
    want = greedy(l_ref)
    if tok != want:
        gap = float(l_ref[want]) - float(l_ref[tok])
        assert gap <= 2 * e_ref * float(np.abs(l_ref).max()), f"token {tok} != {want} (gap {gap:.3e})"
    # the cache rows the prompt wrote
    s0 = CONTEXT if ctx else 0
    for i in (0, cfg["num_hidden_layers"] - 1):
        for name in ("k", "v"):
            mine = g.layers[i][f"{name}_cache"][:, :s0 + n].cpu().numpy().astype(np.float32)
            r = getattr(ref, name)[i][0, :, :s0 + n].astype(np.float32)
            b = getattr(bf, name)[i][0, :, :s0 + n].astype(np.float32)
            d, e = oracle.normwise_rel(b[:, s0:], r[:, s0:]), oracle.normwise_rel(mine[:, s0:], r[:, s0:])
            print(f"layer {i} {name}: bf16 drift {d:.2e}, device vs reference path {e:.2e}", flush=True)
            assert e < max(2 * d, LOGIT_TOL), f"layer {i} {name}"
            if ctx:
                assert np.array_equal(mine[:, :s0], r[:, :s0]), f"layer {i} {name}: the context moved"
    assert g.position == s0 + n and int(g.pos.item()) == s0 + n
    # decode from the prompt's end, teacher-forced on the bf16 oracle's tokens
    g.capture()
    t_bf = greedy(l_bf)
    for step in range(steps):
        l_b = bf.logits(t_bf)
        g.set_token(t_bf)
        g.step()
        e = oracle.normwise_rel(g.logits.cpu().numpy().reshape(-1), l_b)
        print(f"decode step {step} after the prompt: {e:.2e} from the bf16 oracle", flush=True)
        assert e < max(drift / 2, LOGIT_TOL), f"decode step {step} after the prompt: {e:.2e}"
        t_bf = greedy(l_b)


def test_prefill_argument_errors(model):
    from hetero.gpu_model import GpuStage
    cfg, w, ks, vs = model
    g = GpuStage(cfg, w, None, None, max_new=2)
    with pytest.raises(ValueError):
        g.prefill([])
    with pytest.raises(ValueError):
        g.prefill([1, 2], chunk=0)


def test_cache_growth_and_capture_after_eager_steps(model):
    """A stage whose cache must grow twice while decoding, with two eager
    steps before the graph is captured, gives the logits of a stage built
    large enough, step for step, bit for bit (the attention of a position
    does not depend on the capacity past it)."""
    import torch
    from hetero.gpu_model import GpuStage, KV_STEP
    cfg, w, ks, vs = model
    steps = 2 * KV_STEP + 6
    big = GpuStage(cfg, w, ks, vs, max_new=steps)
    small = GpuStage(cfg, w, ks, vs, max_new=2)
    cap0 = small.cap
    toks = _ids(steps, seed=3)
    for i, t in enumerate(toks):
        for g in (big, small):
            g.set_token(t)
            g.step()
            if i == 1 and g is small:
                g.capture()                      # after two eager steps: the position carries on
        a = big.logits.cpu().numpy().reshape(-1)
        b = small.logits.cpu().numpy().reshape(-1)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"step {i}"
    torch.cuda.synchronize()
    assert small.cap > cap0 + KV_STEP and small.position == CONTEXT + steps
    assert int(small.pos.item()) == CONTEXT + steps


def test_qwen7b_prompt_full_size_vs_reference_fixture():
    """The 512-token prompt forward of the 28-layer model against the
    reference path's fixture."""
    import torch
    from hetero.gpu_model import GpuStage
    from test_gpu_decode import _checksum_torch
    with open(os.path.join(GOLDEN, "prompt_qwen7b.json")) as f:
        meta = json.load(f)
    fx = np.load(os.path.join(GOLDEN, "prompt_qwen7b.npz"))
    with open(os.path.join(GOLDEN, "decode_qwen7b.json")) as f:
        sums = json.load(f)
    assert sums["seed"] == meta["seed"] and sums["config"] == meta["config"]
    cfg, dev = meta["config"], torch.device("cuda")
    print("generating the 28-layer model on the GPU", flush=True)
    w = qwen2.synthetic_weights_torch(cfg, meta["seed"], dev)
    bad = [k for k, v in sums["input_checksums"].items() if k in w and int(v) != _checksum_torch(w[k])]
    assert not bad, f"generated weights differ from the fixture's: {bad[:5]}"
    g = GpuStage(cfg, w, None, None, max_new=4)
    del w
    ids = fx["ids"].tolist()
    print(f"prefill of {len(ids)} tokens", flush=True)
    tok = g.prefill(ids, chunk=len(ids))
    lg = g.logits.cpu().numpy().reshape(-1)
    ref, bfl = fx["ref_logits"], fx["bf16_logits"]
    drift = meta["bf16_drift"]["logits"]
    e_ref, e_bf = oracle.normwise_rel(lg, ref), oracle.normwise_rel(lg, bfl)
    print(f"bf16 drift {drift:.2e}; device vs reference path {e_ref:.2e}, vs bf16 run {e_bf:.2e}", flush=True)
    failures = []
    if not e_ref < max(2 * drift, LOGIT_TOL):
        failures.append(f"logits {e_ref:.2e} from the reference path")
    if not e_bf < max(drift, LOGIT_TOL):
        failures.append(f"logits {e_bf:.2e} from the bf16 run")
    want = int(np.argmax(ref))
    if tok != want:
        gap = float(ref[want]) - float(ref[tok])
        if gap > 2 * e_ref * float(np.abs(ref).max()):
            failures.append(f"token {tok} != {want} (gap {gap:.3e})")
    for l in meta["kv_layers"]:
        for kv in "kv":
            mine = g.layers[l][f"{kv}_cache"][:, :len(ids)].cpu().numpy().astype(np.float32)
            e = oracle.normwise_rel(mine, fx[f"kv_{l}_{kv}"].astype(np.float32))
            d = meta["bf16_drift"][f"kv_{l}_{kv}"]
            print(f"layer {l} {kv}: {e:.2e} from the reference path (bf16 drift {d:.2e})", flush=True)
            if not e < max(2 * d, LOGIT_TOL):
                failures.append(f"layer {l} {kv}: {e:.2e}")
    assert not failures, failures
