"""GPU checks of the prefill contraction q4_gemm_bf16_dev (bf16 MFMA GEMM with
the group-64 dequantisation fused into the weight-tile load).

Two references:
  * exact-operand: x and the dequantised weights rounded to bf16 (round to
    nearest even, the rule of q4_dequant_bf16_dev) and multiplied in fp64 --
    the kernel may differ only by its fp32 accumulation order (tolerance
    1e-5 norm-wise, stated here);
  * the reference's own contraction, fp32 dequant-matmul
    (hetero/cpu_model.py:119-136), computed here in fp64: the bf16 rounding
    of both operands sets the error; the maximum relative error is reported
    and bounded at 1e-2 norm-wise.
"""
import numpy as np
import pytest

from hetero import q4, synth
import oracle

pytestmark = pytest.mark.gpu

EXACT_OPERAND_TOL = 1e-5
BF16_TOL = 1e-2


def bf16_round(a):
    b = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return b.astype(np.uint32).view(np.float32)


# Shapes that take each tile height and split: (37, 200, 512) and
# (130, 96, 1024) partial 128-row and 256-column tiles; (512, 3584, 3584) and
# (512, 512, 3584) split along K; (500, 16600, 1024) a partial last tile of
# both kinds; (512, 18944, 3584) gate/up of a 512-token prompt unsplit;
# (512, 3584, 18944) and (64, 3584, 18944) down_proj, split along K
@pytest.mark.parametrize("m,n_out,n_in", [(37, 200, 512), (130, 96, 1024), (512, 3584, 3584),
                                          (512, 512, 3584), (64, 3584, 18944), (500, 16600, 1024),
                                          (512, 18944, 3584), (512, 3584, 18944)])
def test_gemm_bf16(m, n_out, n_in):
    import torch
    print(f"gemm m={m} n={n_out} k={n_in}", flush=True)
    w, s, b = synth.qlinear(700 + n_out, n_out, n_in, 64)
    x = synth.activations(701, m, n_in)
    tw, ts, tb, tx = (torch.from_numpy(a).cuda() for a in (w, s.view(np.int16), b.view(np.int16), x))
    got = q4.gemm_bf16_dev(tw, ts, tb, tx)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    wd = oracle.dequant_np(w, s, b, 64)
    exact = bf16_round(x).astype(np.float64) @ bf16_round(wd).astype(np.float64).T
    assert oracle.normwise_rel(got, exact) < EXACT_OPERAND_TOL
    ref = x.astype(np.float64) @ wd.astype(np.float64).T
    rel = oracle.normwise_rel(got, ref)
    print(f"max relative error vs fp32 dequant-matmul: {rel:.3e}")
    assert rel < BF16_TOL


def test_gemm_bf16_dequant_matches_bf16_dequant_kernel():
    """The weights the GEMM multiplies are exactly q4_dequant_bf16_dev's: with x
    a one-hot row selector the product returns dequantised columns."""
    import torch
    n_out, n_in = 64, 512
    w, s, b = synth.qlinear(710, n_out, n_in, 64)
    x = np.zeros((n_in, n_in), np.float32)
    x[np.arange(n_in), np.arange(n_in)] = 1.0
    tw, ts, tb, tx = (torch.from_numpy(a).cuda() for a in (w, s.view(np.int16), b.view(np.int16), x))
    got = q4.gemm_bf16_dev(tw, ts, tb, tx)             # [n_in, n_out] = W^T in bf16
    deq = q4.dequant_dev(tw, ts, tb, bf16=True).float()
    torch.cuda.synchronize()
    assert torch.equal(got.t().contiguous(), deq)


def _plan(monkeypatch, plan):
    if plan is None:
        monkeypatch.delenv("Q4_GEMM_PLAN", raising=False)
    else:
        monkeypatch.setenv("Q4_GEMM_PLAN", plan)


def _operands(seed, m, n_out, n_in):
    import torch
    w, s, b = synth.qlinear(seed, n_out, n_in, 64)
    x = synth.activations(seed + 1, m, n_in)
    dev = [torch.from_numpy(a).cuda() for a in (w, s.view(np.int16), b.view(np.int16), x)]
    exact = bf16_round(x).astype(np.float64) @ bf16_round(oracle.dequant_np(w, s, b, 64)).astype(np.float64).T
    return dev, exact


# Stream-K plans: P workgroups over tiles x G iterations, in 8 XCD groups
# when P is a multiple of 8 and there are at least 8 tiles (one group
# otherwise).  P = tiles gives every workgroup one whole tile (no partials);
# P = tiles + 1 cuts every range across two tiles (a partial and an owner
# segment each); the largest P gives ranges of one or two K steps, so an
# owner adds many partials (up to G - 1 of them).  (300, 600, 1024) and
# (500, 16600, 1024): ragged last tiles in both dimensions; the latter's 130
# tiles split 16/17 over the groups.  (512, 3584, 18944): 37-step ranges in
# 296-step tiles, 8 partials per owner.
@pytest.mark.parametrize("m,n_out,n_in,ps", [(37, 200, 512, (1, 3, 8)),
                                             (300, 600, 1024, (6, 7, 50, 96)),
                                             (512, 3584, 3584, (28, 29, 200, 256)),
                                             (500, 16600, 1024, (136, 256)),
                                             (512, 3584, 18944, (224,)),
                                             (512, 18944, 3584, (148, 256))])
def test_gemm_bf16_stream_k(monkeypatch, m, n_out, n_in, ps):
    import torch
    (tw, ts, tb, tx), exact = _operands(720 + m, m, n_out, n_in)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for p in ps:
        p = min(p, cus)
        print(f"stream-K m={m} n={n_out} k={n_in} P={p}", flush=True)
        _plan(monkeypatch, f"sk:{p}")
        a = q4.gemm_bf16_dev(tw, ts, tb, tx)
        b2 = q4.gemm_bf16_dev(tw, ts, tb, tx)
        torch.cuda.synchronize()
        got = a.cpu().numpy()
        assert np.isfinite(got).all(), "a tile's partials did not arrive"
        assert oracle.normwise_rel(got, exact) < EXACT_OPERAND_TOL
        assert torch.equal(a, b2), "stream-K sums in a fixed order: runs agree bit for bit"
        assert q4.prefill_errors() == 0, "a partial missed its wait"
    _plan(monkeypatch, None)


def test_gemm_bf16_stream_k_graph_replays(monkeypatch):
    """Each launch waits for flags carrying its own epoch, which the launch
    before it advanced, so a captured stream-K launch replays correctly:
    every replay equals the eager result bit for bit, and no partial ever
    misses its wait."""
    import torch
    m, n_out, n_in = 512, 3584, 3584
    (tw, ts, tb, tx), exact = _operands(760, m, n_out, n_in)
    _plan(monkeypatch, "sk:200")
    eager = q4.gemm_bf16_dev(tw, ts, tb, tx)            # workspace sized before capture
    torch.cuda.synchronize()
    out = torch.full_like(eager, float("nan"))
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        q4.gemm_bf16_dev(tw, ts, tb, tx, out=out, stream=s)   # this stream's workspace
        s.synchronize()
        with torch.cuda.graph(g, stream=s):
            q4.gemm_bf16_dev(tw, ts, tb, tx, out=out, stream=s)
    for r in range(4):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r}"
        q4.gemm_bf16_dev(tw, ts, tb, tx)                # eager work between replays
    assert q4.prefill_errors(stream=s) == 0 and q4.prefill_errors() == 0
    assert oracle.normwise_rel(eager.cpu().numpy(), exact) < EXACT_OPERAND_TOL
    _plan(monkeypatch, None)


@pytest.mark.parametrize("plan", ["sk:0", "sk:100000", "dp:64:1", "dp:256:3", "splitk"])
def test_gemm_bf16_plan_override_rejected(monkeypatch, plan):
    """A plan the shape cannot take is an error, not a silent fallback."""
    import torch
    (tw, ts, tb, tx), _ = _operands(770, 64, 512, 512)   # one tile of G = 8 K steps
    _plan(monkeypatch, plan)
    if plan == "dp:256:3":
        q4.gemm_bf16_dev(tw, ts, tb, tx)                # splits of 3, 3 and 2 steps: valid
        torch.cuda.synchronize()
    else:
        with pytest.raises(RuntimeError, match="Q4_GEMM_PLAN"):
            q4.gemm_bf16_dev(tw, ts, tb, tx)
    _plan(monkeypatch, None)


# Several matrices sharing x in one launch: q/k/v and gate/up of the Qwen
# shapes at M=512, and a ragged set -- 300 rows (a partial block), a matrix
# of no rows and 700 rows -- at M=200, under the default plan and forced
# data-parallel, split-K and stream-K plans.  Each output against its own
# exact-operand product; two runs agree bit for bit.
@pytest.mark.parametrize("m,n_in,n_outs,plans", [
    (512, 3584, (3584, 512, 512), (None, "dp:128:4", "sk:40")),
    (512, 3584, (18944, 18944), (None, "dp:256:1")),
    (200, 1024, (300, 0, 700), (None, "dp:256:3", "sk:8", "sk:5")),
])
def test_gemm_bf16_multi(monkeypatch, m, n_in, n_outs, plans):
    import torch
    mats, exacts = [], []
    x = synth.activations(780 + m, m, n_in)
    xr = bf16_round(x).astype(np.float64)
    for i, n in enumerate(n_outs):
        w, s, b = synth.qlinear(781 + i + n, max(n, 1), n_in, 64)
        w, s, b = w[:n], s[:n], b[:n]
        mats.append(tuple(torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (w, s.view(np.int16), b.view(np.int16))))
        exacts.append(xr @ bf16_round(oracle.dequant_np(w, s, b, 64)).astype(np.float64).T if n else None)
    tx = torch.from_numpy(x).cuda()
    for plan in plans:
        print(f"multi m={m} k={n_in} n={n_outs} plan={plan}", flush=True)
        _plan(monkeypatch, plan)
        a = q4.gemm_bf16_multi_dev(mats, tx)
        b2 = q4.gemm_bf16_multi_dev(mats, tx)
        torch.cuda.synchronize()
        for n, got, again, exact in zip(n_outs, a, b2, exacts):
            assert got.shape == (m, n)
            if n == 0:
                continue
            g = got.cpu().numpy()
            assert np.isfinite(g).all()
            assert oracle.normwise_rel(g, exact) < EXACT_OPERAND_TOL, (plan, n)
            assert torch.equal(got, again), (plan, n)
    _plan(monkeypatch, None)
