"""GPU checks of the prompt forward's bf16 operand path: the producers that
store the prefill GEMM's x operand in bf16 themselves, and the GEMM entry
points that take it so.

Each is pinned bit for bit to an fp32 entry point that is checked elsewhere
(test_gpu_prefill.py, test_gpu_decode_kernels.py, test_gpu_prompt.py),
followed by round-to-nearest-even to bf16 (torch's float32 -> bfloat16
conversion, the rule of x_to_bf16_kernel):
  * q4_gemm_bf16in_multi_dev(bf16(x)) == q4_gemm_bf16_multi_dev(x);
  * q4_gemm_bf16in_gate_up_silu_dev(bf16(x)) == bf16(SiLU(g) * u) with g, u
    from q4_gemm_bf16_multi_dev on {gate, up} under the unsplit plan and
    SiLU * u from q4_silu_mul_dev, in its one-workgroup-per-tile form; its
    stream-K form (tiles past one round of CUs, or forced) adds a tile's
    partial sums, so it is held next to that (a bf16 unit, more where a
    sum cancels), and to
    the float64 product of the same bf16 operands;
  * q4_add_rmsnorm_rows_bf16_dev == bf16(q4_add_rmsnorm_rows_dev), the
    residual written back the same, on the 16-byte and the scalar path;
  * q4_prompt_attention_bf16_dev == bf16(q4_prompt_attention_dev).
"""
import ctypes

import numpy as np
import pytest

from hetero import q4, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as t
    return t


@pytest.fixture(scope="module")
def lib():
    return q4.load()


def _sp(torch):
    return torch.cuda.current_stream().cuda_stream


def _mats(torch, seed, n_outs, n_in):
    mats = []
    for i, n in enumerate(n_outs):
        w, s, b = synth.qlinear(seed + i + n, max(n, 1), n_in, 64)
        w, s, b = w[:n], s[:n], b[:n]
        mats.append(tuple(torch.from_numpy(np.ascontiguousarray(a)).cuda()
                          for a in (w, s.view(np.int16), b.view(np.int16))))
    return mats


def _plan(monkeypatch, plan):
    if plan is None:
        monkeypatch.delenv("Q4_GEMM_PLAN", raising=False)
    else:
        monkeypatch.setenv("Q4_GEMM_PLAN", plan)


def _pair_plan(monkeypatch, plan):
    if plan is None:
        monkeypatch.delenv("Q4_PAIR_PLAN", raising=False)
    else:
        monkeypatch.setenv("Q4_PAIR_PLAN", plan)


def _bits(t):
    import torch
    return t.contiguous().view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32)


@pytest.mark.parametrize("m,n_in,n_outs,plan", [
    (512, 3584, (3584, 512, 512), None),          # q/k/v of a 512-token chunk, split along K
    (512, 18944, (3584,), None),                  # down
    (200, 1024, (300, 0, 700), "sk:8"),           # ragged, stream-K
    (37, 512, (200,), None),
])
def test_gemm_bf16in_equals_fp32_entry(torch, monkeypatch, m, n_in, n_outs, plan):
    print(f"bf16in m={m} k={n_in} n={n_outs} plan={plan}", flush=True)
    _plan(monkeypatch, plan)
    mats = _mats(torch, 900, n_outs, n_in)
    x = torch.from_numpy(synth.activations(901 + m, m, n_in)).cuda()
    want = q4.gemm_bf16_multi_dev(mats, x)
    got = q4.gemm_bf16_multi_dev(mats, x.to(torch.bfloat16))
    torch.cuda.synchronize()
    for n, a, b in zip(n_outs, got, want):
        assert a.shape == (m, n)
        assert torch.equal(_bits(a), _bits(b)), n
    _plan(monkeypatch, None)


@pytest.mark.parametrize("m,n_inter,n_in", [(512, 18944, 3584), (300, 1000, 1024), (37, 200, 512), (1, 130, 64)])
def test_gate_up_silu_epilogue_equals_separate_calls(torch, lib, monkeypatch, m, n_inter, n_in):
    print(f"gate/up silu m={m} n={n_inter} k={n_in}", flush=True)
    gate, up = _mats(torch, 920, (n_inter, n_inter), n_in)
    xb = torch.from_numpy(synth.activations(921 + m, m, n_in)).cuda().to(torch.bfloat16)
    _plan(monkeypatch, "dp:256:1")              # every K step in one workgroup, as the paired tiles
    g, u = q4.gemm_bf16_multi_dev([gate, up], xb)
    _plan(monkeypatch, None)
    h32 = torch.empty_like(g)
    assert lib.q4_silu_mul_dev(g.data_ptr(), u.data_ptr(), h32.data_ptr(), g.numel(), _sp(torch)) == 0
    _pair_plan(monkeypatch, "dp")
    got = q4.gemm_bf16_gate_up_silu_dev(gate, up, xb)
    again = q4.gemm_bf16_gate_up_silu_dev(gate, up, xb)
    _pair_plan(monkeypatch, None)
    torch.cuda.synchronize()
    assert got.dtype == torch.bfloat16 and got.shape == (m, n_inter)
    assert torch.isfinite(got.float()).all()
    assert torch.equal(_bits(got), _bits(h32.to(torch.bfloat16)))
    assert torch.equal(_bits(got), _bits(again))


# the default plan of a 512-token prompt (296 tiles: stream-K over the
# CUs), and forced stream-K plans on small shapes: 8 and 5 workgroups
# (fewer than the tiles: ranges of several tiles), 64 (more than the
# tiles: several partials per tile), 3 over a single tile row
@pytest.mark.parametrize("m,n_inter,n_in,plan", [(512, 18944, 3584, None), (300, 1000, 1024, "sk:8"),
                                                 (300, 1000, 1024, "sk:5"), (300, 1000, 1024, "sk:64"),
                                                 (37, 200, 512, "sk:3")])
def test_gate_up_silu_stream_k(torch, lib, monkeypatch, m, n_inter, n_in, plan):
    print(f"gate/up silu stream-K m={m} n={n_inter} k={n_in} plan={plan}", flush=True)
    gate, up = _mats(torch, 940, (n_inter, n_inter), n_in)
    xb = torch.from_numpy(synth.activations(941 + m, m, n_in)).cuda().to(torch.bfloat16)
    _pair_plan(monkeypatch, "dp")
    want = q4.gemm_bf16_gate_up_silu_dev(gate, up, xb)
    _pair_plan(monkeypatch, plan)
    got = q4.gemm_bf16_gate_up_silu_dev(gate, up, xb)
    again = q4.gemm_bf16_gate_up_silu_dev(gate, up, xb)
    _pair_plan(monkeypatch, None)
    torch.cuda.synchronize()
    assert lib.q4_prefill_errors(_sp(torch)) == 0
    assert torch.equal(_bits(got), _bits(again))
    assert torch.isfinite(got.float()).all()
    # next to the one-workgroup-per-tile result: the fp32 sums differ in
    # their last places (relative to the sum of the terms' magnitudes, so
    # more near a cancelling sum), and the bf16 rounding may then move by a
    # unit: |diff| <= 2^-7 |want| + 1e-5 max |want|
    g32, w32 = got.float(), want.float()
    diff = (g32 - w32).abs()
    moved = int((_bits(got) != _bits(want)).sum())
    print(f"stream-K vs one workgroup per tile: {moved} of {got.numel()} values moved, largest "
          f"{float(diff.max()) / float(w32.abs().max()):.2e} of max |h|", flush=True)
    assert bool((diff <= 2.0 ** -7 * w32.abs() + 1e-5 * w32.abs().max()).all())
    # and against float64 with the same bf16 operands
    import oracle
    xr = xb.float().cpu().numpy().astype(np.float64)
    wg, wu = (oracle.dequant_np(*synth.qlinear(940 + i + n_inter, n_inter, n_in, 64), 64) for i in (0, 1))
    bf = lambda a: torch.from_numpy(a.astype(np.float32)).to(torch.bfloat16).float().numpy().astype(np.float64)
    g64, u64 = xr @ bf(wg).T, xr @ bf(wu).T
    ref = g64 / (1 + np.exp(-g64)) * u64
    err = oracle.normwise_rel(got.float().cpu().numpy(), ref)
    print(f"normwise error vs float64: {err:.2e}", flush=True)
    assert err < 8e-3                             # bf16 output rounding, 2^-8 relative at most


def test_gate_up_silu_argument_errors(torch, lib):
    gate, up = _mats(torch, 930, (64, 64), 128)
    xb = torch.zeros((4, 128), dtype=torch.bfloat16, device="cuda")
    h = torch.empty((4, 64), dtype=torch.bfloat16, device="cuda")
    P = lambda t: t.data_ptr()
    args = lambda gs, x=xb: (*(P(t) for t in gate), *(P(t) for t in up), P(x), P(h), 4, 64, 128, gs, _sp(torch))
    assert lib.q4_gemm_bf16in_gate_up_silu_dev(*args(32)) == -1             # the reference's shape code
    assert lib.q4_gemm_bf16in_gate_up_silu_dev(*args(128)) == q4.Q4_EARG     # the GEMM takes group size 64
    assert lib.q4_gemm_bf16in_gate_up_silu_dev(*args(64, xb[:, 1:])) == q4.Q4_EARG   # x not 16-byte aligned
    assert lib.q4_gemm_bf16in_gate_up_silu_dev(*args(64)) == 0


@pytest.mark.parametrize("n,aligned,with_delta", [(3584, True, True), (3584, True, False), (1000, True, True),
                                                  (100, True, True), (3584, False, True)])
def test_norm_rows_bf16_equals_fp32_entry(torch, lib, n, aligned, with_delta):
    """n = 3584 and 1000 take the 16-byte path when aligned; n = 100 (not a
    multiple of 8) and a buffer one float off alignment take the scalar one."""
    print(f"norm rows bf16 n={n} aligned={aligned} delta={with_delta}", flush=True)
    rng = np.random.default_rng(n)
    rows, off = 7, 0 if aligned else 1
    x = rng.normal(0, 3, (rows, n)).astype(np.float32)
    d = rng.normal(0, 1, (rows, n)).astype(np.float32)
    w = rng.normal(1, 0.1, n).astype(np.float32)

    def dev(a):                                   # [rows][n] starting `off` floats into its buffer
        buf = torch.zeros(a.size + off, dtype=torch.float32, device="cuda")
        v = buf[off:].view(a.shape)
        v.copy_(torch.from_numpy(a))
        return v
    tw = dev(w)
    x1, x2 = dev(x), dev(x)
    td = dev(d) if with_delta else None
    y32 = torch.empty((rows, n), device="cuda")
    yb = torch.empty(rows * n + 8, dtype=torch.bfloat16, device="cuda")[off:off + rows * n].view(rows, n)
    dp = td.data_ptr() if with_delta else None
    assert lib.q4_add_rmsnorm_rows_dev(x1.data_ptr(), dp, tw.data_ptr(), 1e-6, y32.data_ptr(), rows, n,
                                       _sp(torch)) == 0
    assert lib.q4_add_rmsnorm_rows_bf16_dev(x2.data_ptr(), dp, tw.data_ptr(), 1e-6, yb.data_ptr(), rows, n,
                                            _sp(torch)) == 0, q4.last_error(lib)
    torch.cuda.synchronize()
    assert torch.equal(_bits(x1), _bits(x2))
    assert torch.equal(_bits(yb), _bits(y32.to(torch.bfloat16)))


def test_prompt_attention_bf16_equals_fp32_entry(torch, lib):
    nh, nkv, d, cap, pos0, rows = 28, 4, 128, 320, 64, 200
    rng = np.random.default_rng(77)
    q = torch.from_numpy(rng.normal(0, 1, (rows, nh * d)).astype(np.float32)).cuda()
    kc = torch.from_numpy(rng.normal(0, 1, (nkv, cap, d)).astype(np.float16)).cuda()
    vc = torch.from_numpy(rng.normal(0, 1, (nkv, cap, d)).astype(np.float16)).cuda()
    o32 = torch.empty((rows, nh * d), device="cuda")
    ob = torch.empty((rows, nh * d), dtype=torch.bfloat16, device="cuda")
    scale = ctypes.c_float(d ** -0.5).value
    P = lambda t: t.data_ptr()
    assert lib.q4_prompt_attention_dev(P(q), P(kc), P(vc), P(o32), rows, pos0, nh, nkv, d, cap, scale,
                                       _sp(torch)) == 0
    assert lib.q4_prompt_attention_bf16_dev(P(q), P(kc), P(vc), P(ob), rows, pos0, nh, nkv, d, cap, scale,
                                            _sp(torch)) == 0, q4.last_error(lib)
    torch.cuda.synchronize()
    assert torch.equal(_bits(ob), _bits(o32.to(torch.bfloat16)))
