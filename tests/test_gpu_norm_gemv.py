"""GEMVs with the residual add + RMSNorm folded into their prologue
(q4_norm_gemv_multi_dev, q4_norm_gate_up_silu_dev in include/q4decode.h).

The fused launch must equal, bit for bit, the two launches it replaces:
q4_add_rmsnorm_dev (the residual add hetero/cpu_model.py:305-306 and the
RMSNorm of :164-166) followed by q4_gemv_multi_dev / q4_gate_up_silu_dev,
which other tests pin to the oracle.  x_out must receive x + delta bit for
bit, and the input x must stay untouched.  The composition is also checked
against the oracle GEMV of an fp64 RMSNorm (north-star 1e-3 norm-wise).
"""
import numpy as np
import pytest

from hetero import q4, synth
import oracle

pytestmark = pytest.mark.gpu

OUT_TOL = 1e-3
EPS = 1e-6


def tensors(*arrays):
    import torch
    return [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in arrays]


def mats(seed, n_out, n_in):
    w, s, b = synth.qlinear(seed, n_out, n_in, 64)
    return (w, s, b), tuple(tensors(w, s.view(np.int16), b.view(np.int16)))


def unfused_input(lib, x, delta, nw):
    """q4_add_rmsnorm_dev on copies: (x + delta, y)."""
    import torch
    xc = x.clone()
    y = torch.empty_like(x)
    rc = lib.q4_add_rmsnorm_dev(xc.data_ptr(), None if delta is None else delta.data_ptr(), nw.data_ptr(), EPS,
                                y.data_ptr(), x.numel(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, q4.last_error(lib)
    return xc, y


@pytest.mark.parametrize("n_in,n_outs", [(3584, (3584, 512, 512)), (3584, (4097,)), (896, (896, 128, 128)),
                                         (8192, (1000, 24)), (64, (300,))])
@pytest.mark.parametrize("with_delta", [True, False])
def test_norm_gemv_multi_matches_two_launches(n_in, n_outs, with_delta):
    import torch
    print(f"norm gemv n_in={n_in} n_outs={n_outs} delta={with_delta}", flush=True)
    lib = q4.load()
    rng = np.random.default_rng(n_in + len(n_outs))
    ms = [mats(700 + k, n, n_in) for k, n in enumerate(n_outs)]
    x_np = rng.normal(0, 1, n_in).astype(np.float32)
    d_np = rng.normal(0, 1, n_in).astype(np.float32)
    w_np = rng.normal(1, 0.2, n_in).astype(np.float32)
    x, d, nw = tensors(x_np, d_np, w_np)
    delta = d if with_delta else None
    x_out = torch.full_like(x, 7.0)
    outs = q4.norm_gemv_multi_dev([t for _, t in ms], x, delta, nw, EPS, x_out=x_out, lib=lib)
    xs_ref, y = unfused_input(lib, x, delta, nw)
    refs = q4.gemv_multi_dev([t for _, t in ms], y.reshape(1, -1), lib=lib)
    torch.cuda.synchronize()
    for o, r in zip(outs, refs):
        assert torch.equal(o.view(torch.int32), r.view(torch.int32))
    assert np.array_equal(x.cpu().numpy(), x_np)                  # x is read only
    if with_delta:
        assert torch.equal(x_out.view(torch.int32), xs_ref.view(torch.int32))
    else:
        assert bool((x_out == 7.0).all())                         # nothing written without delta
    # against the oracle GEMV of an fp64 RMSNorm
    orc = oracle.Oracle()
    xs = (x_np + d_np if with_delta else x_np).astype(np.float64)
    y64 = (xs / np.sqrt((xs * xs).mean() + EPS) * w_np).astype(np.float32)
    for (nm, _), o in zip(ms, outs):
        assert oracle.normwise_rel(o.cpu().numpy()[0], orc.gemv(*nm, y64, 64)) < OUT_TOL


@pytest.mark.parametrize("n_in,n_inter", [(3584, 18944), (896, 4864)])
def test_norm_gate_up_matches_two_launches(n_in, n_inter):
    import torch
    print(f"norm gate/up n_in={n_in} n_inter={n_inter}", flush=True)
    lib = q4.load()
    rng = np.random.default_rng(n_inter)
    (_, gt), (_, ut) = mats(720, n_inter, n_in), mats(721, n_inter, n_in)
    x, d, nw = tensors(rng.normal(0, 1, n_in).astype(np.float32), rng.normal(0, 1, n_in).astype(np.float32),
                       rng.normal(1, 0.2, n_in).astype(np.float32))
    x_out = torch.empty_like(x)
    h = q4.norm_gate_up_silu_dev(gt, ut, x, d, nw, EPS, x_out=x_out, lib=lib)
    xs_ref, y = unfused_input(lib, x, d, nw)
    h_ref = q4.gate_up_silu_dev(gt, ut, y.reshape(1, -1), lib=lib)
    torch.cuda.synchronize()
    assert torch.equal(h.view(torch.int32), h_ref.view(torch.int32))
    assert torch.equal(x_out.view(torch.int32), xs_ref.view(torch.int32))


def test_norm_gemv_argument_errors():
    import torch
    lib = q4.load()
    (_, t) = mats(730, 64, 256)
    x = torch.zeros(256, device="cuda")
    with pytest.raises(RuntimeError):               # x_out aliasing x
        q4.norm_gemv_multi_dev([t], x, x, x, EPS, x_out=x, lib=lib)
    with pytest.raises(RuntimeError):               # n_in past the norm prologue's limit
        (_, big) = mats(731, 64, 8256)
        xb = torch.zeros(8256, device="cuda")
        q4.norm_gemv_multi_dev([big], xb, None, xb, EPS, lib=lib)


# The greedy token taken in lm_head's own launch (q4_norm_gemv_argmax_dev)
# against q4_norm_gemv_multi_dev followed by q4_argmax_dev (whose NumPy
# argmax rule other tests pin): logits bit for bit, token, history slot and
# position.  Planted: nothing; a tie (the argmax row copied to a lower row:
# the first index wins); NaN rows (fp16 NaN scales: the first NaN wins).
# Shapes: the Qwen vocabulary, and vocabularies that leave workgroups with
# no row.  Three calls in a row check that the arrival counter starts at 0
# each launch.
@pytest.mark.parametrize("n_in,n_out", [(3584, 152064), (512, 1000), (256, 37)])
def test_norm_gemv_argmax_matches_two_launches(n_in, n_out):
    import torch
    print(f"norm gemv argmax n_in={n_in} n_out={n_out}", flush=True)
    lib = q4.load()
    rng = np.random.default_rng(n_out)
    (w, s, b), _ = mats(900, n_out, n_in)
    x, d, nw = tensors(rng.normal(0, 1, n_in).astype(np.float32), rng.normal(0, 1, n_in).astype(np.float32),
                       rng.normal(1, 0.2, n_in).astype(np.float32))
    st = torch.cuda.current_stream().cuda_stream

    def state():
        return (torch.zeros(1, dtype=torch.int64, device="cuda"), torch.full((4,), -1, dtype=torch.int64, device="cuda"),
                torch.tensor([11], dtype=torch.int64, device="cuda"))

    def two_launches(mat):
        lg = q4.norm_gemv_multi_dev([mat], x, d, nw, EPS, lib=lib)[0]
        tok, hist, pos = state()
        rc = lib.q4_argmax_dev(lg.data_ptr(), n_out, tok.data_ptr(), hist.data_ptr(), pos.data_ptr(), 10, 4, st)
        assert rc == 0, q4.last_error(lib)
        return lg, tok, hist, pos

    def fused(mat, calls=1):
        tok, hist, pos = state()
        for _ in range(calls):
            lg = q4.norm_gemv_argmax_dev(mat, x, d, nw, EPS, tok, pos, hist=hist, s0=10, lib=lib)
        return lg, tok, hist, pos

    r = int(np.argmax(two_launches(tuple(tensors(w, s.view(np.int16), b.view(np.int16))))[0].cpu().numpy()))
    cases = [("none", w, s, b, r)]
    if r > 0:
        lo = r // 2
        w2, s2, b2 = w.copy(), s.copy(), b.copy()
        w2[lo], s2[lo], b2[lo] = w[r], s[r], b[r]
        cases.append(("tie", w2, s2, b2, lo))
    a, c = n_out // 3, n_out - 1
    s3 = s.copy()
    s3.view(np.uint16)[[a, c]] = 0x7E00                  # fp16 NaN
    cases.append(("nan", w, s3, b, a))
    for name, cw, cs, cb, expect in cases:
        mat = tuple(tensors(cw, cs.view(np.int16), cb.view(np.int16)))
        ref = two_launches(mat)
        got = fused(mat)
        torch.cuda.synchronize()
        assert torch.equal(got[0].view(torch.int32), ref[0].view(torch.int32)), name
        assert int(np.argmax(ref[0].cpu().numpy())) == expect, name
        for g, e in zip(got[1:], ref[1:]):
            assert torch.equal(g, e), (name, g, e)
        assert int(got[1].item()) == expect, name
    tok, hist, pos = fused(mat, calls=3)[1:]
    torch.cuda.synchronize()
    assert int(pos.item()) == 14 and hist.cpu().tolist() == [-1, a, a, a]


def test_greedy_and_argmax_on_two_streams():
    """Calls on two streams at once use arrays of their own (a set per
    stream): each stream's greedy token (q4_norm_gemv_argmax_dev, the Qwen
    vocabulary) and argmax (q4_argmax_dev) equal the same call alone, over
    rounds in which the two streams' launches overlap."""
    import torch
    lib = q4.load()
    n_in, n_out = 3584, 152064
    rng = np.random.default_rng(5)
    _, mat = mats(901, n_out, n_in)
    xs = [tensors(rng.normal(0, 1, n_in).astype(np.float32), rng.normal(1, 0.2, n_in).astype(np.float32))
          for _ in range(2)]
    logits = [torch.from_numpy(rng.normal(0, 1, 200003).astype(np.float32)).cuda() for _ in range(2)]
    want_g = [int(torch.argmax(q4.norm_gemv_multi_dev([mat], x, None, nw, EPS, lib=lib)[0]).item()) for x, nw in xs]
    want_a = [int(torch.argmax(lg).item()) for lg in logits]
    assert want_g[0] != want_g[1] and want_a[0] != want_a[1]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for rnd in range(8):
        toks = [torch.zeros(2, dtype=torch.int64, device="cuda") for _ in range(2)]
        poss = [torch.zeros(2, dtype=torch.int64, device="cuda") for _ in range(2)]
        torch.cuda.synchronize()                        # the fills above ran on the default stream
        for i in range(2):
            with torch.cuda.stream(streams[i]):
                x, nw = xs[i]
                q4.norm_gemv_argmax_dev(mat, x, None, nw, EPS, toks[i][:1], poss[i][:1], stream=streams[i], lib=lib)
                rc = lib.q4_argmax_dev(logits[i].data_ptr(), logits[i].numel(), toks[i][1:].data_ptr(), None,
                                       poss[i][1:].data_ptr(), 0, 0, streams[i].cuda_stream)
                assert rc == 0, q4.last_error(lib)
        torch.cuda.synchronize()
        for i in range(2):
            assert toks[i].cpu().tolist() == [want_g[i], want_a[i]], (rnd, i)
            assert poss[i].cpu().tolist() == [1, 1], (rnd, i)
