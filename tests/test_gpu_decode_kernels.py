"""Decode-step kernels (include/q4decode.h) against references of the same ops.

* embedding row: bit-exact with the dequantisation of that row (the oracle's
  restatement of hetero/cpu_model.py:67-81);
* RoPE + bias + KV-cache write: bit-exact with the reference's fp32
  expressions (hetero/cpu_model.py:195-204) evaluated by NumPy, the cache as
  NumPy's float16 rounding of the same values;
* residual add + RMSNorm: the add bit-exact; y bit-exact with the
  reference's NumPy expression (hetero/cpu_model.py:164-166) for the row
  lengths NumPy's pairwise sum halves exactly (the Qwen2 hidden sizes
  among them), one row and several; other lengths within 1e-6 (norm-wise)
  of an fp64 evaluation (a tree sum there);
* attention: within 1e-5 (norm-wise) of an fp64 masked GQA softmax over the
  fp16 cache (hetero/cpu_model.py:233-252), at positions on both sides of
  the 64-position chunk boundaries;
* fused RoPE + attention: bit-exact (output and both caches) with
  q4_rope_kv_dev followed by q4_attention_dev over a run of decode positions;
* argmax: the first index of the maximum, with planted ties, and the step
  bookkeeping (token, history slot, position + 1).
"""
import numpy as np
import pytest

import oracle
from hetero import q4

pytestmark = pytest.mark.gpu

RMS_TOL = 1e-6
ATTN_TOL = 1e-5


@pytest.fixture(scope="module")
def torch():
    import torch as t
    return t


@pytest.fixture(scope="module")
def lib():
    return q4.load()


def sp(torch):
    return torch.cuda.current_stream().cuda_stream


def test_embed_row_bit_exact(torch, lib):
    rng = np.random.default_rng(3)
    n_rows, n_in, gs = 300, 3584, 64
    w = rng.integers(0, 2**32, (n_rows, n_in // 8), dtype=np.uint64).astype(np.uint32)
    s = (np.abs(rng.normal(0, 0.02, (n_rows, n_in // gs))).astype(np.float16)).view(np.uint16)
    b = (rng.normal(0, 0.02, (n_rows, n_in // gs)).astype(np.float16)).view(np.uint16)
    dev = torch.device("cuda")
    tw = torch.from_numpy(w.view(np.int32)).to(dev)
    ts = torch.from_numpy(s.view(np.int16)).to(dev)
    tb = torch.from_numpy(b.view(np.int16)).to(dev)
    out = torch.empty(n_in, device=dev)
    for t in (0, 17, n_rows - 1):
        tok = torch.tensor([t], dtype=torch.int64, device=dev)
        rc = lib.q4_embed_dev(tw.data_ptr(), ts.data_ptr(), tb.data_ptr(), tok.data_ptr(), out.data_ptr(),
                              n_rows, n_in, gs, sp(torch))
        assert rc == 0, q4.last_error(lib)
        ref = oracle.dequant_np(w[t:t + 1], s[t:t + 1].view(np.float16), b[t:t + 1].view(np.float16),
                                gs).reshape(-1)
        assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32)), t


PAIRWISE_EXACT = (3584, 896, 1536, 2048, 5120, 8192, 64, 120)


def test_add_rmsnorm(torch, lib):
    from hetero.numpy_stage import rms_norm
    rng = np.random.default_rng(4)
    dev = torch.device("cuda")
    for n in PAIRWISE_EXACT + (1000, 4104):
        x = rng.normal(0, 1, n).astype(np.float32)
        d = rng.normal(0, 1, n).astype(np.float32)
        w = rng.normal(1, 0.1, n).astype(np.float32)
        tx, td, tw = (torch.from_numpy(a).to(dev) for a in (x, d, w))
        y = torch.empty(n, device=dev)
        rc = lib.q4_add_rmsnorm_dev(tx.data_ptr(), td.data_ptr(), tw.data_ptr(), 1e-6, y.data_ptr(), n, sp(torch))
        assert rc == 0, q4.last_error(lib)
        xs = x + d                                   # fp32 add, as x + attn in the reference
        assert np.array_equal(tx.cpu().numpy(), xs)
        x64 = xs.astype(np.float64)
        ref = x64 / np.sqrt((x64 * x64).mean() + 1e-6) * w
        assert oracle.normwise_rel(y.cpu().numpy(), ref) < RMS_TOL, n
        if n in PAIRWISE_EXACT:
            want = rms_norm(xs, w, 1e-6)
            assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32)), n
        # no residual: x untouched
        rc = lib.q4_add_rmsnorm_dev(tx.data_ptr(), None, tw.data_ptr(), 1e-6, y.data_ptr(), n, sp(torch))
        assert rc == 0 and np.array_equal(tx.cpu().numpy(), xs)
    assert lib.q4_add_rmsnorm_dev(tx.data_ptr(), None, tw.data_ptr(), 1e-6, y.data_ptr(), 8193, None) == q4.Q4_EARG


def test_add_rmsnorm_rows_bit_exact_with_numpy(torch, lib):
    """A prompt's rows: each as the one-row kernel, all equal to NumPy's
    rms_norm over the [rows, n] block (the reduction runs per row)."""
    from hetero.numpy_stage import rms_norm
    rng = np.random.default_rng(5)
    dev = torch.device("cuda")
    rows, n = 5, 3584
    x = rng.normal(0, 3, (rows, n)).astype(np.float32)
    d = rng.normal(0, 1, (rows, n)).astype(np.float32)
    w = rng.normal(1, 0.1, n).astype(np.float32)
    tx, td, tw = (torch.from_numpy(a).to(dev) for a in (x, d, w))
    y = torch.empty((rows, n), device=dev)
    rc = lib.q4_add_rmsnorm_rows_dev(tx.data_ptr(), td.data_ptr(), tw.data_ptr(), 1e-6, y.data_ptr(), rows, n,
                                     sp(torch))
    assert rc == 0, q4.last_error(lib)
    xs = x + d
    assert np.array_equal(tx.cpu().numpy(), xs)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), rms_norm(xs[None], w, 1e-6)[0].view(np.uint32))


def rope_np(x, cos, sin):
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * cos - x2 * sin, x1 * sin + x2 * cos], axis=-1)


def test_rope_kv_bit_exact(torch, lib):
    rng = np.random.default_rng(5)
    nh, nkv, d, cap = 28, 4, 128, 300
    half = d // 2
    inv = 1e6 ** (-np.arange(0, half, dtype=np.float32) * 2.0 / d)
    ang = np.arange(cap, dtype=np.float32)[:, None] * inv[None, :]
    cos, sin = np.cos(ang), np.sin(ang)
    dev = torch.device("cuda")
    q = rng.normal(0, 1, nh * d).astype(np.float32)
    k = rng.normal(0, 1, nkv * d).astype(np.float32)
    v = rng.normal(0, 1, nkv * d).astype(np.float32)
    bias = rng.normal(0, 0.1, (nh + 2 * nkv) * d).astype(np.float32)
    tq, tk, tv, tb, tc, ts = (torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in (q, k, v, bias, cos, sin))
    kc = torch.zeros((nkv, cap, d), dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    qo = torch.empty(nh * d, device=dev)
    for p in (0, 1, 137, cap - 1):
        pos = torch.tensor([p], dtype=torch.int64, device=dev)
        rc = lib.q4_rope_kv_dev(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), tb.data_ptr(), tc.data_ptr(),
                                ts.data_ptr(), pos.data_ptr(), kc.data_ptr(), vc.data_ptr(), qo.data_ptr(),
                                nh, nkv, d, cap, sp(torch))
        assert rc == 0, q4.last_error(lib)
        qb = (q + bias[:nh * d]).reshape(nh, d)
        kb = (k + bias[nh * d:(nh + nkv) * d]).reshape(nkv, d)
        vb = (v + bias[(nh + nkv) * d:]).reshape(nkv, d)
        q_ref = rope_np(qb, cos[p], sin[p]).reshape(-1)
        k_ref = rope_np(kb, cos[p], sin[p]).astype(np.float16)
        assert np.array_equal(qo.cpu().numpy().view(np.uint32), q_ref.view(np.uint32)), p
        assert np.array_equal(kc[:, p].cpu().numpy().view(np.uint16), k_ref.view(np.uint16)), p
        assert np.array_equal(vc[:, p].cpu().numpy().view(np.uint16), vb.astype(np.float16).view(np.uint16)), p
    # a position outside the cache writes no row (and leaves the others)
    before = kc.clone()
    pos = torch.tensor([cap], dtype=torch.int64, device=dev)
    rc = lib.q4_rope_kv_dev(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), tb.data_ptr(), tc.data_ptr(),
                            ts.data_ptr(), pos.data_ptr(), kc.data_ptr(), vc.data_ptr(), qo.data_ptr(),
                            nh, nkv, d, cap, sp(torch))
    assert rc == 0 and torch.equal(before, kc)


def attention_ref(q, kc, vc, pos, nh, nkv, scale):
    g = nh // nkv
    q64 = q.reshape(nkv, g, -1).astype(np.float64)
    k64 = kc[:, :pos + 1].astype(np.float64)
    v64 = vc[:, :pos + 1].astype(np.float64)
    s = np.einsum("kgd,ksd->kgs", q64, k64) * scale
    s -= s.max(-1, keepdims=True)
    e = np.exp(s)
    e /= e.sum(-1, keepdims=True)
    return np.einsum("kgs,ksd->kgd", e, v64).reshape(-1)


@pytest.mark.parametrize("nh,nkv", [(28, 4), (8, 8), (16, 2)])
def test_attention(torch, lib, nh, nkv):
    rng = np.random.default_rng(6)
    d, cap = 128, 200
    scale = np.float32(d ** -0.5)
    dev = torch.device("cuda")
    kc_np = rng.normal(0, 1, (nkv, cap, d)).astype(np.float16)
    vc_np = rng.normal(0, 1, (nkv, cap, d)).astype(np.float16)
    q_np = rng.normal(0, 1, nh * d).astype(np.float32)
    kc, vc, tq = (torch.from_numpy(a).to(dev) for a in (kc_np, vc_np, q_np))
    out = torch.empty(nh * d, device=dev)
    scratch = torch.zeros(lib.q4_attention_scratch_floats(nh, d, cap), device=dev)
    for p in (0, 5, 63, 64, 65, 127, 128, cap - 1):
        pos = torch.tensor([p], dtype=torch.int64, device=dev)
        rc = lib.q4_attention_dev(tq.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(), out.data_ptr(),
                                  scratch.data_ptr(), nh, nkv, d, cap, float(scale), sp(torch))
        assert rc == 0, q4.last_error(lib)
        ref = attention_ref(q_np, kc_np, vc_np, p, nh, nkv, float(scale))
        assert oracle.normwise_rel(out.cpu().numpy(), ref) < ATTN_TOL, p


def test_attention_long_context(torch, lib):
    """Contexts past one round of the merge's loads (36 chunks of 64
    positions): up to 79 chunks, the ones past the first round merged by
    the loop after it, against the fp64 reference; the arrival counters
    are back at zero after every call, and repeated calls give the same
    bits whichever chunk arrives last."""
    rng = np.random.default_rng(9)
    nh, nkv, d, cap = 28, 4, 128, 5000
    scale = np.float32(d ** -0.5)
    dev = torch.device("cuda")
    kc_np = rng.normal(0, 1, (nkv, cap, d)).astype(np.float16)
    vc_np = rng.normal(0, 1, (nkv, cap, d)).astype(np.float16)
    q_np = rng.normal(0, 1, nh * d).astype(np.float32)
    kc, vc, tq = (torch.from_numpy(a).to(dev) for a in (kc_np, vc_np, q_np))
    out = torch.empty(nh * d, device=dev)
    scratch = torch.zeros(lib.q4_attention_scratch_floats(nh, d, cap), device=dev)
    for p in (2303, 2304, 2559, 2560, 2561, 4095, 4096, cap - 1):
        pos = torch.tensor([p], dtype=torch.int64, device=dev)
        rc = lib.q4_attention_dev(tq.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(), out.data_ptr(),
                                  scratch.data_ptr(), nh, nkv, d, cap, float(scale), sp(torch))
        assert rc == 0, q4.last_error(lib)
        ref = attention_ref(q_np, kc_np, vc_np, p, nh, nkv, float(scale))
        assert oracle.normwise_rel(out.cpu().numpy(), ref) < ATTN_TOL, p
        assert int(scratch[-512 * 32:].view(torch.int32).abs().sum().item()) == 0, p
        first = out.clone()
        for _ in range(4):
            lib.q4_attention_dev(tq.data_ptr(), kc.data_ptr(), vc.data_ptr(), pos.data_ptr(), out.data_ptr(),
                                 scratch.data_ptr(), nh, nkv, d, cap, float(scale), sp(torch))
            assert torch.equal(out.view(torch.int32), first.view(torch.int32)), p


@pytest.mark.parametrize("nh,nkv", [(28, 4), (8, 8), (16, 2)])
def test_attention_rope_matches_separate_calls(torch, lib, nh, nkv):
    rng = np.random.default_rng(8)
    d, cap = 128, 150
    half = d // 2
    scale = float(np.float32(d ** -0.5))
    inv = 1e6 ** (-np.arange(0, half, dtype=np.float32) * 2.0 / d)
    ang = np.arange(cap, dtype=np.float32)[:, None] * inv[None, :]
    dev = torch.device("cuda")
    tc = torch.from_numpy(np.cos(ang)).to(dev)
    ts = torch.from_numpy(np.sin(ang)).to(dev)
    tb = torch.from_numpy(rng.normal(0, 0.1, (nh + 2 * nkv) * d).astype(np.float32)).to(dev)
    # both caches start from the same history
    kc_a = torch.from_numpy(rng.normal(0, 1, (nkv, cap, d)).astype(np.float16)).to(dev)
    vc_a = torch.from_numpy(rng.normal(0, 1, (nkv, cap, d)).astype(np.float16)).to(dev)
    kc_b, vc_b = kc_a.clone(), vc_a.clone()
    q_rot = torch.empty(nh * d, device=dev)
    out_a, out_b = torch.empty(nh * d, device=dev), torch.empty(nh * d, device=dev)
    scratch = torch.zeros(lib.q4_attention_scratch_floats(nh, d, cap), device=dev)
    for p in (0, 1, 2, 62, 63, 64, 65, 100, 127, 128, cap - 1, cap, cap + 5):
        q, k, v = (torch.from_numpy(rng.normal(0, 1, n * d).astype(np.float32)).to(dev) for n in (nh, nkv, nkv))
        pos = torch.tensor([p], dtype=torch.int64, device=dev)
        rc = lib.q4_rope_kv_dev(q.data_ptr(), k.data_ptr(), v.data_ptr(), tb.data_ptr(), tc.data_ptr(), ts.data_ptr(),
                                pos.data_ptr(), kc_a.data_ptr(), vc_a.data_ptr(), q_rot.data_ptr(), nh, nkv, d, cap,
                                sp(torch))
        assert rc == 0, q4.last_error(lib)
        rc = lib.q4_attention_dev(q_rot.data_ptr(), kc_a.data_ptr(), vc_a.data_ptr(), pos.data_ptr(),
                                  out_a.data_ptr(), scratch.data_ptr(), nh, nkv, d, cap, scale, sp(torch))
        assert rc == 0, q4.last_error(lib)
        rc = lib.q4_attention_rope_dev(q.data_ptr(), k.data_ptr(), v.data_ptr(), tb.data_ptr(), tc.data_ptr(),
                                       ts.data_ptr(), pos.data_ptr(), kc_b.data_ptr(), vc_b.data_ptr(),
                                       out_b.data_ptr(), scratch.data_ptr(), nh, nkv, d, cap, scale, sp(torch))
        assert rc == 0, q4.last_error(lib)
        assert torch.equal(out_a.view(torch.int32), out_b.view(torch.int32)), p
        assert torch.equal(kc_a.view(torch.int16), kc_b.view(torch.int16)), p
        assert torch.equal(vc_a.view(torch.int16), vc_b.view(torch.int16)), p


def test_argmax_first_index_and_bookkeeping(torch, lib):
    rng = np.random.default_rng(7)
    dev = torch.device("cuda")
    n = 152064
    logits = rng.normal(0, 1, n).astype(np.float32)
    for planted in ((77, 150000), (5, 6), (n - 3, n - 1)):
        lg = logits.copy()
        lg[list(planted)] = 50.0                     # a tie: the first index wins
        t = torch.from_numpy(lg).to(dev)
        tok = torch.zeros(1, dtype=torch.int64, device=dev)
        hist = torch.full((8,), -1, dtype=torch.int64, device=dev)
        pos = torch.tensor([12], dtype=torch.int64, device=dev)
        rc = lib.q4_argmax_dev(t.data_ptr(), n, tok.data_ptr(), hist.data_ptr(), pos.data_ptr(), 10, 8, sp(torch))
        assert rc == 0, q4.last_error(lib)
        assert int(tok.item()) == planted[0] == int(np.argmax(lg))
        assert int(pos.item()) == 13
        assert hist.cpu().tolist() == [-1, -1, planted[0], -1, -1, -1, -1, -1]
    # odd length (tail past the last float4)
    lg = rng.normal(0, 1, 1001).astype(np.float32)
    t = torch.from_numpy(lg).to(dev)
    rc = lib.q4_argmax_dev(t.data_ptr(), 1001, tok.data_ptr(), hist.data_ptr(), pos.data_ptr(), 0, 0, sp(torch))
    assert rc == 0 and int(tok.item()) == int(np.argmax(lg))


def test_argmax_nan_and_special_values_match_numpy(torch, lib):
    """NumPy's argmax takes NaN as the largest value (the first NaN wins),
    -inf and +inf order as numbers, and a tie keeps the first index; the
    GPU argmax must return np.argmax for each planted case, across the
    slices its first launch splits the vector into (n = 152064: 38 slices)
    and for the short tail past the last float4."""
    rng = np.random.default_rng(8)
    dev = torch.device("cuda")
    tok = torch.zeros(1, dtype=torch.int64, device=dev)
    hist = torch.full((4,), -1, dtype=torch.int64, device=dev)
    pos = torch.tensor([0], dtype=torch.int64, device=dev)
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    for n in (152064, 4099, 7, 1):
        base = rng.normal(0, 1, n).astype(np.float32)
        cases = [{}, {n - 1: nan}, {n // 2: nan, n - 1: nan}, {n // 3: inf, n // 2: nan}, {n // 4: inf, n - 1: inf},
                 {0: nan}, {n // 5: 9.0, n - 1: 9.0}]
        for planted in cases:
            lg = base.copy()
            for k, v in planted.items():
                lg[k] = v
            if not planted and n > 2:
                lg[:] = -inf                                   # all -inf: index 0
            t = torch.from_numpy(lg).to(dev)
            rc = lib.q4_argmax_dev(t.data_ptr(), n, tok.data_ptr(), hist.data_ptr(), pos.data_ptr(), 0, 4, sp(torch))
            assert rc == 0, q4.last_error(lib)
            assert int(tok.item()) == int(np.argmax(lg)), (n, planted)
