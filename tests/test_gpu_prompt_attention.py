"""GPU checks of the prompt chunk's causal attention, q4_prompt_attention_dev
(head_dim 128 on the matrix cores with two-term fp16 operands, 64 and 32 on
the vector ALUs), against the reference's sdpa with causal=True
(hetero/cpu_model.py:233-252) evaluated in float64 here: query row i of a
chunk at positions [pos0, pos0 + rows) sees the cache positions
[0, pos0 + i], query head h reads kv head h / (nh / nkv),
o = softmax((q . k) * scale) v.

Both kernels evaluate the softmax online (tile by tile) and sum in fp32, so
the bar is fp32 rounding, not bit equality: normwise relative error (max
|diff| / max |ref|) below ATTN_TOL = 2e-6, stated here.  A planted
mistake -- one position too many or too few, the wrong kv head, a missing
scale -- moves the output by far more (checked on the reference below).
"""
import ctypes

import numpy as np
import pytest

import oracle
from hetero import q4

ATTN_TOL = 2e-6


def sdpa_causal(q, kc, vc, pos0, nh, nkv, scale, extra=0, head_shift=0):
    """float64 reference; `extra` / `head_shift` plant mistakes."""
    rows, d = q.shape[0], kc.shape[2]
    qh = q.reshape(rows, nh, d).astype(np.float64)
    out = np.empty((rows, nh, d))
    g = nh // nkv
    for h in range(nh):
        kvh = (h // g + head_shift) % nkv
        n = pos0 + rows + extra
        k = kc[kvh, :n].astype(np.float64)
        v = vc[kvh, :n].astype(np.float64)
        s = qh[:, h] @ k.T * scale
        mask = np.arange(n)[None, :] <= (pos0 + np.arange(rows) + extra)[:, None]
        s = np.where(mask, s, -np.inf)
        p = np.exp(s - s.max(1, keepdims=True))
        out[:, h] = (p / p.sum(1, keepdims=True)) @ v
    return out.reshape(rows, nh * d)


# (heads, kv heads, head_dim, rows, pos0, cap): a 512-token Qwen2.5-7B chunk
# (7 heads per kv head, 8 tiles); a chunk after a context; a single row;
# 1 and 8 heads per kv head; head_dim 64 and 32 (vector path); ragged row
# blocks and tiles throughout
CASES = [(28, 4, 128, 512, 0, 512), (28, 4, 128, 70, 64, 200), (28, 4, 128, 1, 300, 301),
         (8, 8, 128, 33, 100, 140), (16, 2, 128, 40, 5, 45), (4, 2, 128, 24, 0, 24),
         (8, 2, 64, 50, 10, 64), (4, 4, 32, 17, 3, 20)]


@pytest.mark.gpu
@pytest.mark.parametrize("nh,nkv,d,rows,pos0,cap", CASES, ids=lambda v: str(v))
def test_prompt_attention_vs_float64(nh, nkv, d, rows, pos0, cap):
    import torch
    print(f"prompt attention nh={nh} nkv={nkv} d={d} rows={rows} pos0={pos0} cap={cap}", flush=True)
    rng = np.random.default_rng(nh * 1000 + rows + pos0)
    q = rng.normal(0, 2, (rows, nh * d)).astype(np.float32)
    kc = rng.normal(0, 1, (nkv, cap, d)).astype(np.float16)
    vc = rng.normal(0, 1, (nkv, cap, d)).astype(np.float16)
    scale = ctypes.c_float(d ** -0.5).value
    lib = q4.load()
    tq, tk, tv = (torch.from_numpy(a).cuda() for a in (q, kc, vc))
    out = torch.full((rows, nh * d), float("nan"), device="cuda")
    rc = lib.q4_prompt_attention_dev(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), out.data_ptr(), rows, pos0, nh,
                                     nkv, d, cap, scale, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, q4.last_error(lib)
    got = out.cpu().numpy()
    ref = sdpa_causal(q, kc, vc, pos0, nh, nkv, scale)
    err = oracle.normwise_rel(got, ref)
    print(f"normwise error vs float64: {err:.2e}", flush=True)
    assert np.isfinite(got).all()
    assert err < ATTN_TOL
    again = torch.empty_like(out)
    lib.q4_prompt_attention_dev(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), again.data_ptr(), rows, pos0, nh, nkv,
                                d, cap, scale, torch.cuda.current_stream().cuda_stream)
    assert torch.equal(out, again)


def test_planted_mistakes_exceed_the_bar():
    """The reference with a mistake planted differs from the true one by far
    more than ATTN_TOL (so the bar above can see such a mistake)."""
    rng = np.random.default_rng(3)
    nh, nkv, d, rows, pos0, cap = 8, 2, 128, 20, 7, 40
    q = rng.normal(0, 2, (rows, nh * d)).astype(np.float32)
    kc = rng.normal(0, 1, (nkv, cap, d)).astype(np.float16)
    vc = rng.normal(0, 1, (nkv, cap, d)).astype(np.float16)
    scale = d ** -0.5
    ref = sdpa_causal(q, kc, vc, pos0, nh, nkv, scale)
    for bad in (sdpa_causal(q, kc, vc, pos0, nh, nkv, scale, extra=1),
                sdpa_causal(q, kc, vc, pos0, nh, nkv, scale, extra=-1),
                sdpa_causal(q, kc, vc, pos0, nh, nkv, scale, head_shift=1),
                sdpa_causal(q, kc, vc, pos0, nh, nkv, 1.0)):
        assert oracle.normwise_rel(bad, ref) > 1e3 * ATTN_TOL
