"""GPU checks of the fused MLP path (gate/up + SiLU*mul, then down).

Oracle: the reference's composition, hetero/cpu_model.py:291-292 with the
NumPy float32 silu of :169-170, over the oracle GEMV.  gate and up are
bit-exact q4_gemv results inside the kernel, but exp differs from NumPy's
float32 exp in the last place, so h is compared with a tight relative bound
and the block output (whose down projection re-quantises h to int16) within
the north-star 1e-3 norm-wise tolerance, also against an fp64 brute force.
"""
import numpy as np
import pytest

from hetero import q4, synth
import oracle

pytestmark = pytest.mark.gpu

H_TOL = 2e-6      # norm-wise, h vs NumPy float32 silu of the oracle's gate/up
OUT_TOL = 1e-3    # norm-wise, MLP output vs the composition and vs fp64


def silu_np(g):
    g = g.astype(np.float32)
    return g / (np.float32(1.0) + np.exp(-g, dtype=np.float32))


def tensors(*arrays):
    import torch
    return [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in arrays]


def mats(seed, n_out, n_in):
    w, s, b = synth.qlinear(seed, n_out, n_in, 64)
    return (w, s, b), tuple(tensors(w, s.view(np.int16), b.view(np.int16)))


@pytest.mark.parametrize("hidden,inter,m", [(1024, 2816, 1), (1024, 2816, 2), (1024, 2816, 3), (1024, 2816, 5),
                                            (1024, 2816, 8), (3584, 18944, 1), (3584, 18944, 2),
                                            (3584, 18944, 4), (3584, 18944, 8)])
def test_gate_up_silu_and_mlp(hidden, inter, m):
    import torch
    print(f"mlp hidden={hidden} inter={inter} m={m}", flush=True)
    orc = oracle.Oracle()
    (gn, gt), (un, ut), (dn, dt) = (mats(600, inter, hidden), mats(601, inter, hidden),
                                    mats(602, hidden, inter))
    x = synth.activations(603, m, hidden)
    tx = tensors(x)[0]
    h = q4.gate_up_silu_dev(gt, ut, tx)
    out = q4.mlp_dev(gt, ut, dt, tx)
    torch.cuda.synchronize()
    h = h.cpu().numpy()
    out = out.cpu().numpy()
    for r in range(m):
        g = orc.gemv(*gn, x[r], 64)
        u = orc.gemv(*un, x[r], 64)
        h_ref = (silu_np(g) * u).astype(np.float32)
        assert oracle.normwise_rel(h[r], h_ref) < H_TOL
        out_ref = orc.gemv(*dn, h_ref, 64)
        assert oracle.normwise_rel(out[r], out_ref) < OUT_TOL
        # fp64 brute force of the whole block
        g64 = oracle.gemv_fp64(*gn, x[r], 64)
        u64 = oracle.gemv_fp64(*un, x[r], 64)
        h64 = g64 / (1.0 + np.exp(-g64)) * u64
        assert oracle.normwise_rel(out[r], oracle.gemv_fp64(*dn, h64, 64)) < OUT_TOL


def test_gate_up_silu_sign_structure():
    """SiLU(g) has the sign of g, so h = SiLU(g) * u has sign(g) * sign(u) for
    the oracle's exact g and u (a check independent of exp's last bits)."""
    import torch
    hidden, inter = 512, 640
    (gn, gt), (un, ut) = mats(610, inter, hidden), mats(611, inter, hidden)
    x = synth.activations(612, 1, hidden)
    h = q4.gate_up_silu_dev(gt, ut, tensors(x)[0]).cpu().numpy()[0]
    torch.cuda.synchronize()
    orc = oracle.Oracle()
    g = orc.gemv(*gn, x[0], 64)
    u = orc.gemv(*un, x[0], 64)
    nz = (g != 0) & (u != 0)
    assert np.array_equal(np.sign(h[nz]), np.sign(g[nz]) * np.sign(u[nz]))


@pytest.mark.parametrize("hidden,inter", [(1024, 2816), (3584, 18944), (512, 200), (4096, 40)])
def test_gate_up_silu_rows_match_one_row_launches(hidden, inter):
    """Several rows (the matrix-core path) against each row on its own (the
    streaming path): the same gate/up dots and the same SiLU*mul, so h is
    bit-identical; inter 200 and 40 leave a partial 16-row tile."""
    import torch
    (_, gt), (_, ut) = mats(620, inter, hidden), mats(621, inter, hidden)
    x = synth.activations(622, 8, hidden)
    tx = tensors(x)[0]
    ones = [q4.gate_up_silu_dev(gt, ut, tx[r:r + 1].contiguous()).cpu().numpy()[0] for r in range(8)]
    for m in (2, 3, 5, 8):
        print(f"gate/up rows hidden={hidden} inter={inter} m={m}", flush=True)
        h = q4.gate_up_silu_dev(gt, ut, tx[:m].contiguous())
        torch.cuda.synchronize()
        h = h.cpu().numpy()
        for r in range(m):
            assert np.array_equal(h[r].view(np.uint32), ones[r].view(np.uint32)), f"m={m} row {r}"


def test_gate_up_silu_rows_odd_group_count():
    """The fused gate/up tiles with 13 groups per row (per-group scale/bias
    loads) and a partial tile: 3..8 rows against the one-row launches."""
    import torch
    hidden, inter = 832, 100
    (_, gt), (_, ut) = mats(630, inter, hidden), mats(631, inter, hidden)
    x = synth.activations(632, 8, hidden)
    tx = tensors(x)[0]
    ones = [q4.gate_up_silu_dev(gt, ut, tx[r:r + 1].contiguous()).cpu().numpy()[0] for r in range(8)]
    for m in (3, 8):
        h = q4.gate_up_silu_dev(gt, ut, tx[:m].contiguous())
        torch.cuda.synchronize()
        h = h.cpu().numpy()
        for r in range(m):
            assert np.array_equal(h[r].view(np.uint32), ones[r].view(np.uint32)), f"m={m} row {r}"
