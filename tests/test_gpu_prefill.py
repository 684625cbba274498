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
