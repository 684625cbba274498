"""The summation order the device RMSNorm reproduces (row_sum_numpy in
hetero-infer_amd/csrc/q4_common.h), restated on the CPU and checked bit for
bit against NumPy's own float32 reductions: np.add.reduce over a row, and
the mean of squares the reference's rms_norm takes
(hetero/cpu_model.py:164-166).  Rows whose pairwise split is not exact are
outside the claim.  A plainly sequential sum differs from NumPy's on some
rows, which shows the comparison can fail."""
import numpy as np
import pytest

PERFECT = (64, 120, 896, 1536, 2048, 3584, 4096, 5120, 8192)


def perfect_split(n):
    """(blocks, block length) of a row NumPy halves exactly, else None."""
    m, L = n, 1
    if n < 8 or n % 8:
        return None
    while m > 128:
        if m % 16:
            return None
        m, L = m // 2, L * 2
    return L, m


def device_order_sum(a):
    """The device's order: block b's accumulator j adds values j, j + 8, ...
    of the block in order; then lane-xor pairs (accumulators, then blocks)."""
    L, m = perfect_split(a.size)
    f = np.float32
    blk = a.reshape(L, m)
    acc = blk[:, 0:8].astype(np.float32).copy()
    for i in range(8, m, 8):
        acc = (acc + blk[:, i:i + 8]).astype(np.float32)
    vals = [f(v) for v in acc.reshape(-1)]         # lane 8b + j
    s = 1
    while s < len(vals):
        vals = [f(vals[i] + vals[i ^ s]) if i % (2 * s) == 0 else vals[i] for i in range(len(vals))]
        s *= 2
    return vals[0]


@pytest.mark.parametrize("n", PERFECT)
def test_device_order_is_numpy_pairwise(n):
    rng = np.random.default_rng(n)
    for _ in range(200):
        a = (rng.standard_normal(n) * rng.choice([1e-3, 1.0, 1e3])).astype(np.float32)
        sq = a * a
        assert device_order_sum(sq).view(np.uint32) == np.add.reduce(sq).view(np.uint32)
        assert device_order_sum(a).view(np.uint32) == np.add.reduce(a).view(np.uint32)
        # the mean of squares: the float32 sum divided by the count in float64
        mean = np.float32(np.float64(device_order_sum(sq)) / np.float64(n))
        assert mean.view(np.uint32) == (a * a).mean(-1, keepdims=True)[0].view(np.uint32)


def test_split_claims():
    assert perfect_split(3584) == (32, 112) and perfect_split(8192) == (64, 128)
    assert perfect_split(1000) is None and perfect_split(4104) is None


def test_sequential_order_differs_from_numpy():
    """A plainly sequential sum differs from NumPy's on some rows: the
    comparison above is not vacuous."""
    rng = np.random.default_rng(0)
    diff = 0
    for _ in range(50):
        a = rng.standard_normal(3584).astype(np.float32)
        seq = np.float32(0)
        for v in a:
            seq = np.float32(seq + v)
        diff += int(seq.view(np.uint32) != np.add.reduce(a).view(np.uint32))
    assert diff > 0
