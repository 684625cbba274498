"""CPU checks of the oracle (oracle/q4oracle.c) -- no GPU needed.

Each oracle function is pinned by something other than a restatement of its
own formula:
  * golden vectors written by the reference kernel/q4gemv.c compiled from
    source (tests/golden/make_golden.py), bit-exact, every ROWS build;
  * the reference libraries themselves (oracle/_ref) on fresh seeded inputs;
  * library routines and closed forms: NumPy's float16 conversion for all
    65536 bit patterns, the nibble closed form (w >> 4j) & 0xF, q*s+b, a
    sequential NumPy cumsum for the group sums, integer dot products in
    int64, exact scaling by two, row permutation, zero inputs;
  * an fp64 brute force within the north-star tolerance (1e-3 norm-wise).
"""
import json
import os

import numpy as np
import pytest

import oracle
from hetero import synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def orc():
    return oracle.Oracle()


@pytest.fixture(scope="module")
def manifest():
    with open(os.path.join(GOLDEN, "manifest.json")) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def small():
    return np.load(os.path.join(GOLDEN, "golden_small.npz"))


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_f16_to_f32_exhaustive(orc):
    """All 65536 fp16 bit patterns vs NumPy's conversion (NaN: NaN-ness only)."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([orc.lib.oq_f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got[~nan]), bits(want[~nan]))


def test_unpack_closed_form(orc):
    """Every nibble value in every position: oracle unpack == (w >> 4j) & 0xF."""
    w = np.zeros((16, 8), np.uint32)
    for v in range(16):
        for j in range(8):
            w[v, j] = np.uint32(v << (4 * j)) | np.uint32(((15 - v) << (4 * ((j + 1) % 8))))
    got = orc.unpack(w)
    assert np.array_equal(got, oracle.unpack_np(w))
    assert got.max() == 15 and got.min() == 0


def test_dequant_closed_form(orc):
    w, s, b = synth.qlinear(21, 40, 512, 64)
    s[0, :] = np.float16(0.0)                                   # zero scale
    s[1, :] = (s[1, :].view(np.uint16) & np.uint16(0x03FF)).view(np.float16)   # subnormal
    w[2, :] = 0                                                 # q = 0
    w[3, :] = 0xFFFFFFFF                                        # q = 15
    got = orc.dequant(w, s, b, 64)
    want = oracle.dequant_np(w, s, b, 64)
    assert np.array_equal(bits(got), bits(want))
    assert np.array_equal(bits(orc.dequant(w, s, b, 64, 5, 17)), bits(want[5:17]))


def test_dequant_golden(orc, manifest, small):
    for name, c in manifest["cases"].items():
        if not name.startswith("d_"):
            continue
        p = c["params"]
        w, s, b = (small[f"{name}.{k}"] for k in ("w", "scales", "biases"))
        got = orc.dequant(w, s, b, p["gs"], p["row0"], p["row1"])
        assert np.array_equal(bits(got), bits(small[f"{name}.out"])), name


def test_gemv_small_golden_all_rows(orc, manifest, small):
    """Bit-exact vs the reference for ROWS = 1, 2, 4, 8 (incl. the fp32 tail rows)."""
    for name, c in manifest["cases"].items():
        if not name.startswith("g_"):
            continue
        p = c["params"]
        w, s, b, x = (small[f"{name}.{k}"] for k in ("w", "scales", "biases", "x"))
        for r in (1, 2, 4, 8):
            got = orc.gemv(w, s, b, x, p["gs"], rows_block=r)
            assert np.array_equal(bits(got), bits(small[f"{name}.out_rows{r}"])), (name, r)


@pytest.mark.parametrize("name", ["config0_q_proj", "q_proj", "k_proj", "down_proj"])
def test_gemv_qwen7b_golden(orc, manifest, name):
    c = manifest["qwen7b"][name]
    w, s, b = synth.qlinear(c["seed"], c["n_out"], c["n_in"], 64)
    x = synth.activations(c["seed"], c["m"], c["n_in"])
    assert synth.sha256(w, s, b) == c["sha256_w_s_b"]
    assert synth.sha256(x) == c["sha256_x"]
    want = np.load(os.path.join(GOLDEN, "golden_qwen7b.npz"))[name]
    for m in range(min(c["m"], 2)):
        assert np.array_equal(bits(orc.gemv(w, s, b, x[m], 64)), bits(want[m])), (name, m)


def test_return_codes(orc, manifest):
    rcs = manifest["return_codes"]
    w, s, b = synth.qlinear(120, 4, 256, 64)
    x = synth.activations(120, 1, 256)[0]
    out = np.empty(4, np.float32)
    args = (w.ctypes.data, s.ctypes.data, b.ctypes.data, x.ctypes.data, out.ctypes.data)
    assert orc.lib.oq_q4_gemv(*args, 4, 256, 32, 1) == rcs["gemv_gs32"] == -1
    assert orc.lib.oq_q4_gemv(*args, 4, 200, 64, 1) == rcs["gemv_nin_not_multiple"] == -1
    assert orc.lib.oq_q4_gemv(*args, 4, 192, 96, 1) == rcs["gemv_gs96"] == -1
    buf = np.empty((2, 256), np.float32)
    dargs = (w.ctypes.data, s.ctypes.data, b.ctypes.data, buf.ctypes.data)
    assert orc.lib.oq_q4_dequant(*dargs, 0, 2, 256, 12) == rcs["dequant_gs12"] == -1
    assert orc.lib.oq_q4_dequant(*dargs, 3, 3, 256, 64) == rcs["dequant_empty"] == 0
    assert orc.lib.oq_q4_dequant(*dargs, 3, 1, 256, 64) == rcs["dequant_reversed"] == 0


def test_xprep_closed_form(orc):
    """Prologue: sequential group sums (NumPy cumsum), amax/32767, int16 rounding."""
    x = synth.activations(31, 1, 1024)[0] * np.float32(3.0)
    xq, xsum, xscale = orc.xprep(x, 64)
    want_sum = np.array([np.cumsum(x[g * 64:(g + 1) * 64], dtype=np.float32)[-1]
                         for g in range(16)], np.float32)
    assert np.array_equal(bits(xsum), bits(want_sum))
    amax = np.float32(np.max(np.abs(x)))
    assert xscale == np.float32(amax / np.float32(32767.0))
    inv = np.float32(1.0) / np.float32(xscale)
    a = (x * inv).astype(np.float32)
    r = np.where(a < 0, a - np.float32(0.5), a + np.float32(0.5)).astype(np.float32)
    assert np.array_equal(xq, np.trunc(r).astype(np.int32).astype(np.int16))
    assert np.abs(xq.astype(np.int32)).max() == 32767


def test_gemv_integer_path_closed_form(orc):
    """s = 1, b = 0: out = sequential sum_g fl(xscale * idot_g), idot in int64."""
    w, s, b = synth.qlinear(32, 24, 512, 64)
    s[:] = np.float16(1.0)
    b[:] = np.float16(0.0)
    x = synth.activations(32, 1, 512)[0]
    xq, _, xscale = orc.xprep(x, 64)
    q = oracle.unpack_np(w).astype(np.int64)
    idot = (q.reshape(24, 8, 64) * xq.astype(np.int64).reshape(1, 8, 64)).sum(-1)
    want = np.zeros(24, np.float32)
    for g in range(8):
        want = (want + (np.float32(xscale) * idot[:, g].astype(np.float32))).astype(np.float32)
    assert np.array_equal(bits(orc.gemv(w, s, b, x, 64)), bits(want))


def test_gemv_zero_weights_closed_form(orc):
    """q = 0: out = sequential sum_g fl(b_g * xsum_g)."""
    w, s, b = synth.qlinear(33, 10, 384, 64)
    w[:] = 0
    x = synth.activations(33, 1, 384)[0]
    _, xsum, _ = orc.xprep(x, 64)
    want = np.zeros(10, np.float32)
    for g in range(6):
        want = (want + (b[:, g].astype(np.float32) * xsum[g])).astype(np.float32)
    assert np.array_equal(bits(orc.gemv(w, s, b, x, 64)), bits(want))


def test_gemv_invariants(orc):
    """x = 0 gives 0; doubling the scales (b = 0) doubles the output exactly;
    permuting rows permutes outputs."""
    w, s, b = synth.qlinear(34, 32, 1024, 64)
    x = synth.activations(34, 1, 1024)[0]
    assert np.array_equal(orc.gemv(w, s, b, np.zeros(1024, np.float32), 64), np.zeros(32, np.float32))
    b0 = np.zeros_like(b)
    one = orc.gemv(w, s, b0, x, 64)
    two = orc.gemv(w, (s.astype(np.float32) * 2).astype(np.float16), b0, x, 64)
    assert np.array_equal(bits(two), bits(one * np.float32(2)))
    perm = np.random.default_rng(0).permutation(32)
    got = orc.gemv(np.ascontiguousarray(w[perm]), np.ascontiguousarray(s[perm]),
                   np.ascontiguousarray(b[perm]), x, 64)
    assert np.array_equal(bits(got), bits(orc.gemv(w, s, b, x, 64)[perm]))


def test_gemv_vs_fp64_brute_force(orc):
    """Within the stated fp32-reordering tolerance of the exact product."""
    for seed, n_out, n_in in ((40, 64, 3584), (41, 16, 18944)):
        w, s, b = synth.qlinear(seed, n_out, n_in, 64)
        x = synth.activations(seed, 1, n_in)[0]
        rel = oracle.normwise_rel(orc.gemv(w, s, b, x, 64), oracle.gemv_fp64(w, s, b, x, 64))
        assert rel < 1e-3, rel


@pytest.mark.skipif(not os.path.exists(oracle.ref_path(1)), reason="oracle/_ref not built")
def test_oracle_vs_reference_library_fresh_inputs(orc):
    """The restatement equals the compiled reference on fresh seeded shapes."""
    os.environ.setdefault("HETERO_KERNEL_THREADS", "4")
    refs = {r: oracle.load_ref(r) for r in (1, 2, 4, 8)}
    for seed, n_out, n_in, gs in ((50, 35, 640, 64), (51, 17, 1280, 128), (52, 96, 3584, 64),
                                  (53, 9, 4480, 320)):
        w, s, b = synth.qlinear(seed, n_out, n_in, gs)
        x = synth.activations(seed, 1, n_in)[0]
        for r, lib in refs.items():
            out = np.empty(n_out, np.float32)
            rc = lib.q4_gemv(w.ctypes.data, s.ctypes.data, b.ctypes.data, x.ctypes.data,
                             out.ctypes.data, n_out, n_in, gs, 4)
            assert rc == 0
            assert np.array_equal(bits(orc.gemv(w, s, b, x, gs, rows_block=r)), bits(out)), (seed, r)
        d = np.empty((n_out, n_in), np.float32)
        assert refs[1].q4_dequant(w.ctypes.data, s.ctypes.data, b.ctypes.data, d.ctypes.data,
                                  0, n_out, n_in, gs, 4) == 0
        assert np.array_equal(bits(orc.dequant(w, s, b, gs)), bits(d))


def test_synth_is_deterministic():
    """Same seed, same bits; the stream does not depend on how much is drawn."""
    a = synth.u64(7, "w", 1000)
    assert np.array_equal(a[:10], synth.u64(7, "w", 10))
    assert np.array_equal(a[500:], synth.u64(7, "w", 500, start=500))
    s1, b1 = synth.scales_biases(3, 4, 8)
    s2, b2 = synth.scales_biases(3, 4, 8)
    assert np.array_equal(s1.view(np.uint16), s2.view(np.uint16))
    n = synth.normal(5, "x", 200000)
    assert abs(n.mean()) < 0.01 and abs(n.std() - 1) < 0.01
