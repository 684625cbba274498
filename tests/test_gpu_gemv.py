"""GPU parity of the HIP int4 GEMV path, called through the C-ABI.

Bar: bit-exact against the golden vectors written from the reference
kernel/q4gemv.c compiled from source (tests/golden/make_golden.py), and
against the oracle on seeded inputs; dequantised weights bit-exact.
"""
import json
import os

import numpy as np
import pytest

from hetero import q4, synth
import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_bit_exact(got, want, what):
    got, want = bits(got), bits(want)
    bad = np.nonzero(got != want)[0] if got.ndim == 1 else np.argwhere(got != want)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    assert bad.size == 0, f"{what}: {len(bad)} of {got.size} differ, first at {bad[:5].tolist()}"


@pytest.fixture(scope="module")
def lib():
    return q4.load()


@pytest.fixture(scope="module")
def manifest():
    with open(os.path.join(GOLDEN, "manifest.json")) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def small():
    return np.load(os.path.join(GOLDEN, "golden_small.npz"))


def gemv_cases(man):
    return [k for k in man["cases"] if k.startswith("g_")]


def test_small_golden_host_abi(lib, manifest, small):
    """q4_gemv (host pointers) vs the reference on every small golden case."""
    for name in gemv_cases(manifest):
        p = manifest["cases"][name]["params"]
        w, s, b, x = (small[f"{name}.{k}"] for k in ("w", "scales", "biases", "x"))
        print(f"case {name} {p}", flush=True)
        out = q4.gemv_host(lib, w, s.view(np.uint16), b.view(np.uint16), x, p["gs"])
        ref = small[f"{name}.out_rows1"]
        assert_bit_exact(out, ref, name)
        if p["n_out"] % 8 == 0:
            assert_bit_exact(out, small[f"{name}.out_rows8"], name + " rows8")


def test_small_golden_dev_abi(lib, manifest, small):
    """q4_gemv_dev (device pointers, torch tensors) vs the reference."""
    import torch
    for name in gemv_cases(manifest):
        p = manifest["cases"][name]["params"]
        print(f"case {name} {p}", flush=True)
        w, s, b, x = (torch.from_numpy(np.ascontiguousarray(small[f"{name}.{k}"])).cuda()
                      for k in ("w", "scales", "biases", "x"))
        out = q4.gemv_dev(w, s.view(torch.int16), b.view(torch.int16), x.reshape(1, -1))
        torch.cuda.synchronize()
        assert_bit_exact(out.cpu().numpy()[0], small[f"{name}.out_rows1"], name)


@pytest.mark.parametrize("rows", [2, 4, 8])
def test_rows_tail_golden(lib, manifest, small, rows):
    """With the reference build's ROWS set (q4_set_rows), the last
    n_out % ROWS rows take its fp32 tail path (kernel/q4gemv.c:185-200):
    bit-exact against the reference compiled with that ROWS, through the
    host ABI, the device ABI at 1 and 3 rows of x (streaming and
    matrix-core paths) and grouped calls of two matrices."""
    import torch
    o = oracle.Oracle()
    prev = q4.set_rows(rows, lib)
    try:
        for name in gemv_cases(manifest):
            p = manifest["cases"][name]["params"]
            w, s, b, x = (small[f"{name}.{k}"] for k in ("w", "scales", "biases", "x"))
            gs = p["gs"]
            print(f"case {name} {p} rows {rows}", flush=True)
            want = small[f"{name}.out_rows{rows}"]
            assert_bit_exact(q4.gemv_host(lib, w, s.view(np.uint16), b.view(np.uint16), x, gs), want,
                             f"{name} host")
            x3 = np.stack([x, synth.activations(130 + rows, 1, x.size)[0], -x])
            want3 = np.stack([o.gemv(w, s, b, xr, gs, rows_block=rows) for xr in x3])
            assert_bit_exact(want3[0], want, f"{name} oracle")
            tw, ts, tb = (torch.from_numpy(np.ascontiguousarray(a)).cuda()
                          for a in (w, s.view(np.int16), b.view(np.int16)))
            tx3 = torch.from_numpy(x3).cuda()
            for m in (1, 3):
                got = q4.gemv_dev(tw, ts, tb, tx3[:m])
                got2 = q4.gemv_multi_dev([(tw, ts, tb), (tw, ts, tb)], tx3[:m])
                torch.cuda.synchronize()
                assert_bit_exact(got.cpu().numpy(), want3[:m], f"{name} dev m={m}")
                for k, g in enumerate(got2):
                    assert_bit_exact(g.cpu().numpy(), want3[:m], f"{name} multi m={m} matrix {k}")
            lib.q4_release(w.ctypes.data)
    finally:
        q4.set_rows(prev, lib)
    assert q4.set_rows(1, lib) == 1


def test_return_codes(lib, manifest):
    """Invalid shapes give the reference's return codes."""
    rcs = manifest["return_codes"]
    w, s, b = synth.qlinear(120, 4, 256, 64)
    x = synth.activations(120, 1, 256)[0]
    out = np.empty(4, np.float32)
    args = (w.ctypes.data, s.ctypes.data, b.ctypes.data, x.ctypes.data, out.ctypes.data)
    assert lib.q4_gemv(*args, 4, 256, 32, 1) == rcs["gemv_gs32"]
    assert lib.q4_gemv(*args, 4, 200, 64, 1) == rcs["gemv_nin_not_multiple"]
    assert lib.q4_gemv(*args, 4, 192, 96, 1) == rcs["gemv_gs96"]
    buf = np.empty((2, 256), np.float32)
    dargs = (w.ctypes.data, s.ctypes.data, b.ctypes.data, buf.ctypes.data)
    assert lib.q4_dequant(*dargs, 0, 2, 256, 12, 1) == rcs["dequant_gs12"]
    assert lib.q4_dequant(*dargs, 3, 3, 256, 64, 1) == rcs["dequant_empty"]
    assert lib.q4_dequant(*dargs, 3, 1, 256, 64, 1) == rcs["dequant_reversed"]


def test_dequant_golden(lib, manifest, small):
    """q4_dequant (host ABI) bit-exact vs the reference, incl. row sub-ranges and gs=32."""
    for name, c in manifest["cases"].items():
        if not name.startswith("d_"):
            continue
        p = c["params"]
        w, s, b = (small[f"{name}.{k}"] for k in ("w", "scales", "biases"))
        out = np.empty((p["row1"] - p["row0"], p["n_in"]), np.float32)
        rc = lib.q4_dequant(w.ctypes.data, s.ctypes.data, b.ctypes.data, out.ctypes.data,
                            p["row0"], p["row1"], p["n_in"], p["gs"], 4)
        assert rc == 0, q4.last_error(lib)
        assert_bit_exact(out, small[f"{name}.out"], name)


def test_dequant_dev_vs_closed_form(lib):
    """fp32 and bf16 device dequant vs q*s+b (NumPy) on a seeded matrix."""
    import torch
    w, s, b = synth.qlinear(7, 96, 1024, 64)
    ref = oracle.dequant_np(w, s, b, 64)
    tw, ts, tb = (torch.from_numpy(a).cuda() for a in (w, s.view(np.int16), b.view(np.int16)))
    got = q4.dequant_dev(tw, ts, tb).cpu().numpy()
    assert_bit_exact(got, ref, "dequant fp32")
    got16 = q4.dequant_dev(tw, ts, tb, 10, 90, bf16=True).cpu()
    want16 = torch.from_numpy(ref[10:90]).to(torch.bfloat16)
    assert torch.equal(got16.view(torch.int16), want16.view(torch.int16))


def test_unpack_nibbles(lib):
    """Integer nibbles: with scale 1 and bias 0 the dequantised value is q itself."""
    import torch
    w, s, b = synth.qlinear(8, 16, 512, 64)
    s[:] = np.float16(1.0)
    b[:] = np.float16(0.0)
    tw, ts, tb = (torch.from_numpy(a).cuda() for a in (w, s.view(np.int16), b.view(np.int16)))
    got = q4.dequant_dev(tw, ts, tb).cpu().numpy()
    assert np.array_equal(got.astype(np.uint8), oracle.unpack_np(w))
    assert np.array_equal(got, got.astype(np.uint8).astype(np.float32))


@pytest.mark.parametrize("name", [n for n, _, _ in synth.QWEN7B_SHAPES] + ["config0_q_proj"])
def test_qwen7b_shapes(lib, manifest, name):
    """Every Qwen2.5-7B projection at M=1 (and M=8 where stored) vs the reference."""
    import torch
    c = manifest["qwen7b"][name]
    print(f"shape {name} K={c['n_in']} N={c['n_out']} m={c['m']}", flush=True)
    w, s, b = synth.qlinear(c["seed"], c["n_out"], c["n_in"], 64)
    x = synth.activations(c["seed"], c["m"], c["n_in"])
    assert synth.sha256(w, s, b) == c["sha256_w_s_b"], "generator drift: inputs differ"
    assert synth.sha256(x) == c["sha256_x"]
    want = np.load(os.path.join(GOLDEN, "golden_qwen7b.npz"))[name]
    got = q4.gemv_host(lib, w, s.view(np.uint16), b.view(np.uint16), x[0], 64)
    assert_bit_exact(got, want[0], name + " host")
    if c["m"] > 1:
        out = np.empty((c["m"], c["n_out"]), np.float32)
        rc = lib.q4_gemv_batched(w.ctypes.data, s.ctypes.data, b.ctypes.data, x.ctypes.data,
                                 out.ctypes.data, c["m"], c["n_out"], c["n_in"], 64, 0)
        assert rc == 0, q4.last_error(lib)
        assert_bit_exact(out, want, name + " batched")
        tw, ts, tb, tx = (torch.from_numpy(a).cuda() for a in (w, s.view(np.int16), b.view(np.int16), x))
        for m in (1, 2, 3, 4, 5, 8):
            o = q4.gemv_dev(tw, ts, tb, tx[:m].contiguous())
            torch.cuda.synchronize()
            assert_bit_exact(o.cpu().numpy(), want[:m], f"{name} dev m={m}")
    lib.q4_release(w.ctypes.data)


def test_zero_sizes(lib):
    """n_out = 0 is a no-op; n_in = 0 gives zeros (empty sums)."""
    w = np.zeros((4, 0), np.uint32)
    s = np.zeros((4, 0), np.uint16)
    out = np.full(4, np.nan, np.float32)
    x = np.zeros(0, np.float32)
    rc = lib.q4_gemv(w.ctypes.data, s.ctypes.data, s.ctypes.data, x.ctypes.data, out.ctypes.data,
                     4, 0, 64, 1)
    assert rc == 0, q4.last_error(lib)
    assert np.array_equal(out, np.zeros(4, np.float32))
    assert lib.q4_gemv(w.ctypes.data, s.ctypes.data, s.ctypes.data, x.ctypes.data,
                       out.ctypes.data, 0, 64, 64, 1) == 0


def test_generic_group_size(lib):
    """gs = 192 (a multiple of 64, not a power of two) vs the oracle, bit-exact."""
    o = oracle.Oracle()
    w, s, b = synth.qlinear(9, 33, 192 * 5, 192)
    x = synth.activations(9, 1, 192 * 5)[0]
    got = q4.gemv_host(lib, w, s.view(np.uint16), b.view(np.uint16), x, 192)
    assert_bit_exact(got, o.gemv(w, s, b, x, 192), "gs192")


def test_residency_detects_replaced_weights(lib):
    """A matrix overwritten in place at the same address is re-uploaded."""
    o = oracle.Oracle()
    w, s, b = synth.qlinear(10, 64, 1024, 64)
    x = synth.activations(10, 1, 1024)[0]
    first = q4.gemv_host(lib, w, s.view(np.uint16), b.view(np.uint16), x, 64)
    assert_bit_exact(first, o.gemv(w, s, b, x, 64), "first")
    w2, s2, b2 = synth.qlinear(11, 64, 1024, 64)
    w[:], s[:], b[:] = w2, s2, b2
    second = q4.gemv_host(lib, w, s.view(np.uint16), b.view(np.uint16), x, 64)
    assert_bit_exact(second, o.gemv(w, s, b, x, 64), "second")
    assert lib.q4_release(w.ctypes.data) >= 1


def test_residency_full_check_sees_an_edit_between_samples(lib, monkeypatch):
    """Q4_RESIDENCY_CHECK=full hashes every byte: one word edited in place,
    away from the 16 offsets the default fingerprint samples (byte 2708 of
    32768; samples at multiples of 32767/15), is re-uploaded."""
    o = oracle.Oracle()
    w, s, b = synth.qlinear(12, 64, 1024, 64)
    x = synth.activations(12, 1, 1024)[0]
    monkeypatch.setenv("Q4_RESIDENCY_CHECK", "full")
    first = q4.gemv_host(lib, w, s.view(np.uint16), b.view(np.uint16), x, 64)
    assert_bit_exact(first, o.gemv(w, s, b, x, 64), "first")
    w[5, 37] ^= np.uint32(0x11111111)
    second = q4.gemv_host(lib, w, s.view(np.uint16), b.view(np.uint16), x, 64)
    assert_bit_exact(second, o.gemv(w, s, b, x, 64), "after the edit")
    assert lib.q4_release(w.ctypes.data) >= 1


def test_multi_dev_grouped(lib):
    """q4_gemv_multi_dev (q/k/v and gate/up style groups) vs the oracle, bit-exact."""
    import torch
    o = oracle.Oracle()
    for m, shapes in ((1, [(3584, 3584), (3584, 512), (3584, 512)]),
                      (2, [(1024, 1536), (1024, 2560)]),
                      (4, [(2048, 96), (2048, 64), (2048, 8), (2048, 40)]),
                      (3, [(3584, 512), (3584, 128)]), (6, [(1024, 200)]), (8, [(3584, 512), (3584, 256)])):
        k_in = shapes[0][0]
        print(f"multi m={m} shapes={shapes}", flush=True)
        mats_np = [synth.qlinear(300 + i, n, k_in, 64) for i, (_, n) in enumerate(shapes)]
        x = synth.activations(300, m, k_in)
        mats = [tuple(torch.from_numpy(a).cuda() for a in (w, s.view(np.int16), b.view(np.int16)))
                for w, s, b in mats_np]
        outs = q4.gemv_multi_dev(mats, torch.from_numpy(x).cuda())
        torch.cuda.synchronize()
        for (w, s, b), got in zip(mats_np, outs):
            want = o.gemv_rows(w, s, b, x, 64)
            assert_bit_exact(got.cpu().numpy(), want, f"multi m={m} n={w.shape[0]}")


def test_dev_all_m_and_paths(lib):
    """q4_gemv_dev for m = 1..9 at a small and a long K (fused and split paths)."""
    import torch
    o = oracle.Oracle()
    for k_in, n_out in ((1536, 200), (18944, 40), (40960, 16)):
        w, s, b = synth.qlinear(400 + k_in, n_out, k_in, 64)
        x = synth.activations(401, 9, k_in)
        want = o.gemv_rows(w, s, b, x, 64)
        tw, ts, tb, tx = (torch.from_numpy(a).cuda() for a in (w, s.view(np.int16), b.view(np.int16), x))
        for m in range(1, 10):
            print(f"dev K={k_in} N={n_out} m={m}", flush=True)
            got = q4.gemv_dev(tw, ts, tb, tx[:m].contiguous())
            torch.cuda.synchronize()
            assert_bit_exact(got.cpu().numpy(), want[:m], f"K={k_in} m={m}")


@pytest.mark.parametrize("gs", [64, 128])
def test_one_row_five_item_ring(lib, gs):
    """One row at n_in = 9216 (five chunks of 256 words, one row per unit:
    the streaming kernel's five-item ring) and at 8200 (a partial fifth
    chunk), bit-exact vs the oracle, through q4_gemv_dev and a grouped call."""
    import torch
    o = oracle.Oracle()
    for n_in, n_out in ((9216, 1000), (9216, 37), (8192 + gs, 300)):
        print(f"n_in {n_in} n_out {n_out} gs {gs}", flush=True)
        w, s, b = synth.qlinear(140 + n_in + gs + n_out, n_out, n_in, gs)
        x = synth.activations(141 + n_in, 1, n_in)
        want = o.gemv(w, s, b, x[0], gs)
        tw, ts, tb, tx = (torch.from_numpy(np.ascontiguousarray(a)).cuda()
                          for a in (w, s.view(np.int16), b.view(np.int16), x))
        got = q4.gemv_dev(tw, ts, tb, tx)
        got2 = q4.gemv_multi_dev([(tw, ts, tb), (tw, ts, tb)], tx)
        torch.cuda.synchronize()
        assert_bit_exact(got.cpu().numpy()[0], want, f"dev n_in={n_in}")
        for g in got2:
            assert_bit_exact(g.cpu().numpy()[0], want, f"multi n_in={n_in}")


def test_matrix_core_tile_variants(lib):
    """3..8 rows on the matrix cores, bit-exact vs the oracle, for the
    variants the Qwen shapes leave out: group counts not a multiple of 8
    (per-group scale/bias loads; 13 and 44 groups), 16-row tiles with a
    partial last tile (N = 300), 32-row tiles of 8 waves (N = 9000) and of 4
    waves (N = 16400, a partial last tile)."""
    import torch
    o = oracle.Oracle()
    for k_in, n_out in ((832, 300), (2816, 48), (512, 9000), (832, 16400)):
        w, s, b = synth.qlinear(500 + k_in + n_out, n_out, k_in, 64)
        x = synth.activations(501, 8, k_in)
        want = o.gemv_rows(w, s, b, x, 64)
        tw, ts, tb, tx = (torch.from_numpy(a).cuda() for a in (w, s.view(np.int16), b.view(np.int16), x))
        for m in (3, 5, 8):
            print(f"matrix cores K={k_in} N={n_out} m={m}", flush=True)
            got = q4.gemv_dev(tw, ts, tb, tx[:m].contiguous())
            torch.cuda.synchronize()
            assert_bit_exact(got.cpu().numpy(), want[:m], f"K={k_in} N={n_out} m={m}")


def test_matrix_core_group_count_bounds(lib):
    """The matrix-core path at one group (K = 64: a window holds a single
    group, every other group slot past the end) and at 64 and 65 groups
    (K = 4096, 4160), for 16-row and 32-row tiles, with rows past M zero in
    the prepared x.  Bit-exact vs the oracle."""
    import torch
    o = oracle.Oracle()
    for k_in, n_out in ((64, 40), (4096, 3584), (4096, 9000), (4160, 200)):
        w, s, b = synth.qlinear(800 + k_in + n_out, n_out, k_in, 64)
        x = synth.activations(801, 8, k_in)
        want = o.gemv_rows(w, s, b, x, 64)
        tw, ts, tb, tx = (torch.from_numpy(a).cuda() for a in (w, s.view(np.int16), b.view(np.int16), x))
        for m in (3, 7, 8):
            print(f"matrix cores, group bounds K={k_in} N={n_out} m={m}", flush=True)
            got = q4.gemv_dev(tw, ts, tb, tx[:m].contiguous())
            torch.cuda.synchronize()
            assert_bit_exact(got.cpu().numpy(), want[:m], f"K={k_in} N={n_out} m={m}")


def test_matrix_core_uneven_prep_slices(lib):
    """The matrix-core x prep splits each row's groups over up to 8
    workgroups in slices of ceil(G / slices): K = 6208 (97 groups, slices of
    33/33/31) and K = 9024 (141 groups, 36/36/36/33) leave a short last slice,
    and rows past M are zero-filled across uneven slices.  Bit-exact vs the
    oracle at 3, 5 and 8 rows."""
    import torch
    o = oracle.Oracle()
    for k_in, n_out in ((6208, 200), (9024, 96)):
        w, s, b = synth.qlinear(700 + k_in, n_out, k_in, 64)
        x = synth.activations(701, 8, k_in)
        want = o.gemv_rows(w, s, b, x, 64)
        tw, ts, tb, tx = (torch.from_numpy(a).cuda() for a in (w, s.view(np.int16), b.view(np.int16), x))
        for m in (3, 5, 8):
            print(f"uneven prep slices K={k_in} N={n_out} m={m}", flush=True)
            got = q4.gemv_dev(tw, ts, tb, tx[:m].contiguous())
            torch.cuda.synchronize()
            assert_bit_exact(got.cpu().numpy(), want[:m], f"K={k_in} N={n_out} m={m}")


def test_release_drops_dequant_row_blocks(lib):
    """q4_dequant registers each row block it is asked for under the block's
    own address; q4_release(base) must drop those blocks too, so weights
    rewritten in place after a release are uploaded again."""
    o = oracle.Oracle()
    n_out, n_in = 1536, 512
    w, s, b = synth.qlinear(810, n_out, n_in, 64)
    w, s, b = w.copy(), s.view(np.uint16).copy(), b.view(np.uint16).copy()
    out = np.empty((512, n_in), np.float32)

    def dq(r0, r1):
        rc = lib.q4_dequant(w.ctypes.data, s.ctypes.data, b.ctypes.data, out.ctypes.data, r0, r1, n_in, 64, 1)
        assert rc == 0, q4.last_error(lib)
        return out[: r1 - r0].copy()

    lib.q4_release(w.ctypes.data)
    for r0 in (0, 512, 1024):
        assert_bit_exact(dq(r0, r0 + 512), o.dequant(w, s.view(np.float16), b.view(np.float16), 64, r0, r0 + 512),
                         f"rows {r0}..")
    assert lib.q4_release(w.ctypes.data) == 3
    assert lib.q4_release(w.ctypes.data) == 0
    # new weights at the same addresses (every sampled word may even be equal:
    # the release, not the fingerprint, has to make the library read them)
    w2, s2, b2 = synth.qlinear(811, n_out, n_in, 64)
    w[:] = w2
    s[:] = s2.view(np.uint16)
    b[:] = b2.view(np.uint16)
    got = dq(512, 1024)
    assert_bit_exact(got, o.dequant(w, s.view(np.float16), b.view(np.float16), 64, 512, 1024), "after release")
    assert lib.q4_release(w.ctypes.data) == 1


def test_workspace_grown_after_capture_keeps_graph_valid(lib):
    """A graph captured with the stream's workspace at one size must stay
    valid after an eager call on the same stream grows it: the buffers the
    graph holds are retired, not freed.  Replays, with eager work between
    them, match the eager result bit for bit."""
    import torch
    o = oracle.Oracle()
    st = torch.cuda.Stream()
    ws_, ss_, bs_ = synth.qlinear(820, 256, 1536, 64)
    wb_, sb_, bb_ = synth.qlinear(821, 128, 18944, 64)
    xs = synth.activations(822, 4, 1536)
    xb = synth.activations(823, 4, 18944)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    small = (t(ws_), t(ss_.view(np.int16)), t(bs_.view(np.int16)))
    big = (t(wb_), t(sb_.view(np.int16)), t(bb_.view(np.int16)))
    txs, txb = t(xs), t(xb)
    out_s = torch.empty((4, 256), device="cuda")
    torch.cuda.synchronize()
    with torch.cuda.stream(st):
        q4.gemv_dev(*small, txs, out=out_s, stream=st)      # sizes the workspace for the small call
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        q4.gemv_dev(*small, txs, out=out_s, stream=st)
    torch.cuda.synchronize()
    want_s = o.gemv_rows(ws_, ss_, bs_, xs, 64)
    want_b = o.gemv_rows(wb_, sb_, bb_, xb, 64)
    for rep in range(3):
        with torch.cuda.stream(st):
            got_b = q4.gemv_dev(*big, txb, stream=st)       # grows the workspace (first time)
        torch.cuda.synchronize()
        assert_bit_exact(got_b.cpu().numpy(), want_b, f"eager big call {rep}")
        out_s.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(st):
            g.replay()
        torch.cuda.synchronize()
        assert_bit_exact(out_s.cpu().numpy(), want_s, f"graph replay {rep}")


@pytest.mark.parametrize("k_in,n_out", [(3584, 3584), (3584, 512), (18944, 3584), (3584, 18944)])
def test_group_size_128_qwen_shapes(lib, k_in, n_out):
    """Group size 128 (MLX's other common 4-bit layout) at the Qwen2.5-7B
    projection shapes: 1 and 2 rows take the streaming kernel with 128-wide
    groups, 3 and 4 rows the general path; bit-exact vs the oracle, and the
    oracle vs the reference kernel compiled from source where it is built."""
    import torch
    o = oracle.Oracle()
    w, s, b = synth.qlinear(900 + k_in + n_out, n_out, k_in, 128)
    x = synth.activations(901, 4, k_in)
    want = o.gemv_rows(w, s, b, x, 128)
    if os.path.exists(oracle.ref_path(1)):
        # the reference kernel compiled from source, on the first row
        ref = np.empty(n_out, np.float32)
        assert oracle.load_ref(1).q4_gemv(w.ctypes.data, s.ctypes.data, b.ctypes.data, x[0].ctypes.data,
                                          ref.ctypes.data, n_out, k_in, 128, 8) == 0
        assert_bit_exact(want[0], ref, "oracle vs reference kernel")
    tw, ts, tb, tx = (torch.from_numpy(a).cuda() for a in (w, s.view(np.int16), b.view(np.int16), x))
    for m in (1, 2, 3, 4):
        print(f"gs128 K={k_in} N={n_out} m={m}", flush=True)
        got = q4.gemv_dev(tw, ts, tb, tx[:m].contiguous())
        torch.cuda.synchronize()
        assert_bit_exact(got.cpu().numpy(), want[:m], f"gs128 K={k_in} N={n_out} m={m}")


def test_group_size_128_multi_and_gate_up(lib):
    """Group size 128 through q4_gemv_multi_dev (q/k/v) and the gate/up
    pair: the grouped outputs bit-exact vs the oracle, h bit-identical
    between 2-row and 1-row launches and within 2e-6 of NumPy's float32
    SiLU of the oracle's gate and up (exp may differ in the last place)."""
    import torch
    o = oracle.Oracle()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    qkv = [synth.qlinear(910 + i, n, 3584, 128) for i, n in enumerate((3584, 512, 512))]
    x = synth.activations(913, 2, 3584)
    dev = [(t(w), t(s.view(np.int16)), t(b.view(np.int16))) for w, s, b in qkv]
    for m in (1, 2):
        print(f"gs128 q/k/v m={m}", flush=True)
        outs = q4.gemv_multi_dev(dev, t(x[:m]))
        torch.cuda.synchronize()
        for (w, s, b), got in zip(qkv, outs):
            assert_bit_exact(got.cpu().numpy(), o.gemv_rows(w, s, b, x[:m], 128), f"gs128 multi m={m} n={w.shape[0]}")
    gate, up = synth.qlinear(920, 18944, 3584, 128), synth.qlinear(921, 18944, 3584, 128)
    gd, ud = [(t(w), t(s.view(np.int16)), t(b.view(np.int16))) for w, s, b in (gate, up)]
    print("gs128 gate/up", flush=True)
    h2 = q4.gate_up_silu_dev(gd, ud, t(x)).cpu().numpy()
    h1 = [q4.gate_up_silu_dev(gd, ud, t(x[r:r + 1])).cpu().numpy()[0] for r in range(2)]
    torch.cuda.synchronize()
    for r in range(2):
        assert np.array_equal(h2[r].view(np.uint32), h1[r].view(np.uint32)), f"row {r}"
        g, u = o.gemv(*gate, x[r], 128), o.gemv(*up, x[r], 128)
        h_ref = (g / (np.float32(1.0) + np.exp(-g, dtype=np.float32)) * u).astype(np.float32)
        assert oracle.normwise_rel(h2[r], h_ref) < 2e-6, f"row {r}"
