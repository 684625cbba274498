"""q4_gemv_noalloc_dev (the entry point that allocates nothing) against
q4_gemv_dev, called through the C-ABI: bit-identical outputs on two calls in
a row on one stream, the second with a smaller input (the static scratch
keeps the first call's contents), over the paths that use scratch -- 3..8
rows on the matrix cores, group size 128 on the split path -- and the
streaming path (1..2 rows, no scratch).  The size limit is refused on the
host before any launch."""
import numpy as np
import pytest

from hetero import q4, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    return q4.load()


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _call(lib, fn, w, s, b, x, m, n_out, n_in, gs, st):
    import torch
    out = torch.full((m, n_out), float("nan"), device="cuda")
    rc = fn(w.data_ptr(), s.data_ptr(), b.data_ptr(), x.data_ptr(), out.data_ptr(), m, n_out, n_in, gs, st)
    assert rc == 0, q4.last_error(lib)
    return out


CASES = [  # (m, n_out, n_in, gs): each pair is a larger call followed by a smaller one
    ((8, 3584, 3584, 64), (3, 200, 1536, 64)),      # matrix-core prep in the scratch
    ((11, 512, 18944, 64), (5, 96, 6208, 64)),      # 8 + 3 rows; uneven prep slices
    ((4, 300, 4096, 128), (2, 40, 1024, 128)),      # split path (gs 128): planes in the scratch
    ((2, 1024, 3584, 64), (1, 512, 512, 64)),       # streaming kernel: no scratch
]


@pytest.mark.parametrize("big,small", CASES)
def test_noalloc_matches_dev_two_calls(lib, big, small):
    import torch
    st = torch.cuda.Stream()
    outs = []
    for k, (m, n_out, n_in, gs) in enumerate((big, small)):
        print(f"noalloc case m={m} n_out={n_out} n_in={n_in} gs={gs}", flush=True)
        w, s, b = synth.qlinear(900 + 7 * k + n_in, n_out, n_in, gs)
        x = synth.activations(901 + k, m, n_in)
        tw, ts, tb, tx = _dev(w), _dev(s.view(np.int16)), _dev(b.view(np.int16)), _dev(x)
        torch.cuda.synchronize()
        got = _call(lib, lib.q4_gemv_noalloc_dev, tw, ts, tb, tx, m, n_out, n_in, gs, st.cuda_stream)
        want = _call(lib, lib.q4_gemv_dev, tw, ts, tb, tx, m, n_out, n_in, gs, st.cuda_stream)
        torch.cuda.synchronize()
        outs.append((got.cpu().numpy(), want.cpu().numpy()))
    for k, (got, want) in enumerate(outs):
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"call {k}"


def test_noalloc_refuses_beyond_limit(lib):
    import ctypes
    null = ctypes.c_void_p(16)
    rc = lib.q4_gemv_noalloc_dev(null, null, null, null, null, 1, 8, 32768 + 64, 64, None)
    assert rc == q4.Q4_EARG
    assert "32768" in q4.last_error(lib)
