"""The activation wire codec on the GPU (include/q4wire.h, hetero/transport.py
here) against the oracle restatement of hetero/transport.py:193-225 with the
NumPy backend's conversions (hetero/backends.py:100-104): payload bytes and
decoded values bit for bit, both codecs, through the device entry points and
the host-array contract, on the vector and the per-value paths."""
import numpy as np
import pytest

from hetero import q4, transport
from oracle import wire

pytestmark = pytest.mark.gpu


def edge_rows(hidden):
    """Rows the codec treats specially: zeros, ties at k + 1/2 of a
    power-of-two scale, fp16 subnormals and the fp16 range's top."""
    s = 2.0 ** -4
    ties = np.resize(np.array([127, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -127, 3.5], np.float64) * s, hidden)
    sub = np.resize(np.array([1e-7, -3e-8, 2 ** -24, 6e-5, -6.1e-5, 0.0], np.float64), hidden)
    top = np.resize(np.array([65519.0, -65504.0, 1.0, 60000.0, -0.0], np.float64), hidden)
    return np.stack([np.zeros(hidden), ties, sub, top]).astype(np.float32)


def rows_for(seed, rows, hidden):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, hidden)) * np.exp(rng.uniform(-4, 4, (rows, 1)))).astype(np.float32)
    e = edge_rows(hidden)
    k = min(rows, e.shape[0])
    x[:k] = e[:k]
    return x


def check_device_round(x, codec):
    import torch
    print(f"wire {codec} shape={x.shape}", flush=True)
    h_ref, p_ref = wire.stage_encode(x, codec)
    xd = torch.from_numpy(x).cuda()
    h, p = transport.encode(xd, codec)
    assert h == h_ref
    assert p.is_cuda and p.dtype == torch.uint8
    got = p.cpu().numpy().tobytes()
    assert got == p_ref, f"{codec} payload differs at byte {next(i for i in range(len(got)) if got[i] != p_ref[i])}"
    back = transport.decode(h, p)
    assert back.is_cuda and back.dtype == torch.float32 and tuple(back.shape) == x.shape
    want = wire.stage_decode(h_ref, p_ref)
    assert np.array_equal(back.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("codec", ["fp16", "int8"])
@pytest.mark.parametrize("rows,hidden", [(1, 3584), (4, 3584), (256, 3584), (3, 8), (5, 12), (2, 100),
                                         (7, 4096), (2, 18944), (1, 32768), (9, 1)])
def test_codec_matches_oracle(codec, rows, hidden):
    check_device_round(rows_for(rows * 1000 + hidden, rows, hidden), codec)


@pytest.mark.parametrize("codec", ["fp16", "int8"])
def test_codec_three_dim_shape(codec):
    x = rows_for(11, 10, 3584).reshape(2, 5, 3584)
    check_device_round(x, codec)


@pytest.mark.parametrize("codec", ["fp16", "int8"])
def test_codec_unaligned_input(codec):
    """A view one float into its buffer: the per-value path."""
    import torch
    x = rows_for(12, 3, 3584)
    buf = torch.zeros(x.size + 1, dtype=torch.float32, device="cuda")
    buf[1:] = torch.from_numpy(x.reshape(-1)).cuda()
    view = buf[1:].view(3, 3584)
    assert view.data_ptr() % 16 == 4
    h_ref, p_ref = wire.stage_encode(x, codec)
    h, p = transport.encode(view, codec)
    assert p.cpu().numpy().tobytes() == p_ref


@pytest.mark.parametrize("codec", ["fp16", "int8"])
def test_host_contract(codec):
    """NumPy in, bytes out; bytes in, float16 out -- as transport.encode/decode."""
    x = rows_for(13, 6, 3584)
    h_ref, p_ref = wire.stage_encode(x, codec)
    h, p = transport.encode(x.astype(np.float16), codec)     # what the reference's encode receives
    assert h == h_ref and isinstance(p, bytes) and p == p_ref
    back = transport.decode(h_ref, p_ref)
    ref = wire.decode(h_ref, p_ref)
    assert back.dtype == np.float16 and np.array_equal(back.view(np.uint16), ref.view(np.uint16))


def test_empty_and_errors():
    import torch
    h, p = transport.encode(torch.zeros((0, 3584), device="cuda"), "int8")
    assert h == {"codec": "int8", "shape": [0, 3584]} and p.numel() == 0
    with pytest.raises(ValueError):
        transport.encode(torch.zeros((1, 8), device="cuda"), "bf16")
    with pytest.raises(ValueError):
        transport.decode({"codec": "int8", "shape": [2, 8]}, torch.zeros(8, dtype=torch.uint8, device="cuda"))
    lib = q4.load()
    assert lib.q4_wire_encode_dev(None, 1, 8, 0, None, None) == q4.Q4_EARG
    assert lib.q4_wire_encode_dev(None, 1, 40000, 1, None, None) == q4.Q4_EARG
    x = torch.zeros(40000, device="cuda")
    pay = torch.zeros(40004, dtype=torch.uint8, device="cuda")
    assert lib.q4_wire_encode_dev(x.data_ptr(), 1, 40000, 1, pay.data_ptr(), None) == q4.Q4_EARG
    assert "32768" in q4.last_error(lib)


def test_graph_replays_match_eager():
    """Encode + decode captured once, replayed with new inputs in place."""
    import torch
    rows, hidden = 8, 3584
    xs = [rows_for(20 + i, rows, hidden) for i in range(3)]
    x = torch.from_numpy(xs[0]).cuda()
    lib = q4.load()
    n = int(lib.q4_wire_payload_bytes(1, rows, hidden))
    pay = torch.zeros(n, dtype=torch.uint8, device="cuda")
    out = torch.zeros((rows, hidden), dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            st = torch.cuda.current_stream().cuda_stream
            assert lib.q4_wire_encode_dev(x.data_ptr(), rows, hidden, 1, pay.data_ptr(), st) == 0
            assert lib.q4_wire_decode_dev(pay.data_ptr(), rows, hidden, 1, out.data_ptr(), st) == 0
    for xi in xs:
        x.copy_(torch.from_numpy(xi).cuda())
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        h_ref, p_ref = wire.stage_encode(xi, "int8")
        assert pay.cpu().numpy().tobytes() == p_ref
        assert np.array_equal(out.cpu().numpy(), wire.stage_decode(h_ref, p_ref))
