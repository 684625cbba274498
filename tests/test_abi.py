"""C-ABI contract of libq4gemv.so, checked on the CPU (no GPU is touched).

* the library is built in-tree where the reference's loader looks
  (hetero/cpu_model.py:35-37: <package parent>/kernel/libq4gemv.so);
* it exports every function include/*.h declares, and the ctypes
  declarations match the reference's for the two drop-in symbols
  (hetero/cpu_model.py:41-44);
* shape errors return the reference's codes before any HIP call
  (kernel/q4gemv.c:237, :361, :363), other argument errors Q4_EARG.
"""
import ctypes
import os
import re

import numpy as np
import pytest

from hetero import q4

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("q4gemv.h", "q4decode.h", "q4wire.h", "q4chain.h")]


def header_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(q4_\w+)\s*\(", text))
    return sorted(names)


def test_every_header_is_checked():
    assert sorted(HEADERS) == sorted(os.path.join(ROOT, "include", h)
                                     for h in os.listdir(os.path.join(ROOT, "include")) if h.endswith(".h"))


@pytest.fixture(scope="module")
def lib():
    return q4.load()


def test_library_location_mirrors_reference():
    assert q4.LIB_PATH == os.path.join(ROOT, "hetero-infer_amd", "kernel", "libq4gemv.so")
    assert os.path.exists(q4.LIB_PATH), "run python hetero-infer_amd/build.py"


def test_exports_every_declared_function(lib):
    declared = header_functions()
    assert {"q4_gemv", "q4_dequant"} <= set(declared)
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(q4.EXPORTS)


def test_dropin_signatures_match_reference(lib):
    vp, i = ctypes.c_void_p, ctypes.c_int
    assert list(lib.q4_gemv.argtypes) == [vp] * 5 + [i] * 4
    assert list(lib.q4_dequant.argtypes) == [vp] * 4 + [i] * 5
    assert lib.q4_gemv.restype is i and lib.q4_dequant.restype is i


def test_shape_errors_before_any_device_call(lib):
    w = np.zeros((4, 32), np.uint32)
    s = np.zeros((4, 4), np.uint16)
    x = np.zeros(256, np.float32)
    out = np.zeros(4, np.float32)
    a = (w.ctypes.data, s.ctypes.data, s.ctypes.data, x.ctypes.data, out.ctypes.data)
    assert lib.q4_gemv(*a, 4, 256, 32, 1) == -1            # gs % 64 (x86 reference)
    assert lib.q4_gemv(*a, 4, 200, 64, 1) == -1            # n_in % gs
    assert lib.q4_gemv(*a, 4, 256, 0, 1) == -1             # gs <= 0 (reference would trap)
    assert lib.q4_gemv_batched(*a, 1, 4, 200, 64, 1) == -1
    d = (w.ctypes.data, s.ctypes.data, s.ctypes.data, out.ctypes.data)
    assert lib.q4_dequant(*d, 0, 2, 256, 12, 1) == -1      # gs % 8
    assert lib.q4_dequant(*d, 3, 3, 256, 64, 1) == 0       # empty range
    assert lib.q4_dequant(*d, 3, 1, 256, 64, 1) == 0       # reversed range
    assert lib.q4_gemv_dev(*a[:5], 1, 4, 200, 64, None) == -1
    assert lib.q4_dequant_dev(*d, 0, 2, 256, 12, None) == -1


def test_set_rows_rejects_and_restores(lib):
    """ROWS outside [1, 64] is refused (no device call) and leaves the
    setting alone; a valid one returns the previous setting."""
    prev = q4.set_rows(1, lib)
    for bad in (0, -1, 65):
        assert lib.q4_set_rows(bad) == q4.Q4_EARG
    assert q4.set_rows(4, lib) == 1
    assert q4.set_rows(prev, lib) == 4


def test_rows_env_is_read_on_first_use(tmp_path):
    """HETERO_Q4_ROWS sets the ROWS of the reference build being replaced;
    a value outside [1, 64] is reported by the first call that needs it."""
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, {pkg!r}); from hetero import q4; lib = q4.load(); "
            "print(lib.q4_set_rows(1))").format(pkg=os.path.join(ROOT, "hetero-infer_amd"))
    for env, want in (("8", "8"), ("1", "1"), ("0", "1"), ("x", "1")):
        out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                             env=dict(os.environ, HETERO_Q4_ROWS=env), check=True).stdout.strip()
        assert out == want, (env, out)


def test_argument_errors(lib):
    assert lib.q4_gemv(None, None, None, None, None, 4, 256, 64, 1) == q4.Q4_EARG
    assert "null" in q4.last_error(lib)
    assert lib.q4_gemv_dev(None, None, None, None, None, 1, 4, 256, 64, None) == q4.Q4_EARG
    w = np.zeros(64, np.uint32)
    mis = w.ctypes.data + 4                                # not 16-byte aligned
    assert lib.q4_gemv_dev(mis, mis, mis, mis, mis, 1, 4, 256, 64, None) == q4.Q4_EARG
    arr = (ctypes.c_void_p * 5)()
    n = (ctypes.c_int * 5)()
    assert lib.q4_gemv_multi_dev(0, arr, arr, arr, arr, n, None, 1, 256, 64, None) == q4.Q4_EARG
    assert lib.q4_gemv_multi_dev(5, arr, arr, arr, arr, n, None, 1, 256, 64, None) == q4.Q4_EARG


def test_zero_rows_are_noops(lib):
    # n_out == 0 / m == 0: success without touching any pointer or device
    assert lib.q4_gemv(None, None, None, None, None, 0, 256, 64, 1) == 0
    assert lib.q4_gemv_dev(None, None, None, None, None, 0, 4, 256, 64, None) == 0
    assert lib.q4_gemv_dev(None, None, None, None, None, 1, 0, 256, 64, None) == 0


def test_release_without_registrations(lib):
    assert lib.q4_release(None) == 0
    assert lib.q4_release_all() >= 0


def test_decode_kernel_argument_errors(lib):
    """Argument checks of the decode-step entry points, before any launch."""
    assert lib.q4_add_rmsnorm_dev(None, None, None, 1e-6, None, 16, None) == q4.Q4_EARG
    x = np.zeros(16, np.float32)
    p = x.ctypes.data
    assert lib.q4_add_rmsnorm_dev(p, None, p, 1e-6, p, 0, None) == q4.Q4_EARG
    assert lib.q4_add_rmsnorm_dev(p, None, p, 1e-6, p, 8193, None) == q4.Q4_EARG
    assert lib.q4_embed_dev(p, p, p, p, p, 10, 100, 64, None) == q4.Q4_EARG          # n_in % gs
    assert lib.q4_rope_kv_dev(*([p] * 10), 28, 5, 128, 64, None) == q4.Q4_EARG      # heads % kv heads
    assert lib.q4_attention_dev(*([p] * 6), 72, 4, 128, 64, 0.1, None) == q4.Q4_EARG  # 18 heads per kv head
    assert lib.q4_attention_dev(*([p] * 6), 28, 4, 256, 64, 0.1, None) == q4.Q4_EARG  # head_dim > 128
    assert lib.q4_attention_rope_dev(*([p] * 11), 72, 4, 128, 64, 0.1, None) == q4.Q4_EARG
    assert lib.q4_attention_rope_dev(*([p] * 10), None, 28, 4, 128, 64, 0.1, None) == q4.Q4_EARG
    assert lib.q4_argmax_dev(None, 10, p, p, p, 0, 1, None) == q4.Q4_EARG
    # norm-prologue GEMVs: bad count, n_in past 8192, x_out aliasing x, gs != 64
    assert lib.q4_norm_gemv_multi_dev(0, None, None, None, None, None, p, None, p, 1e-6, None, 256, 64,
                                      None) == q4.Q4_EARG
    assert lib.q4_norm_gate_up_silu_dev(*([p] * 6), p, None, p, 1e-6, None, p, 64, 8256, 64, None) == q4.Q4_EARG
    assert lib.q4_norm_gate_up_silu_dev(*([p] * 6), p, p, p, 1e-6, p, p, 64, 256, 64, None) == q4.Q4_EARG
    assert lib.q4_norm_gate_up_silu_dev(*([p] * 6), p, None, p, 1e-6, None, p, 64, 256, 128, None) == q4.Q4_EARG
    # the chunks' parts, then 512 arrival counters, one per 128-byte line
    assert lib.q4_attention_scratch_floats(28, 128, 2048) == 28 * 32 * 130 + 512 * 32
    assert lib.q4_attention_scratch_floats(28, 128, 2049) == 28 * 33 * 130 + 512 * 32
    assert lib.q4_attention_dev(*([p] * 6), 520, 65, 128, 64, 0.1, None) == q4.Q4_EARG   # 520 query heads


def test_wire_codec_argument_errors(lib):
    """Payload sizes (host arithmetic) and the codec's checks before any launch."""
    assert lib.q4_wire_payload_bytes(0, 3, 3584) == 2 * 3 * 3584
    assert lib.q4_wire_payload_bytes(1, 3, 3584) == 3 * 4 + 3 * 3584
    assert lib.q4_wire_payload_bytes(1, 0, 3584) == 0
    assert lib.q4_wire_payload_bytes(2, 3, 3584) == -1
    assert lib.q4_wire_payload_bytes(0, -1, 3584) == -1
    assert lib.q4_wire_payload_bytes(0, 1, 0) == -1
    x = np.zeros(16, np.float32)
    p = x.ctypes.data
    assert lib.q4_wire_encode_dev(p, 1, 16, 7, p, None) == q4.Q4_EARG                 # unknown codec
    assert lib.q4_wire_encode_dev(p, -1, 16, 0, p, None) == q4.Q4_EARG
    assert lib.q4_wire_encode_dev(None, 1, 16, 1, p, None) == q4.Q4_EARG
    assert lib.q4_wire_encode_dev(p, 1, 40000, 1, p, None) == q4.Q4_EARG             # int8 row past 32768
    assert lib.q4_wire_encode_dev(p, 1, 16, 1, p + 2, None) == q4.Q4_EARG            # payload not 4-aligned
    assert lib.q4_wire_decode_dev(p, 1, 16, 3, p, None) == q4.Q4_EARG
    assert lib.q4_wire_decode_dev(None, 1, 16, 0, p, None) == q4.Q4_EARG
    assert lib.q4_wire_decode_dev(p + 2, 1, 16, 1, p, None) == q4.Q4_EARG
    assert lib.q4_wire_encode_dev(None, 0, 16, 1, None, None) == 0                    # no rows: no-op
    assert lib.q4_wire_decode_dev(None, 0, 16, 1, None, None) == 0


def test_chain_argument_errors(lib):
    """q4_chain_create rejects bad phases with Q4_EARG before any device call."""
    fake = 1 << 20                                       # 16-byte aligned, never dereferenced

    def phase(**kw):
        ph = q4.ChainPhase()
        ph.count, ph.pair, ph.n_in, ph.gs, ph.x = 1, 0, 256, 64, fake
        ph.w[0] = ph.scales[0] = ph.biases[0] = fake
        ph.out[0] = fake + (1 << 16)                     # apart from x
        ph.n_out[0] = 8
        for k, v in kw.items():
            setattr(ph, k, v)
        return ph

    def create(*phs):
        arr = (q4.ChainPhase * len(phs))(*phs)
        plan = ctypes.c_void_p()
        return lib.q4_chain_create(arr, len(phs), ctypes.byref(plan)), plan

    for bad in (dict(count=0), dict(count=5), dict(pair=1), dict(gs=128), dict(n_in=100), dict(n_in=0),
                dict(n_in=24576 + 64), dict(x=fake + 4), dict(x=0)):
        rc, plan = create(phase(**bad))
        assert rc == q4.Q4_EARG and not plan.value, bad
    ph = phase()
    ph.w[0] = fake + 8                                   # misaligned weights
    assert create(ph)[0] == q4.Q4_EARG
    ph = phase(count=2, pair=1)                          # pair with unequal rows / a null matrix
    ph.w[1] = ph.scales[1] = ph.biases[1] = ph.out[1] = fake
    ph.n_out[1] = 16
    assert create(ph)[0] == q4.Q4_EARG
    ph.n_out[1], ph.w[1] = 8, 0
    assert create(ph)[0] == q4.Q4_EARG
    assert create(phase(), phase(n_in=96))[0] == q4.Q4_EARG      # any bad phase
    rc, plan = create(phase())                           # valid: fails later only without a device
    assert rc != q4.Q4_EARG
    if plan.value:
        lib.q4_chain_destroy(plan)
    ph = phase()
    ph.out[0] = fake + 1020                              # the last value of x: the output overlaps it
    assert create(ph)[0] == q4.Q4_EARG
    assert lib.q4_chain_create(None, 1, ctypes.byref(ctypes.c_void_p())) == q4.Q4_EARG
    assert lib.q4_chain_run(None, None) == q4.Q4_EARG
    assert lib.q4_chain_destroy(None) == 0


def test_gemm_multi_argument_errors(lib):
    """q4_gemm_bf16_multi_dev checks its arguments before any device call:
    count, group size, shapes; a call with no rows or no columns is a no-op."""
    fake = 1 << 20                                       # 16-byte aligned, never dereferenced
    vp = ctypes.c_void_p

    def call(count, n_out, n_in=256, gs=64, m=4, x=fake, w=fake):
        k = max(count, 1)
        arr = lambda v: (vp * k)(*([v] * k))
        return lib.q4_gemm_bf16_multi_dev(count, arr(w), arr(fake), arr(fake), arr(fake),
                                          (ctypes.c_int * k)(*([n_out] * k)), x, m, n_in, gs, None)

    assert call(0, 8) == q4.Q4_EARG
    assert call(5, 8) == q4.Q4_EARG
    assert call(2, 8, gs=128) == q4.Q4_EARG                 # the prefill GEMM takes gs 64
    assert call(2, 8, n_in=100) != 0                          # n_in not a multiple of gs: the shape code
    assert call(2, -1) != 0
    assert call(2, 8, m=-1) == q4.Q4_EARG
    assert call(2, 8, m=0, x=None) == 0                       # nothing to compute
    assert call(2, 0, x=None) == 0
    assert call(2, 8, x=fake + 4) == q4.Q4_EARG               # misaligned x
    assert call(2, 8, w=fake + 8) == q4.Q4_EARG               # misaligned weights


def test_norm_gemv_argmax_argument_errors(lib):
    """q4_norm_gemv_argmax_dev checks its arguments before any device call:
    the GEMV shape, the norm-prologue limits, and the token, position and
    history pointers."""
    fake = 1 << 20                                       # 16-byte aligned, never dereferenced

    def call(n_out=1000, n_in=512, gs=64, w=fake, x=fake, norm_w=fake, tok=fake, pos=fake, hist=fake, hist_len=4):
        return lib.q4_norm_gemv_argmax_dev(w, fake, fake, fake, n_out, x, None, norm_w, 1e-6, None, n_in, gs,
                                           tok, hist, pos, 0, hist_len, None)

    assert call(n_out=0) == q4.Q4_EARG                  # no logits, no token
    assert call(n_out=-1) != 0
    assert call(tok=None) == q4.Q4_EARG
    assert call(pos=None) == q4.Q4_EARG
    assert call(hist=None) == q4.Q4_EARG                # hist_len > 0 needs the history
    assert call(w=fake + 8) == q4.Q4_EARG
    assert call(x=None) == q4.Q4_EARG
    assert call(x=fake + 4) == q4.Q4_EARG
    assert call(norm_w=None) == q4.Q4_EARG
    assert call(gs=128, n_in=512) == q4.Q4_EARG          # the norm prologue takes gs 64
    assert call(n_in=16384) == q4.Q4_EARG                # past the norm prologue's 8192
    assert call(n_in=100) != 0                           # not a multiple of gs
