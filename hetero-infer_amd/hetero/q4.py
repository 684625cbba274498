"""ctypes binding of libq4gemv.so, the gfx950 int4 GEMV library.

The drop-in entry points keep the reference's argument types exactly
(hetero/cpu_model.py:41-44): q4_gemv takes [c_void_p]*5 + [c_int]*4 and
q4_dequant [c_void_p]*4 + [c_int]*5, both returning c_int.  The additional
entry points (batched, device-pointer, release) are declared the same way;
their C declarations are in include/q4gemv.h.

There is no fallback: if the library is missing, load() raises.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

PKG_PARENT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_PARENT, "kernel", "libq4gemv.so")

EXPORTS = ("q4_gemv", "q4_dequant", "q4_gemv_batched", "q4_release", "q4_release_all",
           "q4_last_error", "q4_gemv_dev", "q4_gemv_noalloc_dev", "q4_gemv_multi_dev", "q4_gate_up_silu_dev",
           "q4_mlp_dev", "q4_gemm_bf16_dev", "q4_gemm_bf16_multi_dev", "q4_gemm_bf16in_multi_dev",
           "q4_gemm_bf16in_gate_up_silu_dev", "q4_set_rows", "q4_prefill_errors",
           "q4_dequant_dev",
           "q4_dequant_bf16_dev",
           # decode-step kernels (include/q4decode.h)
           "q4_embed_dev", "q4_add_rmsnorm_dev", "q4_rope_kv_dev", "q4_attention_scratch_floats",
           "q4_attention_dev", "q4_attention_rope_dev", "q4_argmax_dev",
           "q4_norm_gemv_multi_dev", "q4_norm_gate_up_silu_dev", "q4_norm_gemv_argmax_dev",
           # the prompt forward (include/q4decode.h)
           "q4_embed_rows_dev", "q4_add_rmsnorm_rows_dev", "q4_rope_kv_rows_dev", "q4_silu_mul_dev",
           "q4_prompt_attention_dev", "q4_add_rmsnorm_rows_bf16_dev", "q4_prompt_attention_bf16_dev",
           # activation wire codec (include/q4wire.h)
           "q4_wire_payload_bytes", "q4_wire_encode_dev", "q4_wire_decode_dev",
           # chained GEMV programs (include/q4chain.h)
           "q4_chain_create", "q4_chain_run", "q4_chain_stamps", "q4_chain_errors", "q4_chain_destroy")

Q4_EHIP, Q4_ENOMEM, Q4_EARG = -2, -3, -4

_VP, _I, _F, _L = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_long


def declare(lib: ctypes.CDLL) -> ctypes.CDLL:
    """Attach argtypes/restype for every symbol the library exports."""
    lib.q4_gemv.argtypes = [_VP] * 5 + [_I] * 4
    lib.q4_gemv.restype = _I
    lib.q4_dequant.argtypes = [_VP] * 4 + [_I] * 5
    lib.q4_dequant.restype = _I
    if hasattr(lib, "q4_gemv_batched"):
        lib.q4_gemv_batched.argtypes = [_VP] * 5 + [_I] * 5
        lib.q4_gemv_batched.restype = _I
        lib.q4_release.argtypes = [_VP]
        lib.q4_release.restype = _I
        lib.q4_release_all.argtypes = []
        lib.q4_release_all.restype = _I
        lib.q4_last_error.argtypes = []
        lib.q4_last_error.restype = ctypes.c_char_p
        lib.q4_gemv_dev.argtypes = [_VP] * 5 + [_I] * 4 + [_VP]
        lib.q4_gemv_dev.restype = _I
        lib.q4_gemv_noalloc_dev.argtypes = [_VP] * 5 + [_I] * 4 + [_VP]
        lib.q4_gemv_noalloc_dev.restype = _I
        lib.q4_gemv_multi_dev.argtypes = [_I] + [_VP] * 6 + [_I] * 3 + [_VP]
        lib.q4_gemv_multi_dev.restype = _I
        lib.q4_gate_up_silu_dev.argtypes = [_VP] * 8 + [_I] * 4 + [_VP]
        lib.q4_gate_up_silu_dev.restype = _I
        lib.q4_mlp_dev.argtypes = [_VP] * 12 + [_I] * 4 + [_VP]
        lib.q4_mlp_dev.restype = _I
        lib.q4_gemm_bf16_dev.argtypes = [_VP] * 5 + [_I] * 4 + [_VP]
        lib.q4_gemm_bf16_dev.restype = _I
        lib.q4_gemm_bf16_multi_dev.argtypes = [_I] + [_VP] * 6 + [_I] * 3 + [_VP]
        lib.q4_gemm_bf16_multi_dev.restype = _I
        lib.q4_gemm_bf16in_multi_dev.argtypes = [_I] + [_VP] * 6 + [_I] * 3 + [_VP]
        lib.q4_gemm_bf16in_multi_dev.restype = _I
        lib.q4_gemm_bf16in_gate_up_silu_dev.argtypes = [_VP] * 8 + [_I] * 4 + [_VP]
        lib.q4_gemm_bf16in_gate_up_silu_dev.restype = _I
        lib.q4_set_rows.argtypes = [_I]
        lib.q4_set_rows.restype = _I
        lib.q4_prefill_errors.argtypes = [_VP]
        lib.q4_prefill_errors.restype = _I
        lib.q4_dequant_dev.argtypes = [_VP] * 4 + [_I] * 4 + [_VP]
        lib.q4_dequant_dev.restype = _I
        lib.q4_dequant_bf16_dev.argtypes = [_VP] * 4 + [_I] * 4 + [_VP]
        lib.q4_dequant_bf16_dev.restype = _I
    if hasattr(lib, "q4_embed_dev"):
        lib.q4_embed_dev.argtypes = [_VP] * 5 + [_I] * 3 + [_VP]
        lib.q4_embed_dev.restype = _I
        lib.q4_add_rmsnorm_dev.argtypes = [_VP] * 3 + [_F, _VP, _I, _VP]
        lib.q4_add_rmsnorm_dev.restype = _I
        lib.q4_rope_kv_dev.argtypes = [_VP] * 10 + [_I] * 4 + [_VP]
        lib.q4_rope_kv_dev.restype = _I
        lib.q4_attention_scratch_floats.argtypes = [_I] * 3
        lib.q4_attention_scratch_floats.restype = _L
        lib.q4_attention_dev.argtypes = [_VP] * 6 + [_I] * 4 + [_F, _VP]
        lib.q4_attention_dev.restype = _I
        lib.q4_attention_rope_dev.argtypes = [_VP] * 11 + [_I] * 4 + [_F, _VP]
        lib.q4_attention_rope_dev.restype = _I
        lib.q4_norm_gemv_multi_dev.argtypes = [_I] + [_VP] * 8 + [_F, _VP, _I, _I, _VP]
        lib.q4_norm_gemv_multi_dev.restype = _I
        lib.q4_norm_gate_up_silu_dev.argtypes = [_VP] * 9 + [_F, _VP, _VP, _I, _I, _I, _VP]
        lib.q4_norm_gate_up_silu_dev.restype = _I
        lib.q4_argmax_dev.argtypes = [_VP, _I, _VP, _VP, _VP, ctypes.c_int64, _I, _VP]
        lib.q4_argmax_dev.restype = _I
        lib.q4_norm_gemv_argmax_dev.argtypes = ([_VP] * 4 + [_I] + [_VP] * 3 + [_F, _VP, _I, _I] + [_VP] * 3
                                                + [ctypes.c_int64, _I, _VP])
        lib.q4_norm_gemv_argmax_dev.restype = _I
        lib.q4_embed_rows_dev.argtypes = [_VP] * 4 + [_I, _VP] + [_I] * 3 + [_VP]
        lib.q4_embed_rows_dev.restype = _I
        lib.q4_add_rmsnorm_rows_dev.argtypes = [_VP] * 3 + [_F, _VP, _I, _I, _VP]
        lib.q4_add_rmsnorm_rows_dev.restype = _I
        lib.q4_rope_kv_rows_dev.argtypes = [_VP] * 6 + [ctypes.c_int64, _I] + [_VP] * 3 + [_I] * 4 + [_VP]
        lib.q4_rope_kv_rows_dev.restype = _I
        lib.q4_silu_mul_dev.argtypes = [_VP] * 3 + [_L, _VP]
        lib.q4_silu_mul_dev.restype = _I
        lib.q4_prompt_attention_dev.argtypes = [_VP] * 4 + [_I, ctypes.c_int64] + [_I] * 4 + [_F, _VP]
        lib.q4_prompt_attention_dev.restype = _I
        lib.q4_add_rmsnorm_rows_bf16_dev.argtypes = [_VP] * 3 + [_F, _VP, _I, _I, _VP]
        lib.q4_add_rmsnorm_rows_bf16_dev.restype = _I
        lib.q4_prompt_attention_bf16_dev.argtypes = [_VP] * 4 + [_I, ctypes.c_int64] + [_I] * 4 + [_F, _VP]
        lib.q4_prompt_attention_bf16_dev.restype = _I
    if hasattr(lib, "q4_wire_encode_dev"):
        lib.q4_wire_payload_bytes.argtypes = [_I] * 3
        lib.q4_wire_payload_bytes.restype = ctypes.c_longlong
        lib.q4_wire_encode_dev.argtypes = [_VP, _I, _I, _I, _VP, _VP]
        lib.q4_wire_encode_dev.restype = _I
        lib.q4_wire_decode_dev.argtypes = [_VP, _I, _I, _I, _VP, _VP]
        lib.q4_wire_decode_dev.restype = _I
    if hasattr(lib, "q4_chain_create"):
        lib.q4_chain_create.argtypes = [ctypes.POINTER(ChainPhase), _I, ctypes.POINTER(_VP)]
        lib.q4_chain_create.restype = _I
        lib.q4_chain_run.argtypes = [_VP, _VP]
        lib.q4_chain_run.restype = _I
        lib.q4_chain_stamps.argtypes = [_VP, _VP, _L]
        lib.q4_chain_stamps.restype = _I
        lib.q4_chain_errors.argtypes = [_VP]
        lib.q4_chain_errors.restype = _I
        lib.q4_chain_destroy.argtypes = [_VP]
        lib.q4_chain_destroy.restype = _I
    return lib


class ChainPhase(ctypes.Structure):
    """q4_chain_phase of include/q4chain.h."""
    _fields_ = [("count", _I), ("pair", _I), ("w", _VP * 4), ("scales", _VP * 4), ("biases", _VP * 4),
                ("out", _VP * 4), ("n_out", _I * 4), ("x", _VP), ("n_in", _I), ("gs", _I)]


_LIB: Optional[ctypes.CDLL] = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise if it is not built."""
    global _LIB
    if _LIB is not None and path == LIB_PATH:
        return _LIB
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built: run `python hetero-infer_amd/build.py`")
    # One HIP runtime per process.  PyTorch-ROCm ships its own libamdhip64
    # (same SONAME, libamdhip64.so.7); if it is imported after this library
    # has pulled in /opt/rocm's copy, torch finds no GPU.  Importing torch
    # first makes the dynamic linker bind this library to torch's runtime.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = declare(ctypes.CDLL(path))
    if path == LIB_PATH:
        _LIB = lib
    return lib


def last_error(lib: ctypes.CDLL) -> str:
    return lib.q4_last_error().decode(errors="replace")


def check(lib: ctypes.CDLL, rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed with {rc}: {last_error(lib)}")


# ---- device-pointer helpers over torch tensors (torch is only plumbing) ----

def _ptr(t) -> int:
    return t.data_ptr()


# The entry points take raw device pointers and sizes, so nothing below the
# wrappers can tell a buffer of the wrong type or size: the wrappers check
# every tensor they pass (a too-small buffer would be read or written past
# its end by a kernel) and raise before any library call.

def _need(t, name, dtypes, numel=None, shape=None):
    import torch
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: a torch tensor, got {type(t).__name__}")
    if t.dtype not in dtypes:
        raise TypeError(f"{name}: dtype {t.dtype}, expected {' or '.join(str(d) for d in dtypes)}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: shape {tuple(t.shape)}, expected {tuple(shape)}")
    if numel is not None and t.numel() != numel:
        raise ValueError(f"{name}: {t.numel()} elements, expected {numel}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: not contiguous")
    return t


def _gpu(*ts):
    """Every tensor given (None skipped) on one GPU; after the type and size
    checks, so that those report first."""
    ts = [t for t in ts if t is not None]
    for t in ts:
        if t.device.type != "cuda":
            raise ValueError(f"a tensor on {t.device}: the library takes GPU tensors")
    if len({t.device for t in ts}) > 1:
        raise ValueError("tensors on more than one GPU")


def _f32():
    import torch
    return (torch.float32,)


def _mat(mat, name="w"):
    """(n_out, n_in, gs) of a (w, scales, biases) triple: int32 words
    [n_out, n_in / 8], 16-bit scales and biases [n_out, n_in / gs]."""
    import torch
    w, sc, b = mat
    if w.dim() != 2 or sc.dim() != 2:
        raise ValueError(f"{name}: w and scales are 2-D")
    n_out, n_in = w.shape[0], w.shape[1] * 8
    if sc.shape[1] == 0 or n_in % sc.shape[1]:
        raise ValueError(f"{name}: {sc.shape[1]} scale groups do not divide n_in {n_in}")
    gs = n_in // sc.shape[1]
    _need(w, name, (torch.int32, torch.uint32))
    for t, k in ((sc, "scales"), (b, "biases")):
        _need(t, f"{name} {k}", (torch.int16, torch.float16), shape=(n_out, n_in // gs))
    return n_out, n_in, gs


def _same_in(mats, name="mats"):
    dims = [_mat(m, f"{name}[{i}]") for i, m in enumerate(mats)]
    if not dims:
        raise ValueError(f"{name}: no matrices")
    if any(d[1:] != dims[0][1:] for d in dims):
        raise ValueError(f"{name}: the matrices differ in n_in or group size")
    return dims


def _ptr_or_null(t):
    return None if t is None else _ptr(t)


def _stream(stream=None) -> int:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def gemv_dev(w, scales, biases, x, out=None, stream=None, lib=None):
    """out[m, n_out] = x[m, n_in] @ W^T on the GPU (torch tensors on one device)."""
    import torch
    n_out, n_in, gs = _mat((w, scales, biases))
    x2 = _need(x, "x", _f32()).reshape(-1, n_in)
    if out is None:
        out = torch.empty((x2.shape[0], n_out), dtype=torch.float32, device=x.device)
    _need(out, "out", _f32(), numel=x2.shape[0] * n_out)
    _gpu(w, scales, biases, x2, out)
    lib = lib or load()
    rc = lib.q4_gemv_dev(_ptr(w), _ptr(scales), _ptr(biases), _ptr(x2), _ptr(out),
                         x2.shape[0], n_out, n_in, gs, _stream(stream))
    check(lib, rc, "q4_gemv_dev")
    return out


def gemv_multi_dev(mats, x, outs=None, stream=None, lib=None):
    """Several (w, scales, biases) sharing x in one launch; returns the outputs."""
    import torch
    dims = _same_in(mats)
    n_in, gs = dims[0][1], dims[0][2]
    x2 = _need(x, "x", _f32()).reshape(-1, n_in)
    m = x2.shape[0]
    if outs is None:
        outs = [torch.empty((m, d[0]), dtype=torch.float32, device=x.device) for d in dims]
    for i, (o, d) in enumerate(zip(outs, dims)):
        _need(o, f"outs[{i}]", _f32(), numel=m * d[0])
    k = len(mats)
    _gpu(x2, *outs, *(t for m in mats for t in m))
    lib = lib or load()
    arr = lambda vals: (ctypes.c_void_p * k)(*vals)
    rc = lib.q4_gemv_multi_dev(k, arr([_ptr(a[0]) for a in mats]), arr([_ptr(a[1]) for a in mats]),
                               arr([_ptr(a[2]) for a in mats]), arr([_ptr(o) for o in outs]),
                               (ctypes.c_int * k)(*[a[0].shape[0] for a in mats]),
                               _ptr(x2), m, n_in, gs, _stream(stream))
    check(lib, rc, "q4_gemv_multi_dev")
    return outs


def _norm_args(n_in, x, delta, norm_w, x_out):
    """One row of x, delta (optional), norm weights and x_out (optional), fp32."""
    _need(x, "x", _f32(), numel=n_in)
    _need(norm_w, "norm_w", _f32(), numel=n_in)
    if delta is not None:
        _need(delta, "delta", _f32(), numel=n_in)
    if x_out is not None:
        _need(x_out, "x_out", _f32(), numel=n_in)


def norm_gemv_multi_dev(mats, x, delta, norm_w, eps, x_out=None, outs=None, stream=None, lib=None):
    """gemv_multi_dev of rmsnorm(x + delta) * norm_w (one row), the norm in
    the GEMV prologue; x_out (if given, with delta) receives x + delta."""
    import torch
    dims = _same_in(mats)
    n_in, gs = dims[0][1], dims[0][2]
    _norm_args(n_in, x, delta, norm_w, x_out)
    if outs is None:
        outs = [torch.empty((1, d[0]), dtype=torch.float32, device=x.device) for d in dims]
    for i, (o, d) in enumerate(zip(outs, dims)):
        _need(o, f"outs[{i}]", _f32(), numel=d[0])
    k = len(mats)
    _gpu(x, delta, norm_w, x_out, *outs, *(t for m in mats for t in m))
    lib = lib or load()
    arr = lambda vals: (ctypes.c_void_p * k)(*vals)
    rc = lib.q4_norm_gemv_multi_dev(k, arr([_ptr(a[0]) for a in mats]), arr([_ptr(a[1]) for a in mats]),
                                    arr([_ptr(a[2]) for a in mats]), arr([_ptr(o) for o in outs]),
                                    (ctypes.c_int * k)(*[a[0].shape[0] for a in mats]), _ptr(x),
                                    _ptr_or_null(delta), _ptr(norm_w), eps, _ptr_or_null(x_out), n_in, gs,
                                    _stream(stream))
    check(lib, rc, "q4_norm_gemv_multi_dev")
    return outs


def norm_gemv_argmax_dev(mat, x, delta, norm_w, eps, tok, pos, hist=None, s0=0, x_out=None, logits=None,
                         stream=None, lib=None):
    """norm_gemv_multi_dev of one matrix plus the greedy token: *tok = argmax
    of the logits (NumPy's rule), hist[*pos - s0] = *tok when in range, *pos
    += 1 -- all in the GEMV's launch.  Returns the logits."""
    import torch
    w, s, b = mat
    n_out, n_in, gs = _mat(mat)
    _norm_args(n_in, x, delta, norm_w, x_out)
    if logits is None:
        logits = torch.empty((1, n_out), dtype=torch.float32, device=x.device)
    _need(logits, "logits", _f32(), numel=n_out)
    _need(tok, "tok", (torch.int64,), numel=1)
    _need(pos, "pos", (torch.int64,), numel=1)
    if hist is not None:
        _need(hist, "hist", (torch.int64,))
    _gpu(w, s, b, x, delta, norm_w, x_out, logits, tok, pos, hist)
    lib = lib or load()
    rc = lib.q4_norm_gemv_argmax_dev(_ptr(w), _ptr(s), _ptr(b), _ptr(logits), n_out, _ptr(x), _ptr_or_null(delta),
                                     _ptr(norm_w), eps, _ptr_or_null(x_out), n_in, gs, _ptr(tok), _ptr_or_null(hist),
                                     _ptr(pos), s0, 0 if hist is None else hist.numel(), _stream(stream))
    check(lib, rc, "q4_norm_gemv_argmax_dev")
    return logits


def _pair(gate, up):
    """(n_inter, n_in, gs) of a gate/up pair of equal shapes."""
    d = _mat(gate, "gate")
    if _mat(up, "up") != d:
        raise ValueError("gate and up differ in shape or group size")
    return d


def norm_gate_up_silu_dev(gate, up, x, delta, norm_w, eps, x_out=None, h=None, stream=None, lib=None):
    """gate_up_silu_dev of rmsnorm(x + delta) * norm_w (one row), the norm in
    the GEMV prologue; x_out (if given, with delta) receives x + delta."""
    import torch
    n_inter, n_in, gs = _pair(gate, up)
    _norm_args(n_in, x, delta, norm_w, x_out)
    if h is None:
        h = torch.empty((1, n_inter), dtype=torch.float32, device=x.device)
    _need(h, "h", _f32(), numel=n_inter)
    _gpu(*gate, *up, x, delta, norm_w, x_out, h)
    lib = lib or load()
    rc = lib.q4_norm_gate_up_silu_dev(*(_ptr(t) for t in gate), *(_ptr(t) for t in up), _ptr(x),
                                      _ptr_or_null(delta), _ptr(norm_w), eps, _ptr_or_null(x_out), _ptr(h),
                                      n_inter, n_in, gs, _stream(stream))
    check(lib, rc, "q4_norm_gate_up_silu_dev")
    return h


def gate_up_silu_dev(gate, up, x, h=None, stream=None, lib=None):
    """h[m, n_inter] = SiLU(x @ gate^T) * (x @ up^T); gate/up = (w, scales, biases)."""
    import torch
    n_inter, n_in, gs = _pair(gate, up)
    x2 = _need(x, "x", _f32()).reshape(-1, n_in)
    if h is None:
        h = torch.empty((x2.shape[0], n_inter), dtype=torch.float32, device=x.device)
    _need(h, "h", _f32(), numel=x2.shape[0] * n_inter)
    _gpu(*gate, *up, x2, h)
    lib = lib or load()
    rc = lib.q4_gate_up_silu_dev(*(_ptr(t) for t in gate), *(_ptr(t) for t in up), _ptr(x2), _ptr(h),
                                 x2.shape[0], n_inter, n_in, gs, _stream(stream))
    check(lib, rc, "q4_gate_up_silu_dev")
    return h


def mlp_dev(gate, up, down, x, h=None, out=None, stream=None, lib=None):
    """down(SiLU(gate(x)) * up(x)) for 4-bit (w, scales, biases) triples."""
    import torch
    n_inter, n_hidden, gs = _pair(gate, up)
    if _mat(down, "down") != (n_hidden, n_inter, gs):
        raise ValueError("down must map n_inter back to n_hidden with the same group size")
    x2 = _need(x, "x", _f32()).reshape(-1, n_hidden)
    m = x2.shape[0]
    if h is None:
        h = torch.empty((m, n_inter), dtype=torch.float32, device=x.device)
    if out is None:
        out = torch.empty((m, n_hidden), dtype=torch.float32, device=x.device)
    _need(h, "h", _f32(), numel=m * n_inter)
    _need(out, "out", _f32(), numel=m * n_hidden)
    _gpu(*gate, *up, *down, x2, h, out)
    lib = lib or load()
    rc = lib.q4_mlp_dev(*(_ptr(t) for t in gate), *(_ptr(t) for t in up), *(_ptr(t) for t in down),
                        _ptr(x2), _ptr(h), _ptr(out), m, n_hidden, n_inter, gs, _stream(stream))
    check(lib, rc, "q4_mlp_dev")
    return out


def gemm_bf16_dev(w, scales, biases, x, out=None, stream=None, lib=None):
    """Prefill: out[m, n_out] = bf16(x) @ bf16(dequant(W))^T with fp32 accumulation."""
    import torch
    n_out, n_in, gs = _mat((w, scales, biases))
    x2 = _need(x, "x", _f32()).reshape(-1, n_in)             # rounded to bf16 by the call
    if out is None:
        out = torch.empty((x2.shape[0], n_out), dtype=torch.float32, device=x.device)
    _need(out, "out", _f32(), numel=x2.shape[0] * n_out)
    _gpu(w, scales, biases, x2, out)
    lib = lib or load()
    rc = lib.q4_gemm_bf16_dev(_ptr(w), _ptr(scales), _ptr(biases), _ptr(x2), _ptr(out),
                              x2.shape[0], n_out, n_in, gs, _stream(stream))
    check(lib, rc, "q4_gemm_bf16_dev")
    return out


def gemm_bf16_multi_dev(mats, x, outs=None, stream=None, lib=None):
    """Prefill for several (w, scales, biases) sharing x in one launch; returns
    the outputs.  x in fp32 (rounded to bf16 by the call) or already bf16."""
    import torch
    dims = _same_in(mats)
    n_in, gs = dims[0][1], dims[0][2]
    x2 = _need(x, "x", (torch.float32, torch.bfloat16)).reshape(-1, n_in)
    m = x2.shape[0]
    if outs is None:
        outs = [torch.empty((m, d[0]), dtype=torch.float32, device=x.device) for d in dims]
    for i, (o, d) in enumerate(zip(outs, dims)):
        _need(o, f"outs[{i}]", _f32(), numel=m * d[0])
    k = len(mats)
    _gpu(x2, *outs, *(t for m in mats for t in m))
    lib = lib or load()
    arr = lambda vals: (ctypes.c_void_p * k)(*vals)
    fn = lib.q4_gemm_bf16in_multi_dev if x2.dtype == torch.bfloat16 else lib.q4_gemm_bf16_multi_dev
    rc = fn(k, arr([_ptr(a[0]) for a in mats]), arr([_ptr(a[1]) for a in mats]),
            arr([_ptr(a[2]) for a in mats]), arr([_ptr(o) for o in outs]),
            (ctypes.c_int * k)(*[a[0].shape[0] for a in mats]),
            _ptr(x2), m, n_in, gs, _stream(stream))
    check(lib, rc, fn.__name__)
    return outs


def gemm_bf16_gate_up_silu_dev(gate, up, xb, h=None, stream=None, lib=None):
    """Prefill MLP activations from bf16 x: h[m, n_inter] = bf16(SiLU(x @
    gate^T) * (x @ up^T)), the down projection's bf16 operand."""
    import torch
    n_inter, n_in, gs = _pair(gate, up)
    x2 = _need(xb, "x", (torch.bfloat16,)).reshape(-1, n_in)
    if h is None:
        h = torch.empty((x2.shape[0], n_inter), dtype=torch.bfloat16, device=xb.device)
    _need(h, "h", (torch.bfloat16,), numel=x2.shape[0] * n_inter)
    _gpu(*gate, *up, x2, h)
    lib = lib or load()
    rc = lib.q4_gemm_bf16in_gate_up_silu_dev(*(_ptr(t) for t in gate), *(_ptr(t) for t in up), _ptr(x2), _ptr(h),
                                             x2.shape[0], n_inter, n_in, gs, _stream(stream))
    check(lib, rc, "q4_gemm_bf16in_gate_up_silu_dev")
    return h


def set_rows(rows: int, lib=None) -> int:
    """The reference build's ROWS whose fp32 tail rows the plain GEMV entry
    points reproduce (kernel/q4gemv.c:185-200); returns the previous value."""
    lib = lib or load()
    prev = lib.q4_set_rows(int(rows))
    if prev < 0:
        check(lib, prev, "q4_set_rows")
    return prev


def prefill_errors(stream=None, lib=None) -> int:
    """Stream-K partial sums on `stream` that missed their bounded wait since
    the last call (0 in a correct run); synchronises the stream."""
    lib = lib or load()
    rc = lib.q4_prefill_errors(_stream(stream))
    if rc < 0:
        check(lib, rc, "q4_prefill_errors")
    return rc


def dequant_dev(w, scales, biases, row0=0, row1=None, out=None, bf16=False, stream=None, lib=None):
    import torch
    n_out, n_in, gs = _mat((w, scales, biases))
    row1 = n_out if row1 is None else row1
    rows = max(row1 - row0, 0)
    odt = torch.bfloat16 if bf16 else torch.float32
    if out is None:
        out = torch.empty((rows, n_in), dtype=odt, device=w.device)
    _need(out, "out", (odt,), numel=rows * n_in)
    _gpu(w, scales, biases, out)
    lib = lib or load()
    fn = lib.q4_dequant_bf16_dev if bf16 else lib.q4_dequant_dev
    rc = fn(_ptr(w), _ptr(scales), _ptr(biases), _ptr(out), row0, row1, n_in, gs, _stream(stream))
    check(lib, rc, "q4_dequant_dev")
    return out


class Chain:
    """A chained GEMV program (include/q4chain.h): `phases` is a list of
    (mats, x, outs, pair) with mats a list of (w, scales, biases) device
    tensors sharing the one-row input x, outs their output tensors (pair:
    gate/up, one output h = SiLU(gate x) * (up x)).  The phases run in order
    in one launch; a phase may read the outputs of the phases before it."""

    def __init__(self, phases, lib=None):
        self.lib = lib or load()
        self._keep = []
        table = (ChainPhase * len(phases))()
        for i, (mats, x, outs, pair) in enumerate(phases):
            ph = table[i]
            dims = _same_in(mats, f"phase {i}")
            n_in = dims[0][1]
            _need(x, f"phase {i} x", _f32(), numel=n_in)
            n_outs = [dims[0][0]] if pair else [d[0] for d in dims]
            if len(outs) < len(n_outs):
                raise ValueError(f"phase {i}: {len(outs)} outputs for {len(n_outs)}")
            for k, n in enumerate(n_outs):
                _need(outs[k], f"phase {i} outs[{k}]", _f32(), numel=n)
            _gpu(x, *outs[:len(n_outs)], *(t for m in mats for t in m))
            ph.count, ph.pair = len(mats), int(bool(pair))
            ph.n_in, ph.gs = n_in, dims[0][2]
            ph.x = _ptr(x)
            for k, (w, sc, b) in enumerate(mats):
                ph.w[k], ph.scales[k], ph.biases[k] = _ptr(w), _ptr(sc), _ptr(b)
                ph.n_out[k] = w.shape[0]
                ph.out[k] = _ptr(outs[0] if pair else outs[k])
            self._keep.append((mats, x, outs))
        self._plan = _VP()
        check(self.lib, self.lib.q4_chain_create(table, len(phases), ctypes.byref(self._plan)), "q4_chain_create")

    def run(self, stream=None):
        check(self.lib, self.lib.q4_chain_run(self._plan, _stream(stream)), "q4_chain_run")

    def stamps(self, buf):
        """Record per-phase event times (include/q4chain.h: q4_chain_stamps)
        into the int64 device tensor `buf` on later runs; None stops."""
        check(self.lib, self.lib.q4_chain_stamps(self._plan, None if buf is None else _ptr(buf),
                                                 0 if buf is None else buf.numel()), "q4_chain_stamps")

    def errors(self) -> int:
        """Barrier waits that ran out of time since the last call (synchronises)."""
        n = self.lib.q4_chain_errors(self._plan)
        if n < 0:
            check(self.lib, n, "q4_chain_errors")
        return n

    def close(self):
        if self._plan:
            plan, self._plan = self._plan, _VP()
            self._keep = []
            check(self.lib, self.lib.q4_chain_destroy(plan), "q4_chain_destroy")
        self._keep = []

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- host-pointer calls (the reference's ABI) over NumPy arrays ----

def gemv_host(lib, w: np.ndarray, scales: np.ndarray, biases: np.ndarray, x: np.ndarray,
              gs: int, nthreads: int = 0) -> np.ndarray:
    if w.ndim != 2 or w.dtype not in (np.uint32, np.int32) or not w.flags.c_contiguous:
        raise TypeError("w: C-contiguous [n_out, n_in / 8] uint32")
    n_out, n_in = w.shape[0], w.shape[1] * 8
    for a, k in ((scales, "scales"), (biases, "biases")):
        if a.dtype.itemsize != 2 or a.size != n_out * (n_in // gs) or not a.flags.c_contiguous:
            raise TypeError(f"{k}: C-contiguous [n_out, n_in / gs] of 16-bit values")
    xc = np.ascontiguousarray(x, dtype=np.float32)
    if xc.size != n_in:
        raise ValueError(f"x: {xc.size} values, expected {n_in}")
    out = np.empty(n_out, dtype=np.float32)
    rc = lib.q4_gemv(w.ctypes.data, scales.ctypes.data, biases.ctypes.data, xc.ctypes.data,
                     out.ctypes.data, n_out, n_in, gs, nthreads)
    if rc != 0:
        raise RuntimeError(f"q4_gemv failed with {rc}")
    return out
