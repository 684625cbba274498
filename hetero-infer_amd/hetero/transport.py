"""The activation codec of the reference's transport (hetero/transport.py:193-225),
run on the GPU by libq4gemv.so (include/q4wire.h).

Only the codec is here.  The reference's framing, sockets and link shaping
move bytes between hosts and stay the reference's.  What changes is where
the codec runs:

  * a device tensor (the hidden state of a GPU stage) is encoded in HBM, and
    the payload comes back as a device uint8 tensor, so only the payload
    crosses to the host.  A device payload decodes straight into a device
    fp32 hidden state;
  * a NumPy array or a bytes payload takes the reference's host-side
    contract: encode returns (header, bytes) and decode returns a float16
    array.  The data goes to the GPU and back.

encode rounds its input to fp16 first, as the NumPy backend's to_wire does
before every encode (hetero/backends.py:100-101; hetero/engine.py:97).  An
fp16 input is therefore encoded exactly as the reference encodes it.  A
device decode ends with the backend's from_wire (hetero/backends.py:103-104:
fp16 -> fp32).

Headers are the reference's: {"codec": name, "shape": [...]}.
There is no CPU fallback: a missing library raises from q4.load().
"""
from __future__ import annotations

from typing import Tuple

import numpy as np

from . import q4

CODECS = {"fp16": 0, "int8": 1}        # include/q4wire.h: Q4_WIRE_FP16, Q4_WIRE_INT8


def _codec_id(codec: str) -> int:
    if codec not in CODECS:
        raise ValueError(f"unknown codec {codec}")            # hetero/transport.py:212, :225
    return CODECS[codec]


def _rows_hidden(shape) -> Tuple[int, int]:
    shape = tuple(int(s) for s in shape)
    if len(shape) == 0:
        return 1, 1
    hidden = shape[-1]
    rows = int(np.prod(shape[:-1], dtype=np.int64)) if len(shape) > 1 else 1
    return rows, hidden


def payload_bytes(codec: str, shape) -> int:
    """Bytes of the payload of an activation of `shape` under `codec`."""
    rows, hidden = _rows_hidden(shape)
    if hidden == 0 or rows == 0:
        return 0
    return int(q4.load().q4_wire_payload_bytes(_codec_id(codec), rows, hidden))


def _is_device_tensor(a) -> bool:
    try:
        import torch
    except ImportError:
        return False
    return isinstance(a, torch.Tensor) and a.is_cuda


def encode(arr, codec: str = "fp16", stream=None, lib=None):
    """hetero/transport.py:198-211.  A device tensor gives (header, device
    uint8 payload); a NumPy array gives (header, bytes)."""
    import torch
    lib = lib or q4.load()
    cid = _codec_id(codec)
    on_device = _is_device_tensor(arr)
    if on_device:
        x = arr.detach().to(torch.float32).contiguous()
    else:   # host arrays: copy, encode and copy back on the current stream
        x = torch.from_numpy(np.ascontiguousarray(np.asarray(arr, dtype=np.float32))).cuda()
        stream = None
    shape = list(x.shape)
    rows, hidden = _rows_hidden(shape)
    header = {"codec": codec, "shape": shape}
    if rows * hidden == 0:
        payload = torch.empty(0, dtype=torch.uint8, device=x.device)
    else:
        n = int(lib.q4_wire_payload_bytes(cid, rows, hidden))
        payload = torch.empty(n, dtype=torch.uint8, device=x.device)
        q4.check(lib, lib.q4_wire_encode_dev(x.data_ptr(), rows, hidden, cid, payload.data_ptr(),
                                             q4._stream(stream)), "q4_wire_encode_dev")
    if on_device:
        return header, payload
    return header, payload.cpu().numpy().tobytes()


def decode(header: dict, payload, stream=None, lib=None):
    """hetero/transport.py:214-225.  A device uint8 payload decodes to a
    device fp32 tensor (the backend's from_wire included); a bytes payload to
    a NumPy float16 array, as the reference returns it."""
    import torch
    lib = lib or q4.load()
    cid = _codec_id(header["codec"])
    shape = tuple(int(s) for s in header["shape"])
    rows, hidden = _rows_hidden(shape)
    on_device = _is_device_tensor(payload)
    if on_device:
        p = payload.contiguous()
    else:   # host bytes: copy, decode and copy back on the current stream
        p = torch.from_numpy(np.frombuffer(bytes(payload), dtype=np.uint8).copy()).cuda()
        stream = None
    out = torch.empty(shape, dtype=torch.float32, device=p.device)
    if rows * hidden:
        need = int(lib.q4_wire_payload_bytes(cid, rows, hidden))
        if p.numel() != need:                                  # the reshape of transport.py:217, :222
            raise ValueError(f"payload of {p.numel()} bytes for {header['codec']} {list(shape)}, "
                             f"which takes {need}")
        q4.check(lib, lib.q4_wire_decode_dev(p.data_ptr(), rows, hidden, cid, out.data_ptr(),
                                             q4._stream(stream)), "q4_wire_decode_dev")
    if on_device:
        return out
    return out.cpu().numpy().astype(np.float16)
