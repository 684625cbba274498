"""The device wrappers of hetero/q4.py check every tensor before the library
sees its pointer: the entry points take raw device pointers and sizes, so a
buffer of the wrong type or size would be read or written past its end by a
kernel.  CPU tensors here: each wrong argument raises before any library
call (a CPU tensor of the right type raises for its device)."""
import pytest
import torch

from hetero import q4


def mat(n_out=64, n_in=256, gs=64, wdt=torch.int32, sdt=torch.int16):
    return (torch.zeros((n_out, n_in // 8), dtype=wdt), torch.zeros((n_out, n_in // gs), dtype=sdt),
            torch.zeros((n_out, n_in // gs), dtype=sdt))


def test_wrong_types_and_sizes_raise_before_the_library():
    m = mat()
    x32 = torch.zeros((1, 256))
    with pytest.raises(TypeError):
        q4.gemv_dev(*m, x32.to(torch.bfloat16))                   # fp32 x only
    with pytest.raises(TypeError):
        q4.gemm_bf16_dev(*m, x32.to(torch.bfloat16))              # rounds fp32 x itself
    with pytest.raises(TypeError):
        q4.gemv_dev(*mat(wdt=torch.float32), x32)                 # packed words
    with pytest.raises(TypeError):
        q4.gemv_dev(*mat(sdt=torch.float32), x32)                 # 16-bit scales
    with pytest.raises(ValueError):
        q4.gemv_dev(m[0], m[1][:, :2], m[2], x32)                 # scales of another group size
    with pytest.raises(ValueError):
        q4.gemv_dev(*m, x32, out=torch.zeros((1, 32)))            # output too small
    with pytest.raises(ValueError):
        q4.gemv_multi_dev([m, mat(n_in=512)], x32)                # n_in differs
    with pytest.raises(TypeError):
        q4.gemm_bf16_gate_up_silu_dev(m, m, x32)                  # bf16 x only
    with pytest.raises(ValueError):
        q4.gate_up_silu_dev(m, mat(n_out=32), x32)                # gate and up differ
    with pytest.raises(ValueError):
        q4.mlp_dev(m, m, mat(n_out=128, n_in=64), x32)            # down does not map back
    with pytest.raises(ValueError):
        q4.norm_gemv_multi_dev([m], x32, None, torch.zeros(128), 1e-6)   # norm weights too short
    with pytest.raises(ValueError):
        q4.dequant_dev(*m, out=torch.zeros((64, 128)))            # output too small
    with pytest.raises(TypeError):
        q4.norm_gemv_argmax_dev(m, x32, None, torch.zeros(256), 1e-6, torch.zeros(1, dtype=torch.int32),
                                torch.zeros(1, dtype=torch.int64))
    with pytest.raises(ValueError, match="GPU tensors"):
        q4.gemv_dev(*m, x32)                                      # right types, but on the CPU
