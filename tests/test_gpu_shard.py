"""Loading a checkpoint shard straight into HBM (hetero/shard.py,
load_shard(framework="hip")): every tensor's device bytes equal the file's
(whatever the staging size, so chunks split tensors and span several), the
residency registry's accounting and its refusal of a shard that does not
fit, and a device-resident decode stage built from the loaded tensors giving
the logits of one built from the NumPy arrays, bit for bit."""
import os

import numpy as np
import pytest

from hetero import qwen2
from hetero.shard import Residency, ShardSpec, WeightIndex
from test_shard import tiny_cfg, write_checkpoint, write_raw

pytestmark = pytest.mark.gpu


def device_bytes(t):
    return t.reshape(-1).view(__import__("torch").uint8).cpu().numpy().tobytes() if t.numel() else b""


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("ckpt_gpu"))
    cfg = tiny_cfg(layers=3)
    w = qwen2.synthetic_weights(cfg, seed=5)
    write_checkpoint(d, cfg, w, split_at=2)
    return d, cfg, w


@pytest.mark.parametrize("staging", [1 << 20, 3 * 4096 + 4, 64 << 20])
@pytest.mark.parametrize("spec", [ShardSpec(0, 3, True, True), ShardSpec(1, 2, False, False), ShardSpec(2, 3, False, True)])
def test_device_bytes_equal_file(ckpt, staging, spec):
    d, cfg, w = ckpt
    print(f"shard load spec={spec} staging={staging}", flush=True)
    idx = WeightIndex(d)
    got = idx.load_shard(spec, framework="hip", staging_bytes=staging)
    assert set(got) == set(idx.owned(spec))
    for n, t in got.items():
        assert t.is_cuda and list(t.shape) == list(w[n].shape)
        assert device_bytes(t) == np.ascontiguousarray(w[n]).tobytes(), n


def test_bf16_and_empty_tensors(tmp_path):
    import torch
    d = str(tmp_path)
    bf = (np.arange(4096, dtype=np.uint32) * 2654435761 % 65536).astype(np.uint16)
    write_raw(os.path.join(d, "m.safetensors"),
              {"model.norm.weight": ("BF16", (4096,), bf.tobytes()), "lm_head.bias": ("F32", (0,), b""),
               "lm_head.weight": ("U32", (7, 3), np.arange(21, dtype=np.uint32).tobytes())})
    with open(os.path.join(d, "config.json"), "w") as f:
        import json
        json.dump(tiny_cfg(), f)
    got = WeightIndex(d).load_shard(ShardSpec(0, 0, False, True), framework="hip", staging_bytes=1 << 20)
    assert got["model.norm.weight"].dtype == torch.bfloat16
    assert device_bytes(got["model.norm.weight"]) == bf.tobytes()
    assert got["lm_head.bias"].numel() == 0
    assert device_bytes(got["lm_head.weight"]) == np.arange(21, dtype=np.uint32).tobytes()


def test_residency(ckpt):
    import torch
    d, cfg, w = ckpt
    idx = WeightIndex(d)
    res = Residency()
    a = idx.load_shard(ShardSpec(0, 1, True, False), framework="hip", residency=res)
    b = idx.load_shard(ShardSpec(1, 3, False, True), framework="hip", residency=res)
    assert res.nbytes() == idx.total_bytes()
    assert res.layer_bytes() == dict(enumerate(idx.layer_bytes()))
    with pytest.raises(KeyError):
        res.add(a)
    free, _ = torch.cuda.mem_get_info()
    with pytest.raises(MemoryError):
        Residency(headroom=free).reserve(1)            # refused before anything is read
    assert res.release("model.layers.1.") == idx.layer_bytes()[1]
    assert res.nbytes() == idx.total_bytes() - idx.layer_bytes()[1]
    assert "lm_head.weight" in res and res["lm_head.weight"] is b["lm_head.weight"]
    assert res.release() == idx.total_bytes() - idx.layer_bytes()[1] and res.nbytes() == 0


def test_stage_from_loaded_checkpoint_matches_numpy(tmp_path):
    import torch
    from hetero.gpu_model import GpuStage
    from test_gpu_decode import small_cfg
    cfg = small_cfg()
    w = qwen2.synthetic_weights(cfg, seed=21)
    kk, vv = qwen2.synthetic_context(cfg, 64, seed=22)
    write_checkpoint(str(tmp_path), cfg, w)
    dev_w = WeightIndex(str(tmp_path)).load_shard(ShardSpec(0, cfg["num_hidden_layers"], True, True),
                                                 framework="hip")
    stages = [GpuStage(cfg, ww, kk, vv, max_new=6) for ww in (w, dev_w)]
    tokens = []
    for g in stages:
        g.set_token(7)
        g.capture()
        seq, logits = [], []
        for _ in range(6):
            seq.append(g.step())
            logits.append(g.logits.cpu().numpy().copy())
        tokens.append((seq, logits))
    torch.cuda.synchronize()
    assert tokens[0][0] == tokens[1][0]
    for a, b in zip(tokens[0][1], tokens[1][1]):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
