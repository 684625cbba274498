"""Checkpoint index and ownership (hetero/shard.py here; the reference's
hetero/shard.py:17-159): header parsing and byte ranges against the
safetensors package's own reader, the ownership rule for every kind of
tensor, tied embeddings, byte accounting and the NumPy load."""
from __future__ import annotations

import json
import os
import struct

import numpy as np
import pytest

from hetero import qwen2
from hetero.shard import ShardSpec, WeightIndex, read_header


def tiny_cfg(tied=False, layers=3):
    cfg = qwen2.qwen2_7b_config(layers=layers)
    cfg.update(hidden_size=128, intermediate_size=256, num_attention_heads=2, num_key_value_heads=1,
               vocab_size=96, tie_word_embeddings=tied)
    return cfg


def write_checkpoint(d, cfg, w, split_at=1):
    """Two files as a sharded MLX snapshot lays them out: the embedding and
    the layers below split_at in the first, the rest in the second."""
    from safetensors.numpy import save_file
    first = {n: a for n, a in w.items()
             if n.startswith("model.embed_tokens") or (n.startswith("model.layers.") and int(n.split(".")[2]) < split_at)}
    rest = {n: a for n, a in w.items() if n not in first}
    save_file(first, os.path.join(d, "model-00001-of-00002.safetensors"), metadata={"format": "mlx"})
    save_file(rest, os.path.join(d, "model-00002-of-00002.safetensors"), metadata={"format": "mlx"})
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(cfg, f)


def write_raw(path, tensors, metadata=None):
    """A safetensors file by its format (8-byte LE header length, JSON
    header with data_offsets, data): lets a test store dtypes NumPy lacks."""
    head, blobs, off = {}, [], 0
    for name, (dt, shape, raw) in tensors.items():
        head[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    if metadata:
        head["__metadata__"] = metadata
    hb = json.dumps(head).encode()
    hb += b" " * (-len(hb) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb)) + hb + b"".join(blobs))


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = str(tmp_path_factory.mktemp("ckpt"))
    cfg = tiny_cfg()
    w = qwen2.synthetic_weights(cfg, seed=3)
    write_checkpoint(d, cfg, w)
    return d, cfg, w


def test_reader_matches_safetensors_package(ckpt):
    from safetensors import safe_open
    d, cfg, w = ckpt
    idx = WeightIndex(d)
    assert set(idx.names()) == set(w)
    for name in idx.names():
        path = idx.entries[name][0]
        with safe_open(path, framework="numpy") as f:
            ref = f.get_tensor(name)
        got = idx._numpy(name)
        assert got.dtype == ref.dtype and got.shape == ref.shape
        assert got.tobytes() == ref.tobytes() == np.ascontiguousarray(w[name]).tobytes()


def test_read_header_drops_metadata(ckpt):
    d, _, _ = ckpt
    h = read_header(os.path.join(d, "model-00001-of-00002.safetensors"))
    assert "__metadata__" not in h
    assert all({"dtype", "shape", "data_offsets"} <= set(v) for v in h.values())


def test_ownership(ckpt):
    d, cfg, w = ckpt
    idx = WeightIndex(d)
    first = ShardSpec(0, 1, True, False)
    mid = ShardSpec(1, 2, False, False)
    last = ShardSpec(2, 3, False, True)
    owned = {s: set(idx.owned(s)) for s in (first, mid, last)}
    assert owned[first] == {n for n in w if n.startswith("model.embed_tokens") or n.startswith("model.layers.0.")}
    assert owned[mid] == {n for n in w if n.startswith("model.layers.1.")}
    assert owned[last] == {n for n in w if n.startswith("model.layers.2.") or n.startswith("lm_head")
                           or n == "model.norm.weight"}
    assert set().union(*owned.values()) == set(w)          # a partition of the model
    assert not (owned[first] & owned[mid] or owned[mid] & owned[last] or owned[first] & owned[last])
    with pytest.raises(KeyError):
        idx.owns("model.rotary.inv_freq", first)
    # layer names split on their index, not a prefix: layer 10 is not layer 1
    assert not idx.owns("model.layers.10.mlp.up_proj.weight", ShardSpec(1, 2, False, False))
    assert ShardSpec.from_json(json.loads(json.dumps(first.to_json()))) == first and mid.n_layers == 1


def test_tied_head_owns_the_embedding(tmp_path):
    cfg = tiny_cfg(tied=True, layers=2)
    w = qwen2.synthetic_weights(cfg, seed=4)
    for k in [k for k in w if k.startswith("lm_head")]:
        del w[k]
    write_checkpoint(str(tmp_path), cfg, w)
    idx = WeightIndex(str(tmp_path))
    assert idx.tied
    head = ShardSpec(1, 2, False, True)
    assert {n for n in idx.owned(head) if n.startswith("model.embed_tokens")} == \
        {"model.embed_tokens.weight", "model.embed_tokens.scales", "model.embed_tokens.biases"}
    assert idx.head_bytes() == idx.embed_bytes() + idx.nbytes("model.norm.weight")


def test_byte_accounting(ckpt):
    d, cfg, w = ckpt
    idx = WeightIndex(d)
    assert all(idx.nbytes(n) == w[n].nbytes for n in w)
    lb = idx.layer_bytes()
    assert len(lb) == cfg["num_hidden_layers"]
    for i, b in enumerate(lb):
        assert b == sum(a.nbytes for n, a in w.items() if n.startswith(f"model.layers.{i}."))
    assert idx.embed_bytes() == sum(a.nbytes for n, a in w.items() if n.startswith("model.embed_tokens"))
    assert idx.total_bytes() == sum(a.nbytes for a in w.values()) == sum(lb) + idx.embed_bytes() + idx.head_bytes()
    assert idx.shard_bytes(ShardSpec(0, 3, True, True)) == idx.total_bytes()
    data = sum(os.path.getsize(os.path.join(d, f)) - 8 - struct.unpack("<Q", open(os.path.join(d, f), "rb").read(8))[0]
               for f in os.listdir(d) if f.endswith(".safetensors"))
    assert data == idx.total_bytes()


def test_numpy_load_is_the_owned_tensors(ckpt):
    d, _, w = ckpt
    idx = WeightIndex(d)
    spec = ShardSpec(1, 3, False, True)
    got = idx.load_shard(spec, framework="numpy")
    assert set(got) == set(idx.owned(spec))
    for n, a in got.items():
        assert a.dtype == w[n].dtype and np.array_equal(a, w[n])


def test_bf16_and_bad_files(tmp_path):
    d = str(tmp_path)
    raw = np.arange(12, dtype=np.uint16).tobytes()
    write_raw(os.path.join(d, "a.safetensors"),
              {"model.norm.weight": ("BF16", (12,), raw), "lm_head.weight": ("U32", (2, 3), bytes(24))},
              metadata={"format": "mlx"})
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(tiny_cfg(), f)
    idx = WeightIndex(d)
    assert idx.nbytes("model.norm.weight") == 24 and idx.entries["model.norm.weight"][1] == "BF16"
    with pytest.raises(TypeError):                  # NumPy has no bfloat16, as in the reference
        idx.load_shard(ShardSpec(0, 0, False, True), framework="numpy")
    assert idx.load_shard(ShardSpec(0, 0, False, False), framework="numpy") == {}
    write_raw(os.path.join(d, "a.safetensors"), {"lm_head.weight": ("U32", (2, 3), bytes(20))})
    with pytest.raises(ValueError):                 # offsets disagree with shape x dtype
        WeightIndex(d)
    with pytest.raises(FileNotFoundError):
        WeightIndex(os.path.join(d, "missing"))
    with pytest.raises(ValueError):
        idx.load_shard(ShardSpec(0, 0, False, True), framework="mlx")
