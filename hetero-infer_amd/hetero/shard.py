"""Shard specification, selective weight loading and device residency.

The interface is the reference's hetero/shard.py: ShardSpec (:26-47), read_header
(:63-69), and WeightIndex (:72-159) with its ownership rule and byte accounting.  A
stage reads the safetensors headers (no tensor data), keeps the tensors it owns
and loads those alone.  What this module adds is a device target:

  * load_shard(spec, framework="hip") streams the owned tensors straight into
    HBM.  It reads their byte ranges from the files into two pinned staging
    buffers, several threads per buffer.  Each filled buffer is copied to the
    device asynchronously on a copy stream while the next range is read.  No
    host copy of the shard is ever whole, and the tensors come back as device
    tensors in the file's dtype.
  * Residency tracks what a device holds (name -> tensor, bytes per layer)
    and refuses a shard that does not fit in the free HBM, before reading
    anything.

Local model directories only: there is no download (the reference's
snapshot_dir falls back to huggingface_hub, hetero/shard.py:50-60).
framework="numpy" returns NumPy arrays as the reference's
load_shard(..., framework="numpy") does.  It is read through a memory map
here, not through the safetensors package.
"""
from __future__ import annotations

import json
import os
import struct
from dataclasses import asdict, dataclass
from typing import Dict, List, Optional, Tuple

import numpy as np

# hetero/shard.py:17-22
_DTYPE_BYTES = {
    "BOOL": 1, "U8": 1, "I8": 1, "F8_E4M3": 1, "F8_E5M2": 1,
    "U16": 2, "I16": 2, "F16": 2, "BF16": 2,
    "U32": 4, "I32": 4, "F32": 4,
    "U64": 8, "I64": 8, "F64": 8,
}
_NUMPY = {"BOOL": np.bool_, "U8": np.uint8, "I8": np.int8, "U16": np.uint16, "I16": np.int16,
          "F16": np.float16, "U32": np.uint32, "I32": np.int32, "F32": np.float32, "U64": np.uint64,
          "I64": np.int64, "F64": np.float64}


def _torch_dtype(torch, dt: str):
    return {"BOOL": torch.bool, "U8": torch.uint8, "I8": torch.int8, "U16": torch.uint16,
            "I16": torch.int16, "F16": torch.float16, "BF16": torch.bfloat16, "U32": torch.uint32,
            "I32": torch.int32, "F32": torch.float32, "U64": torch.uint64, "I64": torch.int64,
            "F64": torch.float64, "F8_E4M3": torch.float8_e4m3fn, "F8_E5M2": torch.float8_e5m2}[dt]


@dataclass(frozen=True)
class ShardSpec:
    """Layers [start, end) plus the embedding and/or the output norm + lm_head
    (hetero/shard.py:26-47)."""
    start: int
    end: int
    embed: bool
    head: bool

    @property
    def n_layers(self) -> int:
        return self.end - self.start

    def to_json(self) -> dict:
        return asdict(self)

    @staticmethod
    def from_json(d: dict) -> "ShardSpec":
        return ShardSpec(int(d["start"]), int(d["end"]), bool(d["embed"]), bool(d["head"]))


def _header(path: str) -> Tuple[Dict[str, dict], int]:
    """The header of a safetensors file and the offset its data starts at:
    8 bytes of little-endian header length, the JSON header, then the data
    (tensor offsets are relative to that)."""
    with open(path, "rb") as f:
        raw = f.read(8)
        if len(raw) != 8:
            raise ValueError(f"{path}: not a safetensors file")
        (n,) = struct.unpack("<Q", raw)
        head = json.loads(f.read(n))
    return head, 8 + n


def read_header(path: str) -> Dict[str, dict]:
    """hetero/shard.py:63-69: {name: {"dtype", "shape", "data_offsets"}}, no data read."""
    head, _ = _header(path)
    head.pop("__metadata__", None)
    return head


class WeightIndex:
    """name -> (file, dtype, shape, nbytes) across a model directory
    (hetero/shard.py:72-159), plus each tensor's absolute byte range."""

    def __init__(self, model_dir: str):
        if not os.path.isdir(model_dir):
            raise FileNotFoundError(f"{model_dir} is not a local model directory (no downloads here)")
        self.dir = model_dir
        files = sorted(os.path.join(model_dir, f) for f in os.listdir(model_dir) if f.endswith(".safetensors"))
        if not files:
            raise FileNotFoundError(f"no safetensors in {model_dir}")
        self.entries: Dict[str, Tuple[str, str, List[int], int]] = {}
        self.ranges: Dict[str, Tuple[int, int]] = {}
        for path in files:
            head, base = _header(path)
            head.pop("__metadata__", None)
            for name, meta in head.items():
                shape = [int(s) for s in meta["shape"]]
                nb = _DTYPE_BYTES[meta["dtype"]]
                for s in shape:
                    nb *= s
                b0, b1 = (int(o) for o in meta["data_offsets"])
                if b1 - b0 != nb:
                    raise ValueError(f"{path}: {name} spans {b1 - b0} bytes, its shape and dtype {nb}")
                self.entries[name] = (path, meta["dtype"], shape, nb)
                self.ranges[name] = (base + b0, base + b1)
        with open(os.path.join(model_dir, "config.json")) as f:
            self.config = json.load(f)

    @property
    def tied(self) -> bool:
        return bool(self.config.get("tie_word_embeddings", False))

    # ---- ownership and byte accounting (hetero/shard.py:96-134) ----
    # Every tensor falls in one class: a decoder layer's (by layer number),
    # the embedding table, or the head's (lm_head, final norm).  A stage owns
    # the layers of its range, the embedding when it is the first stage (or,
    # with tied weights, the head stage too), and the head's tensors when it
    # is the last.

    @staticmethod
    def _tensor_class(name: str) -> Tuple[str, int]:
        parts = name.split(".")
        if parts[:2] == ["model", "layers"]:
            return "layer", int(parts[2])
        if name.startswith("model.embed_tokens"):
            return "embed", -1
        if name.startswith("lm_head") or name == "model.norm.weight":
            return "head", -1
        raise KeyError(f"unclassified tensor {name}")

    def owns(self, name: str, spec: ShardSpec) -> bool:
        cls, layer = self._tensor_class(name)
        if cls == "layer":
            return layer in range(spec.start, spec.end)
        if cls == "embed":
            return spec.embed or (spec.head and self.tied)
        return spec.head

    def names(self) -> List[str]:
        return list(self.entries)

    def nbytes(self, name: str) -> int:
        return self.entries[name][3]

    def _class_bytes(self, cls: str) -> int:
        return sum(self.nbytes(n) for n in self.entries if self._tensor_class(n)[0] == cls)

    def layer_bytes(self) -> List[int]:
        per_layer = [0] * int(self.config["num_hidden_layers"])
        for n in self.entries:
            cls, layer = self._tensor_class(n)
            if cls == "layer":
                per_layer[layer] += self.nbytes(n)
        return per_layer

    def embed_bytes(self) -> int:
        return self._class_bytes("embed")

    def head_bytes(self) -> int:
        """The head stage's bytes; with tied weights it also holds the embedding."""
        return self._class_bytes("head") + (self._class_bytes("embed") if self.tied else 0)

    def total_bytes(self) -> int:
        return sum(self.nbytes(n) for n in self.entries)

    def shard_bytes(self, spec: ShardSpec) -> int:
        return sum(self.nbytes(n) for n in self.owned(spec))

    def owned(self, spec: ShardSpec) -> List[str]:
        return [n for n in self.entries if self.owns(n, spec)]

    # ---- loading ----

    def load_shard(self, spec: ShardSpec, framework: str = "numpy", device="cuda",
                   residency: Optional["Residency"] = None, staging_bytes: int = 64 << 20,
                   readers: int = 4):
        """Read only this stage's tensors (hetero/shard.py:131-159).

        framework="numpy": {name: ndarray} (BF16 has no NumPy dtype and
        raises, as in the reference).  framework="hip": {name: device tensor}
        in the file's dtype, streamed into HBM; recorded in `residency` if
        given (which first checks that the shard fits)."""
        names = self.owned(spec)
        if framework == "numpy":
            return {n: self._numpy(n) for n in names}
        if framework not in ("hip", "torch"):
            raise ValueError(f"unknown framework {framework}")
        if residency is not None:
            residency.reserve(sum(self.nbytes(n) for n in names))
        out = self._to_device(names, device, staging_bytes, readers)
        if residency is not None:
            residency.add(out)
        return out

    def _numpy(self, name: str) -> np.ndarray:
        path, dt, shape, nb = self.entries[name]
        if dt not in _NUMPY:
            raise TypeError(f"{name}: dtype {dt} has no NumPy equivalent")
        b0, _ = self.ranges[name]
        mm = np.memmap(path, dtype=np.uint8, mode="r", offset=b0, shape=(nb,)) if nb else np.zeros(0, np.uint8)
        return np.array(mm).view(_NUMPY[dt]).reshape(shape)

    def _to_device(self, names: List[str], device, staging_bytes: int, readers: int):
        import torch
        from concurrent.futures import ThreadPoolExecutor
        dev = torch.device(device)
        out = {}
        # one device buffer per tensor, in the file's dtype; reads go file by
        # file in offset order, neighbouring tensors merged into one span
        by_file: Dict[str, List[str]] = {}
        for n in names:
            by_file.setdefault(self.entries[n][0], []).append(n)
        spans = []                          # (path, file offset, [(device byte view, bytes)])
        for path, ns in sorted(by_file.items()):
            ns.sort(key=lambda n: self.ranges[n][0])
            cur = None
            for n in ns:
                _, dt, shape, nb = self.entries[n]
                t = torch.empty(shape, dtype=_torch_dtype(torch, dt), device=dev)
                out[n] = t
                if nb == 0:
                    continue
                dst = t.view(-1).view(torch.uint8) if t.dim() else t.reshape(1).view(torch.uint8)
                b0, b1 = self.ranges[n]
                if cur is not None and cur[1] + cur[2] == b0:
                    cur[3].append(dst)
                    cur[2] += nb
                else:
                    cur = [path, b0, nb, [dst]]
                    spans.append(cur)
        if not spans:
            return out
        chunk = max(1 << 20, min(staging_bytes, max(s[2] for s in spans)))
        stage = [torch.empty(chunk, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        views = [memoryview(s.numpy()) for s in stage]
        done = [None, None]
        copy_stream = torch.cuda.Stream(device=dev)
        pool = ThreadPoolExecutor(max(1, readers))
        k = 0

        def read(fd, mv, at):               # one reader's part of a chunk (preadv drops the GIL)
            got = 0
            while got < len(mv):
                r = os.preadv(fd, [mv[got:]], at + got)
                if r <= 0:
                    break
                got += r
            return got

        for path, off, total, dsts in spans:
            with open(path, "rb", buffering=0) as f:
                di, dpos = 0, 0             # destination tensor and the bytes of it written
                pos = 0
                while pos < total:
                    n = min(chunk, total - pos)
                    slot = k % 2
                    if done[slot] is not None:
                        done[slot].synchronize()          # the copy out of this buffer has finished
                    # the chunk in `readers` page-aligned parts, read in parallel
                    step = max(4096, -(-n // max(1, readers)) + 4095 & ~4095)
                    parts = [(a, min(n, a + step)) for a in range(0, n, step)]
                    got = sum(fu.result() for fu in [pool.submit(read, f.fileno(), views[slot][a:b], off + pos + a)
                                                     for a, b in parts])
                    if got != n:
                        pool.shutdown()
                        raise IOError(f"{path}: short read at {off + pos} ({got} of {n} bytes)")
                    with torch.cuda.stream(copy_stream):
                        s = 0
                        while s < n:                      # scatter the chunk over its tensors
                            d = dsts[di]
                            m = min(n - s, d.numel() - dpos)
                            d[dpos:dpos + m].copy_(stage[slot][s:s + m], non_blocking=True)
                            s += m
                            dpos += m
                            if dpos == d.numel():
                                di, dpos = di + 1, 0
                        ev = torch.cuda.Event()
                        ev.record(copy_stream)
                    done[slot] = ev
                    pos += n
                    k += 1
        pool.shutdown()
        copy_stream.synchronize()
        torch.cuda.current_stream(dev).wait_stream(copy_stream)
        return out


class Residency:
    """What one device holds: name -> tensor, with bytes in total, per
    decoder layer and for the embedding/head.  reserve() refuses a load that
    would not fit in the device's free HBM, less `headroom` bytes, before
    anything is read."""

    def __init__(self, device="cuda", headroom: int = 2 << 30):
        self.device = device
        self.headroom = headroom
        self.tensors: Dict[str, object] = {}

    def reserve(self, nbytes: int) -> None:
        import torch
        free, _ = torch.cuda.mem_get_info(torch.device(self.device))
        if nbytes + self.headroom > free:
            raise MemoryError(f"shard of {nbytes / 2**30:.2f} GiB does not fit: {free / 2**30:.2f} GiB free, "
                              f"{self.headroom / 2**30:.2f} GiB kept back")

    def add(self, tensors: Dict[str, object]) -> None:
        dup = set(tensors) & set(self.tensors)
        if dup:
            raise KeyError(f"already resident: {sorted(dup)[:4]}")
        self.tensors.update(tensors)

    def __getitem__(self, name: str):
        return self.tensors[name]

    def __contains__(self, name: str) -> bool:
        return name in self.tensors

    def get(self, name: str, default=None):
        return self.tensors.get(name, default)

    def keys(self):
        return self.tensors.keys()

    def nbytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.tensors.values())

    def layer_bytes(self) -> Dict[int, int]:
        out: Dict[int, int] = {}
        for n, t in self.tensors.items():
            if n.startswith("model.layers."):
                i = int(n.split(".")[2])
                out[i] = out.get(i, 0) + t.numel() * t.element_size()
        return out

    def release(self, prefix: str = "") -> int:
        """Drop the tensors whose names start with `prefix` (all by default);
        returns the bytes released."""
        gone = [n for n in self.tensors if n.startswith(prefix)]
        nb = sum(self.tensors[n].numel() * self.tensors[n].element_size() for n in gone)
        for n in gone:
            del self.tensors[n]
        return nb
