"""Build libq4gemv.so for gfx950 from csrc/ into kernel/ (in-tree).

The library sits where the reference's ctypes loader looks for its CPU
kernel (hetero/cpu_model.py:35-37: <package parent>/kernel/libq4gemv.so), so
hetero/cpu_model.py here loads it the same way.

csrc/q4gemv.hip (host code, C-ABI and the other kernels), csrc/q4_decode.hip
(the decode-step kernels of include/q4decode.h), csrc/q4_prompt.hip (the
prompt forward's causal attention, also include/q4decode.h), csrc/q4_chain.hip (the
chained GEMV programs of include/q4chain.h), csrc/q4_gemm.hip (the prefill
GEMM) and the instances of the
streaming GEMV kernel (csrc/q4_stream_inst.hip, once per activation rows x
gate/up pair x ring size) are compiled as separate objects in parallel, then
linked into one shared library.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
SRC = os.path.join(CSRC, "q4gemv.hip")
DECODE = os.path.join(CSRC, "q4_decode.hip")
PROMPT = os.path.join(CSRC, "q4_prompt.hip")
WIRE = os.path.join(CSRC, "q4_wire.hip")
CHAIN = os.path.join(CSRC, "q4_chain.hip")
GEMM = os.path.join(CSRC, "q4_gemm.hip")
INST = os.path.join(CSRC, "q4_stream_inst.hip")
OUT = os.path.join(HERE, "kernel", "libq4gemv.so")

HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument",
]

# (activation rows, gate/up pair, ring size, group size 64 << gsh) of the
# streaming kernel objects
STREAM_INSTANCES = [(mr, pair, ring, gsh) for gsh in (0, 1) for mr in (1, 2) for pair in (0, 1)
                    for ring in (1, 2)] + [(1, 0, 5, 0), (1, 0, 5, 1)]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found")


def _run(cmd, what, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed ({r.returncode}) building {what}")


def build(verbose: bool = False, jobs: int | None = None, out: str = OUT, defines=()) -> str:
    """Compile every object in parallel and link `out`; `defines` are extra
    -D flags for every object."""
    os.makedirs(os.path.dirname(out), exist_ok=True)
    cc = hipcc()
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
    jobs = jobs or min(16, os.cpu_count() or 4)
    with tempfile.TemporaryDirectory(prefix="q4build") as tmpd:
        units = [(SRC, os.path.join(tmpd, "q4gemv.o"), []), (DECODE, os.path.join(tmpd, "q4_decode.o"), []),
                 (PROMPT, os.path.join(tmpd, "q4_prompt.o"), []),
                 (WIRE, os.path.join(tmpd, "q4_wire.o"), []), (CHAIN, os.path.join(tmpd, "q4_chain.o"), []),
                 (GEMM, os.path.join(tmpd, "q4_gemm.o"), [])]
        for mr, pair, ring, gsh in STREAM_INSTANCES:
            obj = os.path.join(tmpd, f"stream_m{mr}_p{pair}_r{ring}_g{gsh}.o")
            units.append((INST, obj, [f"-DQ4_MR={mr}", f"-DQ4_PAIR={pair}", f"-DQ4_RING={ring}", f"-DQ4_GSH={gsh}"]))
        with ThreadPoolExecutor(max_workers=jobs) as ex:
            futs = [ex.submit(_run, [cc, *HIPCC_FLAGS, *inc, *defines, *defs, "-c", "-o", obj, src],
                              f"{os.path.basename(src)} {' '.join(defs)}", verbose)
                    for src, obj, defs in units]
            for f in futs:
                f.result()
        tmp = out + ".tmp"
        _run([cc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *[o for _, o, _ in units]],
             "link", verbose)
        os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
