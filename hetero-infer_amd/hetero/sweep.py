"""The Qwen2.5-7B int4 projection sweep at one activation row.

28 decoder layers of seven projections (q, k, v, o 3584 -> 3584/512/512/3584,
gate/up 3584 -> 18944, down 18944 -> 3584) plus lm_head 3584 -> 152064, group
size 64, every layer with its own weights: 3,987,750,912 algorithmic bytes
(packed weights, fp16 scales and biases, fp32 x and y of every projection).
In decode order the projections that share an input run together, so a
sweep is 4 phases per layer (q/k/v, o, gate+up, down) and lm_head: 113
phases.  This module holds that definition for the benchmark and the tests:
the weights (generated on the device), the phase list, and the two ways of
running it -- one launch per phase, or one chained program
(include/q4chain.h).

The shapes are those of the reference's model config (Qwen2.5-7B: hidden
3584, intermediate 18944, 28 heads of 128 with 4 KV heads, vocab 152064), the
projections its stage calls q4_gemv for (hetero/cpu_model.py:269-275,
:291-292, :367).
"""
from __future__ import annotations

import ctypes

from . import q4

LAYERS = 28
GS = 64
HIDDEN, INTER, VOCAB = 3584, 18944, 152064
# (name, n_in, n_out)
LAYER_SHAPES = [("q_proj", HIDDEN, HIDDEN), ("k_proj", HIDDEN, 512), ("v_proj", HIDDEN, 512),
                ("o_proj", HIDDEN, HIDDEN), ("gate_proj", HIDDEN, INTER), ("up_proj", HIDDEN, INTER),
                ("down_proj", INTER, HIDDEN)]
HEAD_SHAPE = ("lm_head", HIDDEN, VOCAB)
# the phases of a layer: indices into LAYER_SHAPES that share x
LAYER_PHASES = [(0, 1, 2), (3,), (4, 5), (6,)]


def gemv_bytes(m, n_out, n_in, gs=GS):
    """Algorithmic bytes of one GEMV call: packed W, fp16 scales and biases,
    fp32 x and y."""
    return n_out * n_in // 2 + 4 * n_out * (n_in // gs) + 4 * m * n_in + 4 * m * n_out


def sweep_bytes(layers=LAYERS):
    return layers * sum(gemv_bytes(1, n_out, n_in) for _, n_in, n_out in LAYER_SHAPES) \
        + gemv_bytes(1, HEAD_SHAPE[2], HEAD_SHAPE[1])


def make_weights(torch, gen, n_out, n_in, dev, gs=GS):
    """One projection's (w int32 [n_out][n_in/8], scales, biases as int16
    bit patterns [n_out][n_in/gs]) on `dev`: uniform 4-bit values, scales
    |N(0, 0.02)|, biases -8 scale + N(0, 0.002), from `gen`."""
    w = torch.randint(-2**31, 2**31, (n_out, n_in // 8), dtype=torch.int64, device=dev,
                      generator=gen).to(torch.int32)
    g = n_in // gs
    s = (torch.randn((n_out, g), device=dev, generator=gen) * 0.02).abs().half()
    b = (-8.0 * s.float() + torch.randn((n_out, g), device=dev, generator=gen) * 0.002).half()
    return w, s.view(torch.int16), b.view(torch.int16)


def make_model(torch, dev, seed=1234, layers=LAYERS):
    """(layers, head, xs): `layers` lists of the seven projections' weights,
    the lm_head weights and the two inputs x[1][3584], x[1][18944]."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    lw = [[make_weights(torch, gen, n_out, n_in, dev) for _, n_in, n_out in LAYER_SHAPES] for _ in range(layers)]
    head = make_weights(torch, gen, HEAD_SHAPE[2], HEAD_SHAPE[1], dev)
    xs = {k: torch.randn((1, k), device=dev, generator=gen) for k in (HIDDEN, INTER)}
    return lw, head, xs


def phases(layers, head, xs, outs):
    """The sweep as (mats, x, outs, pair) phases (q4.Chain's form), in decode
    order.  outs(p, n_outs) gives phase p's output tensors."""
    out, p = [], 0
    for layer in layers:
        for idx in LAYER_PHASES:
            mats = [layer[i] for i in idx]
            n_in = LAYER_SHAPES[idx[0]][1]
            out.append((mats, xs[n_in], outs(p, [LAYER_SHAPES[i][2] for i in idx]), False))
            p += 1
    out.append(([head], xs[HIDDEN], outs(p, [HEAD_SHAPE[2]]), False))
    return out


def distinct_outputs(torch, dev, fill=float("nan")):
    """outs() for phases(): every phase its own output tensors."""
    return lambda p, n_outs: [torch.full((1, n), fill, device=dev) for n in n_outs]


def run_launches(phase_list, stream, lib=None):
    """Every phase as one grouped launch (q4_gemv_multi_dev) on `stream`."""
    lib = lib or q4.load()
    sp = stream.cuda_stream
    for mats, x, outs, pair in phase_list:
        assert not pair
        k = len(mats)
        n_in = mats[0][0].shape[1] * 8
        arr = lambda vals: (ctypes.c_void_p * k)(*vals)
        rc = lib.q4_gemv_multi_dev(k, arr([m[0].data_ptr() for m in mats]), arr([m[1].data_ptr() for m in mats]),
                                   arr([m[2].data_ptr() for m in mats]), arr([o.data_ptr() for o in outs]),
                                   (ctypes.c_int * k)(*[m[0].shape[0] for m in mats]), x.data_ptr(), 1, n_in,
                                   n_in // mats[0][1].shape[1], sp)
        q4.check(lib, rc, "q4_gemv_multi_dev")


def mismatches(torch, a_list, b_list):
    """Phases whose outputs differ in any bit: [(phase, matrix, differing values)]."""
    bad = []
    for p, (pa, pb) in enumerate(zip(a_list, b_list)):
        for k, (ta, tb) in enumerate(zip(pa[2], pb[2])):
            n = int((ta.view(torch.int32) != tb.view(torch.int32)).sum().item())
            if n:
                bad.append((p, k, n))
    return bad
