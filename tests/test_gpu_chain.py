"""GPU parity of chained GEMV programs (include/q4chain.h): phases run in one
persistent launch with a grid barrier between them.

Bar: every phase output bit-exact against the oracle on the inputs the
phase actually read (for gate/up: bit-identical to q4_gate_up_silu_dev, and
within 2e-6 of NumPy's float32 SiLU of the oracle's gate and up, whose exp
may differ in the last place); outputs of separate launches of the same
projections bit-identical; no barrier wait ever runs out of time; graph
replays equal to the eager run.
"""
import numpy as np
import pytest

from hetero import q4, synth
import oracle

pytestmark = pytest.mark.gpu


def dev(*arrays):
    import torch
    return [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in arrays]


def mat(seed, n_out, n_in):
    w, s, b = synth.qlinear(seed, n_out, n_in, 64)
    return (w, s, b), tuple(dev(w, s.view(np.int16), b.view(np.int16)))


def silu_np(g):
    with np.errstate(over="ignore"):          # exp(-g) of a large negative g is inf: SiLU(g) = -0.0
        return g / (np.float32(1.0) + np.exp(-g, dtype=np.float32))


def bits(t):
    return t.cpu().numpy().view(np.uint32)


def test_dependent_qwen_layers_bit_exact():
    """Two Qwen2.5-7B layers of projections, each phase reading the output of
    the one before: q/k/v -> o -> gate/up -> down -> next layer."""
    import torch
    H, I = 3584, 18944
    o = oracle.Oracle()
    x0 = synth.activations(1000, 1, H)
    tx0 = dev(x0)[0]
    layers, phases, bufs = [], [], []
    x = tx0
    for l in range(2):
        m = [mat(1010 + 10 * l + i, n, k) for i, (n, k) in
             enumerate(((H, H), (512, H), (512, H), (H, H), (I, H), (I, H), (H, I)))]
        layers.append(m)
        q_, k_, v_, o_, h_, d_ = (torch.empty((1, n), device="cuda") for n in (H, 512, 512, H, I, H))
        phases += [([m[0][1], m[1][1], m[2][1]], x, [q_, k_, v_], False), ([m[3][1]], q_, [o_], False),
                   ([m[4][1], m[5][1]], o_, [h_], True), ([m[6][1]], h_, [d_], False)]
        bufs.append((q_, k_, v_, o_, h_, d_))
        x = d_
    ch = q4.Chain(phases)
    ch.run()
    torch.cuda.synchronize()
    assert ch.errors() == 0
    xin = x0
    for l, (m, (q_, k_, v_, o_, h_, d_)) in enumerate(zip(layers, bufs)):
        print(f"layer {l}", flush=True)
        for (wsb, _), got in zip(m[:3], (q_, k_, v_)):
            assert np.array_equal(bits(got)[0], o.gemv(*wsb, xin[0], 64).view(np.uint32))
        q_in = q_.cpu().numpy()
        assert np.array_equal(bits(o_)[0], o.gemv(*m[3][0], q_in[0], 64).view(np.uint32))
        o_in = o_.cpu().numpy()
        g, u = o.gemv(*m[4][0], o_in[0], 64), o.gemv(*m[5][0], o_in[0], 64)
        h = h_.cpu().numpy()[0]
        assert oracle.normwise_rel(h, silu_np(g) * u) < 2e-6
        sep = q4.gate_up_silu_dev(m[4][1], m[5][1], o_)
        torch.cuda.synchronize()
        assert np.array_equal(h.view(np.uint32), bits(sep)[0])
        assert np.array_equal(bits(d_)[0], o.gemv(*m[6][0], h, 64).view(np.uint32))
        xin = d_.cpu().numpy()
    ch.close()


@pytest.mark.parametrize("n_in,counts,pair", [
    (512, (8,), False),                 # one chunk: ring 1
    (832, (300, 40), False),            # 13 groups, partial chunk, two matrices
    (3584, (96, 64, 8, 40), False),     # four matrices of uneven rows: ring 2
    (6144, (200,), False),              # three chunks: ring 1
    (18944, (3584,), False),            # ten chunks: ring 2
    (9216, (1000,), False),             # five chunks: ring 5
    (24576, (64,), False),              # the longest row: twelve chunks
    (3584, (152064,), False),           # lm_head: eight rows per unit, ring 2
    (2048, (1000, 1000), True),         # gate/up, one chunk: ring 2
    (3584, (18944, 18944), True),       # gate/up, Qwen shape: two rows per unit, ring 2
    (320, (48, 48), True),              # gate/up, five groups
])
def test_phase_shapes_vs_separate_launches(n_in, counts, pair):
    """One phase shape per ring size and row layout, run three times in one
    chain (a dependency-free program, so the barrier is exercised with
    identical phases), each bit-identical to the separate launch and, for
    plain phases, to the oracle."""
    import torch
    o = oracle.Oracle()
    mats = [mat(1100 + n_in + i + n, n, n_in) for i, n in enumerate(counts)]
    x = synth.activations(1101 + n_in, 1, n_in)
    tx = dev(x)[0]
    n_outs = counts[:1] if pair else counts
    outs = [[torch.full((1, n), float("nan"), device="cuda") for n in n_outs] for _ in range(3)]
    ch = q4.Chain([([m[1] for m in mats], tx, outs[r], pair) for r in range(3)])
    ch.run()
    torch.cuda.synchronize()
    assert ch.errors() == 0
    if pair:
        want = [q4.gate_up_silu_dev(mats[0][1], mats[1][1], tx)]
    else:
        want = q4.gemv_multi_dev([m[1] for m in mats], tx)
    torch.cuda.synchronize()
    for r in range(3):
        for k, (got, ref) in enumerate(zip(outs[r], want)):
            assert np.array_equal(bits(got), bits(ref)), f"repeat {r} matrix {k}"
    if not pair:
        for (wsb, _), got in zip(mats, outs[0]):
            assert np.array_equal(bits(got)[0], o.gemv(*wsb, x[0], 64).view(np.uint32))
    ch.close()


def test_mixed_dependencies_vs_launches_in_order():
    """A program whose barriers order different things: x from outside the
    program (loaded before the barrier), x written by the phase just before
    (after it), x written two phases back (before the barrier, so the
    writer's stores complete one barrier earlier), and an output buffer
    written again by a later phase.  Every buffer ends bit-identical to the
    same phases run as separate launches in order, on two runs."""
    import torch
    from hetero import sweep
    n = 1024
    mats = [mat(1300 + i, n, n)[1] for i in range(7)]
    x1, x2 = dev(synth.activations(1301, 1, n), synth.activations(1302, 1, n))

    def program():
        a, b, c, d, e, f = (torch.full((1, n), float("nan"), device="cuda") for _ in range(6))
        ph = [([mats[0]], x1, [a], False),      # outside x
              ([mats[1]], x2, [b], False),      # outside x, no dependency on the phase before
              ([mats[2]], a, [c], False),       # x from two phases back
              ([mats[3]], c, [d], False),       # x from the phase before
              ([mats[4]], x1, [a], False),      # writes a again
              ([mats[5]], a, [e], False),       # reads the new a
              ([mats[6], mats[0]], d, [f, b], False)]   # x from three back; writes b again
        return ph, (a, b, c, d, e, f)

    ph, bufs = program()
    ch = q4.Chain(ph)
    ref_ph, ref = program()
    sweep.run_launches(ref_ph, torch.cuda.current_stream())
    for r in range(2):
        for t in bufs:
            t.fill_(float("nan"))
        ch.run()
        torch.cuda.synchronize()
        assert ch.errors() == 0
        for i, (got, want) in enumerate(zip(bufs, ref)):
            assert np.array_equal(bits(got), bits(want)), f"run {r} buffer {'abcdef'[i]}"
    ch.close()


def test_graph_replays_and_barrier_reset():
    """A chain captured in a HIP graph: replays with eager work between them
    equal the eager run (the barrier state returns to zero after every
    launch), and the plan runs again eagerly afterwards."""
    import torch
    H = 3584
    mats = [mat(1200 + i, H, H) for i in range(4)]
    x = dev(synth.activations(1201, 1, H))[0]
    bufs = [torch.empty((1, H), device="cuda") for _ in range(4)]
    phases, xin = [], x
    for m, b in zip(mats, bufs):
        phases.append(([m[1]], xin, [b], False))
        xin = b
    ch = q4.Chain(phases)
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        ch.run(st)
    torch.cuda.synchronize()
    want = [bits(b) for b in bufs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        ch.run(st)
    for rep in range(3):
        for b in bufs:
            b.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert all(np.array_equal(bits(b), w) for b, w in zip(bufs, want)), f"replay {rep}"
        y = q4.gemv_dev(*mats[0][1], x)          # eager work between replays
        torch.cuda.synchronize()
        assert np.array_equal(bits(y), want[0])
    ch.run()
    torch.cuda.synchronize()
    assert all(np.array_equal(bits(b), w) for b, w in zip(bufs, want))
    assert ch.errors() == 0
    ch.close()


def test_headline_sweep_at_full_size():
    """The benchmark's headline program at the size it is timed: the 113
    phases of the Qwen2.5-7B sweep (28 layers of distinct weights generated
    on the GPU, q/k/v, o, gate+up and down each, plus lm_head's 152,064
    rows at eight rows per unit) in one chained launch, twice.  Every
    phase's outputs are bit-identical to the same phase run as its own
    launch; layers 0 and 27 and lm_head are bit-exact against the oracle."""
    import torch
    from hetero import sweep
    dev = torch.device("cuda:0")
    layers, head, xs = sweep.make_model(torch, dev, seed=1234)
    phases = sweep.phases(layers, head, xs, sweep.distinct_outputs(torch, dev))
    assert len(phases) == 113
    ch = q4.Chain(phases)
    ch.run()
    torch.cuda.synchronize()
    assert ch.errors() == 0
    first = [[t.clone() for t in ph[2]] for ph in phases]
    for ph in phases:
        for t in ph[2]:
            t.fill_(float("nan"))
    ch.run()
    torch.cuda.synchronize()
    assert ch.errors() == 0
    ch.close()
    for p, ph in enumerate(phases):
        for k, t in enumerate(ph[2]):
            assert torch.equal(t.view(torch.int32), first[p][k].view(torch.int32)), f"run 2, phase {p} matrix {k}"
    check = sweep.phases(layers, head, xs, sweep.distinct_outputs(torch, dev))
    sweep.run_launches(check, torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert sweep.mismatches(torch, phases, check) == []
    o = oracle.Oracle()
    xh = {n: t.cpu().numpy()[0] for n, t in xs.items()}

    def host(wsb):
        w, sc, b = (t.cpu().numpy() for t in wsb)
        return w.view(np.uint32), sc.view(np.float16), b.view(np.float16)

    for l in (0, 27):
        for j, idx in enumerate(sweep.LAYER_PHASES):
            ph = phases[4 * l + j]
            for k, i in enumerate(idx):
                _, n_in, n_out = sweep.LAYER_SHAPES[i]
                print(f"layer {l} {sweep.LAYER_SHAPES[i][0]}", flush=True)
                want = o.gemv(*host(layers[l][i]), xh[n_in], 64)
                assert np.array_equal(bits(ph[2][k])[0], want.view(np.uint32)), f"layer {l} projection {i}"
    print("lm_head", flush=True)
    want = o.gemv(*host(head), xh[3584], 64)
    assert np.array_equal(bits(phases[-1][2][0])[0], want.view(np.uint32))


def test_inputs_change_between_runs():
    """A program whose every x comes from outside it (each prepared once at
    the program's start and read through the L2s) run again after x has
    changed: eagerly, and as graph replays with x rewritten in between.
    Every run's outputs are bit-identical to separate launches on that run's
    x: nothing of an earlier run's x survives in any cache."""
    import torch
    from hetero import sweep
    H, I = 3584, 18944
    m = [mat(1400 + i, n, k)[1] for i, (n, k) in enumerate(((H, H), (512, H), (I, H), (I, H), (H, I)))]
    xh, xi = (torch.empty((1, k), device="cuda") for k in (H, I))

    def program():
        a, b, c, d = (torch.full((1, n), float("nan"), device="cuda") for n in (H, 512, I, H))
        return [([m[0], m[1]], xh, [a, b], False), ([m[2], m[3]], xh, [c], True), ([m[4]], xi, [d], False)], \
            (a, b, c, d)

    ph, bufs = program()
    ch = q4.Chain(ph)
    st = torch.cuda.Stream()

    def check(tag):
        ref_ph, ref = program()
        q4.gate_up_silu_dev(m[2], m[3], xh, h=ref[2])
        sweep.run_launches([ref_ph[0], ref_ph[2]], torch.cuda.current_stream())
        torch.cuda.synchronize()
        assert ch.errors() == 0
        for i, (got, want) in enumerate(zip(bufs, ref)):
            assert np.array_equal(bits(got), bits(want)), f"{tag} buffer {i}"

    for r in range(3):
        xh.copy_(torch.from_numpy(synth.activations(1410 + r, 1, H)))
        xi.copy_(torch.from_numpy(synth.activations(1420 + r, 1, I)))
        with torch.cuda.stream(st):
            ch.run(st)
        torch.cuda.synchronize()
        check(f"eager run {r}")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        ch.run(st)
    for r in range(3):
        xh.copy_(torch.from_numpy(synth.activations(1430 + r, 1, H)))
        xi.copy_(torch.from_numpy(synth.activations(1440 + r, 1, I)))
        for t in bufs:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        check(f"replay {r}")
    ch.close()


@pytest.mark.parametrize("n_in,n_out,phases", [(64, 300, 1), (24576, 700, 1), (24576, 700, 2), (64, 40, 3)])
def test_prepared_x_edges(n_in, n_out, phases):
    """Programs of one to three phases whose x is prepared at the program's
    start, at the smallest and largest n_in (one group; 12 chunks of planes,
    the most a prepared x holds): with one phase the preparation stage's
    barrier is the program's only one.  Every phase bit-exact against the
    oracle and bit-identical to its own launch, on two runs."""
    import torch
    o = oracle.Oracle()
    mats = [mat(1500 + n_in % 97 + p, n_out, n_in) for p in range(phases)]
    x = synth.activations(1501 + n_in % 89, 1, n_in)
    tx = dev(x)[0]
    outs = [torch.full((1, n_out), float("nan"), device="cuda") for _ in range(phases)]
    ch = q4.Chain([([m[1]], tx, [outs[p]], False) for p, m in enumerate(mats)])
    for r in range(2):
        for t in outs:
            t.fill_(float("nan"))
        ch.run()
        torch.cuda.synchronize()
        assert ch.errors() == 0
        for p, (m, got) in enumerate(zip(mats, outs)):
            assert np.array_equal(bits(got)[0], o.gemv(*m[0], x[0], 64).view(np.uint32)), f"run {r} phase {p}"
            assert np.array_equal(bits(got), bits(q4.gemv_dev(*m[1], tx))), f"run {r} phase {p} vs launch"
    ch.close()


def test_stamps_leave_outputs_unchanged():
    """Event stamps on (q4_chain_stamps) in a program with prepared x, an x
    from the phase before and an x from two phases back: outputs
    bit-identical to the run without stamps, and every workgroup's events
    of a phase in order (arrival before release, x staged before planes
    ready, planes before wave 0 is done)."""
    import torch
    n = 3584
    mats = [mat(1600 + i, n, n)[1] for i in range(4)]
    x = dev(synth.activations(1601, 1, n))[0]
    a, b, c, d = (torch.empty((1, n), device="cuda") for _ in range(4))
    ch = q4.Chain([([mats[0]], x, [a], False), ([mats[1]], a, [b], False),
                   ([mats[2]], x, [c], False), ([mats[3]], b, [d], False)])
    ch.run()
    torch.cuda.synchronize()
    want = [bits(t) for t in (a, b, c, d)]
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    buf = torch.zeros(5 * cus * 8, dtype=torch.int64, device="cuda")
    ch.stamps(buf)
    for t in (a, b, c, d):
        t.fill_(float("nan"))
    ch.run()
    torch.cuda.synchronize()
    ch.stamps(None)
    assert ch.errors() == 0
    assert all(np.array_equal(bits(t), w) for t, w in zip((a, b, c, d), want))
    ev = buf.cpu().numpy().reshape(5, cus, 8)
    for p in range(1, 4):
        arrived, released, staged, planes, done = (ev[p, :, e] for e in range(1, 6))
        assert (released.min() >= arrived.max() - 1), f"phase {p}: released before the last arrival"
        assert (staged <= planes).all() and (planes <= done).all(), f"phase {p}: events out of order"
    ch.close()
