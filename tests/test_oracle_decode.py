"""Pins of the decode-step oracle (oracle/decode.py) and the NumPy stage of
the product (hetero/numpy_stage.py), on the CPU.

* The oracle against a float64 decode written from the textbook
  definitions here -- dequantised weights, explicit per-head loops over the
  grouped KV heads, rotation angles in float64, softmax by definition, the
  new key and value rounded to the cache's fp16 -- within the tolerance the
  int16 quantisation of x in every GEMV leaves (1e-3, max |diff| / max |ref|).
  Planted mistakes in the oracle (KV head mapping, rotation sign, a dropped
  residual) must fail the same comparison.
* The oracle's prompt path (L > 1 rows, causal attention, the q4_dequant +
  BLAS contraction above 16 rows) against the same float64 decode: in
  exact arithmetic a causal prompt's last row has the logits of decoding
  its tokens one by one.  Planted mistakes (a causal mask shifted by one
  position, RoPE at offset 0 instead of the cache position, the chunk's
  keys written one position late) must fail it.
* The product's NumPy stage on the reference kernel compiled from source
  against the oracle on the same kernel: logits bit-identical step for step.
* The generators the fixtures and the GPU tests share: NumPy and torch
  draws bit-identical.
"""
import os

import numpy as np
import pytest

import oracle
from oracle import decode as odec
from hetero import numpy_stage, qwen2, synth

TOL = 1e-3

needs_ref = pytest.mark.skipif(not os.path.exists(oracle.ref_path(1)), reason="oracle/_ref not built")


def tiny_cfg(layers=2):
    cfg = qwen2.qwen2_7b_config(layers)
    cfg.update(hidden_size=256, intermediate_size=512, num_attention_heads=8, num_key_value_heads=2,
               vocab_size=300)
    return cfg


@pytest.fixture(scope="module")
def tiny():
    cfg = tiny_cfg()
    w = qwen2.synthetic_weights(cfg, seed=31)
    ks, vs = qwen2.synthetic_context(cfg, 37, seed=32)
    return cfg, w, ks, vs


def textbook_decode(cfg, w, ks, vs, tokens):
    """float64 logits of each step consuming tokens[i] at position S0 + i."""
    gs = cfg["quantization"]["group_size"]
    H, nh, nkv = cfg["hidden_size"], cfg["num_attention_heads"], cfg["num_key_value_heads"]
    d, eps, theta = H // nh, cfg["rms_norm_eps"], cfg["rope_theta"]
    W = lambda n: oracle.dequant_np(w[f"{n}.weight"], w[f"{n}.scales"], w[f"{n}.biases"], gs).astype(np.float64)
    f64 = lambda n: np.asarray(w[n], np.float64)
    K = [k.astype(np.float64) for k in ks]
    V = [v.astype(np.float64) for v in vs]
    s0 = ks[0].shape[1]
    E = W("model.embed_tokens")
    half = d // 2
    freq = theta ** (-2.0 * np.arange(half) / d)

    def norm(x, g):
        return x / np.sqrt(np.mean(x * x) + eps) * g

    def rot(x, pos):
        a, b = x[:half], x[half:]
        c, s = np.cos(pos * freq), np.sin(pos * freq)
        return np.concatenate([a * c - b * s, a * s + b * c])

    out = []
    for t, tok in enumerate(tokens):
        pos = s0 + t
        x = E[tok].copy()
        for i in range(cfg["num_hidden_layers"]):
            p = f"model.layers.{i}"
            h = norm(x, f64(f"{p}.input_layernorm.weight"))
            q = W(f"{p}.self_attn.q_proj") @ h + f64(f"{p}.self_attn.q_proj.bias")
            k = W(f"{p}.self_attn.k_proj") @ h + f64(f"{p}.self_attn.k_proj.bias")
            v = W(f"{p}.self_attn.v_proj") @ h + f64(f"{p}.self_attn.v_proj.bias")
            kn = np.stack([rot(k[j * d:(j + 1) * d], pos) for j in range(nkv)])
            vn = v.reshape(nkv, d)
            # the cache stores fp16
            K[i] = np.concatenate([K[i], kn.astype(np.float16).astype(np.float64)[:, None]], axis=1)
            V[i] = np.concatenate([V[i], vn.astype(np.float16).astype(np.float64)[:, None]], axis=1)
            att = np.zeros(H)
            for hh in range(nh):
                kv = hh // (nh // nkv)
                qh = rot(q[hh * d:(hh + 1) * d], pos)
                sc = K[i][kv] @ qh / np.sqrt(d)
                pr = np.exp(sc - sc.max())
                pr /= pr.sum()
                att[hh * d:(hh + 1) * d] = pr @ V[i][kv]
            x = x + W(f"{p}.self_attn.o_proj") @ att
            h = norm(x, f64(f"{p}.post_attention_layernorm.weight"))
            g, u = W(f"{p}.mlp.gate_proj") @ h, W(f"{p}.mlp.up_proj") @ h
            x = x + W(f"{p}.mlp.down_proj") @ (g / (1 + np.exp(-g)) * u)
        out.append(W("lm_head") @ norm(x, f64("model.norm.weight")))
    return out


def run_oracle(cfg, w, ks, vs, tokens, lib):
    orc = odec.DecodeOracle(cfg, w, ks, vs, lib, extra=len(tokens))
    return [orc.logits(t) for t in tokens]


TOKENS = [5, 299, 0, 77]


@needs_ref
def test_oracle_matches_textbook_decode(tiny):
    cfg, w, ks, vs = tiny
    got = run_oracle(cfg, w, ks, vs, TOKENS, oracle.load_ref(1))
    want = textbook_decode(cfg, w, ks, vs, TOKENS)
    for i, (a, b) in enumerate(zip(got, want)):
        assert oracle.normwise_rel(a, b) < TOL, i


def _planted(monkeypatch, which):
    if which == "kv head mapping":
        def sdpa(q, k, v, scale):
            B, H, L, D = q.shape
            rep = np.tile(np.arange(k.shape[1]), H // k.shape[1])      # h % KH instead of h // G
            kk, vv = k[:, rep].astype(np.float32), v[:, rep].astype(np.float32)
            s = np.einsum("bhld,bhsd->bhls", q, kk) * scale
            e = np.exp(s - s.max(-1, keepdims=True))
            e /= e.sum(-1, keepdims=True)
            return np.einsum("bhls,bhsd->bhld", e, vv)
        monkeypatch.setattr(odec, "_sdpa", sdpa)
    elif which == "rotation sign":
        orig = odec._rope
        monkeypatch.setattr(odec, "_rope", lambda x, c, s: orig(x, c, -s))
    elif which == "dropped mlp residual":
        orig = odec.DecodeOracle.project

        def project(self, name, x):
            y = orig(self, name, x)
            return np.zeros_like(y) if name.endswith("down_proj") else y
        monkeypatch.setattr(odec.DecodeOracle, "project", project)


@needs_ref
@pytest.mark.parametrize("which", ["kv head mapping", "rotation sign", "dropped mlp residual"])
def test_textbook_comparison_catches_planted_mistakes(tiny, monkeypatch, which):
    cfg, w, ks, vs = tiny
    want = textbook_decode(cfg, w, ks, vs, TOKENS)
    _planted(monkeypatch, which)
    got = run_oracle(cfg, w, ks, vs, TOKENS, oracle.load_ref(1))
    assert max(oracle.normwise_rel(a, b) for a, b in zip(got, want)) > 10 * TOL, which


PROMPT = [7, 3, 250, 41, 0, 299, 12, 12, 5, 88, 140, 2, 61, 33, 9, 170, 203, 4, 77, 150]   # 20 tokens


@needs_ref
@pytest.mark.parametrize("chunks", [(5,), (20,), (12, 8), (17, 3)], ids=lambda c: "+".join(map(str, c)))
def test_oracle_prompt_matches_textbook(tiny, chunks):
    """Prompt chunks of <= 16 rows take the per-row GEMV, longer ones the
    q4_dequant + BLAS contraction; either way the last row's logits are the
    textbook decode's of the same tokens."""
    cfg, w, ks, vs = tiny
    n = sum(chunks)
    want = textbook_decode(cfg, w, ks, vs, PROMPT[:n])[-1]
    orc = odec.DecodeOracle(cfg, w, ks, vs, oracle.load_ref(1), extra=n)
    lo = 0
    for c in chunks:
        got = orc.prompt(PROMPT[lo:lo + c])
        lo += c
    assert orc.pos == ks[0].shape[1] + n
    assert oracle.normwise_rel(got, want) < TOL


def _planted_prompt(monkeypatch, which):
    if which == "causal mask shifted":
        orig = odec._sdpa

        def sdpa(q, k, v, scale, causal=False):
            if not causal:
                return orig(q, k, v, scale)
            # every row also sees the next position
            B, H, L, D = q.shape
            KH, S = k.shape[1], k.shape[2]
            s = np.einsum("bkgld,bksd->bkgls", q.reshape(B, KH, H // KH, L, D), k) * scale
            s = np.where(np.arange(S)[None, :] <= np.arange(L)[:, None] + (S - L) + 1, s, -np.inf)
            e = np.exp(s - s.max(-1, keepdims=True))
            e /= e.sum(-1, keepdims=True)
            return np.einsum("bkgls,bksd->bkgld", e, v).reshape(B, H, L, D)
        monkeypatch.setattr(odec, "_sdpa", sdpa)
    elif which == "rope at offset 0":
        orig = odec.DecodeOracle.prompt

        def prompt(self, ids):
            c, s_ = self.cos, self.sin
            self.cos, self.sin = np.roll(c, self.pos, axis=0), np.roll(s_, self.pos, axis=0)
            try:
                return orig(self, ids)
            finally:
                self.cos, self.sin = c, s_
        monkeypatch.setattr(odec.DecodeOracle, "prompt", prompt)
    elif which == "keys one position late":
        orig = odec._rope
        state = {"n": 0}

        def rope(x, cos, sin):
            y = orig(x, cos, sin)
            state["n"] += 1
            if state["n"] % 2 == 0 and x.shape[2] > 1:             # the keys: shift by one position
                y = np.concatenate([np.zeros_like(y[:, :, :1]), y[:, :, :-1]], axis=2)
            return y
        monkeypatch.setattr(odec, "_rope", rope)


@needs_ref
@pytest.mark.parametrize("which", ["causal mask shifted", "rope at offset 0", "keys one position late"])
def test_prompt_comparison_catches_planted_mistakes(tiny, monkeypatch, which):
    cfg, w, ks, vs = tiny
    want = textbook_decode(cfg, w, ks, vs, PROMPT)[-1]
    _planted_prompt(monkeypatch, which)
    orc = odec.DecodeOracle(cfg, w, ks, vs, oracle.load_ref(1), extra=len(PROMPT))
    got = orc.prompt(PROMPT)
    assert oracle.normwise_rel(got, want) > 10 * TOL, which


@needs_ref
def test_oracle_bf16_contraction_moves_logits_slightly(tiny):
    """gemm_bf16 changes only the contraction's operands: a prompt of <= 16
    rows is unchanged bit for bit, a longer one moves by bf16 rounding."""
    cfg, w, ks, vs = tiny
    lib = oracle.load_ref(1)
    a = odec.DecodeOracle(cfg, w, ks, vs, lib, extra=20).prompt(PROMPT[:12])
    b = odec.DecodeOracle(cfg, w, ks, vs, lib, extra=20, gemm_bf16=True).prompt(PROMPT[:12])
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    a = odec.DecodeOracle(cfg, w, ks, vs, lib, extra=20).prompt(PROMPT)
    b = odec.DecodeOracle(cfg, w, ks, vs, lib, extra=20, gemm_bf16=True).prompt(PROMPT)
    assert 1e-5 < oracle.normwise_rel(b, a) < 5e-2


def test_bf16_round_is_nearest_even():
    import torch
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-20, 20, 100000),
                        np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -1.0 - 2 ** -8, 0.0, -0.0], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(odec.bf16_round(x).view(np.uint32), want.view(np.uint32))


@needs_ref
def test_numpy_stage_bit_identical_to_oracle(tiny):
    """The product's NumPy stage and the oracle, both on the reference
    kernel, give the same logits bit for bit (two codings of the reference
    stage; the projections are the same kernel's)."""
    cfg, w, ks, vs = tiny
    lib = oracle.load_ref(1)
    want = run_oracle(cfg, w, ks, vs, TOKENS, lib)
    st = numpy_stage.Stage(cfg, w, lib=lib)
    caches = st.new_caches(ks, vs, extra=len(TOKENS), dtype=np.float16)
    for i, tok in enumerate(TOKENS):
        got = st(np.array([[tok]]), caches, last_only=True).reshape(-1)
        assert np.array_equal(got.view(np.uint32), want[i].view(np.uint32)), i


@needs_ref
def test_numpy_stage_prompt_matches_decode(tiny):
    """A 5-token prompt through the stage's prompt path (causal attention
    over the prompt's own positions; the per-row GEMV quantises each row
    alone) gives, at its last position, the logits of five decode steps up
    to the summation order of the attention's BLAS calls and softmax sums,
    which moves the int16 rounding of a few inputs of later GEMVs (measured
    9e-5 here; a wrong causal mask is off by far more)."""
    cfg, w, ks, vs = tiny
    lib = oracle.load_ref(1)
    st = numpy_stage.Stage(cfg, w, lib=lib)
    ids = np.array([[3, 1, 4, 1, 5]])
    c1 = st.new_caches(ks, vs, extra=8, dtype=np.float16)
    prompt = st(ids, c1, last_only=True).reshape(-1)
    c2 = st.new_caches(ks, vs, extra=8, dtype=np.float16)
    for t in ids[0]:
        step = st(np.array([[t]]), c2, last_only=True).reshape(-1)
    assert oracle.normwise_rel(prompt, step) < TOL


def test_kv_cache_grows_past_capacity():
    c = numpy_stage.KVCache(2, 4, capacity=3, dtype=np.float16)
    rng = np.random.default_rng(0)
    ks = [rng.standard_normal((1, 2, n, 4)).astype(np.float32) for n in (2, 3, 1)]
    for k in ks:
        kk, vv = c.update_and_fetch(k, -k)
    allk = np.concatenate(ks, axis=2).astype(np.float16)
    assert c.offset == 6 and np.array_equal(kk, allk) and np.array_equal(vv, -allk)


def test_ih_draws_numpy_torch_identical():
    import torch
    w, s, b = synth.qlinear_ih_np(5, 70, 512, 64, tag="t.")
    tw, ts, tb = synth.qlinear_ih_torch(5, 70, 512, 64, "cpu", tag="t.")
    assert np.array_equal(w.view(np.int32), tw.numpy())
    assert np.array_equal(s.view(np.int16), ts.numpy()) and np.array_equal(b.view(np.int16), tb.numpy())
    z = synth.ih_normal_np(6, "z", 100001, 0.5)
    assert np.array_equal(z, synth.ih_normal_torch(6, "z", 100001, 0.5, "cpu").numpy())
    assert abs(float(z.std()) - 0.5) < 0.01 and abs(float(z.mean())) < 0.01
    # u64 wraps identically: the first outputs of a stream
    assert np.array_equal(synth.u64(9, "k", 5).view(np.int64), synth.u64_torch(9, "k", 5, "cpu").numpy())


def test_synthetic_model_numpy_torch_identical():
    cfg = tiny_cfg(1)
    a = qwen2.synthetic_weights(cfg, 3)
    b = qwen2.synthetic_weights_torch(cfg, 3, "cpu")
    assert sorted(a) == sorted(b)
    for k in a:
        x, y = np.ascontiguousarray(a[k]), b[k].numpy()
        assert x.dtype.itemsize == y.dtype.itemsize and np.array_equal(x.view(y.dtype), y), k
    ks, vs = qwen2.synthetic_context(cfg, 9, 4)
    tk, tv = qwen2.synthetic_context_torch(cfg, 9, 4, "cpu")
    assert np.array_equal(ks[0].view(np.int16), tk[0].view(__import__("torch").int16).numpy())
    assert np.array_equal(vs[0].view(np.int16), tv[0].view(__import__("torch").int16).numpy())
