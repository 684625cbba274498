"""Decode-step parity (a Qwen2-architecture stage with random 4-bit weights).

1. Drop-in: the NumPy stage (hetero/cpu_model.py, the reference's
   cpu_model restated) running on libq4gemv.so through the reference C-ABI
   must give the same logits, bit for bit, as the same stage running on the
   reference kernel compiled from source (oracle/_ref) -- every step, and
   therefore the same greedy tokens.
2. Device-resident: hetero/gpu_model.py (everything in HBM, HIP graph) vs
   the NumPy stage on the reference kernel: RMSNorm, softmax and exp round
   differently on the GPU, so logits agree within a stated norm-wise
   tolerance and greedy tokens are compared step by step (teacher-forced).
"""
import copy
import os

import numpy as np
import pytest

import oracle
from hetero import cpu_model, q4

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3      # norm-wise, device-resident vs NumPy reference logits


def small_cfg():
    cfg = cpu_model.qwen2_7b_config(layers=2)
    cfg.update(hidden_size=512, intermediate_size=1024, num_attention_heads=4,
               num_key_value_heads=2, vocab_size=1000)
    return cfg


@pytest.fixture(scope="module")
def model():
    cfg = small_cfg()
    w = cpu_model.synthetic_weights(cfg, seed=11)
    caches = cpu_model.synthetic_kv(cfg, context=64, seed=12)
    return cfg, w, caches


@pytest.mark.skipif(not os.path.exists(oracle.ref_path(1)), reason="oracle/_ref not built")
def test_dropin_stage_bit_identical_to_reference_kernel(model):
    cfg, w, caches = model
    ours = cpu_model.Stage(cfg, w, lib=q4.load())
    ref = cpu_model.Stage(cfg, w, lib=oracle.load_ref(1))
    c1, c2 = copy.deepcopy(caches), copy.deepcopy(caches)
    tok_a = tok_b = 7
    for step in range(6):
        la = ours(np.array([[tok_a]]), c1, last_only=True)
        lb = ref(np.array([[tok_b]]), c2, last_only=True)
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), f"step {step}"
        tok_a, tok_b = cpu_model.greedy(la), cpu_model.greedy(lb)
        assert tok_a == tok_b
    # a 20-row prompt goes through q4_gemv_batched (rows <= 16) and q4_dequant
    # + BLAS (rows > 16) on both sides
    ids = (np.arange(20) * 37 % cfg["vocab_size"]).reshape(1, -1)
    pa = ours(ids, copy.deepcopy(caches))
    pb = ref(ids, copy.deepcopy(caches))
    assert np.array_equal(pa.view(np.uint32), pb.view(np.uint32))
    pa = ours(ids[:, :12], copy.deepcopy(caches))
    pb = ref(ids[:, :12], copy.deepcopy(caches))
    assert np.array_equal(pa.view(np.uint32), pb.view(np.uint32))


@pytest.mark.skipif(not os.path.exists(oracle.ref_path(1)), reason="oracle/_ref not built")
def test_device_resident_decode_vs_reference(model):
    import torch
    from hetero.gpu_model import GpuStage
    cfg, w, caches = model
    steps = 8
    ref = cpu_model.Stage(cfg, w, lib=oracle.load_ref(1))
    c = copy.deepcopy(caches)
    ref_tokens, ref_logits = [], []
    tok = 7
    for _ in range(steps):
        lg = ref(np.array([[tok]]), c, last_only=True).reshape(-1)
        ref_logits.append(lg)
        tok = cpu_model.greedy(lg)
        ref_tokens.append(tok)
    g = GpuStage(cfg, w, [cc.keys[0, :, :cc.offset] for cc in caches],
                 [cc.values[0, :, :cc.offset] for cc in caches], max_new=steps)
    g.set_token(7)
    g.capture()
    inputs = [7] + ref_tokens[:-1]
    agree = 0
    for i in range(steps):
        g.set_token(inputs[i])
        t = g.step()
        lg = g.logits.cpu().numpy().reshape(-1)
        assert oracle.normwise_rel(lg, ref_logits[i]) < LOGIT_TOL, i
        agree += int(t == ref_tokens[i])
    torch.cuda.synchronize()
    assert agree == steps, f"greedy tokens agree on {agree}/{steps} teacher-forced steps"
