"""Device-resident Qwen2 decode step on one MI355X.

The reference's Qwen2 stage (hetero/cpu_model.py:164-368; the host
counterpart here is hetero/numpy_stage.py) with every tensor resident in HBM
and every operation a kernel of libq4gemv.so:
  * 4-bit projections through the streaming GEMV: q/k/v in one grouped
    launch, o_proj, the fused gate/up/SiLU*mul launch, down and lm_head --
    every GEMV result is the reference q4_gemv's bit for bit given the same
    input.  Each residual add and RMSNorm is folded into the prologue of the
    GEMV that follows it (q4_norm_gemv_multi_dev for q/k/v,
    q4_norm_gate_up_silu_dev for gate/up; include/q4decode.h), and lm_head
    takes the greedy argmax with the step's bookkeeping in its own launch
    (q4_norm_gemv_argmax_dev);
  * the rest from include/q4decode.h: the embedding row (q4_embed_dev) and
    bias + RoPE + the fp16 KV-cache write fused with GQA attention split over
    the context (q4_attention_rope_dev).
The token id and the position live in device tensors and attention covers
positions [0, pos] of a fixed-size cache, so one decode step is
position-independent and is captured once as a HIP graph; generating n
tokens is n graph replays with no host work in between.  torch only
allocates the buffers and captures the graph.
"""
from __future__ import annotations

from typing import Dict, List, Optional

import numpy as np

from . import q4


class GpuStage:
    def __init__(self, cfg: dict, w: Dict[str, np.ndarray], kv_k: List[np.ndarray],
                 kv_v: List[np.ndarray], max_new: int, device="cuda", lib=None):
        """w: reference-named weights, NumPy arrays (qwen2.synthetic_weights)
        or device tensors (qwen2.synthetic_weights_torch,
        shard.WeightIndex.load_shard(..., framework="hip"));
        kv_k / kv_v: per layer [KH, S0, D] context already in the cache
        (NumPy arrays or tensors; stored as fp16); max_new: decode steps the
        cache must hold."""
        import torch
        self.torch = torch
        self.lib = lib or q4.load()
        self.cfg = cfg
        self.dev = torch.device(device)
        self.gs = cfg["quantization"]["group_size"]
        self.eps = cfg["rms_norm_eps"]
        self.h = cfg["hidden_size"]
        self.nh, self.nkv = cfg["num_attention_heads"], cfg["num_key_value_heads"]
        self.hd = self.h // self.nh
        self.inter = cfg["intermediate_size"]
        self.s0 = kv_k[0].shape[1]
        self.max_new = int(max_new)
        self.cap = self.s0 + self.max_new
        self.steps_done = 0       # decode steps since the last reset (the cache holds max_new)
        dev = self.dev

        def t(a, dtype=None):
            if isinstance(a, torch.Tensor):           # already loaded (hetero/shard.py)
                return a.to(dev) if dtype is None else a.to(dev, dtype)
            a = np.ascontiguousarray(a)
            tt = torch.from_numpy(a.view(np.int16) if a.dtype == np.float16 else a)
            return tt.to(dev) if dtype is None else tt.to(dev, dtype)

        def f16_bits(a):
            """scales/biases as fp16 bit patterns (cpu_model.py:102-103 takes
            them as float16; a bf16 or fp32 checkpoint is rounded to nearest
            fp16 once, here)."""
            if isinstance(a, torch.Tensor):
                a = a.to(dev)
                return (a if a.dtype == torch.float16 else a.to(torch.float32).to(torch.float16)).view(torch.int16)
            return t(np.asarray(a, dtype=np.float16))

        def f32(a):
            """.astype(np.float32) of a host array or a device tensor"""
            if isinstance(a, torch.Tensor):
                return a.to(dev, torch.float32)
            return t(np.asarray(a).astype(np.float32))

        def f16(a):
            """a KV context block [KH, S0, D] as fp16 values on the device"""
            if isinstance(a, torch.Tensor):
                return a.to(dev, torch.float16)
            return t(np.asarray(a).astype(np.float16)).view(torch.float16)

        def mat(name):
            return (t(w[f"{name}.weight"]), f16_bits(w[f"{name}.scales"]), f16_bits(w[f"{name}.biases"]))

        self.embed = mat("model.embed_tokens")
        self.layers = []
        for i in range(cfg["num_hidden_layers"]):
            p = f"model.layers.{i}"
            L = {
                "qkv": [mat(f"{p}.self_attn.{x}_proj") for x in ("q", "k", "v")],
                "qkv_bias": torch.cat([f32(w[f"{p}.self_attn.{x}_proj.bias"]).reshape(-1)
                                       for x in ("q", "k", "v")]),
                "o": mat(f"{p}.self_attn.o_proj"),
                "gate": mat(f"{p}.mlp.gate_proj"), "up": mat(f"{p}.mlp.up_proj"),
                "down": mat(f"{p}.mlp.down_proj"),
                "in_w": f32(w[f"{p}.input_layernorm.weight"]),                      # cpu_model.py:298-299
                "post_w": f32(w[f"{p}.post_attention_layernorm.weight"]),
            }
            kc = torch.zeros((self.nkv, self.cap, self.hd), dtype=torch.float16, device=dev)
            vc = torch.zeros_like(kc)
            kc[:, :self.s0] = f16(kv_k[i])
            vc[:, :self.s0] = f16(kv_v[i])
            L["k_cache"], L["v_cache"] = kc, vc
            self.layers.append(L)
        self.norm_w = f32(w["model.norm.weight"])
        tied = bool(cfg.get("tie_word_embeddings", False))
        self.lm_head = self.embed if tied else mat("lm_head")                # cpu_model.py:324-329
        # RoPE table exactly as the reference builds it (cpu_model.py:180-193)
        half = self.hd // 2
        inv = cfg["rope_theta"] ** (-np.arange(0, half, dtype=np.float32) * 2.0 / self.hd)
        ang = np.arange(self.cap, dtype=np.float32)[:, None] * inv[None, :]
        self.cos, self.sin = t(np.cos(ang)), t(np.sin(ang))
        # step state and static buffers
        self.tok = torch.zeros(1, dtype=torch.int64, device=dev)
        self.pos = torch.full((1,), self.s0, dtype=torch.int64, device=dev)
        # the residual stream, in two buffers: each fused norm + GEMV reads
        # one and writes x + delta to the other
        self.xbuf = (torch.zeros(self.h, dtype=torch.float32, device=dev),
                     torch.zeros(self.h, dtype=torch.float32, device=dev))
        self.hbuf = torch.zeros((1, self.inter), dtype=torch.float32, device=dev)
        self.mlp_out = torch.zeros((1, self.h), dtype=torch.float32, device=dev)
        self.q = torch.zeros((1, self.h), dtype=torch.float32, device=dev)
        kvd = self.nkv * self.hd
        self.k = torch.zeros((1, kvd), dtype=torch.float32, device=dev)
        self.v = torch.zeros((1, kvd), dtype=torch.float32, device=dev)
        self.attn = torch.zeros((1, self.h), dtype=torch.float32, device=dev)
        self.o = torch.zeros((1, self.h), dtype=torch.float32, device=dev)
        self.logits = torch.zeros((1, cfg["vocab_size"]), dtype=torch.float32, device=dev)
        self.positions = torch.arange(self.cap, device=dev)
        self.hist = torch.zeros(max_new, dtype=torch.int64, device=dev)   # token of each step
        n_scr = self.lib.q4_attention_scratch_floats(self.nh, self.hd, self.cap)
        self.attn_scratch = torch.zeros(n_scr, dtype=torch.float32, device=dev)
        self.scale = float(np.float32(self.hd ** -0.5))            # cpu_model.py:261
        self.stream = torch.cuda.Stream(device=dev)
        self.graph = None

    # -- one step -----------------------------------------------------------
    def _step(self):
        lib = self.lib
        st = self.torch.cuda.current_stream().cuda_stream
        ck = lambda rc, what: q4.check(lib, rc, what)
        P = lambda t: t.data_ptr()
        h, gs = self.h, self.gs
        ew, es, eb = self.embed
        # embedding row (cpu_model.py:334-338)
        cur, other = self.xbuf
        ck(lib.q4_embed_dev(P(ew), P(es), P(eb), P(self.tok), P(cur), ew.shape[0], h, gs, st), "embed")
        delta = None
        for L in self.layers:                                           # cpu_model.py:304-306
            # x = x + mlp (of the layer before); q/k/v of rms_norm(x, in_w)
            q4.norm_gemv_multi_dev(L["qkv"], cur, delta, L["in_w"], self.eps,
                                   x_out=other if delta is not None else None, outs=[self.q, self.k, self.v],
                                   lib=lib)
            if delta is not None:
                cur, other = other, cur
            # bias + RoPE + the KV-cache write fused into the attention launches
            ck(lib.q4_attention_rope_dev(P(self.q), P(self.k), P(self.v), P(L["qkv_bias"]), P(self.cos),
                                         P(self.sin), P(self.pos), P(L["k_cache"]), P(L["v_cache"]), P(self.attn),
                                         P(self.attn_scratch), self.nh, self.nkv, self.hd, self.cap, self.scale, st),
               "attention")
            q4.gemv_dev(*L["o"], self.attn, out=self.o, lib=lib)
            # x = x + attn; SiLU(gate) * up of rms_norm(x, post_w), then down
            q4.norm_gate_up_silu_dev(L["gate"], L["up"], cur, self.o, L["post_w"], self.eps, x_out=other,
                                     h=self.hbuf, lib=lib)
            cur, other = other, cur
            q4.gemv_dev(*L["down"], self.hbuf, out=self.mlp_out, lib=lib)
            delta = self.mlp_out
        # x = x + mlp; lm_head of the final norm (cpu_model.py:367), and in the
        # same launch the greedy token (backends.py:106-109), its history
        # slot and position + 1
        q4.norm_gemv_argmax_dev(self.lm_head, cur, delta, self.norm_w, self.eps, self.tok, self.pos,
                                hist=self.hist, s0=self.s0, logits=self.logits, lib=lib)

    # -- driving --------------------------------------------------------------
    def _eager_step(self):
        """One step on the stage's stream, ordered after the caller's stream
        (the state set up or copied there: token, caches, clones) and before
        its later work (a read of the token).  torch's side streams do not
        synchronise with the default stream by themselves."""
        cur = self.torch.cuda.current_stream()
        self.stream.wait_stream(cur)
        with self.torch.cuda.stream(self.stream):
            self._step()
        cur.wait_stream(self.stream)

    def capture(self):
        """Run one step eagerly (sizes every workspace), restore the state and
        capture the step as a HIP graph.  The decode state (token, position,
        caches, steps taken) is what it was before the call."""
        torch = self.torch
        tok0, pos0 = self.tok.clone(), self.pos.clone()
        caches = [(L["k_cache"].clone(), L["v_cache"].clone()) for L in self.layers]
        self._eager_step()
        torch.cuda.synchronize()
        self.tok.copy_(tok0)
        self.pos.copy_(pos0)
        for L, (kc, vc) in zip(self.layers, caches):
            L["k_cache"].copy_(kc)
            L["v_cache"].copy_(vc)
        del caches
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self._step()
        torch.cuda.synchronize()

    def set_token(self, tok: int):
        self.tok.fill_(int(tok))

    def reset(self, tok: int):
        """Back to the initial context (positions past it are masked and
        rewritten as decoding proceeds) with `tok` as the next input."""
        self.pos.fill_(self.s0)
        self.tok.fill_(int(tok))
        self.steps_done = 0

    def _take(self, n: int):
        """Claim n steps of the cache; past max_new the kernels would clamp
        the position and decode wrong tokens without an error."""
        if n < 0 or self.steps_done + n > self.max_new:
            raise ValueError(f"{n} more decode steps after {self.steps_done} exceed max_new={self.max_new}; "
                             "reset() first or build the stage with a larger max_new")
        self.steps_done += n

    def run(self, n: int) -> List[int]:
        """n free-running steps from the last reset() as back-to-back graph
        replays (no host sync in between); returns the n greedy tokens."""
        if self.steps_done:
            raise ValueError("run() starts from the initial context: reset() first")
        self._take(n)
        for _ in range(n):
            self.graph.replay()
        self.torch.cuda.synchronize()
        return self.hist[:n].tolist()

    def step(self) -> int:
        """One decode step (graph replay once captured); returns the greedy token."""
        self._take(1)
        if self.graph is None:
            self._eager_step()
        else:
            self.graph.replay()
        return int(self.tok.item())

    def generate(self, n: int, tokens_in: Optional[List[int]] = None) -> List[int]:
        """n steps free-running from the current token, or teacher-forced on
        tokens_in (step i consumes tokens_in[i])."""
        out = []
        for i in range(n):
            if tokens_in is not None:
                self.set_token(tokens_in[i])
            out.append(self.step())
        return out
