"""Device-resident Qwen2 decode step on one MI355X.

The same stage as hetero/cpu_model.py (the reference's
hetero/cpu_model.py:164-368), with every tensor resident in HBM:
  * 4-bit projections through libq4gemv.so's device entry points: q/k/v in
    one grouped launch (q4_gemv_multi_dev), o_proj and lm_head as single
    launches, the MLP as the fused gate/up/SiLU*mul launch plus down
    (q4_mlp_dev) -- every GEMV result is the reference q4_gemv's bit for bit;
  * RMSNorm, RoPE, the fp16 KV cache and GQA attention as torch fp32 ops
    (torch is plumbing here: device memory, streams, graph capture);
  * greedy argmax on the device.
The token id and the position live in device tensors and attention runs
over the whole fixed-size cache with a position mask, so one decode step is
position-independent and is captured once as a HIP graph; generating n
tokens is n graph replays with no host work in between.
"""
from __future__ import annotations

from typing import Dict, List, Optional

import numpy as np

from . import q4


class GpuStage:
    def __init__(self, cfg: dict, w: Dict[str, np.ndarray], kv_k: List[np.ndarray],
                 kv_v: List[np.ndarray], max_new: int, device="cuda", lib=None):
        """w: reference-named numpy weights (cpu_model.synthetic_weights);
        kv_k / kv_v: per layer [KH, S0, D] context already in the cache
        (fp16 as stored); max_new: decode steps the cache must hold."""
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
        self.cap = self.s0 + max_new
        dev = self.dev

        def t(a, dtype=None):
            a = np.ascontiguousarray(a)
            tt = torch.from_numpy(a.view(np.int16) if a.dtype == np.float16 else a)
            return tt.to(dev) if dtype is None else tt.to(dev, dtype)

        def mat(name):
            return (t(w[f"{name}.weight"]), t(w[f"{name}.scales"]), t(w[f"{name}.biases"]))

        self.embed = mat("model.embed_tokens")
        self.layers = []
        for i in range(cfg["num_hidden_layers"]):
            p = f"model.layers.{i}"
            L = {
                "qkv": [mat(f"{p}.self_attn.{x}_proj") for x in ("q", "k", "v")],
                "qkv_bias": t(np.concatenate([w[f"{p}.self_attn.{x}_proj.bias"] for x in ("q", "k", "v")])),
                "o": mat(f"{p}.self_attn.o_proj"),
                "gate": mat(f"{p}.mlp.gate_proj"), "up": mat(f"{p}.mlp.up_proj"),
                "down": mat(f"{p}.mlp.down_proj"),
                "in_w": t(w[f"{p}.input_layernorm.weight"]),
                "post_w": t(w[f"{p}.post_attention_layernorm.weight"]),
            }
            kc = torch.zeros((self.nkv, self.cap, self.hd), dtype=torch.float16, device=dev)
            vc = torch.zeros_like(kc)
            kc[:, :self.s0] = t(kv_k[i].astype(np.float16)).view(torch.float16)
            vc[:, :self.s0] = t(kv_v[i].astype(np.float16)).view(torch.float16)
            L["k_cache"], L["v_cache"] = kc, vc
            self.layers.append(L)
        self.norm_w = t(w["model.norm.weight"])
        self.lm_head = mat("lm_head")
        # RoPE table exactly as the reference builds it (cpu_model.py:180-193)
        half = self.hd // 2
        inv = cfg["rope_theta"] ** (-np.arange(0, half, dtype=np.float32) * 2.0 / self.hd)
        ang = np.arange(self.cap, dtype=np.float32)[:, None] * inv[None, :]
        self.cos, self.sin = t(np.cos(ang)), t(np.sin(ang))
        # step state and static buffers
        self.tok = torch.zeros(1, dtype=torch.int64, device=dev)
        self.pos = torch.full((1,), self.s0, dtype=torch.int64, device=dev)
        self.x = torch.zeros((1, self.h), dtype=torch.float32, device=dev)
        self.hbuf = torch.zeros((1, self.inter), dtype=torch.float32, device=dev)
        self.mlp_out = torch.zeros((1, self.h), dtype=torch.float32, device=dev)
        self.q = torch.zeros((1, self.h), dtype=torch.float32, device=dev)
        kvd = self.nkv * self.hd
        self.k = torch.zeros((1, kvd), dtype=torch.float32, device=dev)
        self.v = torch.zeros((1, kvd), dtype=torch.float32, device=dev)
        self.attn = torch.zeros((1, self.h), dtype=torch.float32, device=dev)
        self.o = torch.zeros((1, self.h), dtype=torch.float32, device=dev)
        self.logits = torch.zeros((1, cfg["vocab_size"]), dtype=torch.float32, device=dev)
        self.emb_rows = [torch.zeros((1,) + tuple(a.shape[1:]), dtype=a.dtype, device=dev) for a in self.embed]
        self.positions = torch.arange(self.cap, device=dev)
        self.hist = torch.zeros(max_new, dtype=torch.int64, device=dev)   # token of each step
        self.stream = torch.cuda.Stream(device=dev)
        self.graph = None

    # -- pieces -------------------------------------------------------------
    def _rms(self, x, w):                                               # cpu_model.py:164-166
        return x * (1.0 / self.torch.sqrt((x * x).mean(-1, keepdim=True) + self.eps)) * w

    def _rope(self, x, nheads):                                         # cpu_model.py:195-204
        torch = self.torch
        xh = x.view(nheads, self.hd)
        cos = self.cos.index_select(0, self.pos)                        # [1, half]
        sin = self.sin.index_select(0, self.pos)
        half = self.hd // 2
        x1, x2 = xh[:, :half], xh[:, half:]
        return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1)

    def _attention(self, q, L):                                         # cpu_model.py:233-252
        torch = self.torch
        g = self.nh // self.nkv
        kf = L["k_cache"].float()                                       # [KH, cap, D]
        vf = L["v_cache"].float()
        qh = q.view(self.nkv, g, self.hd).transpose(1, 2).contiguous()  # [KH, D, G]
        s = torch.matmul(kf, qh) * (self.hd ** -0.5)                    # [KH, cap, G]
        mask = (self.positions > self.pos).view(1, -1, 1)
        s = s.masked_fill(mask, float("-inf"))
        s = s - s.amax(dim=1, keepdim=True)
        e = torch.exp(s)
        e = e / e.sum(dim=1, keepdim=True)
        p = e.transpose(1, 2).contiguous()                              # [KH, G, cap]
        return torch.matmul(p, vf).reshape(1, self.h)                   # [KH, G, D] -> [1, H]

    def _step(self):
        torch = self.torch
        lib = self.lib
        # embedding: gather the packed row on the device, dequantise it (cpu_model.py:334-338)
        for dst, src in zip(self.emb_rows, self.embed):
            dst.copy_(src.index_select(0, self.tok))
        q4.dequant_dev(*self.emb_rows, 0, 1, out=self.x, lib=lib)
        x = self.x
        kvd = self.nkv * self.hd
        for L in self.layers:                                           # cpu_model.py:304-306
            hn = self._rms(x, L["in_w"]).contiguous()
            q4.gemv_multi_dev(L["qkv"], hn, outs=[self.q, self.k, self.v], lib=lib)
            b = L["qkv_bias"]
            q = self._rope(self.q + b[:self.h], self.nh)
            k = self._rope(self.k + b[self.h:self.h + kvd], self.nkv)
            v = (self.v + b[self.h + kvd:]).view(self.nkv, self.hd)
            L["k_cache"].index_copy_(1, self.pos, k.to(torch.float16).unsqueeze(1))
            L["v_cache"].index_copy_(1, self.pos, v.to(torch.float16).unsqueeze(1))
            self.attn.copy_(self._attention(q, L))
            q4.gemv_dev(*L["o"], self.attn, out=self.o, lib=lib)
            x = x + self.o
            hn2 = self._rms(x, L["post_w"]).contiguous()
            q4.mlp_dev(L["gate"], L["up"], L["down"], hn2, h=self.hbuf, out=self.mlp_out, lib=lib)
            x = x + self.mlp_out
        xn = self._rms(x, self.norm_w).contiguous()
        q4.gemv_dev(*self.lm_head, xn, out=self.logits, lib=lib)
        self.tok.copy_(self.logits.argmax(dim=-1))                      # backends.py:106-109
        self.hist.index_copy_(0, (self.pos - self.s0).clamp_(0, self.hist.numel() - 1), self.tok)
        self.pos.add_(1)

    # -- driving --------------------------------------------------------------
    def capture(self):
        """Run one step eagerly (sizes every workspace), restore the state and
        capture the step as a HIP graph."""
        torch = self.torch
        tok0, pos0 = self.tok.clone(), self.pos.clone()
        caches = [(L["k_cache"].clone(), L["v_cache"].clone()) for L in self.layers]
        with torch.cuda.stream(self.stream):
            self._step()
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

    def run(self, n: int) -> List[int]:
        """n free-running steps as back-to-back graph replays (no host sync in
        between); returns the n greedy tokens."""
        for _ in range(n):
            self.graph.replay()
        self.torch.cuda.synchronize()
        return self.hist[:n].tolist()

    def step(self) -> int:
        """One decode step (graph replay once captured); returns the greedy token."""
        if self.graph is None:
            with self.torch.cuda.stream(self.stream):
                self._step()
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
