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
positions [0, pos] of the cache, so one decode step is position-independent
and is captured once as a HIP graph; generating n tokens is n graph replays
with no host work in between.  torch only allocates the buffers and captures
the graph.

A prompt runs through the same layers on the device (prefill), in chunks of
rows as the reference's coordinator sends them (hetero/coordinator.py:
175-182): the chunk's embedding rows, per layer RMSNorm, the q/k/v
projections -- up to 16 rows the GEMV (each row bit-identical to a q4_gemv
call), above that the bf16 matrix-core GEMM, as the reference switches from
q4_gemv to q4_dequant + BLAS (hetero/cpu_model.py:139-158) -- bias, RoPE and
the KV-cache write at the chunk's positions, causal attention over the
cache, o_proj, the MLP, and for the last chunk the final norm, lm_head and
the greedy token of its last row (hetero/cpu_model.py:357-368).

The KV cache grows as the reference's does (hetero/cpu_model.py:216-230):
when a prompt or a decode step needs positions past its capacity, by the
needed count rounded up to 256 positions; the captured graph then refers to
the old buffers and is captured again before the next replay.
"""
from __future__ import annotations

from typing import Dict, List, Optional

import numpy as np

from . import q4


# the reference cache's growth step (hetero/cpu_model.py:214)
KV_STEP = 256
# positions the attention kernels address (include/q4decode.h)
KV_MAX = 65536


class GpuStage:
    def __init__(self, cfg: dict, w: Dict[str, np.ndarray], kv_k: Optional[List[np.ndarray]] = None,
                 kv_v: Optional[List[np.ndarray]] = None, max_new: int = KV_STEP, device="cuda", lib=None):
        """w: reference-named weights, NumPy arrays (qwen2.synthetic_weights)
        or device tensors (qwen2.synthetic_weights_torch,
        shard.WeightIndex.load_shard(..., framework="hip"));
        kv_k / kv_v: per layer [KH, S0, D] context already in the cache
        (NumPy arrays or tensors; stored as fp16), or None for an empty
        cache; max_new: decode steps the cache holds before it first grows."""
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
        self.s0 = 0 if kv_k is None else kv_k[0].shape[1]
        self.max_new = int(max_new)
        self.cap = max(self.s0 + self.max_new, 1)
        if self.cap > KV_MAX:
            raise ValueError(f"{self.cap} cache positions: the attention kernels address at most {KV_MAX}")
        self.steps_done = 0       # decode steps since the last reset or prompt
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
            if self.s0:
                kc[:, :self.s0] = f16(kv_k[i])
                vc[:, :self.s0] = f16(kv_v[i])
            L["k_cache"], L["v_cache"] = kc, vc
            self.layers.append(L)
        self.norm_w = f32(w["model.norm.weight"])
        tied = bool(cfg.get("tie_word_embeddings", False))
        self.lm_head = self.embed if tied else mat("lm_head")                # cpu_model.py:324-329
        self._tables()
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
        self.hist = torch.zeros(max(self.max_new, 1), dtype=torch.int64, device=dev)   # token of each step
        self._scratch()
        self.scale = float(np.float32(self.hd ** -0.5))            # cpu_model.py:261
        self.stream = torch.cuda.Stream(device=dev)
        self.graph = None

    # -- capacity -------------------------------------------------------------
    def _tables(self):
        """RoPE cos/sin [cap][d/2] exactly as the reference builds them
        (cpu_model.py:180-193): rows do not depend on the table's length."""
        half = self.hd // 2
        inv = self.cfg["rope_theta"] ** (-np.arange(0, half, dtype=np.float32) * 2.0 / self.hd)
        ang = np.arange(self.cap, dtype=np.float32)[:, None] * inv[None, :]
        self.cos = self.torch.from_numpy(np.cos(ang)).to(self.dev)
        self.sin = self.torch.from_numpy(np.sin(ang)).to(self.dev)

    def _scratch(self):
        n_scr = self.lib.q4_attention_scratch_floats(self.nh, self.hd, self.cap)
        self.attn_scratch = self.torch.zeros(n_scr, dtype=self.torch.float32, device=self.dev)

    @property
    def position(self) -> int:
        """The position the next token is written at (host view of self.pos)."""
        return self.s0 + self.steps_done

    def _ensure(self, n: int):
        """Room for n more positions after the current one: past the
        capacity the caches grow by n rounded up to KV_STEP positions (the
        reference's KVCache.update_and_fetch, cpu_model.py:216-226) and the
        decode graph is dropped (it holds the old buffers)."""
        torch = self.torch
        need = self.position + n
        if need > self.cap:
            new_cap = self.position + ((n + KV_STEP - 1) // KV_STEP) * KV_STEP
            if need > KV_MAX:
                raise ValueError(f"{need} cache positions: the attention kernels address at most {KV_MAX}")
            new_cap = min(new_cap, KV_MAX)
            torch.cuda.synchronize()
            keep = self.position
            for L in self.layers:
                for name in ("k_cache", "v_cache"):
                    old = L[name]
                    new = torch.zeros((self.nkv, new_cap, self.hd), dtype=torch.float16, device=self.dev)
                    new[:, :keep] = old[:, :keep]
                    L[name] = new
            self.cap = new_cap
            self._tables()
            self._scratch()
            self.graph = None
        if self.steps_done + n > self.hist.numel():
            torch.cuda.synchronize()
            hist = torch.zeros(self.steps_done + ((n + KV_STEP - 1) // KV_STEP) * KV_STEP, dtype=torch.int64,
                               device=self.dev)
            hist[:self.hist.numel()] = self.hist
            self.hist = hist
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
        caches, steps taken, the last step's logits and the token history)
        is what it was before the call."""
        torch = self.torch
        self._ensure(1)                            # the eager step writes one position
        p = self.position
        saved = [self.tok.clone(), self.pos.clone(), self.logits.clone(), self.hist.clone()]
        rows = [(L["k_cache"][:, p].clone(), L["v_cache"][:, p].clone()) for L in self.layers]
        self._eager_step()
        torch.cuda.synchronize()
        for t, v in zip((self.tok, self.pos, self.logits, self.hist), saved):
            t.copy_(v)
        for L, (kr, vr) in zip(self.layers, rows):
            L["k_cache"][:, p] = kr
            L["v_cache"][:, p] = vr
        del saved, rows
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self._step()
        torch.cuda.synchronize()

    def set_token(self, tok: int):
        self.tok.fill_(int(tok))

    def reset(self, tok: int):
        """Back to the initial context -- the one the stage was built with, or
        the last prompt (positions past it are masked and rewritten as
        decoding proceeds) -- with `tok` as the next input."""
        self.pos.fill_(self.s0)
        self.tok.fill_(int(tok))
        self.steps_done = 0

    def truncate(self, n: int = 0):
        """Keep the first n cache positions and drop the rest (they are
        masked and rewritten by what comes next): the context becomes those
        n positions, decoding and prompts continue from position n."""
        if not 0 <= n <= self.position:
            raise ValueError(f"truncate({n}) with {self.position} positions held")
        self.s0 = n
        self.steps_done = 0
        self.pos.fill_(n)
        self.graph = None                          # s0 is an argument of the captured step

    def _take(self, n: int):
        """Claim n steps: the cache and the token history grow first when
        they lack room (the kernels would otherwise clamp the position and
        decode wrong tokens without an error)."""
        if n < 0:
            raise ValueError(f"{n} decode steps")
        self._ensure(n)
        self.steps_done += n

    def run(self, n: int) -> List[int]:
        """n free-running steps from the last reset() or prompt as
        back-to-back graph replays (no host sync in between); returns the n
        greedy tokens."""
        if self.steps_done:
            raise ValueError("run() starts from the initial context: reset() first")
        self._take(n)
        if self.graph is None:
            self.steps_done -= n                   # capture() runs its step from the state before them
            self.capture()
            self.steps_done += n
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

    # -- prompts --------------------------------------------------------------
    def prefill(self, ids, chunk: int = 512) -> int:
        """Run the prompt token ids through the stage from the current
        position, `chunk` rows per pass (hetero/coordinator.py:175-182),
        appending their keys and values to the cache; returns the greedy
        token of the last position (its logits in self.logits).  Decoding
        then continues from the prompt's end: the prompt becomes the
        context reset() returns to, and the decode graph is captured again
        on the next run()."""
        torch = self.torch
        ids = [int(t) for t in np.asarray(ids).reshape(-1)]
        if not ids:
            raise ValueError("an empty prompt")
        if chunk < 1:
            raise ValueError(f"chunk={chunk}")
        self._ensure(len(ids))
        p0 = self.position
        cur = torch.cuda.current_stream()
        self.stream.wait_stream(cur)
        with torch.cuda.stream(self.stream):
            ids_d = torch.tensor(ids, dtype=torch.int64, device=self.dev)
            for lo in range(0, len(ids), chunk):
                hi = min(lo + chunk, len(ids))
                self._prefill_chunk(ids_d[lo:hi], p0 + lo, last=hi == len(ids))
        cur.wait_stream(self.stream)
        self.s0 = p0 + len(ids)
        self.steps_done = 0
        self.graph = None                          # s0 is an argument of the captured step
        return int(self.tok.item())

    def _proj(self, mats, x, outs):
        """y = x W^T for [rows][n_in] x: the GEMV up to 16 rows (each row as
        q4_gemv computes it), the bf16 matrix-core GEMM above -- the
        reference's QLinear switch (hetero/cpu_model.py:139-158)."""
        if x.shape[0] <= 16:
            q4.gemv_multi_dev(mats, x, outs=outs, lib=self.lib)
        else:
            q4.gemm_bf16_multi_dev(mats, x, outs=outs, lib=self.lib)

    def _prefill_chunk(self, ids, pos0: int, last: bool):
        torch, lib = self.torch, self.lib
        st = torch.cuda.current_stream().cuda_stream
        ck = lambda rc, what: q4.check(lib, rc, what)
        P = lambda t: t.data_ptr()
        rows, h, dev = ids.numel(), self.h, self.dev
        f32 = lambda *shape: torch.empty(shape, dtype=torch.float32, device=dev)
        ew, es, eb = self.embed
        x = f32(rows, h)
        ck(lib.q4_embed_rows_dev(P(ew), P(es), P(eb), P(ids), rows, P(x), ew.shape[0], h, self.gs, st), "embed rows")
        # above 16 rows the projections are bf16 matrix-core GEMMs: the norms,
        # the attention and the gate/up epilogue store their outputs in bf16
        # (rounded as the GEMM would round them), and SiLU * up is the
        # gate/up GEMM's epilogue
        gemm = rows > 16
        act = (lambda *shape: torch.empty(shape, dtype=torch.bfloat16, device=dev)) if gemm else f32
        norm_rows = lib.q4_add_rmsnorm_rows_bf16_dev if gemm else lib.q4_add_rmsnorm_rows_dev
        attention = lib.q4_prompt_attention_bf16_dev if gemm else lib.q4_prompt_attention_dev
        hn, attn, o = act(rows, h), act(rows, h), f32(rows, h)
        kvd = self.nkv * self.hd
        q, k, v, qr = f32(rows, h), f32(rows, kvd), f32(rows, kvd), f32(rows, h)
        hb, mlp = act(rows, self.inter), f32(rows, h)
        delta = None
        for L in self.layers:                                           # cpu_model.py:304-306
            ck(norm_rows(P(x), None if delta is None else P(delta), P(L["in_w"]), self.eps, P(hn), rows, h, st),
               "input norm")
            self._proj(L["qkv"], hn, [q, k, v])
            ck(lib.q4_rope_kv_rows_dev(P(q), P(k), P(v), P(L["qkv_bias"]), P(self.cos), P(self.sin), pos0, rows,
                                       P(L["k_cache"]), P(L["v_cache"]), P(qr), self.nh, self.nkv, self.hd,
                                       self.cap, st), "rope/kv rows")
            ck(attention(P(qr), P(L["k_cache"]), P(L["v_cache"]), P(attn), rows, pos0, self.nh, self.nkv, self.hd,
                         self.cap, self.scale, st), "prompt attention")
            self._proj([L["o"]], attn, [o])
            ck(norm_rows(P(x), P(o), P(L["post_w"]), self.eps, P(hn), rows, h, st), "post-attention norm")
            if gemm:
                q4.gemm_bf16_gate_up_silu_dev(L["gate"], L["up"], hn, h=hb, lib=lib)
            else:
                q4.gate_up_silu_dev(L["gate"], L["up"], hn, h=hb, lib=lib)
            self._proj([L["down"]], hb, [mlp])
            delta = mlp
        if last:
            # x + mlp of the last row; lm_head of its final norm and the
            # greedy token (cpu_model.py:363-367, backends.py:106-109); the
            # launch moves pos from the last row's position to the next
            self.pos.fill_(pos0 + rows - 1)
            q4.norm_gemv_argmax_dev(self.lm_head, x[rows - 1], delta[rows - 1], self.norm_w, self.eps, self.tok,
                                    self.pos, hist=None, s0=0, logits=self.logits, lib=lib)

    def generate(self, n: int, tokens_in: Optional[List[int]] = None) -> List[int]:
        """n steps free-running from the current token, or teacher-forced on
        tokens_in (step i consumes tokens_in[i])."""
        out = []
        for i in range(n):
            if tokens_in is not None:
                self.set_token(tokens_in[i])
            out.append(self.step())
        return out
