"""Greedy single-sequence INT8 decoder on gfx950: the reference's Qwen2 / Llama-3 single-token forward
(src/source/model/qwen2.cpp:690-830, llama3.cpp:705-818) on the HIP operators of this package.

Every launch goes to the HIP libraries (libsq8.so: the INT8 matmul and include/sq8_decode.h);
torch supplies device memory, streams and graph capture only. One decode step is

    embedding -> per layer: [add +] RMSNorm -> fused QKV GEMV -> RoPE + KV write -> attention ->
    O GEMV -> add + RMSNorm -> fused gate/up GEMV -> SwiGLU -> down GEMV
    -> add + final RMSNorm -> classifier GEMV -> argmax -> (pos, token) advance

with the residual add of each block folded into the next RMSNorm. With ``fused=True`` (the
default) every add + RMSNorm runs inside the prologue of the projection that consumes it
(sq8_matmul_rmsnorm, the residual stream ping-ponging between two buffers), SwiGLU in the
gate/up projection's epilogue (sq8_matmul_rmsnorm_swiglu: one wave computes a gate row and its up
row) and RoPE + cache write inside attention (sq8_rope_attention_decode): 5 launches per layer
instead of 9; the step ends with one launch for argmax, position advance and the next token's
embedding (sq8_argmax_advance). Positions and tokens live in device memory, so the step is
captured once into a HIP graph and replayed per token.

Weights come from an INT8 model file (model_file.py / the reference layout) or from an on-device
random init of the same distribution (for benchmarks of the large shapes without writing a file).
The projections of a layer that read the same input are fused at upload: QKV = [wq; wk; wv] and
gate/up = [w1; w3], rows stacked and their scales concatenated in the same order (each output
row is unchanged because groups never cross rows).
"""
from __future__ import annotations

import numpy as np

from . import (Workspace, add_rmsnorm, argmax, argmax_advance, attention_decode,
               decode_attention_workspace_bytes, embedding, lib,
               matmul, matmul_rmsnorm, matmul_rmsnorm_swiglu, matmul_swiglu, quantize, rmsnorm,
               rope_attention_decode, rope_kv, rope_tables, step_advance, swiglu)
from .model_file import ModelConfig, ModelFile

EPS = 1e-6


class Int8Decoder:
    def __init__(self, cfg: ModelConfig, weights: dict, group_size: int, max_seq: int,
                 device="cuda", fused: bool = True):
        import torch
        self.torch = torch
        self.cfg, self.gs, self.max_seq, self.device = cfg, group_size, max_seq, device
        self.hs = cfg.dim // cfg.head_num
        self.kv_dim = cfg.kv_dim
        L, d, kv, h = cfg.layer_num, cfg.dim, cfg.kv_dim, cfg.hidden_dim
        self.w = weights
        f32 = dict(dtype=torch.float32, device=device)
        i32 = dict(dtype=torch.int32, device=device)
        self.kcache = torch.zeros((L, max_seq, kv), **f32)
        self.vcache = torch.zeros((L, max_seq, kv), **f32)
        self.sin = torch.empty((max_seq, self.hs), **f32)
        self.cos = torch.empty((max_seq, self.hs), **f32)
        rope_tables(self.sin, self.cos, self.hs, max_seq, float(cfg.rope_theta))
        self.fused = fused
        self.x = torch.zeros(d, **f32)        # residual stream
        self.x2 = torch.zeros(d, **f32)       # its other half when the norms are fused
        self.xn = torch.zeros(d, **f32)       # normalised input of the next projection
        self.qkv = torch.zeros(d + 2 * kv, **f32)
        self.att = torch.zeros(d, **f32)
        self.proj = torch.zeros(d, **f32)     # O or down projection output (residual branch)
        self.gu = torch.zeros(2 * h, **f32)
        self.hid = torch.zeros(h, **f32)
        self.logits = torch.zeros(cfg.vocab, **f32)
        self.pos = torch.zeros(1, **i32)
        self.token = torch.zeros(1, **i32)
        self.next = torch.zeros(1, **i32)
        self.ws = Workspace(device)
        self.argmax_ws = Workspace(device)  # sized now: nothing is allocated during capture
        self.argmax_ws.get(int(lib().sq8_argmax_workspace_bytes(cfg.vocab)))
        # Split-position attention: zero-filled once, every call leaves its tickets zero.
        att = decode_attention_workspace_bytes(cfg.head_num, self.hs, max_seq)
        self.att_ws = torch.zeros((att + 3) // 4, **i32) if att > 0 else None
        self.graph = None

    # ------------------------------------------------------------------ construction
    @classmethod
    def from_file(cls, path, max_seq: int, device="cuda", fused: bool = True) -> "Int8Decoder":
        """Load an INT8 model file (reference layout) and upload fused projections."""
        return cls.from_model(ModelFile(path), max_seq, device, fused)

    @classmethod
    def from_model(cls, m, max_seq: int, device="cuda", fused: bool = True) -> "Int8Decoder":
        """Upload fused projections from a host model with ModelFile's accessors (a ModelFile or
        a model_file.RandomModel)."""
        import torch
        cfg, gs = m.config, m.group_size

        def dev(a, dtype):
            a = np.ascontiguousarray(a)
            if not a.flags.writeable:      # a read-only memmap view: stage through a host copy
                a = a.copy()
            return torch.from_numpy(a).to(device=device, dtype=dtype)

        def fused(names, layer):
            qs, ss = zip(*(m.quant(n, layer) for n in names))
            return (dev(np.concatenate(qs, axis=0), torch.int8),
                    dev(np.concatenate(ss), torch.float32))

        L = cfg.layer_num
        w = {"qkv": [fused(("wq", "wk", "wv"), l) for l in range(L)],
             "o": [fused(("wo",), l) for l in range(L)],
             "gu": [fused(("w1", "w3"), l) for l in range(L)],
             "down": [fused(("w2",), l) for l in range(L)],
             "cls": fused(("cls",), 0),
             "emb": dev(m.fp32("embedding"), torch.float32),
             "norm": [dev(m.fp32("rmsnorm", i).reshape(-1), torch.float32)
                      for i in range(2 * L + 1)]}
        return cls(cfg, w, gs, max_seq, device, fused)

    @classmethod
    def random(cls, cfg: ModelConfig, max_seq: int, group_size: int = 64, seed: int = 0,
               w_std: float = 0.02, device="cuda", fused: bool = True) -> "Int8Decoder":
        """Random-init model on the device: projections ~ N(0, w_std) quantised per group by
        sq8_quantize (bit-identical to the model-file quantiser), embedding ~ N(0, 1), unit norms."""
        import torch
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        d, kv, h, L = cfg.dim, cfg.kv_dim, cfg.hidden_dim, cfg.layer_num

        def qmat(rows, cols):
            wf = torch.randn((rows, cols), generator=gen, dtype=torch.float32, device=device)
            wf.mul_(w_std)
            q = torch.empty((rows, cols), dtype=torch.int8, device=device)
            s = torch.empty(rows * cols // group_size, dtype=torch.float32, device=device)
            quantize(wf, q, s, group_size)
            del wf
            return q, s

        w = {"qkv": [qmat(d + 2 * kv, d) for _ in range(L)],
             "o": [qmat(d, d) for _ in range(L)],
             "gu": [qmat(2 * h, d) for _ in range(L)],
             "down": [qmat(d, h) for _ in range(L)],
             "cls": qmat(cfg.vocab, d),
             "emb": torch.randn((cfg.vocab, d), generator=gen, dtype=torch.float32, device=device),
             "norm": [torch.ones(d, dtype=torch.float32, device=device) for _ in range(2 * L + 1)]}
        torch.cuda.synchronize()
        return cls(cfg, w, group_size, max_seq, device, fused)

    def weight_bytes(self) -> int:
        """Bytes of weights one decode step reads (int8 + scales of every projection)."""
        total = 0
        for key in ("qkv", "o", "gu", "down"):
            for q, s in self.w[key]:
                total += q.numel() + 4 * s.numel()
        q, s = self.w["cls"]
        return total + q.numel() + 4 * s.numel()

    # ------------------------------------------------------------------ one step
    def _mm(self, x, qs, y, stream):
        q, s = qs
        matmul(x, q, s, y, group_size=self.gs, workspace=self.ws, stream=stream)

    def _launch_step(self, stream, want_logits: bool = True):
        if self.fused:
            self._launch_step_fused(stream, want_logits)
        else:
            self._launch_step_plain(stream, want_logits)

    def _mm_norm(self, x, res, x_out, norm, qs, y, stream):
        q, s = qs
        matmul_rmsnorm(x, res, x_out, norm, q, s, y, self.gs, EPS, stream=stream)

    def _launch_step_fused(self, stream, want_logits: bool):
        """A prompt step (want_logits False) embeds self.token itself; a decode step starts from
        self.x, which the previous step's sq8_argmax_advance (or begin_decode) filled."""
        cfg = self.cfg
        L, d, kv = cfg.layer_num, cfg.dim, self.kv_dim
        w = self.w
        cur, other = self.x, self.x2
        if not want_logits:
            embedding(w["emb"], self.token, cur, stream=stream)
        for l in range(L):
            if l == 0:
                self._mm_norm(cur, None, None, w["norm"][0], w["qkv"][0], self.qkv, stream)
            else:
                self._mm_norm(cur, self.proj, other, w["norm"][l], w["qkv"][l], self.qkv, stream)
                cur, other = other, cur
            rope_attention_decode(self.qkv, cfg.head_num, cfg.kv_head_num, self.hs, self.pos,
                                  self.sin, self.cos, self.kcache[l], self.vcache[l], self.att,
                                  self.max_seq, workspace=self.att_ws, stream=stream)
            self._mm(self.att, w["o"][l], self.proj, stream)
            q, s = w["gu"][l]
            matmul_rmsnorm_swiglu(cur, self.proj, other, w["norm"][L + l], q, s, self.hid,
                                  self.gs, EPS, stream=stream)
            cur, other = other, cur
            self._mm(self.hid, w["down"][l], self.proj, stream)
        if want_logits:
            self._mm_norm(cur, self.proj, None, w["norm"][2 * L], w["cls"], self.logits, stream)
            argmax_advance(self.logits, self.pos, self.token, w["emb"], self.x, self.argmax_ws,
                           stream=stream)
        else:
            step_advance(self.pos, self.token, self.token, stream=stream)

    def begin_decode(self, stream=None):
        """Embed self.token into the first step's input (the fused decode step does not embed:
        sq8_argmax_advance leaves the next token's row in place)."""
        if self.fused:
            embedding(self.w["emb"], self.token, self.x, stream=stream)

    def _launch_step_plain(self, stream, want_logits: bool):
        """Enqueue one token: reads self.token / self.pos, writes self.next (when want_logits)
        and advances pos (and token = next)."""
        cfg = self.cfg
        L, d, kv, h = cfg.layer_num, cfg.dim, self.kv_dim, cfg.hidden_dim
        w = self.w
        embedding(w["emb"], self.token, self.x, stream=stream)
        for l in range(L):
            if l == 0:
                rmsnorm(self.x, w["norm"][0], self.xn, EPS, stream=stream)
            else:  # residual of the previous FFN, then this layer's attention norm
                add_rmsnorm(self.x, self.proj, w["norm"][l], self.xn, EPS, stream=stream)
            self._mm(self.xn, w["qkv"][l], self.qkv, stream)
            rope_kv(self.qkv, d, kv, self.hs, self.pos, self.sin, self.cos, self.kcache[l],
                    self.vcache[l], self.max_seq, stream=stream)
            attention_decode(self.qkv[:d], self.kcache[l], self.vcache[l], self.pos, self.att,
                             cfg.head_num, cfg.kv_head_num, self.hs, self.max_seq, stream=stream)
            self._mm(self.att, w["o"][l], self.proj, stream)
            add_rmsnorm(self.x, self.proj, w["norm"][L + l], self.xn, EPS, stream=stream)
            self._mm(self.xn, w["gu"][l], self.gu, stream)
            swiglu(self.gu[:h], self.gu[h:], self.hid, stream=stream)
            self._mm(self.hid, w["down"][l], self.proj, stream)
        if want_logits:
            add_rmsnorm(self.x, self.proj, w["norm"][2 * L], self.xn, EPS, stream=stream)
            self._mm(self.xn, w["cls"], self.logits, stream)
            argmax(self.logits, self.next, workspace=self.argmax_ws, stream=stream)
            step_advance(self.pos, self.token, self.next, stream=stream)
        else:
            # A prompt token: the residual stream of the last layer is not needed further.
            step_advance(self.pos, self.token, self.token, stream=stream)

    def reset(self):
        self.pos.zero_()
        self.kcache.zero_()
        self.vcache.zero_()

    def capture(self):
        """Capture one logits-producing step into a HIP graph (replayed by generate). Capturing
        records the launches without running them, so the decoder's state is unchanged."""
        torch = self.torch
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            self._launch_step(s, want_logits=True)
        self.graph = g
        self.graph_stream = s

    def generate(self, prompt, n_new: int, use_graph: bool = True):
        """Greedy generation: prompt tokens one per step without logits, then n_new tokens, each
        fed back on the device. Returns the generated token ids."""
        torch = self.torch
        self.reset()
        stream = torch.cuda.current_stream()
        for t in prompt[:-1]:
            self.token.fill_(int(t))
            self._launch_step(stream, want_logits=False)
        self.token.fill_(int(prompt[-1]))
        out = torch.empty(n_new, dtype=torch.int32, device=self.device)
        if use_graph and self.graph is None:
            self.capture()
        self.begin_decode(stream)
        for i in range(n_new):
            if use_graph:
                self.graph.replay()
            else:
                self._launch_step(stream, want_logits=True)
            out[i:i + 1].copy_(self.token)  # token == next after the advance
        torch.cuda.synchronize()
        return out.cpu().tolist()
