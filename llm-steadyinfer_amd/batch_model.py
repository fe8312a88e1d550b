"""Batched forward over a paged KV cache on gfx950: the reference's forward_batch
(src/source/model/llama3.cpp:996-1194) for rows of many sequences, each at its own position, as
the continuous-batching scheduler (scheduler.py) hands them over. Every launch goes to
libsq8.so (the INT8 matmul, include/sq8_decode.h and include/sq8_batch.h); torch supplies
device memory only.

Per step, for the B rows (decode rows first):
    embedding -> per layer: [add +] RMSNorm (rows) -> fused QKV matmul (M = B) ->
    paged RoPE + KV write (every row's k, v at its position) -> paged attention (row r over
    positions 0 .. pos[r] of its sequence) -> O matmul -> add + RMSNorm -> fused gate/up matmul ->
    SwiGLU (rows) -> down matmul
    -> add + final RMSNorm -> classifier matmul on the decode rows only -> argmax per row.
Where the matmul kernel for B rows fuses epilogues (the prefill GEMM, sq8_epilogue_fused), the
residual adds run in the O and down matmuls' output stage (in place on the residual stream x,
followed by a plain RMSNorm) and the SwiGLU in the gate/up matmul's, as
sq8_matmul_epilogue does.

All rows write their KV before any row attends, so prefill rows of one sequence in the same step
see each other causally.

A decode-only step (every row a decode row) launches the same kernels for the same row count B
every time: its inputs (tokens, positions, block tables) live in fixed device buffers. The first
such step at each B runs eagerly and then captures the launch sequence into a HIP graph; later
decode-only steps at that B replay it (one launch instead of ~15 per layer), the way the
reference captures its decode steps (src/source/model/model.cpp:189-238). The matmul workspace is
sized for every row count up front, so no later step can move a buffer a graph points to. The KV pool is [layers][num_blocks][block_size][kv_dim] fp32 for keys
and for values (KVManager's paged layout, src/source/scheduler/kv_manager.cpp).

With packed=True the projections are repacked once at start-up into the matrix-core kernels'
load order (sq8_pack_weights: each 16-row tile's 64-wide groups as contiguous 1 KiB blocks) and
every matmul takes the _packed entry points; the model then holds only the packed copies.
"""
from __future__ import annotations

from typing import List

import numpy as np

from . import (SQ8_EPI_NONE, SQ8_EPI_RESIDUAL, SQ8_EPI_SWIGLU, Workspace, add_rmsnorm,
               argmax_rows, embedding, epilogue_fused, lib, matmul, matmul_epilogue,
               matmul_rmsnorm_rows, pack_weights,
               paged_attention, paged_attention_workspace_bytes, paged_rope_kv, rmsnorm,
               rope_tables, swiglu_rows)

EPS = 1e-6


class PagedBatchModel:
    def __init__(self, cfg, weights: dict, group_size: int, max_rows: int, max_seq_len: int,
                 num_blocks: int, block_size: int, device="cuda", use_graphs: bool = True,
                 split_kv: bool = True, fuse_norm: bool = True, packed: bool = False):
        import torch
        self.torch = torch
        self.packed = packed
        if packed:  # one repack per projection at start-up; the model keeps only these copies
            weights = dict(weights)
            for key in ("qkv", "o", "gu", "down"):
                weights[key] = [(pack_weights(q), s) for q, s in weights[key]]
            weights["cls"] = (pack_weights(weights["cls"][0]), weights["cls"][1])
        self.cfg, self.w, self.gs = cfg, weights, group_size
        self.max_rows, self.block_size = max_rows, block_size
        self.max_blocks_per_seq = (max_seq_len + block_size - 1) // block_size
        self.hs = cfg.dim // cfg.head_num
        L, d, kv, h = cfg.layer_num, cfg.dim, cfg.kv_dim, cfg.hidden_dim
        f32 = dict(dtype=torch.float32, device=device)
        i32 = dict(dtype=torch.int32, device=device)
        self.kcache = torch.zeros((L, num_blocks, block_size, kv), **f32)
        self.vcache = torch.zeros((L, num_blocks, block_size, kv), **f32)
        self.sin = torch.empty((max_seq_len, self.hs), **f32)
        self.cos = torch.empty((max_seq_len, self.hs), **f32)
        rope_tables(self.sin, self.cos, self.hs, max_seq_len, float(cfg.rope_theta))
        R = max_rows
        self.x = torch.zeros((R, d), **f32)
        self.xn = torch.zeros((R, d), **f32)
        self.qkv = torch.zeros((R, d + 2 * kv), **f32)
        self.att = torch.zeros((R, d), **f32)
        self.proj = torch.zeros((R, d), **f32)
        self.gu = torch.zeros((R, 2 * h), **f32)
        self.hid = torch.zeros((R, h), **f32)
        self.logits = torch.zeros((R, cfg.vocab), **f32)
        self.tok = torch.zeros(R, **i32)
        self.pos = torch.zeros(R, **i32)
        self.table = torch.zeros((R, self.max_blocks_per_seq), **i32)
        self.next = torch.zeros(R, **i32)
        self.ws = Workspace(device)
        self.rows_run = 0
        self._fuse = {}
        self.use_graphs = use_graphs
        self.fuse_norm = fuse_norm
        self.graphs = {}
        self.graph_replays = 0
        # Workspace for every row count and projection, allocated once (graphs keep its address).
        need = 0
        for B in range(1, R + 1):
            for (N, K) in ((d + 2 * kv, d), (d, d), (2 * h, d), (d, h), (cfg.vocab, d)):
                for epi in (SQ8_EPI_NONE, SQ8_EPI_RESIDUAL, SQ8_EPI_SWIGLU):
                    if packed:
                        need = max(need, int(lib().sq8_epilogue_packed_workspace_bytes(
                            B, N, K, group_size, epi)))
                        if epi != SQ8_EPI_RESIDUAL:
                            need = max(need, int(lib().sq8_rmsnorm_rows_packed_workspace_bytes(
                                B, N, K, group_size, epi)))
                        continue
                    need = max(need, int(lib().sq8_epilogue_workspace_bytes(B, N, K, group_size,
                                                                            epi)))
                    if epi != SQ8_EPI_RESIDUAL:
                        need = max(need, int(lib().sq8_rmsnorm_rows_workspace_bytes(
                            B, N, K, group_size, epi)))
        self.ws.get(need)
        # Split-KV attention workspace (zero-filled once; each call leaves its tickets zero).
        att_need = paged_attention_workspace_bytes(R, cfg.head_num, cfg.kv_head_num, self.hs,
                                                   self.max_blocks_per_seq, block_size)
        self.att_ws = (torch.zeros((att_need + 3) // 4, **i32) if split_kv and att_need > 0
                       else None)

    @classmethod
    def from_decoder(cls, dec, max_rows: int, max_seq_len: int, num_blocks: int,
                     block_size: int, use_graphs: bool = True, split_kv: bool = True,
                     fuse_norm: bool = True, packed: bool = False) -> "PagedBatchModel":
        """Share the fused weights of an Int8Decoder (model file or random init); with packed
        the model holds packed copies of the projections instead (sq8_pack_weights)."""
        return cls(dec.cfg, dec.w, dec.gs, max_rows, max_seq_len, num_blocks, block_size,
                   dec.device, use_graphs=use_graphs, split_kv=split_kv, fuse_norm=fuse_norm,
                   packed=packed)

    def kv_bytes_per_position(self) -> int:
        return 2 * 4 * self.cfg.layer_num * self.cfg.kv_dim

    def _mm(self, x, qs, y, stream):
        q, s = qs
        matmul(x, q, s, y, group_size=self.gs, workspace=self.ws, stream=stream)

    def _mm_epi(self, x, qs, y, epilogue, stream, residual=None):
        q, s = qs
        matmul_epilogue(x, q, s, y, epilogue, residual=residual, group_size=self.gs,
                        workspace=self.ws, stream=stream)

    def _mm_norm(self, x, res, norm_w, qs, y, epilogue, xn, stream):
        """y = epilogue(rmsnorm(x + res) * norm_w . W^T), x += res. With fuse_norm the norm is
        formed inside the matmul's launches (sq8_matmul_rmsnorm_rows); otherwise through xn."""
        q, s = qs
        if self.fuse_norm:
            matmul_rmsnorm_rows(x, res, norm_w, EPS, q, s, y, epilogue, group_size=self.gs,
                                workspace=self.ws, stream=stream)
            return
        if res is not None:
            add_rmsnorm(x, res, norm_w, xn, EPS, stream=stream)
        else:
            rmsnorm(x, norm_w, xn, EPS, stream=stream)
        if epilogue == SQ8_EPI_NONE:
            self._mm(xn, qs, y, stream)
        else:
            self._mm_epi(xn, qs, y, epilogue, stream)

    def fused(self, B: int):
        """(O, gate/up, down) epilogues fused at B rows."""
        if B not in self._fuse:
            cfg, gs = self.cfg, self.gs
            d, h = cfg.dim, cfg.hidden_dim
            pk = self.packed
            self._fuse[B] = (epilogue_fused(B, d, d, gs, pk), epilogue_fused(B, 2 * h, d, gs, pk),
                             epilogue_fused(B, d, h, gs, pk))
        return self._fuse[B]

    def forward(self, rows, tables: List[List[int]]) -> List[int]:
        """Run the batch rows (scheduler.BatchRow, decode rows first) and return the greedy token
        of each decode row."""
        B = len(rows)
        nd = sum(1 for r in rows if r.is_decode)
        if any(r.is_decode for r in rows[nd:]):
            raise ValueError("decode rows must come first")
        tok = np.fromiter((r.token for r in rows), np.int32, B)
        pos = np.fromiter((r.position for r in rows), np.int32, B)
        return self.forward_arrays(tok, pos, np.asarray(tables, np.int32).reshape(B, -1), nd)

    def forward_arrays(self, tok, pos, tab, nd: int) -> List[int]:
        """The same step from int32 arrays: tokens and positions [B], block tables
        [B][max_blocks_per_seq]; the first nd rows are the decode rows (the native scheduler's
        callback hands its rows over this way)."""
        torch = self.torch
        B = len(tok)
        if B == 0 or B > self.max_rows:
            raise ValueError(f"{B} rows for a model sized for {self.max_rows}")
        if len(pos) != B or tab.shape[0] != B or not 0 <= nd <= B:
            raise ValueError("rows, positions, tables and decode count disagree")
        if tab.shape[1] != self.max_blocks_per_seq:
            raise ValueError("block-table width does not match max_seq_len / block_size")
        tok = np.ascontiguousarray(tok, np.int32)
        pos = np.ascontiguousarray(pos, np.int32)
        tab = np.ascontiguousarray(tab, np.int32)
        self.tok[:B].copy_(torch.from_numpy(tok))
        self.pos[:B].copy_(torch.from_numpy(pos))
        self.table[:B].copy_(torch.from_numpy(tab))
        stream = torch.cuda.current_stream()
        graph = self.graphs.get(B) if self.use_graphs and nd == B else None
        if graph is not None:
            graph.replay()
            self.graph_replays += 1
        else:
            self.launch(B, nd, stream)
            if self.use_graphs and nd == B:
                self._capture(B)
        self.rows_run += B
        if nd == 0:
            return []
        return self.next[:nd].cpu().tolist()

    def capture_decode_graphs(self, rows=None) -> float:
        """Capture the decode-only step graphs for the given row counts (default 1..max_rows) up
        front, as a server does at start-up, instead of at the first decode-only step of each
        row count. Each capture follows one eager run on placeholder rows (token 0 at position 0
        of physical block 0), which writes K/V into block 0 of every layer: it is refused once a
        step has run (a sequence may then hold that block). Returns the seconds spent."""
        import time
        if self.rows_run:
            raise RuntimeError("capture_decode_graphs after a forward step would overwrite the "
                               "KV cache of block 0; capture before the first step")
        torch = self.torch
        t0 = time.perf_counter()
        for B in (rows if rows is not None else range(1, self.max_rows + 1)):
            if B in self.graphs:
                continue
            self.tok[:B].zero_()
            self.pos[:B].zero_()
            self.table[:B].zero_()
            self.launch(B, B, torch.cuda.current_stream())
            self._capture(B)
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    def _capture(self, B: int) -> None:
        """Capture the decode-only step at B rows (after one eager run at B)."""
        torch = self.torch
        s = torch.cuda.Stream(device=self.x.device)
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            self.launch(B, B, s)
        torch.cuda.current_stream().wait_stream(s)
        self.graphs[B] = g

    def launch(self, B: int, nd: int, stream) -> None:
        """Enqueue the forward of the first B staged rows (tokens, positions and block tables in
        self.tok / self.pos / self.table); writes the greedy tokens of the first nd rows to
        self.next."""
        cfg, w = self.cfg, self.w
        L, d, kv = cfg.layer_num, cfg.dim, cfg.kv_dim
        x, xn, qkv, att = self.x[:B], self.xn[:B], self.qkv[:B], self.att[:B]
        proj, gu, hid = self.proj[:B], self.gu[:B], self.hid[:B]
        pos, table = self.pos[:B], self.table[:B]
        fuse_o, fuse_gu, fuse_down = self.fused(B)
        embedding(w["emb"], self.tok[:B], x, stream=stream)
        pending = False  # proj holds the FFN output still to be added to x
        for l in range(L):
            # residual of the previous FFN (if pending), this layer's attention norm, QKV
            self._mm_norm(x, proj if pending else None, w["norm"][l], w["qkv"][l], qkv,
                          SQ8_EPI_NONE, xn, stream)
            paged_rope_kv(qkv, cfg.head_num, cfg.kv_head_num, self.hs, pos, table,
                          self.block_size, self.sin, self.cos, self.kcache[l], self.vcache[l],
                          stream=stream)
            paged_attention(qkv, d + 2 * kv, cfg.head_num, cfg.kv_head_num, self.hs, pos, table,
                            self.block_size, self.kcache[l], self.vcache[l], att,
                            workspace=self.att_ws, stream=stream)
            if fuse_o:
                self._mm_epi(att, w["o"][l], x, SQ8_EPI_RESIDUAL, stream, residual=x)
            else:
                self._mm(att, w["o"][l], proj, stream)
            gres = None if fuse_o else proj  # residual still to be added before the FFN norm
            if fuse_gu:
                self._mm_norm(x, gres, w["norm"][L + l], w["gu"][l], hid, SQ8_EPI_SWIGLU, xn,
                              stream)
            else:
                self._mm_norm(x, gres, w["norm"][L + l], w["gu"][l], gu, SQ8_EPI_NONE, xn,
                              stream)
                swiglu_rows(gu, hid, stream=stream)
            if fuse_down:
                self._mm_epi(hid, w["down"][l], x, SQ8_EPI_RESIDUAL, stream, residual=x)
                pending = False
            else:
                self._mm(hid, w["down"][l], proj, stream)
                pending = True
        if nd > 0:
            if pending:
                add_rmsnorm(self.x[:nd], self.proj[:nd], w["norm"][2 * L], self.xn[:nd], EPS,
                            stream=stream)
            else:
                rmsnorm(self.x[:nd], w["norm"][2 * L], self.xn[:nd], EPS, stream=stream)
            self._mm(self.xn[:nd], w["cls"], self.logits[:nd], stream)
            argmax_rows(self.logits[:nd], self.next[:nd], stream=stream)
