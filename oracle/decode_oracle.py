"""CPU restatement (numpy, float64) of the reference's single-token decode step.

TEST INFRASTRUCTURE ONLY: the checker for the HIP decode operators (include/sq8_decode.h) and for
greedy-token identity of the decoder. Only tests/ may import this module.

Each function restates one reference kernel; the whole-model step follows Qwen2Model's
single-token forward (src/source/model/qwen2.cpp:690-830), which LLamaModel shares
(src/source/model/llama3.cpp:705-818):
    x = embedding[token]
    per layer l: xn = rmsnorm(x, attn_norm[l]); q, k, v = xn Wq, xn Wk, xn Wv; rope(q, k, pos);
                 K[l][pos], V[l][pos] = k, v; a = attention(q, K[l], V[l], pos); x += a Wo;
                 xn = rmsnorm(x, ffn_norm[l]); x += (silu(xn W1) * (xn W3)) W2
    logits = rmsnorm(x, final_norm) Wcls; next = first argmax.
The quantised projections use the dequantised weights w * scale (each product formed in fp32 as
the reference kernel does, matmul_kernel.cu:85-88) and float64 sums.
"""
from __future__ import annotations

import numpy as np

EPS = 1e-6  # rmsnorm_kernel.cu:120,144


def rmsnorm(x, w, eps: float = EPS):
    """row_rmsnorm_f32 (rmsnorm_kernel.cu:63-110): x * rsqrt(mean(x^2) + eps) * w, per row."""
    x = np.asarray(x, np.float64)
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return x / np.sqrt(ms + eps) * np.asarray(w, np.float64)


def rope_tables(head_size: int, max_seq: int, theta: float):
    """sin_cos_calc (rope_kernel.cu:39-52): angle[pos][j] = pos / theta^(j / head_size)."""
    j = np.arange(head_size, dtype=np.float64)
    freq = 1.0 / np.power(float(theta), j / head_size)
    ang = np.arange(max_seq, dtype=np.float64)[:, None] * freq[None, :]
    return np.sin(ang), np.cos(ang)


def rope(vec, n_heads: int, head_size: int, pos: int, sin, cos):
    """rope_kernel_cu_fp32 (rope_kernel.cu:4-37): per head, pair (i, i + hs/2) rotates by the
    angle in table column 2i."""
    v = np.array(vec, np.float64).reshape(n_heads, head_size)
    half = head_size // 2
    i = np.arange(half)
    s, c = sin[pos, 2 * i], cos[pos, 2 * i]
    v0, v1 = v[:, :half].copy(), v[:, half:].copy()
    v[:, :half] = c * v0 - s * v1
    v[:, half:] = c * v1 + s * v0
    return v.reshape(-1)


def attention(q, kcache, vcache, pos: int, head_num: int, kv_head_num: int, head_size: int):
    """flash_decoding_kernel + combine (mha_kernel.cu:178-341): softmax(q.K / sqrt(hs)) . V over
    cache rows 0..pos, query head h reading kv head h * kv_head_num / head_num."""
    q = np.asarray(q, np.float64).reshape(head_num, head_size)
    out = np.empty((head_num, head_size))
    for h in range(head_num):
        g = h * kv_head_num // head_num
        k = np.asarray(kcache[:pos + 1, g * head_size:(g + 1) * head_size], np.float64)
        v = np.asarray(vcache[:pos + 1, g * head_size:(g + 1) * head_size], np.float64)
        s = k @ q[h] / np.sqrt(head_size)
        p = np.exp(s - s.max())
        out[h] = (p @ v) / p.sum()
    return out.reshape(-1)


def attention_causal(q, kcache, vcache, pos0: int, head_num: int, kv_head_num: int,
                     head_size: int):
    """attention() for T query rows at positions pos0 .. pos0+T-1 (q: [T, head_num*head_size]):
    row i attends to cache rows 0 .. pos0+i, the paged kernels' causal rule for prefill rows of
    one sequence (paged_kernels.cu:96-294)."""
    q = np.asarray(q, np.float64)
    T = q.shape[0]
    q = q.reshape(T, head_num, head_size)
    n = pos0 + T
    out = np.empty((T, head_num, head_size))
    mask = np.arange(n)[None, :] > (pos0 + np.arange(T))[:, None]
    for h in range(head_num):
        g = h * kv_head_num // head_num
        k = np.asarray(kcache[:n, g * head_size:(g + 1) * head_size], np.float64)
        v = np.asarray(vcache[:n, g * head_size:(g + 1) * head_size], np.float64)
        s = q[:, h] @ k.T / np.sqrt(head_size)
        s[mask] = -np.inf
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h] = (p @ v) / p.sum(axis=1, keepdims=True)
    return out.reshape(T, -1)


def swiglu(a, b):
    """swiglu_kernel_cu_fp32 (swiglu_kernel.cu:4-21): a * sigmoid(a) * b."""
    a = np.asarray(a, np.float64)
    return a / (1.0 + np.exp(-a)) * np.asarray(b, np.float64)


def argmax_first(logits) -> int:
    """ArgmaxSampler::sample (argmax_sampler.cpp:5-13): std::max_element, the first maximum."""
    return int(np.argmax(np.asarray(logits)))


def dequant(q, s, group_size: int):
    """w[n][k] = (float)q[n][k] * scale of its group, formed in fp32 (matmul_kernel.cu:85-88).
    Works through row blocks (whole groups) so the fp32 temporaries stay cache-sized."""
    q = np.asarray(q)
    s = np.asarray(s, np.float32)
    flat = q.reshape(-1)
    out = np.empty(flat.size, np.float64)
    step = group_size * 65536
    for a in range(0, flat.size, step):
        blk = flat[a:a + step].reshape(-1, group_size).astype(np.float32)
        g0 = a // group_size
        out[a:a + blk.size] = (blk * s[g0:g0 + blk.shape[0], None]).reshape(-1)
    return out.reshape(q.shape)


class DecodeModel:
    """The whole decode step on a model file read with llm-steadyinfer_amd/model_file.py."""

    def __init__(self, model_file, max_seq: int):
        self.m = model_file
        cfg = model_file.config
        self.cfg = cfg
        self.gs = model_file.group_size
        self.hs = cfg.dim // cfg.head_num
        self.max_seq = max_seq
        self.sin, self.cos = rope_tables(self.hs, max_seq, cfg.rope_theta)
        L = cfg.layer_num
        self.W = {(n, l): dequant(*model_file.quant(n, l), self.gs)
                  for n in ("wq", "wk", "wv", "wo", "w1", "w2", "w3") for l in range(L)}
        self.cls = dequant(*model_file.quant("cls"), self.gs)
        self.emb = np.asarray(model_file.fp32("embedding"), np.float64)
        self.norm = [np.asarray(model_file.fp32("rmsnorm", i), np.float64).reshape(-1)
                     for i in range(2 * L + 1)]
        self.K = np.zeros((L, max_seq, cfg.kv_dim))
        self.V = np.zeros((L, max_seq, cfg.kv_dim))

    def step(self, token: int, pos: int, want_logits: bool = True):
        cfg, L = self.cfg, self.cfg.layer_num
        x = self.emb[token].copy()
        for l in range(L):
            xn = rmsnorm(x, self.norm[l])
            q = self.W[("wq", l)] @ xn
            k = self.W[("wk", l)] @ xn
            v = self.W[("wv", l)] @ xn
            q = rope(q, cfg.head_num, self.hs, pos, self.sin, self.cos)
            k = rope(k, cfg.kv_head_num, self.hs, pos, self.sin, self.cos)
            self.K[l, pos], self.V[l, pos] = k, v
            a = attention(q, self.K[l], self.V[l], pos, cfg.head_num, cfg.kv_head_num, self.hs)
            x = x + self.W[("wo", l)] @ a
            xn = rmsnorm(x, self.norm[L + l])
            h = swiglu(self.W[("w1", l)] @ xn, self.W[("w3", l)] @ xn)
            x = x + self.W[("w2", l)] @ h
        if not want_logits:
            return None
        return self.cls @ rmsnorm(x, self.norm[2 * L])

    def prefill(self, tokens, pos0: int = 0):
        """Positions pos0 .. pos0+T-1 of tokens in one pass: the same per-position arithmetic as
        T calls of step(want_logits=False) (row-independent projections, norms and RoPE), with
        each position attending causally to cache rows 0..its own position. Matrix products over
        the T rows make long prompts affordable in float64."""
        cfg, L = self.cfg, self.cfg.layer_num
        T = len(tokens)
        if T == 0:
            return
        pos = np.arange(pos0, pos0 + T)
        x = self.emb[np.asarray(tokens, np.int64)].copy()
        hs, H, KV = self.hs, cfg.head_num, cfg.kv_head_num
        for l in range(L):
            xn = rmsnorm(x, self.norm[l])
            q = xn @ self.W[("wq", l)].T
            k = xn @ self.W[("wk", l)].T
            v = xn @ self.W[("wv", l)].T
            q = np.stack([rope(q[i], H, hs, p, self.sin, self.cos) for i, p in enumerate(pos)])
            k = np.stack([rope(k[i], KV, hs, p, self.sin, self.cos) for i, p in enumerate(pos)])
            self.K[l, pos0:pos0 + T], self.V[l, pos0:pos0 + T] = k, v
            a = attention_causal(q, self.K[l], self.V[l], pos0, H, KV, hs)
            x = x + a @ self.W[("wo", l)].T
            xn = rmsnorm(x, self.norm[L + l])
            h = swiglu(xn @ self.W[("w1", l)].T, xn @ self.W[("w3", l)].T)
            x = x + h @ self.W[("w2", l)].T

    def generate(self, prompt, n_new: int, batched_prompt: bool = False):
        """Prompt tokens one at a time without logits (or all at once through prefill() when
        batched_prompt), then greedy tokens (the reference's predict(is_prompt) loop). Returns
        the generated tokens and every step's logits."""
        pos = 0
        if batched_prompt:
            self.prefill([int(t) for t in prompt[:-1]])
            pos = len(prompt) - 1
        else:
            for t in prompt[:-1]:
                self.step(int(t), pos, want_logits=False)
                pos += 1
        tok = int(prompt[-1])
        out, logits = [], []
        for _ in range(n_new):
            lg = self.step(tok, pos)
            logits.append(lg)
            tok = argmax_first(lg)
            out.append(tok)
            pos += 1
        return out, logits
