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


def swiglu(a, b):
    """swiglu_kernel_cu_fp32 (swiglu_kernel.cu:4-21): a * sigmoid(a) * b."""
    a = np.asarray(a, np.float64)
    return a / (1.0 + np.exp(-a)) * np.asarray(b, np.float64)


def argmax_first(logits) -> int:
    """ArgmaxSampler::sample (argmax_sampler.cpp:5-13): std::max_element, the first maximum."""
    return int(np.argmax(np.asarray(logits)))


def dequant(q, s, group_size: int):
    """w[n][k] = (float)q[n][k] * scale of its group, formed in fp32 (matmul_kernel.cu:85-88)."""
    q = np.asarray(q)
    w = q.reshape(-1, group_size).astype(np.float32) * np.asarray(s, np.float32)[:, None]
    return w.reshape(q.shape).astype(np.float64)


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

    def generate(self, prompt, n_new: int):
        """Prompt tokens one at a time without logits, then greedy tokens (the reference's
        predict(is_prompt) loop). Returns the generated tokens and every step's logits."""
        pos = 0
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
