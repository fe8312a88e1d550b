"""CPU pins of the decode-step oracle (oracle/decode_oracle.py): each restated operator against a
closed form or a case small enough to work out by hand, chosen so that a plausible slip (wrong
RoPE pairing or table column, a missing 1/sqrt(head_size), a dropped epsilon, a transposed
projection, a non-causal prefill) fails one of them."""
import importlib
import math

import numpy as np
import pytest

from conftest import load_pkg
from oracle import decode_oracle as do

load_pkg()
mf = importlib.import_module("llm_steadyinfer_amd.model_file")


def test_rmsnorm_closed_forms():
    # A constant row c: mean(x^2) = c^2, so the result is c / sqrt(c^2 + eps) * w.
    w = np.array([1.0, 2.0, -0.5, 3.0])
    for c in (3.0, -0.25, 1e-4):
        got = do.rmsnorm(np.full(4, c), w)
        np.testing.assert_allclose(got, c / math.sqrt(c * c + 1e-6) * w, rtol=1e-15)
    # [3, 4]: mean square 12.5; the epsilon is inside the square root.
    got = do.rmsnorm(np.array([3.0, 4.0]), np.ones(2), eps=0.5)
    np.testing.assert_allclose(got, np.array([3.0, 4.0]) / math.sqrt(13.0), rtol=1e-15)
    # Rows are normalised independently.
    x = np.array([[1.0, 1.0], [2.0, 0.0]])
    np.testing.assert_allclose(do.rmsnorm(x, np.ones(2), eps=0.0),
                               [[1.0, 1.0], [math.sqrt(2.0), 0.0]], rtol=1e-15)


def test_rope_tables_closed_form():
    s, c = do.rope_tables(4, 3, 10000.0)
    # angle[pos][j] = pos / theta^(j / head_size): columns 0..3 at pos 2 are 2, 2/10, 2/100, 2/1000
    for j, ang in enumerate((2.0, 0.2, 0.02, 0.002)):
        assert s[2, j] == pytest.approx(math.sin(ang), rel=1e-14)
        assert c[2, j] == pytest.approx(math.cos(ang), rel=1e-14)
    assert np.all(s[0] == 0) and np.all(c[0] == 1)


def test_rope_hand_case_and_invariants():
    sin, cos = do.rope_tables(4, 4, 10000.0)
    v = np.array([1.0, 2.0, 3.0, 4.0])
    got = do.rope(v, 1, 4, 1, sin, cos)
    # head_size 4: pairs (0, 2) and (1, 3); pair i takes table column 2i, i.e. angles 1 and 0.01
    a, b = 1.0, 0.01
    want = [math.cos(a) * 1 - math.sin(a) * 3, math.cos(b) * 2 - math.sin(b) * 4,
            math.cos(a) * 3 + math.sin(a) * 1, math.cos(b) * 4 + math.sin(b) * 2]
    np.testing.assert_allclose(got, want, rtol=1e-14)
    rng = np.random.default_rng(3)
    s8, c8 = do.rope_tables(8, 50, 1e6)
    x = rng.standard_normal(3 * 8)
    np.testing.assert_array_equal(do.rope(x, 3, 8, 0, s8, c8), x)  # position 0: identity
    for p in (1, 17, 49):
        y = do.rope(x, 3, 8, p, s8, c8)
        for h in range(3):  # each head's norm, and each rotated pair's, is preserved
            xh, yh = x[8 * h:8 * h + 8], y[8 * h:8 * h + 8]
            np.testing.assert_allclose(np.hypot(yh[:4], yh[4:]), np.hypot(xh[:4], xh[4:]),
                                       rtol=1e-13)
    # Rotations compose: the score of q at p and k at p' depends on p - p' only.
    q, k = rng.standard_normal(8), rng.standard_normal(8)
    d1 = do.rope(q, 1, 8, 30, s8, c8) @ do.rope(k, 1, 8, 20, s8, c8)
    d2 = do.rope(q, 1, 8, 12, s8, c8) @ do.rope(k, 1, 8, 2, s8, c8)
    assert d1 == pytest.approx(d2, rel=1e-12)


def test_attention_closed_forms():
    rng = np.random.default_rng(4)
    H, KV, hs = 4, 2, 8
    K = rng.standard_normal((5, KV * hs))
    V = rng.standard_normal((5, KV * hs))
    q = rng.standard_normal(H * hs)
    # One position: every head returns its kv head's value row.
    out = do.attention(q, K, V, 0, H, KV, hs).reshape(H, hs)
    for h in range(H):
        g = h * KV // H
        np.testing.assert_allclose(out[h], V[0, g * hs:(g + 1) * hs], rtol=1e-15)
    # Equal scores (q = 0): the mean of the value rows 0..pos.
    out = do.attention(np.zeros(H * hs), K, V, 3, H, KV, hs).reshape(H, hs)
    for h in range(H):
        g = h * KV // H
        np.testing.assert_allclose(out[h], V[:4, g * hs:(g + 1) * hs].mean(0), rtol=1e-14)
    # Two positions: weights are the softmax of q.k / sqrt(hs) (the scale matters).
    H1, hs1 = 1, 4
    K2 = np.array([[1.0, 0, 0, 0], [0, 0, 0, 0]])
    V2 = np.array([[1.0, 0, 0, 0], [0, 1.0, 0, 0]])
    q1 = np.array([2.0, 0, 0, 0])  # scores 2/2 = 1 and 0
    w1 = math.e / (math.e + 1)
    np.testing.assert_allclose(do.attention(q1, K2, V2, 1, H1, H1, hs1), [w1, 1 - w1, 0, 0],
                               rtol=1e-15)
    # Causal block form equals one attention() per position.
    Kc = rng.standard_normal((9, KV * hs))
    Vc = rng.standard_normal((9, KV * hs))
    Q = rng.standard_normal((4, H * hs))
    blk = do.attention_causal(Q, Kc, Vc, 5, H, KV, hs)
    for i in range(4):
        np.testing.assert_allclose(blk[i], do.attention(Q[i], Kc, Vc, 5 + i, H, KV, hs),
                                   rtol=1e-13)


def test_swiglu_known_values():
    assert do.swiglu(0.0, 5.0) == 0.0                      # silu(0) = 0
    assert do.swiglu(1.0, 1.0) == pytest.approx(1 / (1 + math.exp(-1)), rel=1e-15)
    assert do.swiglu(40.0, 2.0) == pytest.approx(80.0, rel=1e-15)   # silu(a) -> a
    assert abs(do.swiglu(-40.0, 2.0)) < 1e-15                         # silu(a) -> 0
    assert do.swiglu(-1.0, 3.0) == pytest.approx(-3 / (1 + math.e), rel=1e-15)


def test_argmax_first_and_dequant():
    assert do.argmax_first([1.0, 3.0, 3.0, 2.0]) == 1
    q = np.array([[1, -2, 127, 0], [5, 5, -127, 3]], np.int8)
    s = np.array([0.5, 2.0, 0.25, 1.0], np.float32)  # group size 2: flat groups of 2
    np.testing.assert_array_equal(do.dequant(q, s, 2), [[0.5, -1.0, 254.0, 0.0],
                                                        [1.25, 1.25, -127.0, 3.0]])


def test_prefill_equals_steps(tmp_path):
    """The batched prompt pass leaves the same caches and the same next-step logits as one
    step() per position."""
    cfg = mf.ModelConfig(dim=64, hidden_dim=96, layer_num=2, head_num=4, kv_head_num=2,
                         vocab_size=-50, seq_len=32, rope_theta=1e4)
    path = mf.write_random(tmp_path / "m.bin", cfg, 32, seed=9, w_std=0.2)
    prompt = np.random.default_rng(9).integers(0, 50, 13).tolist()
    a = do.DecodeModel(mf.ModelFile(path), max_seq=32)
    b = do.DecodeModel(mf.ModelFile(path), max_seq=32)
    for p, t in enumerate(prompt[:-1]):
        a.step(t, p, want_logits=False)
    b.prefill(prompt[:5])
    b.prefill(prompt[5:-1], pos0=5)   # a second chunk attends to the first
    np.testing.assert_allclose(b.K, a.K, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(b.V, a.V, rtol=1e-12, atol=1e-12)
    la = a.step(prompt[-1], len(prompt) - 1)
    lb = b.step(prompt[-1], len(prompt) - 1)
    np.testing.assert_allclose(lb, la, rtol=1e-12, atol=1e-12)
    ta, _ = do.DecodeModel(mf.ModelFile(path), 32).generate(prompt, 4)
    tb, _ = do.DecodeModel(mf.ModelFile(path), 32).generate(prompt, 4, batched_prompt=True)
    assert ta == tb


def test_decode_step_tiny_by_hand():
    """One layer, dim 2, one head: the whole step written out with scalars (embedding row,
    RMSNorm, q/k/v, RoPE at position 0 = identity, attention over one position = v, O, FFN)."""
    class M:
        pass
    m = M()
    m.config = mf.ModelConfig(dim=2, hidden_dim=2, layer_num=1, head_num=1, kv_head_num=1,
                              vocab_size=-3, seq_len=4, rope_theta=1e4)
    m.group_size = 2
    eye = (np.array([[1, 0], [0, 1]], np.int8), np.array([1.0, 1.0], np.float32))
    swap = (np.array([[0, 1], [1, 0]], np.int8), np.array([1.0, 1.0], np.float32))
    quant = {"wq": eye, "wk": eye, "wv": swap, "wo": eye, "w1": eye, "w3": eye, "w2": eye,
             "cls": (np.array([[1, 0], [0, 1], [1, 1]], np.int8),
                     np.array([1.0, 1.0, 1.0], np.float32))}
    m.quant = lambda name, layer=0: quant[name]
    emb = np.array([[3.0, 4.0], [0, 0], [0, 0]], np.float32)
    m.fp32 = lambda name, i=0: emb if name == "embedding" else np.ones((1, 2), np.float32)
    d = do.DecodeModel(m, max_seq=4)
    lg = d.step(0, 0)
    x = np.array([3.0, 4.0])
    xn = x / math.sqrt(12.5 + 1e-6)
    x = x + xn[::-1]                      # attention over one position returns v = swap(xn)
    xn2 = x / math.sqrt(np.mean(x * x) + 1e-6)
    x = x + xn2 / (1 + np.exp(-xn2)) * xn2
    xf = x / math.sqrt(np.mean(x * x) + 1e-6)
    np.testing.assert_allclose(lg, [xf[0], xf[1], xf[0] + xf[1]], rtol=1e-13)
