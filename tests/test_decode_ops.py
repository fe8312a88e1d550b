"""The decode operators of include/sq8_decode.h against the numpy restatement of the reference
kernels (oracle/decode_oracle.py). CPU tests cover argument validation only (no device work)."""
import numpy as np
import pytest

from oracle import decode_oracle as do
from oracle import sq8_oracle as o

FAKE = 0x1000  # never dereferenced: validation fails first


def test_decode_ops_reject_bad_arguments(sq8):
    L = sq8.lib()
    assert L.sq8_rmsnorm(None, FAKE, FAKE, 1, 8, 1e-6, None) == sq8.SQ8_ERR_NULL
    assert L.sq8_rmsnorm(FAKE, FAKE, FAKE, 0, 8, 1e-6, None) == sq8.SQ8_ERR_DIMS
    assert L.sq8_add_rmsnorm(FAKE, None, FAKE, FAKE, 1, 8, 1e-6, None) == sq8.SQ8_ERR_NULL
    assert L.sq8_rope_kv(FAKE, 96, 64, 64, FAKE, FAKE, FAKE, FAKE, FAKE, 16, None) == sq8.SQ8_ERR_DIMS
    assert L.sq8_rope_kv(FAKE, 128, 256, 64, FAKE, FAKE, FAKE, FAKE, FAKE, 16, None) == sq8.SQ8_ERR_DIMS
    assert L.sq8_attention_decode(FAKE, FAKE, FAKE, FAKE, FAKE, 6, 4, 64, 16, None) == sq8.SQ8_ERR_DIMS
    assert L.sq8_attention_decode(FAKE, FAKE, FAKE, FAKE, FAKE, 8, 2, 512, 16, None) == sq8.SQ8_ERR_DIMS
    assert L.sq8_attention_decode(FAKE, FAKE, FAKE, FAKE, FAKE, 8, 2, 64, 1 << 25, None) == sq8.SQ8_ERR_DIMS
    assert L.sq8_quantize(FAKE, 100, 64, FAKE, FAKE, None) == sq8.SQ8_ERR_GROUP
    assert L.sq8_argmax(FAKE, 0, FAKE, FAKE, 4096, None) == sq8.SQ8_ERR_DIMS
    assert L.sq8_argmax(FAKE, 5000, FAKE, FAKE, 8, None) == sq8.SQ8_ERR_WORKSPACE
    assert L.sq8_argmax_workspace_bytes(151936) == 256 + 38 * 8
    assert L.sq8_swiglu(FAKE, None, FAKE, 4, None) == sq8.SQ8_ERR_NULL
    assert L.sq8_embedding(FAKE, 0, 8, FAKE, 1, FAKE, None) == sq8.SQ8_ERR_DIMS
    assert L.sq8_step_advance(FAKE, None, FAKE, None) == sq8.SQ8_ERR_NULL
    assert L.sq8_matmul_rmsnorm(FAKE, None, None, None, 1e-6, FAKE, FAKE, FAKE, 8, 64, 64, None) == sq8.SQ8_ERR_NULL
    assert L.sq8_matmul_rmsnorm(FAKE, None, None, FAKE, 1e-6, FAKE, FAKE, FAKE, 8, 20000, 16, None) == sq8.SQ8_ERR_DIMS
    assert L.sq8_matmul_swiglu(FAKE, FAKE, FAKE, FAKE, 8, 96, 64, None) == sq8.SQ8_ERR_GROUP
    assert L.sq8_matmul_swiglu(FAKE + 4, FAKE, FAKE, FAKE, 8, 128, 64, None) == sq8.SQ8_ERR_DIMS
    assert L.sq8_matmul_rmsnorm_swiglu(FAKE, None, None, FAKE, 1e-6, FAKE, FAKE, FAKE, 7, 64, 64,
                                       None) == sq8.SQ8_ERR_DIMS   # odd N
    assert L.sq8_matmul_rmsnorm_swiglu(FAKE, None, None, None, 1e-6, FAKE, FAKE, FAKE, 8, 64, 64,
                                       None) == sq8.SQ8_ERR_NULL
    assert L.sq8_argmax_advance(FAKE, 8, FAKE, 4096, None, FAKE, FAKE, 8, 8, FAKE,
                                None) == sq8.SQ8_ERR_NULL
    assert L.sq8_argmax_advance(FAKE, 8, FAKE, 0, FAKE, FAKE, FAKE, 8, 8, FAKE,
                                None) == sq8.SQ8_ERR_WORKSPACE
    assert L.sq8_rope_attention_decode_ws(FAKE, 32, 8, 128, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                                          4096, FAKE, 16, None) == sq8.SQ8_ERR_WORKSPACE
    # the split: up to 16 chunks of a multiple of 64 positions, tickets then partials
    f = sq8.decode_attention_workspace_bytes
    assert f(32, 128, 64) == 0                      # one chunk: no split
    assert f(32, 128, 192) == 256 + 32 * 3 * 130 * 4
    assert f(32, 128, 8192) == 256 + 32 * 16 * 130 * 4
    assert f(100, 64, 1000) == 512 + 100 * 16 * 66 * 4


def _t(a, dev, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dtype is None else t.to(dtype)


def _close(got, ref, rtol, label):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    err = np.max(np.abs(got - ref)) / max(np.max(np.abs(ref)), 1e-30)
    print(f"{label}: max err / max |ref| = {err:.2e}")
    assert np.all(np.isfinite(got)) and err <= rtol, (label, err)


@pytest.mark.gpu
@pytest.mark.parametrize("rows,dim", [(1, 1536), (3, 4096), (2, 100)])
def test_rmsnorm_and_add_rmsnorm(sq8, dev, rows, dim):
    import torch
    rng = np.random.default_rng(rows + dim)
    x = rng.standard_normal((rows, dim)).astype(np.float32) * 3
    r = rng.standard_normal((rows, dim)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, dim).astype(np.float32)
    out = torch.empty((rows, dim), device=dev)
    sq8.rmsnorm(_t(x, dev), _t(w, dev), out)
    _close(out.cpu().numpy(), do.rmsnorm(x, w), 2e-6, "rmsnorm")
    xt = _t(x, dev)
    sq8.add_rmsnorm(xt, _t(r, dev), _t(w, dev), out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(xt.cpu().numpy(), x + r)
    _close(out.cpu().numpy(), do.rmsnorm(x + r, w), 2e-6, "add_rmsnorm")


@pytest.mark.gpu
@pytest.mark.parametrize("head_size,theta", [(64, 1e6), (128, 5e5)])
def test_rope_tables(sq8, dev, head_size, theta):
    import torch
    max_seq = 512
    sin = torch.empty((max_seq, head_size), device=dev)
    cos = torch.empty((max_seq, head_size), device=dev)
    sq8.rope_tables(sin, cos, head_size, max_seq, theta)
    s_ref, c_ref = do.rope_tables(head_size, max_seq, theta)
    # The angle is formed in fp32 (pos * freq), as the reference does: allow its rounding.
    tol = 1e-6 + 2e-7 * np.arange(max_seq)[:, None]
    assert np.all(np.abs(sin.cpu().numpy() - s_ref) <= tol)
    assert np.all(np.abs(cos.cpu().numpy() - c_ref) <= tol)


@pytest.mark.gpu
@pytest.mark.parametrize("heads,kv_heads,hs,pos", [(12, 2, 128, 0), (12, 2, 128, 37), (4, 4, 64, 200)])
def test_rope_kv_writes_cache(sq8, dev, heads, kv_heads, hs, pos):
    import torch
    dim, kv = heads * hs, kv_heads * hs
    max_seq = 256
    rng = np.random.default_rng(pos + hs)
    qkv = rng.standard_normal(dim + 2 * kv).astype(np.float32)
    sin = torch.empty((max_seq, hs), device=dev)
    cos = torch.empty((max_seq, hs), device=dev)
    sq8.rope_tables(sin, cos, hs, max_seq, 1e6)
    kc = torch.full((max_seq, kv), -7.0, device=dev)
    vc = torch.full((max_seq, kv), -7.0, device=dev)
    qt = _t(qkv, dev)
    sq8.rope_kv(qt, dim, kv, hs, _t(np.array([pos], np.int32), dev), sin, cos, kc, vc, max_seq)
    torch.cuda.synchronize()
    s_np, c_np = sin.cpu().numpy().astype(np.float64), cos.cpu().numpy().astype(np.float64)
    _close(qt[:dim].cpu().numpy(), do.rope(qkv[:dim], heads, hs, pos, s_np, c_np), 1e-6, "q")
    _close(kc[pos].cpu().numpy(), do.rope(qkv[dim:dim + kv], kv_heads, hs, pos, s_np, c_np), 1e-6, "k")
    np.testing.assert_array_equal(vc[pos].cpu().numpy(), qkv[dim + kv:])
    other = np.delete(np.arange(max_seq), pos)
    assert np.all(kc.cpu().numpy()[other] == -7.0) and np.all(vc.cpu().numpy()[other] == -7.0)


@pytest.mark.gpu
@pytest.mark.parametrize("heads,kv_heads,hs,pos", [(12, 2, 128, 0), (12, 2, 128, 191), (32, 8, 128, 700),
                                                   (4, 1, 64, 5)])
def test_attention_decode(sq8, dev, heads, kv_heads, hs, pos):
    import torch
    max_seq = 1024
    kv = kv_heads * hs
    rng = np.random.default_rng(pos * 3 + heads)
    q = rng.standard_normal(heads * hs).astype(np.float32)
    kc = rng.standard_normal((max_seq, kv)).astype(np.float32)
    vc = rng.standard_normal((max_seq, kv)).astype(np.float32)
    out = torch.empty(heads * hs, device=dev)
    sq8.attention_decode(_t(q, dev), _t(kc, dev), _t(vc, dev), _t(np.array([pos], np.int32), dev),
                         out, heads, kv_heads, hs, max_seq)
    _close(out.cpu().numpy(), do.attention(q, kc, vc, pos, heads, kv_heads, hs), 2e-6, "attention")


@pytest.mark.gpu
def test_swiglu_add_embedding(sq8, dev):
    import torch
    rng = np.random.default_rng(0)
    a = (rng.standard_normal(8960) * 4).astype(np.float32)
    b = rng.standard_normal(8960).astype(np.float32)
    out = torch.empty(8960, device=dev)
    sq8.swiglu(_t(a, dev), _t(b, dev), out)
    _close(out.cpu().numpy(), do.swiglu(a, b), 1e-6, "swiglu")
    x = _t(a, dev)
    sq8.add(x, _t(b, dev))
    np.testing.assert_array_equal(x.cpu().numpy(), a + b)
    table = rng.standard_normal((300, 96)).astype(np.float32)
    toks = np.array([5, 299, 0, 300, -1], np.int32)   # the last two are out of range
    emb = torch.full((5, 96), 3.0, device=dev)
    sq8.embedding(_t(table, dev), _t(toks, dev), emb)
    e = emb.cpu().numpy()
    np.testing.assert_array_equal(e[:3], table[[5, 299, 0]])
    assert np.all(e[3:] == 3.0)


@pytest.mark.gpu
def test_argmax_first_maximum(sq8, dev):
    import torch
    rng = np.random.default_rng(1)
    out = torch.empty(1, dtype=torch.int32, device=dev)
    for n in (1, 7, 1000, 151936):
        v = rng.standard_normal(n).astype(np.float32)
        sq8.argmax(_t(v, dev), out)
        assert int(out.item()) == do.argmax_first(v), n
    v = rng.standard_normal(151936).astype(np.float32)
    v[[90000, 1234, 151935]] = 50.0            # ties: the first index wins
    sq8.argmax(_t(v, dev), out)
    assert int(out.item()) == 1234
    v = np.full(5000, -np.inf, np.float32)
    sq8.argmax(_t(v, dev), out)
    assert int(out.item()) == 0


@pytest.mark.gpu
def test_device_quantiser_matches_oracle(sq8, dev):
    import torch
    rng = np.random.default_rng(2)
    w = (rng.standard_normal(64 * 4096) * 10.0 ** rng.uniform(-5, 5, 64 * 4096)).astype(np.float32)
    w[:64] = 0
    w[64:128] = np.float32(127.5) * np.arange(64, dtype=np.float32) / 63
    q = torch.empty(w.size, dtype=torch.int8, device=dev)
    s = torch.empty(w.size // 64, device=dev)
    sq8.quantize(_t(w, dev), q, s, 64)
    q2, s2 = o.quantize(w, 64)
    np.testing.assert_array_equal(q.cpu().numpy(), q2.reshape(-1))
    np.testing.assert_array_equal(s.cpu().numpy(), s2)


@pytest.mark.gpu
def test_step_advance(sq8, dev):
    import torch
    pos = torch.tensor([41], dtype=torch.int32, device=dev)
    tok = torch.tensor([3], dtype=torch.int32, device=dev)
    nxt = torch.tensor([977], dtype=torch.int32, device=dev)
    sq8.step_advance(pos, tok, nxt)
    assert int(pos.item()) == 42 and int(tok.item()) == 977


@pytest.mark.gpu
@pytest.mark.parametrize("N,K,with_res", [(2048, 1536, False), (17920, 1536, True), (151936, 1536, True),
                                          (6144, 4096, True), (96, 256, True)])
def test_matmul_rmsnorm_equals_separate_ops(sq8, dev, N, K, with_res):
    """The fused prologue gives the unfused add + RMSNorm + GEMV result (both against the oracle)
    and writes the residual stream once."""
    import torch
    rng = np.random.default_rng(N + K)
    x = (rng.standard_normal(K) * 2).astype(np.float32)
    r = rng.standard_normal(K).astype(np.float32)
    g = rng.uniform(0.5, 1.5, K).astype(np.float32)
    _, q, s = o.make_case(1, N, K, 64, seed=K)
    qt, st = _t(q, dev), _t(s, dev)
    y = torch.empty(N, device=dev)
    xo = torch.full((K,), 9.0, device=dev)
    sq8.matmul_rmsnorm(_t(x, dev), _t(r, dev) if with_res else None, xo, _t(g, dev), qt, st, y)
    xin = (x + r) if with_res else x
    xn = do.rmsnorm(xin, g).astype(np.float32)
    ref = o.matmul_f64(xn.reshape(1, -1), q, s, 64).reshape(-1)
    elem, norm = o.rel_errors(y.cpu().numpy().reshape(1, -1), ref.reshape(1, -1))
    print(f"fused norm N={N} K={K}: elem {elem:.2e} norm {norm:.2e}")
    assert elem <= 1e-3 and norm <= 1e-5
    np.testing.assert_array_equal(xo.cpu().numpy(), xin)


@pytest.mark.gpu
@pytest.mark.parametrize("N,K,with_res", [(17920, 1536, True), (28672, 4096, True),
                                          (28672, 4096, False), (96, 256, True), (8, 2048, True)])
def test_matmul_rmsnorm_swiglu_equals_separate_ops(sq8, dev, N, K, with_res):
    """Add + RMSNorm prologue, fused [w1; w3] GEMV and SwiGLU epilogue in one launch: against the
    oracle's rmsnorm, float64 matmul and swiglu; the residual stream is written once."""
    import torch
    rng = np.random.default_rng(N + 3 * K)
    x = (rng.standard_normal(K) * 2).astype(np.float32)
    r = rng.standard_normal(K).astype(np.float32)
    g = rng.uniform(0.5, 1.5, K).astype(np.float32)
    _, q, s = o.make_case(1, N, K, 64, seed=N + K)
    y = torch.full((N // 2,), float("nan"), device=dev)
    xo = torch.full((K,), 9.0, device=dev)
    sq8.matmul_rmsnorm_swiglu(_t(x, dev), _t(r, dev) if with_res else None, xo, _t(g, dev),
                              _t(q, dev), _t(s, dev), y)
    xin = (x + r) if with_res else x
    xn = do.rmsnorm(xin, g).astype(np.float32)
    gu = o.matmul_f64(xn.reshape(1, -1), q, s, 64).reshape(-1)
    ref = do.swiglu(gu[:N // 2], gu[N // 2:])
    elem, norm = o.rel_errors(y.cpu().numpy().reshape(1, -1), ref.reshape(1, -1))
    print(f"fused norm+swiglu N={N} K={K}: elem {elem:.2e} norm {norm:.2e}")
    assert elem <= 1e-3 and norm <= 1e-5
    np.testing.assert_array_equal(xo.cpu().numpy(), xin)


@pytest.mark.gpu
def test_argmax_advance(sq8, dev):
    """Argmax (first maximum), position advance and the winner's embedding row in one launch;
    the workspace is reused (its ticket is left zero)."""
    import torch
    rng = np.random.default_rng(11)
    vocab, dim = 5003, 96
    emb = rng.standard_normal((vocab, dim)).astype(np.float32)
    emb_t = _t(emb, dev)
    ws = sq8.Workspace(dev)
    pos = torch.tensor([17], dtype=torch.int32, device=dev)
    tok = torch.tensor([3], dtype=torch.int32, device=dev)
    x = torch.zeros(dim, device=dev)
    for i, n in enumerate((vocab, vocab, 4096, 7)):
        v = rng.standard_normal(n).astype(np.float32)
        if i == 1:
            v[[4000, 2500]] = 50.0            # tie: the first index wins
        sq8.argmax_advance(_t(v, dev), pos, tok, emb_t, x, ws)
        want = do.argmax_first(v)
        assert int(tok.item()) == want and int(pos.item()) == 18 + i
        np.testing.assert_array_equal(x.cpu().numpy(), emb[want])


@pytest.mark.gpu
@pytest.mark.parametrize("N,K", [(1536, 8960), (1001, 10240), (2048, 8256), (4096, 14336), (64, 1024)])
def test_matmul_swiglu_equals_separate_ops(sq8, dev, N, K):
    import torch
    rng = np.random.default_rng(K)
    ab = (rng.standard_normal(2 * K) * 3).astype(np.float32)
    _, q, s = o.make_case(1, N, K, 64, seed=N)
    y = torch.empty(N, device=dev)
    sq8.matmul_swiglu(_t(ab, dev), _t(q, dev), _t(s, dev), y)
    h = do.swiglu(ab[:K], ab[K:]).astype(np.float32)
    ref = o.matmul_f64(h.reshape(1, -1), q, s, 64)
    elem, norm = o.rel_errors(y.cpu().numpy().reshape(1, -1), ref)
    print(f"fused swiglu N={N} K={K}: elem {elem:.2e} norm {norm:.2e}")
    assert elem <= 1e-3 and norm <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("heads,kv_heads,hs,pos", [(12, 2, 128, 0), (12, 2, 128, 77), (32, 8, 128, 300),
                                                   (4, 4, 64, 9)])
def test_rope_attention_equals_separate_ops(sq8, dev, heads, kv_heads, hs, pos):
    """The fused launch writes the same cache row and returns the same output as sq8_rope_kv
    followed by sq8_attention_decode (both against the oracle)."""
    import torch
    max_seq = 512
    dim, kv = heads * hs, kv_heads * hs
    rng = np.random.default_rng(pos + heads)
    qkv = rng.standard_normal(dim + 2 * kv).astype(np.float32)
    kc0 = rng.standard_normal((max_seq, kv)).astype(np.float32)
    vc0 = rng.standard_normal((max_seq, kv)).astype(np.float32)
    sin = torch.empty((max_seq, hs), device=dev)
    cos = torch.empty((max_seq, hs), device=dev)
    sq8.rope_tables(sin, cos, hs, max_seq, 1e6)
    p = _t(np.array([pos], np.int32), dev)
    kc, vc, out = _t(kc0, dev), _t(vc0, dev), torch.empty(dim, device=dev)
    sq8.rope_attention_decode(_t(qkv, dev), heads, kv_heads, hs, p, sin, cos, kc, vc, out, max_seq)
    kc2, vc2, out2 = _t(kc0, dev), _t(vc0, dev), torch.empty(dim, device=dev)
    q2 = _t(qkv, dev)
    sq8.rope_kv(q2, dim, kv, hs, p, sin, cos, kc2, vc2, max_seq)
    sq8.attention_decode(q2[:dim], kc2, vc2, p, out2, heads, kv_heads, hs, max_seq)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(kc.cpu().numpy(), kc2.cpu().numpy())
    np.testing.assert_array_equal(vc.cpu().numpy(), vc2.cpu().numpy())
    s_np, c_np = sin.cpu().numpy().astype(np.float64), cos.cpu().numpy().astype(np.float64)
    qr = do.rope(qkv[:dim], heads, hs, pos, s_np, c_np)
    ref = do.attention(qr, kc2.cpu().numpy(), vc2.cpu().numpy(), pos, heads, kv_heads, hs)
    _close(out.cpu().numpy(), ref, 2e-6, "fused rope+attention")
    _close(out2.cpu().numpy(), ref, 2e-6, "separate")


@pytest.mark.gpu
@pytest.mark.parametrize("heads,kv_heads,hs,max_seq", [(32, 8, 128, 192), (12, 2, 128, 4096),
                                                       (4, 4, 64, 1000), (14, 2, 256, 300)])
def test_split_rope_attention_matches_oracle(sq8, dev, heads, kv_heads, hs, max_seq):
    """Positions split over up to 16 workgroups per head (rows past 512 positions), merged by the
    last to finish: the cache row written and the output equal the unsplit launch's (cache
    bitwise, output to the oracle's bound) at positions on and around chunk edges and the split
    threshold, all calls on one workspace (its tickets are zero after each)."""
    import torch
    dim, kv = heads * hs, kv_heads * hs
    nbytes = sq8.decode_attention_workspace_bytes(heads, hs, max_seq)
    assert nbytes > 0
    ws = torch.zeros((nbytes + 3) // 4, dtype=torch.int32, device=dev)
    sin = torch.empty((max_seq, hs), device=dev)
    cos = torch.empty((max_seq, hs), device=dev)
    sq8.rope_tables(sin, cos, hs, max_seq, 1e6)
    s_np, c_np = sin.cpu().numpy().astype(np.float64), cos.cpu().numpy().astype(np.float64)
    rng = np.random.default_rng(heads + max_seq)
    kc0 = rng.standard_normal((max_seq, kv)).astype(np.float32)
    vc0 = rng.standard_normal((max_seq, kv)).astype(np.float32)
    edges = {0, 1, 63, 64, 65, 127, 128, 511, 512, 513, 576, 640, 767, 768, 769}
    for pos in sorted({p for p in edges if p < max_seq} | {max_seq // 2, max_seq - 2, max_seq - 1}):
        qkv = rng.standard_normal(dim + 2 * kv).astype(np.float32)
        p = _t(np.array([pos], np.int32), dev)
        kc, vc, out = _t(kc0, dev), _t(vc0, dev), torch.full((dim,), float("nan"), device=dev)
        sq8.rope_attention_decode(_t(qkv, dev), heads, kv_heads, hs, p, sin, cos, kc, vc, out,
                                  max_seq, workspace=ws)
        kc2, vc2, out2 = _t(kc0, dev), _t(vc0, dev), torch.empty(dim, device=dev)
        sq8.rope_attention_decode(_t(qkv, dev), heads, kv_heads, hs, p, sin, cos, kc2, vc2, out2,
                                  max_seq)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(kc.cpu().numpy(), kc2.cpu().numpy())
        np.testing.assert_array_equal(vc.cpu().numpy(), vc2.cpu().numpy())
        qr = do.rope(qkv[:dim], heads, hs, pos, s_np, c_np)
        ref = do.attention(qr, kc2.cpu().numpy(), vc2.cpu().numpy(), pos, heads, kv_heads, hs)
        _close(out.cpu().numpy(), ref, 2e-6, f"split rope+attention pos {pos}")
        assert int(ws[:heads].abs().sum()) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("nbytes,wpc,u", [(16, 1, 1), (4096 * 16 + 48, 4, 4), (1 << 24, 8, 8),
                                          (3 * (1 << 20) + 16, 2, 2)])
def test_probe_stream_read_sums_every_word(sq8, dev, nbytes, wpc, u):
    """The bandwidth probe reads every byte once: its wrapping uint32 word sum matches numpy."""
    import torch
    rng = np.random.default_rng(nbytes)
    a = rng.integers(0, 2 ** 32, nbytes // 4, dtype=np.uint64).astype(np.uint32)
    buf = torch.from_numpy(a.view(np.int32)).to(dev)
    sink = torch.zeros(1000, dtype=torch.int32, device=dev)
    sq8.probe_stream_read(buf, sink, wpc, u)
    sq8.probe_stream_read(buf, sink, wpc, u)
    want = (2 * int(a.astype(np.uint64).sum())) % (1 << 32)
    got = int(sink.cpu().numpy().view(np.uint32).astype(np.uint64).sum()) % (1 << 32)
    assert got == want
