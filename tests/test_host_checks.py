"""The Python layer's argument checks (MatmulLayer::check, src/source/op/matmul.cpp:19-77): a
wrong shape, dtype or placement raises ValueError before anything reaches the C ABI, whose plain
pointers carry no sizes. Runs on the CPU: every case fails a check before any launch."""
import pytest
import torch

from conftest import load_pkg

sq8 = load_pkg()
M, N, K, GS = 4, 32, 128, 64


def ops(**over):
    t = dict(x=torch.zeros(M, K), w=torch.zeros(N, K, dtype=torch.int8),
             s=torch.zeros(N * K // GS), y=torch.zeros(M, N))
    t.update(over)
    return t


@pytest.mark.parametrize("over,msg", [
    (dict(x=torch.zeros(M, K, dtype=torch.float64)), "input dtype"),
    (dict(w=torch.zeros(N, K)), "weight dtype"),
    (dict(w=torch.zeros(N, K + 64, dtype=torch.int8)), "weight shape"),
    (dict(s=torch.zeros(N * K // GS - 1)), "scales holds"),
    (dict(s=torch.zeros(N * K // GS, dtype=torch.float16)), "scales dtype"),
    (dict(y=torch.zeros(M, N - 1)), "output holds"),
    (dict(y=torch.zeros(N, M).t()), "contiguous"),
    (dict(), "expected a GPU"),
])
def test_matmul_rejects(over, msg):
    t = ops(**over)
    with pytest.raises(ValueError, match=msg):
        sq8.matmul(t["x"], t["w"], t["s"], t["y"], group_size=GS)


def test_matmul_rejects_group_not_dividing():
    t = ops()
    with pytest.raises(ValueError, match="group size"):
        sq8.matmul(t["x"], t["w"], t["s"], t["y"], group_size=3 * 1024 + 7)


def test_epilogue_output_and_residual_shapes():
    t = ops(y=torch.zeros(M, N // 2))
    with pytest.raises(ValueError, match="expected a GPU"):  # SwiGLU: N/2 outputs per row
        sq8.matmul_epilogue(t["x"], t["w"], t["s"], t["y"], sq8.SQ8_EPI_SWIGLU, group_size=GS)
    with pytest.raises(ValueError, match="output holds"):
        sq8.matmul_epilogue(t["x"], t["w"], t["s"], t["y"], sq8.SQ8_EPI_RESIDUAL,
                            residual=torch.zeros(M, N // 2), group_size=GS)
    t = ops()
    with pytest.raises(ValueError, match="residual holds"):
        sq8.matmul_epilogue(t["x"], t["w"], t["s"], t["y"], sq8.SQ8_EPI_RESIDUAL,
                            residual=torch.zeros(M, N // 2), group_size=GS)


def test_rmsnorm_rows_checks_norm_weight_and_residual():
    t = ops()
    with pytest.raises(ValueError, match="norm weight holds"):
        sq8.matmul_rmsnorm_rows(t["x"], None, torch.ones(K - 1), 1e-6, t["w"], t["s"], t["y"],
                                group_size=GS)
    with pytest.raises(ValueError, match="residual holds"):
        sq8.matmul_rmsnorm_rows(t["x"], torch.zeros(M, K + 1), torch.ones(K), 1e-6, t["w"],
                                t["s"], t["y"], group_size=GS)
    with pytest.raises(ValueError, match="expected a GPU"):
        sq8.matmul_rmsnorm_rows(t["x"], torch.zeros(M, K), torch.ones(K), 1e-6, t["w"], t["s"],
                                t["y"], group_size=GS)


def test_packed_weight_shape_is_checked():
    t = ops()
    pw = sq8.PackedWeight(torch.zeros(N * K, dtype=torch.int8), N, K + 64)
    with pytest.raises(ValueError, match="weight shape"):
        sq8.matmul(t["x"], pw, t["s"], t["y"], group_size=GS)


def _paged(rows=3, heads=4, kv_heads=2, hs=64, bs=16, width=8, nb=10, **over):
    t = dict(qkv=torch.zeros(rows, (heads + 2 * kv_heads) * hs),
             pos=torch.zeros(rows, dtype=torch.int32),
             tab=torch.zeros(rows, width, dtype=torch.int32),
             kc=torch.zeros(nb, bs, kv_heads * hs), vc=torch.zeros(nb, bs, kv_heads * hs),
             out=torch.zeros(rows, heads * hs))
    t.update(over)
    return t


@pytest.mark.parametrize("over,msg", [
    (dict(pos=torch.zeros(3, dtype=torch.int64)), "int32"),
    (dict(tab=torch.zeros(2, 8, dtype=torch.int32)), "block table"),
    (dict(kc=torch.zeros(10, 8, 128)), "key cache"),
    (dict(vc=torch.zeros(10, 16, 64)), "value cache"),
    (dict(out=torch.zeros(3, 100)), "output of"),
    (dict(qkv=torch.zeros(2, 512)), "qkv of"),
])
def test_paged_attention_checks_shapes(over, msg):
    t = _paged(**over)
    with pytest.raises(ValueError, match=msg):
        sq8.paged_attention(t["qkv"], 512, 4, 2, 64, t["pos"], t["tab"], 16, t["kc"], t["vc"],
                            t["out"])


def test_paged_rope_kv_checks_shapes():
    t = _paged(qkv=torch.zeros(3, 515))
    with pytest.raises(ValueError, match="q, k and v exactly"):
        sq8.paged_rope_kv(t["qkv"], 4, 2, 64, t["pos"], t["tab"], 16, None, None, t["kc"],
                          t["vc"])
    with pytest.raises(ValueError, match="query heads"):
        sq8.paged_rope_kv(torch.zeros(3, 64 * 9), 5, 2, 64, t["pos"], t["tab"], 16, None, None,
                          t["kc"], t["vc"])
