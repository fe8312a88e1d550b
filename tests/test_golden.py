"""The committed golden fixtures (tests/golden/sq8_golden.npz, made by make_golden.py) against the
C oracle (CPU) and the HIP path (GPU)."""
from pathlib import Path

import numpy as np
import pytest

from oracle import sq8_oracle as o

GOLDEN = Path(__file__).resolve().parent / "golden" / "sq8_golden.npz"


def cases():
    d = np.load(GOLDEN)  # allow_pickle=False (default)
    n = len([k for k in d.files if k.endswith("_shape")])
    for i in range(n):
        M, N, K, gs = (int(v) for v in d[f"c{i}_shape"])
        yield i, M, N, K, gs, d[f"c{i}_x"], d[f"c{i}_w"], d[f"c{i}_q"], d[f"c{i}_s"], d[f"c{i}_y"]


@pytest.mark.parametrize("case", list(cases()), ids=lambda c: f"c{c[0]}_M{c[1]}N{c[2]}K{c[3]}g{c[4]}")
def test_oracle_matches_golden(case):
    i, M, N, K, gs, x, w, q, s, y = case
    q2, s2 = o.quantize(w.reshape(-1), gs)
    np.testing.assert_array_equal(q2.reshape(N, K), q)
    np.testing.assert_array_equal(s2, s)
    np.testing.assert_allclose(o.matmul_f64(x, q, s, gs), y, rtol=1e-12, atol=1e-15)


@pytest.mark.gpu
@pytest.mark.parametrize("case", list(cases()), ids=lambda c: f"c{c[0]}_M{c[1]}N{c[2]}K{c[3]}g{c[4]}")
def test_hip_matches_golden(case, sq8, dev):
    import torch
    i, M, N, K, gs, x, w, q, s, y = case
    out = sq8.matmul(torch.from_numpy(x).to(dev), torch.from_numpy(q).to(dev),
                     torch.from_numpy(s).to(dev), group_size=gs)
    torch.cuda.synchronize()
    elem, norm = o.rel_errors(out.cpu().numpy(), y)
    assert elem <= 1e-3 and norm <= 1e-5, (elem, norm)
