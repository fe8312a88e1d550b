"""Writes tests/golden/sq8_golden.npz: small INT8 group-quant matmul cases with expected outputs.

The reference ships no test vectors for this path (it has no tests at all), so these fixtures are
computed here, independently of the C oracle: the quantiser and the product are pure-Python loops
over the formulas the reference kernel uses (src/source/op/kernels/cuda/matmul_kernel.cu:77,85-88:
scale of (n, k) = scales[(n*K)//gs + k//gs], product x * scale * q formed in fp32), accumulated
in float64. Inputs are drawn from numpy's seeded PCG64. Regenerate with
    python tests/golden/make_golden.py
"""
from pathlib import Path

import numpy as np

CASES = [  # (M, N, K, group_size, seed)
    (1, 3, 64, 64, 1),
    (3, 5, 128, 64, 2),
    (8, 17, 192, 64, 3),
    (2, 7, 96, 32, 4),
    (2, 16, 100, 64, 5),   # K not a multiple of the group size: the reference's flat indexing
    (1, 7, 12, 7, 6),
    (5, 9, 256, 128, 7),
    (17, 4, 64, 16, 8),
]


def quantize(w, gs):
    """Per flat group of gs: s = absmax/127 (fp32), q = round-half-away(w/s) clamped to +-127."""
    flat = [float(v) for v in w.reshape(-1)]
    q = np.zeros(len(flat), np.int8)
    s = np.zeros(len(flat) // gs, np.float32)
    for g in range(len(s)):
        amax = max(abs(np.float32(v)) for v in flat[g * gs:(g + 1) * gs])
        sc = np.float32(np.float32(amax) / np.float32(127.0))
        s[g] = sc
        for i in range(g * gs, (g + 1) * gs):
            if sc == 0:
                continue
            v = float(np.float32(np.float32(flat[i]) / sc))
            r = min(127.0, np.floor(abs(v) + 0.5))
            q[i] = int(-r if v < 0 else r)
    return q.reshape(w.shape), s


def matmul(x, q, s, gs):
    M, K = x.shape
    N = q.shape[0]
    y = np.zeros((M, N), np.float64)
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                xs = np.float32(x[m, k]) * np.float32(s[(n * K) // gs + k // gs])
                acc += float(xs) * float(q[n, k])
            y[m, n] = acc
    return y


def main():
    out = {}
    for i, (M, N, K, gs, seed) in enumerate(CASES):
        rng = np.random.default_rng(seed)
        x = rng.standard_normal((M, K)).astype(np.float32)
        w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
        q, s = quantize(w, gs)
        out[f"c{i}_x"], out[f"c{i}_w"], out[f"c{i}_q"], out[f"c{i}_s"] = x, w, q, s
        out[f"c{i}_y"] = matmul(x, q, s, gs)
        out[f"c{i}_shape"] = np.array([M, N, K, gs], np.int64)
    path = Path(__file__).resolve().parent / "sq8_golden.npz"
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({len(CASES)} cases)")


if __name__ == "__main__":
    main()
