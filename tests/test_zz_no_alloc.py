"""sq8_matmul_noalloc (no workspace argument, no allocation: a fixed device scratch array per GPU)
against sq8_matmul with a caller workspace, through the C ABI: bitwise equal on two calls in a
row, the second with a smaller input, on shapes whose kernels use the scratch (split-K tickets,
packed activations, split-K partials); shapes needing more than the array are refused."""
import numpy as np
import pytest

from conftest import load_pkg
from oracle import sq8_oracle as o

sq8_pkg = load_pkg()


def _case(torch, dev, M, N, K, seed):
    x, q, s = o.make_case(M, N, K, 64, seed=seed)
    return (torch.from_numpy(x).to(dev), torch.from_numpy(q).to(dev),
            torch.from_numpy(s).to(dev))


def _noalloc(sq8, torch, x, q, s, y):
    M, K = x.shape
    N = q.shape[0]
    st = torch.cuda.current_stream(x.device).cuda_stream
    return sq8.lib().sq8_matmul_noalloc(x.data_ptr(), q.data_ptr(), s.data_ptr(), y.data_ptr(),
                                        M, N, K, 64, st)


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry(sq8, dev):
    import torch
    L = sq8.lib()
    cap = int(L.sq8_noalloc_scratch_bytes())
    assert cap == 32 << 20
    # (M, N, K): the decode GEMM with split-K partials, then a smaller tile-kernel call with
    # split-K tickets; then the skinny kernel and the prefill GEMM below the cap.
    for shapes in (((64, 28672, 4096), (16, 4096, 4096)), ((8, 6144, 4096), (5, 4096, 14336)),
                   ((256, 4096, 4096), (96, 1024, 4096))):
        for i, (M, N, K) in enumerate(shapes):
            need = sq8.workspace_bytes(M, N, K, 64)
            assert 0 < need <= cap, (M, N, K, need)
            x, q, s = _case(torch, dev, M, N, K, seed=M + N + i)
            y = torch.full((M, N), float("nan"), device=dev)
            print(f"noalloc M={M} N={N} K={K} path={sq8.path_name(M, N, K, 64)} ws={need}",
                  flush=True)
            assert _noalloc(sq8, torch, x, q, s, y) == sq8.SQ8_OK
            ref = sq8.matmul(x, q, s, group_size=64)
            torch.cuda.synchronize()
            assert torch.equal(y, ref), (M, N, K)
            elem, norm = o.rel_errors(y[:4].cpu().numpy(),
                                      o.matmul_f64(x[:4].cpu().numpy(), q.cpu().numpy(),
                                                   s.cpu().numpy(), 64))
            assert elem <= 1e-3 and norm <= 1e-5


@pytest.mark.gpu
def test_noalloc_refuses_shapes_beyond_the_scratch(sq8, dev):
    import torch
    M, N, K = 2048, 28672, 4096
    assert sq8.workspace_bytes(M, N, K, 64) > int(sq8.lib().sq8_noalloc_scratch_bytes())
    x = torch.zeros((M, K), device=dev)
    q = torch.zeros((N, K), dtype=torch.int8, device=dev)
    s = torch.zeros(N * K // 64, device=dev)
    y = torch.full((M, N), 7.0, device=dev)
    assert _noalloc(sq8, torch, x, q, s, y) == sq8.SQ8_ERR_WORKSPACE
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())  # nothing launched


@pytest.mark.gpu
def test_noalloc_replays_under_graph_capture(sq8, dev):
    """The entry point for code under graph capture, captured into a HIP graph: each of several
    replays, with eager work and synchronisation between them, equals the eager sq8_matmul
    bitwise (split-K tile kernel with tickets, then the decode GEMM with partials)."""
    import torch
    for (M, N, K) in ((16, 4096, 4096), (64, 28672, 4096)):
        x, q, s = _case(torch, dev, M, N, K, seed=3 * M)
        ref = sq8.matmul(x, q, s, group_size=64)
        y = torch.full((M, N), float("nan"), device=dev)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):  # one eager call first: the device's scratch lookup
            assert _noalloc(sq8, torch, x, q, s, y) == sq8.SQ8_OK
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize()
        assert torch.equal(y, ref), (M, N, K)
        g = torch.cuda.CUDAGraph()
        rc = []
        with torch.cuda.graph(g, stream=side):
            rc.append(_noalloc(sq8, torch, x, q, s, y))
        assert rc == [sq8.SQ8_OK]
        print(f"noalloc graph M={M} N={N} K={K} path={sq8.path_name(M, N, K, 64)}", flush=True)
        for rep in range(4):
            y.fill_(float("nan"))
            sq8.matmul(x[: M // 2], q, s, group_size=64)  # eager work between the replays
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, ref), (M, N, K, rep)
        del g
