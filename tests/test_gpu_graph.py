"""The hot path captured into a HIP graph: every replay, with eager work and synchronisations in between,
matches the eager result bit for bit (the path records no memset nodes)."""
import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(gpu):
    import torch
    dev = torch.device("cuda:0")
    N, K, g, M = 6912, 2560, 128, 1
    w, s = synth.ternary_weight((60,), N, K, g)
    qw = gpu.QWeight(gpu.W_TERNARY, N, K, g, w, s)
    x = torch.from_numpy(synth.activations((61,), M, K)).to(dev)
    xq = torch.zeros((M, qw.kpad), dtype=torch.int8, device=dev)
    xs = torch.zeros(M, dtype=torch.float32, device=dev)
    y = torch.zeros((M, N), dtype=torch.float32, device=dev)
    norm = gpu.wht_norm(128)

    def step():
        gpu.prep_rows(x, xq, xs, 128, norm)
        qw.linear(xq, xs, y, path=gpu.PATH_GEMV)

    step()
    torch.cuda.synchronize()
    want = y.cpu().numpy().copy()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for r in range(4):
        y.fill_(float("nan"))
        xq.fill_(3)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {r} differs"
        # eager work between replays
        step()
        torch.cuda.synchronize()
    qw.close()
