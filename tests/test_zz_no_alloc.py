"""eif_hip_qlinear_ex_noalloc: the GEMM's split partials in the library's fixed device scratch instead of a
per-stream workspace. Two calls in a row (the second with fewer tokens) give eif_hip_qlinear_ex's bits; a split
beyond the scratch is refused with EIF_HIP_E_LIMIT and launches nothing. Both shapes split along K at 128 and at
40 tokens (long K loops on few row tiles), so both calls use the scratch."""
import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu


def call(gpu, fn, w, xq, xs, y, M):
    import ctypes as C
    lib = gpu.load()
    f = getattr(lib, fn)
    return f(w.h, gpu.ptr(xq), xq.stride(0), gpu.ptr(xs), None, gpu.ptr(y), y.stride(0), M, gpu.PATH_GEMM,
             gpu.stream_ptr())


@pytest.mark.parametrize("fmt,N,K,g", [("tern", 2560, 6912, 96), ("int8", 896, 4864, 0)])
def test_noalloc_matches_qlinear_ex(gpu, fmt, N, K, g):
    import torch
    dev = torch.device("cuda:0")
    if fmt == "tern":
        codes, sc = synth.ternary_weight((61,), N, K, g)
        w = gpu.QWeight(gpu.W_TERNARY, N, K, g, codes, sc)
    else:
        codes, sc = synth.int8_weight((62,), N, K)
        w = gpu.QWeight(gpu.W_INT8, N, K, 0, codes, sc)
    try:
        kp = w.kpad
        for M in (128, 40):   # two calls in a row, the second smaller (the scratch keeps the first call's data)
            x = torch.from_numpy(synth.activations((63, M), M, K)).to(dev)
            xq = torch.zeros((M, kp), dtype=torch.int8, device=dev)
            xs = torch.zeros(M, dtype=torch.float32, device=dev)
            gpu.prep_rows(x, xq, xs, 128 if fmt == "tern" else 0, gpu.wht_norm(128) if fmt == "tern" else 1.0)
            y_ref = torch.full((M, N), np.nan, dtype=torch.float32, device=dev)
            y_na = torch.full((M, N), np.nan, dtype=torch.float32, device=dev)
            assert call(gpu, "eif_hip_qlinear_ex", w, xq, xs, y_ref, M) == 0
            assert call(gpu, "eif_hip_qlinear_ex_noalloc", w, xq, xs, y_na, M) == 0
            torch.cuda.synchronize()
            a, b = y_ref.cpu().numpy(), y_na.cpu().numpy()
            assert np.isfinite(a).all()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (fmt, M)
    finally:
        w.close()


def test_noalloc_refuses_beyond_scratch(gpu):
    import torch
    lib = gpu.load()
    cap = lib.eif_hip_qlinear_noalloc_max_bytes()
    assert cap == 32 << 20
    dev = torch.device("cuda:0")
    N, K, M = 13824, 2560, 512
    codes, sc = synth.ternary_weight((64,), N, K, 128)
    w = gpu.QWeight(gpu.W_TERNARY, N, K, 128, codes, sc)
    old = lib.eif_hip_set_gemm_split(16)   # 16 splits x 512 x 13824 floats: far beyond the scratch
    try:
        xq = torch.zeros((M, w.kpad), dtype=torch.int8, device=dev)
        xs = torch.ones(M, dtype=torch.float32, device=dev)
        y = torch.full((M, N), 7.0, dtype=torch.float32, device=dev)
        assert call(gpu, "eif_hip_qlinear_ex_noalloc", w, xq, xs, y, M) == gpu.E_LIMIT
        torch.cuda.synchronize()
        assert bool((y == 7.0).all())   # nothing launched
    finally:
        lib.eif_hip_set_gemm_split(old)
        w.close()
