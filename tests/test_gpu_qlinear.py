"""INT8-activation linears (MFMA GEMV and GEMM paths) against the oracle.

Integer accumulators are compared bit for bit; row-scaled outputs bit for bit (same epilogue order as the
reference build) and, for INT8 / INT4, within 1e-6 of the float64 closed form acc * xs[m] * s[r] + bias[r]; group-scaled FP32 outputs to 1e-5 relative to sum_g |s*acc_g|*xs + |bias| and, since the
kernels combine a row's groups in group order as the oracle does, bit for bit.
"""
import numpy as np
import pytest

import closed_form as cf
from conftest import P
import synth

pytestmark = pytest.mark.gpu

GEMV, GEMM = 1, 2
REL_TOL = 1e-5


def dev_inputs(gpu, oracle, x, kpad):
    import torch
    M, K = x.shape
    dev = torch.device("cuda:0")
    xq = np.zeros((M, kpad), np.int8)
    xs = np.zeros(M, np.float32)
    assert oracle.orc_prep_rows(P(x), K, None, M, K, 0, 1.0, P(xq), kpad, P(xs), None, 0) == 0
    return xq, xs, torch.from_numpy(xq).to(dev), torch.from_numpy(xs).to(dev)


def run_linear(gpu, qw, xq_d, xs_d, M, path, bias=None):
    import torch
    y = torch.full((M, qw.rows), float("nan"), dtype=torch.float32, device="cuda:0")
    b = torch.from_numpy(bias).to("cuda:0") if bias is not None else None
    qw.linear(xq_d, xs_d, y, M=M, bias=b, path=path)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def run_acc(gpu, qw, xq_d, M, shape, path):
    import torch
    acc = torch.full(shape, -7, dtype=torch.int32, device="cuda:0")
    qw.acc(xq_d, acc, M=M, path=path)
    torch.cuda.synchronize()
    return acc.cpu().numpy()


TERN_GROUPED = [
    # N, K, g, M, path
    (6912, 2560, 128, 1, GEMV),     # the single BitNet linear
    (2560, 6912, 96, 1, GEMV),      # down projection, g96
    (3840, 2560, 128, 8, GEMV),
    (130, 200, 32, 3, GEMV),        # ragged rows and columns
    (70, 640, 64, 5, GEMV),
    (64, 512, 256, 2, GEMV),
    (6912, 2560, 64, 1, GEMV),      # the one-shape layouts up to 16 rows: SMAX - 2 steps a wave
    (1000, 6912, 32, 1, GEMV),
    (300, 2560, 256, 1, GEMV),
    (700, 2560, 64, 8, GEMV),
    (500, 6912, 32, 16, GEMV),
    (300, 6912, 256, 5, GEMV),
    (6912, 2560, 128, 16, GEMV),    # 9 .. 63 tokens: the GEMV in token chunks
    (3840, 2560, 128, 32, GEMV),
    (2560, 6912, 96, 16, GEMV),     # g96 down: one 16-row token tile per workgroup (int16 group sums in LDS)
    (2560, 6912, 96, 32, GEMV),     #   two 16-row chunks
    (2560, 6912, 96, 63, GEMV),     #   four chunks, the last of 15 rows
    (130, 200, 32, 63, GEMV),
    (70, 640, 64, 17, GEMV),
    (70, 640, 64, 17, GEMM),
    (6912, 2560, 128, 64, GEMM),
    (2560, 6912, 96, 64, GEMM),
    (300, 2560, 128, 200, GEMM),
    (17, 96, 96, 1, GEMM),
    (130, 200, 32, 70, GEMM),       # g32, g64, g256 with 64-token tiles (the compiler's register budget)
    (70, 640, 64, 100, GEMM),
    (64, 512, 256, 40, GEMM),
]


@pytest.mark.parametrize("N,K,g,M,path", TERN_GROUPED)
def test_ternary_grouped(gpu, oracle, N, K, g, M, path):
    w, s = synth.ternary_weight((40, N, K, g), N, K, g)
    x = synth.activations((41, M, K), M, K)
    qw = gpu.QWeight(gpu.W_TERNARY, N, K, g, w, s)
    xq, xs, xq_d, xs_d = dev_inputs(gpu, oracle, x, qw.kpad)
    ng = -(-K // g)
    acc = run_acc(gpu, qw, xq_d, M, (M, N, ng), path)
    oacc = np.zeros((M, N, ng), np.int32)
    oracle.orc_ternary_acc_i32(P(w), P(xq), qw.kpad, M, N, K, g, P(oacc))
    assert np.array_equal(acc, oacc)
    bias = synth.rng(42, N).standard_normal(N).astype(np.float32) if M % 2 else None
    y = run_linear(gpu, qw, xq_d, xs_d, M, path, bias)
    oy = np.zeros((M, N), np.float32)
    oracle.orc_ternary_gemv_grouped(P(w), P(s), g, P(xq), qw.kpad, P(xs), P(bias), P(oy), N, M, N, K)
    mag = np.einsum("mng,ng->mn", np.abs(oacc).astype(np.float64), s.astype(np.float64)) * xs[:, None]
    if bias is not None:
        mag = mag + np.abs(bias)[None, :]
    err = np.abs(y.astype(np.float64) - oy) / (mag + 1e-30)
    assert np.all(np.isfinite(y)) and err.max() <= REL_TOL, err.max()
    # the small-batch GEMV and the unsplit GEMM combine the groups of a row in group order, as the oracle does
    lib = gpu.load()
    old = lib.eif_hip_set_gemm_split(1)
    try:
        y = run_linear(gpu, qw, xq_d, xs_d, M, path, bias)
    finally:
        lib.eif_hip_set_gemm_split(old)
    assert np.array_equal(y.view(np.uint32), oy.view(np.uint32))
    qw.close()


@pytest.mark.parametrize("N,K,g", [(3072, 2560, 128), (1024, 6912, 96), (200, 2560, 128),
                                   (1000, 2560, 64), (300, 2560, 32), (500, 2560, 256), (260, 6912, 64)])
def test_gemv_shape_knobs(gpu, oracle, N, K, g):
    """Row tiles per workgroup, waves per tile and prep columns per thread change the launch, never the result
    (y, acc, fused y); the fused y is the oracle's prep and grouped GEMV bit for bit."""
    import torch
    dev = torch.device("cuda:0")
    lib = gpu.load()
    w, s = synth.ternary_weight((58, N, K, g), N, K, g)
    qw = gpu.QWeight(gpu.W_TERNARY, N, K, g, w, s)
    ng = -(-K // g)
    norm = gpu.wht_norm(128)
    ref = None
    try:
        for M in (1, 5):
            x = synth.activations((59, M, K), M, K)
            xd = torch.from_numpy(x).to(dev)
            xq, xs, xq_d, xs_d = dev_inputs(gpu, oracle, x, qw.kpad)
            oy = np.zeros((M, N), np.float32)
            oracle.orc_ternary_gemv_grouped(P(w), P(s), g, P(xq), qw.kpad, P(xs), None, P(oy), N, M, N, K)
            oacc = np.zeros((M, N, ng), np.int32)
            oracle.orc_ternary_acc_i32(P(w), P(xq), qw.kpad, M, N, K, g, P(oacc))
            # the fused prep's reference: the oracle's WHT-128 prep, then its grouped GEMV
            rq = np.zeros((M, qw.kpad), np.int8)
            rs = np.zeros(M, np.float32)
            assert oracle.orc_prep_rows(P(x), K, None, M, K, 128, norm, P(rq), qw.kpad, P(rs), None, 0) == 0
            fy = np.zeros((M, N), np.float32)
            oracle.orc_ternary_gemv_grouped(P(w), P(s), g, P(rq), qw.kpad, P(rs), None, P(fy), N, M, N, K)
            ref = None
            for rt, ks, e in [(0, 0, 0), (1, 0, 0), (4, 0, 0), (1, 2, 0), (4, 2, 0), (1, 16, 0), (4, 4, 0), (1, 1, 0),
                              (0, 0, 8), (1, 0, 16), (4, 0, 8), (1, 4, 16)]:
                lib.eif_hip_set_gemv_row_tiles(rt)
                lib.eif_hip_set_gemv_ksplit(ks)
                lib.eif_hip_set_gemv_prep_cols(e)
                y = run_linear(gpu, qw, xq_d, xs_d, M, GEMV)
                assert np.array_equal(y.view(np.uint32), oy.view(np.uint32)), (M, rt, ks, e)
                acc = run_acc(gpu, qw, xq_d, M, (M, N, ng), GEMV)
                assert np.array_equal(acc, oacc), (M, rt, ks, e)
                yf = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
                qw.linear_f32(xd, yf, 128, norm)
                yf = yf.cpu().numpy()
                if ref is None:
                    ref = yf
                    assert np.array_equal(yf.view(np.uint32), fy.view(np.uint32)), M
                assert np.array_equal(yf.view(np.uint32), ref.view(np.uint32)), (M, rt, ks, e)
    finally:
        lib.eif_hip_set_gemv_row_tiles(0)
        lib.eif_hip_set_gemv_ksplit(0)
        lib.eif_hip_set_gemv_prep_cols(0)
        qw.close()


@pytest.mark.parametrize("N,K", [(13824, 2560), (2560, 6912), (200, 2560), (70, 640)])
def test_ternary_rowscale_shapes(gpu, oracle, N, K):
    """Ternary with one scale per row through every GEMV launch shape (row tiles 1 / 4, waves per tile, token
    tiles and chunks up to 40 rows) and the fused prep (WHT-128, E columns per thread): y bit-exact against the
    oracle's row-scaled GEMV of the oracle's prep, int32 sums exact."""
    import torch
    dev = torch.device("cuda:0")
    lib = gpu.load()
    w, s = synth.ternary_weight((146, N, K), N, K, 0)
    qw = gpu.QWeight(gpu.W_TERNARY, N, K, 0, w, s)
    codes = synth.unpack_ternary(w, K).astype(np.int64)
    bias = synth.rng(147, N).standard_normal(N).astype(np.float32)
    norm = gpu.wht_norm(128)
    try:
        for M in (1, 3, 8, 20, 40):
            x = synth.activations((148, M, K), M, K)
            xq, xs, xq_d, xs_d = dev_inputs(gpu, oracle, x, qw.kpad)
            oacc = (xq[:, :K].astype(np.int64) @ codes.T).astype(np.int32)
            oy = np.zeros((M, N), np.float32)
            oracle.orc_ternary_gemv_rowscale(P(w), P(s), P(xq), qw.kpad, P(xs), P(bias), P(oy), N, M, N, K)
            # the fused prep's reference: the oracle's WHT-128 prep, then its row-scaled GEMV
            rq = np.zeros((M, qw.kpad), np.int8)
            rs = np.zeros(M, np.float32)
            assert oracle.orc_prep_rows(P(x), K, None, M, K, 128, norm, P(rq), qw.kpad, P(rs), None, 0) == 0
            fy = np.zeros((M, N), np.float32)
            oracle.orc_ternary_gemv_rowscale(P(w), P(s), P(rq), qw.kpad, P(rs), None, P(fy), N, M, N, K)
            xd = torch.from_numpy(x).to(dev)
            for rt, ks in [(0, 0), (1, 0), (4, 0), (1, 2), (4, 2), (1, 16), (4, 4), (1, 1)]:
                lib.eif_hip_set_gemv_row_tiles(rt)
                lib.eif_hip_set_gemv_ksplit(ks)
                case = (M, rt, ks)
                y = run_linear(gpu, qw, xq_d, xs_d, M, GEMV, bias)
                assert np.array_equal(y.view(np.uint32), oy.view(np.uint32)), case
                acc = run_acc(gpu, qw, xq_d, M, (M, N), GEMV)
                assert np.array_equal(acc, oacc), case
                if M <= 8:
                    for e in (0, 8, 16):
                        lib.eif_hip_set_gemv_prep_cols(e)
                        yf = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
                        qw.linear_f32(xd, yf, 128, norm)
                        yf = yf.cpu().numpy()
                        assert np.array_equal(yf.view(np.uint32), fy.view(np.uint32)), case + (e,)
                    lib.eif_hip_set_gemv_prep_cols(0)
    finally:
        lib.eif_hip_set_gemv_row_tiles(0)
        lib.eif_hip_set_gemv_ksplit(0)
        lib.eif_hip_set_gemv_prep_cols(0)
        qw.close()


@pytest.mark.parametrize("fmt,N,K,g,M", [
    ("tern", 200, 2560, 128, 40),    # 20 steps: rounds of 8 with 4 left, of 4 with none
    ("tern", 96, 2688, 128, 17),     # 21 steps: 5, 1 and 1 left for rings of 8, 4, 2
    ("tern", 130, 200, 32, 20),      # g32: 2 steps, fewer than the ring
    ("tern", 2560, 6912, 96, 64),    # g96 down projection, 72 steps
    ("tern", 70, 640, 64, 33),
    ("int8", 896, 4864, 0, 70),
    ("int4", 512, 1024, 0, 48),
    ("int8", 300, 128, 0, 20),       # one step of K
    ("tern", 70, 64, 32, 18),        # g32, one step
])
def test_gemm_forms(gpu, oracle, fmt, N, K, g, M):
    """The GEMM's tiled form with each prefetch ring (2, 4, 8 steps of loads in flight) and its panel form
    (activation panel resident in LDS; rings of 4 and 8), with every token tile, unsplit and split: integer sums
    exact; unsplit outputs bit-exact against the oracle, split ones within tolerance and the same bits in every
    form."""
    lib = gpu.load()
    if fmt == "tern":
        w, s = synth.ternary_weight((65, N, K, g), N, K, g)
        qw = gpu.QWeight(gpu.W_TERNARY, N, K, g, w, s)
    elif fmt == "int8":
        w, s = synth.int8_weight((66, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT8, N, K, 0, w, s)
    else:
        w, s = synth.int4_weight((67, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT4, N, K, 0, w, s)
    x = synth.activations((68, M, K), M, K)
    xq, xs, xq_d, xs_d = dev_inputs(gpu, oracle, x, qw.kpad)
    bias = synth.rng(69, N).standard_normal(N).astype(np.float32)
    oy = np.zeros((M, N), np.float32)
    if fmt == "tern":
        ng = -(-K // g)
        oacc = np.zeros((M, N, ng), np.int32)
        oracle.orc_ternary_acc_i32(P(w), P(xq), qw.kpad, M, N, K, g, P(oacc))
        oracle.orc_ternary_gemv_grouped(P(w), P(s), g, P(xq), qw.kpad, P(xs), P(bias), P(oy), N, M, N, K)
        mag = np.einsum("mng,ng->mn", np.abs(oacc).astype(np.float64), s.astype(np.float64)) * xs[:, None]
        mag = mag + np.abs(bias)[None, :]
    else:
        wi = w.astype(np.int64) if fmt == "int8" else synth.unpack_int4(w, K).astype(np.int64)
        oacc = (xq[:, :K].astype(np.int64) @ wi.T).astype(np.int32)
        fn = oracle.orc_int8_gemv_i8act if fmt == "int8" else oracle.orc_int4_gemv_i8act
        fn(P(w), P(s), P(xq), qw.kpad, P(xs), P(bias), P(oy), N, M, N, K)
    try:
        for tt in (1, 2, 4):
            lib.eif_hip_set_gemm_token_tiles(tt)
            for ks in (1, 3):
                lib.eif_hip_set_gemm_split(ks)
                first = None
                for panel, pf in [(-1, 2), (-1, 4), (-1, 8), (1, 4), (1, 8)]:
                    lib.eif_hip_set_gemm_panel(panel)
                    lib.eif_hip_set_gemm_prefetch(pf)
                    y = run_linear(gpu, qw, xq_d, xs_d, M, GEMM, bias)
                    case = (tt, ks, panel, pf)
                    if fmt != "tern" or ks == 1:
                        assert np.array_equal(y.view(np.uint32), oy.view(np.uint32)), case
                    else:
                        err = np.abs(y.astype(np.float64) - oy) / (mag + 1e-30)
                        assert err.max() <= REL_TOL, (case, err.max())
                    if first is None:
                        first = y
                    assert np.array_equal(y.view(np.uint32), first.view(np.uint32)), case
            acc = run_acc(gpu, qw, xq_d, M, oacc.shape, GEMM)
            assert np.array_equal(acc, oacc), tt
    finally:
        lib.eif_hip_set_gemm_panel(0)
        lib.eif_hip_set_gemm_prefetch(0)
        lib.eif_hip_set_gemm_split(0)
        lib.eif_hip_set_gemm_token_tiles(0)
        qw.close()


@pytest.mark.parametrize("fmt,N,K,g,M", [("tern", 2560, 6912, 96, 64), ("tern", 640, 2560, 128, 40),
                                          ("int8", 896, 4864, 0, 128), ("int4", 512, 1024, 0, 32)])
def test_gemm_split(gpu, oracle, fmt, N, K, g, M):
    """GEMM split along K: integer sums exact and row-scaled outputs bit-exact at every split; grouped FP32
    within tolerance of the oracle, bit-exact unsplit, and the same bits on a repeated launch and on graph
    replays (the arrival counters reset themselves)."""
    import torch
    lib = gpu.load()
    if fmt == "tern":
        w, s = synth.ternary_weight((60, N, K, g), N, K, g)
        qw = gpu.QWeight(gpu.W_TERNARY, N, K, g, w, s)
    elif fmt == "int8":
        w, s = synth.int8_weight((61, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT8, N, K, 0, w, s)
    else:
        w, s = synth.int4_weight((62, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT4, N, K, 0, w, s)
    x = synth.activations((63, M, K), M, K)
    xq, xs, xq_d, xs_d = dev_inputs(gpu, oracle, x, qw.kpad)
    bias = synth.rng(64, N).standard_normal(N).astype(np.float32)
    oy = np.zeros((M, N), np.float32)
    if fmt == "tern":
        ng = -(-K // g)
        oacc = np.zeros((M, N, ng), np.int32)
        oracle.orc_ternary_acc_i32(P(w), P(xq), qw.kpad, M, N, K, g, P(oacc))
        oracle.orc_ternary_gemv_grouped(P(w), P(s), g, P(xq), qw.kpad, P(xs), P(bias), P(oy), N, M, N, K)
        mag = np.einsum("mng,ng->mn", np.abs(oacc).astype(np.float64), s.astype(np.float64)) * xs[:, None]
        mag = mag + np.abs(bias)[None, :]
    else:
        wi = w.astype(np.int64) if fmt == "int8" else synth.unpack_int4(w, K).astype(np.int64)
        oacc = (xq[:, :K].astype(np.int64) @ wi.T).astype(np.int32)
        fn = oracle.orc_int8_gemv_i8act if fmt == "int8" else oracle.orc_int4_gemv_i8act
        fn(P(w), P(s), P(xq), qw.kpad, P(xs), P(bias), P(oy), N, M, N, K)
    try:
        for ks in (1, 2, 5, 16):
            lib.eif_hip_set_gemm_split(ks)
            acc = run_acc(gpu, qw, xq_d, M, oacc.shape, GEMM)
            assert np.array_equal(acc, oacc), ks
            y = run_linear(gpu, qw, xq_d, xs_d, M, GEMM, bias)
            y2 = run_linear(gpu, qw, xq_d, xs_d, M, GEMM, bias)
            assert np.array_equal(y.view(np.uint32), y2.view(np.uint32)), ks
            if fmt != "tern" or ks == 1:
                assert np.array_equal(y.view(np.uint32), oy.view(np.uint32)), ks
            else:
                err = np.abs(y.astype(np.float64) - oy) / (mag + 1e-30)
                assert err.max() <= REL_TOL, (ks, err.max())
        # graph replays of a split launch
        lib.eif_hip_set_gemm_split(5)
        yd = torch.zeros((M, N), dtype=torch.float32, device="cuda:0")
        bd = torch.from_numpy(bias).to("cuda:0")
        cs = torch.cuda.Stream()
        with torch.cuda.stream(cs):
            qw.linear(xq_d, xs_d, yd, M=M, bias=bd, path=GEMM)
        cs.synchronize()
        ref = yd.cpu().numpy()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=cs):
            qw.linear(xq_d, xs_d, yd, M=M, bias=bd, path=GEMM)
        for _ in range(4):
            yd.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert np.array_equal(yd.cpu().numpy().view(np.uint32), ref.view(np.uint32))
        del graph
    finally:
        lib.eif_hip_set_gemm_split(0)
        qw.close()


@pytest.mark.parametrize("N,K,M,path,with_bias", [
    (6912, 2560, 1, GEMV, False), (2560, 6912, 1, GEMV, True), (100, 300, 7, GEMV, True),
    (333, 1000, 70, GEMM, False), (64, 2560, 16, GEMM, True),
])
def test_ternary_rowscale_bit_exact(gpu, oracle, N, K, M, path, with_bias):
    w, s = synth.ternary_weight((43, N, K), N, K, 0)
    x = synth.activations((44, M, K), M, K)
    qw = gpu.QWeight(gpu.W_TERNARY, N, K, 0, w, s)
    xq, xs, xq_d, xs_d = dev_inputs(gpu, oracle, x, qw.kpad)
    acc = run_acc(gpu, qw, xq_d, M, (M, N), path)
    codes = synth.unpack_ternary(w, K)
    assert np.array_equal(acc, xq[:, :K].astype(np.int64) @ codes.astype(np.int64).T)
    bias = synth.rng(45, N).standard_normal(N).astype(np.float32) if with_bias else None
    y = run_linear(gpu, qw, xq_d, xs_d, M, path, bias)
    oy = np.zeros((M, N), np.float32)
    oracle.orc_ternary_gemv_rowscale(P(w), P(s), P(xq), qw.kpad, P(xs), P(bias), P(oy), N, M, N, K)
    assert np.array_equal(y.view(np.uint32), oy.view(np.uint32))
    qw.close()


@pytest.mark.parametrize("fmt,N,K,M,path", [
    ("int8", 4864, 896, 1, GEMV), ("int8", 896, 4864, 1, GEMV), ("int8", 128, 896, 3, GEMV),
    ("int8", 4864, 896, 128, GEMM), ("int8", 77, 100, 20, GEMM),
    ("int8", 4864, 896, 32, GEMV), ("int8", 896, 4864, 63, GEMV), ("int8", 77, 100, 20, GEMV),
    ("int8", 9730, 1024, 24, 0), ("int8", 2600, 2560, 32, 0),   # the auto path's GEMV for large INT8 matrices
    ("int8", 896, 4864, 16, GEMV), ("int8", 896, 4864, 32, GEMV),   # 16 staged rows of 4864 columns: 8 pieces a thread
    ("int4", 3584, 1024, 1, GEMV), ("int4", 1024, 3584, 1, GEMV), ("int4", 3584, 1024, 32, GEMM),
    ("int4", 3584, 1024, 32, GEMV), ("int4", 1024, 3584, 16, GEMV),
    ("int4", 50, 333, 4, GEMV), ("int4", 50, 333, 40, GEMM), ("int4", 50, 333, 40, GEMV),
    # the GEMM's token tiles and splits chosen from the workgroup count: 16-token tiles with 4 splits along K
    # (896x4864 at 128), unsplit 16-token tiles (the stacked q|k|v), 32-token tiles (the stacked gate|up), INT4
    # FFN shapes at 64 and 32 tokens
    ("int8", 896, 4864, 128, GEMM), ("int8", 1152, 896, 128, GEMM), ("int8", 9728, 896, 128, GEMM),
    ("int4", 1024, 3584, 64, GEMM), ("int4", 7168, 1024, 32, GEMM),
])
def test_int_rowscale_bit_exact(gpu, oracle, fmt, N, K, M, path):
    if fmt == "int8":
        w, s = synth.int8_weight((46, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT8, N, K, 0, w, s)
        vals = w
    else:
        w, s = synth.int4_weight((47, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT4, N, K, 0, w, s)
        vals = synth.unpack_int4(w, K)
    x = synth.activations((48, M, K), M, K)
    xq, xs, xq_d, xs_d = dev_inputs(gpu, oracle, x, qw.kpad)
    acc = run_acc(gpu, qw, xq_d, M, (M, N), path)
    assert np.array_equal(acc, xq[:, :K].astype(np.int64) @ vals.astype(np.int64).T)
    fn = oracle.orc_int8_gemv_i8act if fmt == "int8" else oracle.orc_int4_gemv_i8act
    bias = synth.rng(45, N).standard_normal(N).astype(np.float32)
    exact = acc.astype(np.float64)
    for b in (None, bias):
        y = run_linear(gpu, qw, xq_d, xs_d, M, path, bias=b)
        oy = np.zeros((M, N), np.float32)
        fn(P(w), P(s), P(xq), qw.kpad, P(xs), P(b), P(oy), N, M, N, K)
        assert np.array_equal(y.view(np.uint32), oy.view(np.uint32))
        # the FP32 epilogue against the float64 closed form acc * xs[m] * s[r] + bias[r]
        assert cf.rowscale_error(y, exact, xs, s, b) <= cf.ROWSCALE_TOL
    qw.close()


def test_int4_tied_head_full_size(gpu, oracle):
    # the 151936 x 1024 INT4 head at M = 1 and 32 (GEMV) and M = 32 (GEMM): int32 sums against an exact integer
    # product; y (with a bias at 32 rows) bit for bit against the oracle and within 1e-6 of the float64 closed form
    N, K = synth.QWEN35_INT4_HEAD[1:]
    w, s = synth.int4_weight((49,), N, K)
    qw = gpu.QWeight(gpu.W_INT4, N, K, 0, w, s)
    vals = synth.unpack_int4(w, K).astype(np.float64)
    for M, path in ((1, GEMV), (32, GEMV), (32, GEMM)):
        x = synth.activations((50, M), M, K)
        xq, xs, xq_d, xs_d = dev_inputs(gpu, oracle, x, qw.kpad)
        acc = run_acc(gpu, qw, xq_d, M, (M, N), path)
        exact = xq[:, :K].astype(np.float64) @ vals.T          # integer-valued, |sums| < 2^53
        assert np.array_equal(acc.astype(np.float64), exact)
        bias = synth.rng(51, N).standard_normal(N).astype(np.float32) if M > 1 else None
        y = run_linear(gpu, qw, xq_d, xs_d, M, path, bias=bias)
        oy = np.zeros((M, N), np.float32)
        oracle.orc_int4_gemv_i8act(P(w), P(s), P(xq), qw.kpad, P(xs), P(bias), P(oy), N, M, N, K)
        assert np.array_equal(y.view(np.uint32), oy.view(np.uint32)), (M, path)
        # the FP32 epilogue against the float64 closed form acc * xs[m] * s[r] + bias[r]
        assert cf.rowscale_error(y, exact, xs, s, bias) <= cf.ROWSCALE_TOL, (M, path)
    qw.close()


@pytest.mark.parametrize("fmt,N,K,g", [("tern", 3840, 2560, 128), ("tern", 2560, 6912, 96), ("int8", 896, 4864, 0),
                                       ("int4", 3000, 1024, 0)])
def test_gemv_token_chunks(gpu, oracle, fmt, N, K, g):
    """Token rows per workgroup and row tiles per workgroup change the launch of a 40-token GEMV, never the
    result (y and the integer sums, bit for bit against the oracle)."""
    lib = gpu.load()
    M = 40
    if fmt == "tern":
        w, s = synth.ternary_weight((63, N, K, g), N, K, g)
        qw = gpu.QWeight(gpu.W_TERNARY, N, K, g, w, s)
    elif fmt == "int8":
        w, s = synth.int8_weight((64, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT8, N, K, 0, w, s)
    else:
        w, s = synth.int4_weight((65, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT4, N, K, 0, w, s)
    x = synth.activations((66, M, K), M, K)
    xq, xs, xq_d, xs_d = dev_inputs(gpu, oracle, x, qw.kpad)
    oy = np.zeros((M, N), np.float32)
    if fmt == "tern":
        ng = -(-K // g)
        oacc = np.zeros((M, N, ng), np.int32)
        oracle.orc_ternary_acc_i32(P(w), P(xq), qw.kpad, M, N, K, g, P(oacc))
        oracle.orc_ternary_gemv_grouped(P(w), P(s), g, P(xq), qw.kpad, P(xs), None, P(oy), N, M, N, K)
        shape = (M, N, ng)
    else:
        oacc = np.zeros((M, N), np.int32)
        acc_fn = oracle.orc_int8_acc_i32 if fmt == "int8" else oracle.orc_int4_acc_i32
        acc_fn(P(w), P(xq), qw.kpad, M, N, K, P(oacc))
        fn = oracle.orc_int8_gemv_i8act if fmt == "int8" else oracle.orc_int4_gemv_i8act
        fn(P(w), P(s), P(xq), qw.kpad, P(xs), None, P(oy), N, M, N, K)
        shape = (M, N)
    try:
        for ch in (0, 16, 8, 4, 2, 1):
            for rt in (0, 1, 4):
                lib.eif_hip_set_gemv_token_chunk(ch)
                lib.eif_hip_set_gemv_row_tiles(rt)
                y = run_linear(gpu, qw, xq_d, xs_d, M, GEMV)
                assert np.array_equal(y.view(np.uint32), oy.view(np.uint32)), (ch, rt)
                acc = run_acc(gpu, qw, xq_d, M, shape, GEMV)
                assert np.array_equal(acc, oacc), (ch, rt)
    finally:
        lib.eif_hip_set_gemv_token_chunk(0)
        lib.eif_hip_set_gemv_row_tiles(0)
        qw.close()


def test_bitnet_layer_prefill_512(gpu, oracle):
    # every linear of the BitNet-2B-shaped layer at M = 512 through the MFMA GEMM, group sums exact
    import torch
    M = 512
    for name, N, K, g in synth.BITNET_2B_LAYER:
        w, s = synth.ternary_weight((51, N, K, g), N, K, g)
        x = synth.activations((52, K), M, K)
        qw = gpu.QWeight(gpu.W_TERNARY, N, K, g, w, s)
        xq, xs, xq_d, xs_d = dev_inputs(gpu, oracle, x, qw.kpad)
        y = run_linear(gpu, qw, xq_d, xs_d, M, GEMM)
        codes = synth.unpack_ternary(w, K).astype(np.float64)
        ng = K // g
        want = np.zeros((M, N))
        mag = np.zeros((M, N))
        for gi in range(ng):
            a = xq[:, gi * g:(gi + 1) * g].astype(np.float64) @ codes[:, gi * g:(gi + 1) * g].T   # exact ints
            want += a * s[None, :, gi]
            mag += np.abs(a) * s[None, :, gi]
        want *= xs[:, None]
        mag *= xs[:, None]
        err = np.abs(y - want) / (mag + 1e-30)
        assert err.max() <= REL_TOL, (name, err.max())
        qw.close()
        del xq_d, xs_d
        torch.cuda.empty_cache()


FUSED = [
    # fmt, N, K, group, M, wht block, signed
    ("tern", 6912, 2560, 128, 1, 128, False),   # the single BitNet linear, prep fused
    ("tern", 2560, 6912, 96, 1, 128, True),     # down projection
    ("tern", 3840, 2560, 128, 4, 128, True),
    ("tern", 100, 640, 64, 8, 64, False),
    ("tern", 64, 2560, 0, 3, 128, False),       # row scales
    ("tern", 256, 4096, 128, 2, 1024, True),    # largest WHT block of the fused prep
    ("tern", 96, 16384, 128, 1, 128, False),    # longest row of the fused prep
    ("int8", 4864, 896, 0, 1, 0, False),
    ("int4", 3584, 1024, 0, 2, 0, False),
]


@pytest.mark.parametrize("fmt,N,K,g,M,block,signed", FUSED)
def test_fused_prep_linear(gpu, oracle, fmt, N, K, g, M, block, signed):
    """prep fused into the GEMV launch == prep kernel + GEMV, bit for bit; int32 sums == oracle."""
    import ctypes as C
    import torch
    dev = torch.device("cuda:0")
    if fmt == "tern":
        w, s = synth.ternary_weight((53, N, K, g), N, K, g)
        qw = gpu.QWeight(gpu.W_TERNARY, N, K, g, w, s)
    elif fmt == "int8":
        w, s = synth.int8_weight((54, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT8, N, K, 0, w, s)
    else:
        w, s = synth.int4_weight((55, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT4, N, K, 0, w, s)
    x = synth.activations((56, M, K), M, K)
    signs = np.where(synth.rng(57, K).uniform(size=K) > 0.5, 1.0, -1.0).astype(np.float32) if signed else None
    norm = gpu.wht_norm(block) if block else 1.0
    xd = torch.from_numpy(x).to(dev)
    sd = torch.from_numpy(signs).to(dev) if signed else None
    # two-call path
    xq_d = torch.zeros((M, qw.kpad), dtype=torch.int8, device=dev)
    xs_d = torch.zeros(M, dtype=torch.float32, device=dev)
    gpu.prep_rows(xd, xq_d, xs_d, block, norm, signs=sd)
    y2 = run_linear(gpu, qw, xq_d, xs_d, M, GEMV)
    # fused path
    y1 = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    qw.linear_f32(xd, y1, block, norm, signs=sd)
    ng = -(-K // g) if (fmt == "tern" and g > 0) else 0
    acc = torch.full((M, N, ng) if ng else (M, N), -7, dtype=torch.int32, device=dev)
    qw.acc_f32(xd, acc, block, norm, signs=sd)
    torch.cuda.synchronize()
    y1 = y1.cpu().numpy()
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    # oracle: prep + exact integer sums
    xq = np.zeros((M, qw.kpad), np.int8)
    xs = np.zeros(M, np.float32)
    assert oracle.orc_prep_rows(P(x), K, P(signs), M, K, block, C.c_float(norm), P(xq), qw.kpad, P(xs), None, 0) == 0
    if fmt == "tern" and ng:
        oacc = np.zeros((M, N, ng), np.int32)
        oracle.orc_ternary_acc_i32(P(w), P(xq), qw.kpad, M, N, K, g, P(oacc))
    elif fmt == "tern":
        oacc = xq[:, :K].astype(np.int64) @ synth.unpack_ternary(w, K).astype(np.int64).T
    elif fmt == "int8":
        oacc = xq[:, :K].astype(np.int64) @ w.astype(np.int64).T
    else:
        oacc = xq[:, :K].astype(np.int64) @ synth.unpack_int4(w, K).astype(np.int64).T
    assert np.array_equal(acc.cpu().numpy(), oacc)
    qw.close()


@pytest.mark.parametrize("kind", [34, 35, 8])
def test_gguf_ternary_weight(gpu, oracle, kind):
    """GGUF TL1/TL2/Q8_0 projection rows -> 2-bit rows + row scales (eif_gguf_ternary_rows) == the oracle byte for
    byte; the resident weight (eif_hip_qweight_from_gguf_ternary) gives the exact integer sums of those codes."""
    import ctypes as C
    import torch
    from test_oracle_pins import _gguf_blocks
    N, K = 300, 2560
    r = np.random.default_rng(97 + kind)
    raw, _ = _gguf_blocks(r, kind, N, K)
    rb = K // 4
    codes = np.zeros((N, rb), np.uint8)
    sc = np.zeros(N, np.float32)
    assert gpu.load().eif_gguf_ternary_rows(kind, P(raw), N, K, P(codes), P(sc)) == 0
    oc = np.zeros((N, rb), np.uint8)
    osc = np.zeros(N, np.float32)
    oracle.orc_gguf_ternary_rows(kind, P(raw), N, K, P(oc), P(osc))
    assert np.array_equal(codes, oc) and np.array_equal(sc.view(np.uint32), osc.view(np.uint32))
    h = C.c_void_p()
    gpu.check(gpu.load().eif_hip_qweight_from_gguf_ternary(C.byref(h), kind, P(raw), N, K, None),
              "eif_hip_qweight_from_gguf_ternary")
    qw = gpu.QWeight.wrap(h)
    assert (qw.rows, qw.cols, qw.group) == (N, K, 0)
    x = synth.activations((98, 3), 3, K)
    xq, xs, xq_d, xs_d = dev_inputs(gpu, oracle, x, qw.kpad)
    acc = run_acc(gpu, qw, xq_d, 3, (3, N), GEMV)
    want = xq[:, :K].astype(np.int64) @ synth.unpack_ternary(oc, K).astype(np.int64).T
    assert np.array_equal(acc, want)
    qw.close()


@pytest.mark.parametrize("fmt,N,K", [("int4", 151936, 1024), ("int4", 65600, 2048), ("int8", 70001, 512),
                                     ("int8", 65536, 1024)])
def test_stream_gemv(gpu, oracle, fmt, N, K):
    """The streaming GEMV of vocabulary-sized row-scaled matrices (65,536 rows or more, 8 or 16 steps along K)
    at M = 1, 5, 16, 17 and 32, with and without a bias: y and the integer sums bit for bit against the oracle,
    and the same bits with the stream off (the tiled GEMV), at other launch sizes and on the row-tile layout
    instead of the tile-major copy."""
    lib = gpu.load()
    if fmt == "int8":
        w, s = synth.int8_weight((67, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT8, N, K, 0, w, s)
        fn = oracle.orc_int8_gemv_i8act
    else:
        w, s = synth.int4_weight((68, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT4, N, K, 0, w, s)
        fn = oracle.orc_int4_gemv_i8act
    old = lib.eif_hip_set_gemv_stream(0)
    try:
        for M in (1, 5, 16, 17, 32):
            x = synth.activations((69, M, K), M, K)
            xq, xs, xq_d, xs_d = dev_inputs(gpu, oracle, x, qw.kpad)
            bias = synth.rng(70, M).standard_normal(N).astype(np.float32) if M % 2 else None
            oy = np.zeros((M, N), np.float32)
            fn(P(w), P(s), P(xq), qw.kpad, P(xs), P(bias), P(oy), N, M, N, K)
            for wpc in (0, 3, -2, -1):   # -2: the row-tile layout instead of the tile-major copy
                lib.eif_hip_set_gemv_stream(wpc)
                y = run_linear(gpu, qw, xq_d, xs_d, M, GEMV, bias)
                assert np.array_equal(y.view(np.uint32), oy.view(np.uint32)), (M, wpc)
            lib.eif_hip_set_gemv_stream(0)
            if M in (1, 17):
                acc = run_acc(gpu, qw, xq_d, M, (M, N), GEMV)
                oacc = np.zeros((M, N), np.int32)
                (oracle.orc_int8_acc_i32 if fmt == "int8" else oracle.orc_int4_acc_i32)(P(w), P(xq), qw.kpad, M, N,
                                                                                       K, P(oacc))
                assert np.array_equal(acc, oacc), M
    finally:
        lib.eif_hip_set_gemv_stream(old)
    qw.close()


@pytest.mark.parametrize("fmt,N,K,mode", [("int4", 151936, 1024, 0), ("int8", 128256, 2560, 0),
                                          ("int8", 65600, 512, 0), ("int4", 16390, 2048, 0), ("int8", 9730, 2560, 0),
                                          ("int4", 1000, 2048, 1), ("int4", 77, 4096, 1),
                                          ("int8", 130, 1536, 1), ("int8", 64, 2048, 1)])
def test_rowpair_gemv(gpu, oracle, fmt, N, K, mode):
    """The row-pair GEMV (one token row; rows of whole 512-byte runs read half a wave at a time, v_dot4 products
    on the resident layout) on its default shapes (16,384 rows or 20 MB of codes and more: vocabulary heads, ragged
    mid-size matrices on either side of the rule) and, forced on, on small and ragged ones:
    y with and without a bias and the int32 sums bit for bit against the oracle, and the same bits with it off
    (the tiled GEMV)."""
    lib = gpu.load()
    if fmt == "int8":
        w, s = synth.int8_weight((71, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT8, N, K, 0, w, s)
        fn, afn = oracle.orc_int8_gemv_i8act, oracle.orc_int8_acc_i32
    else:
        w, s = synth.int4_weight((72, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT4, N, K, 0, w, s)
        fn, afn = oracle.orc_int4_gemv_i8act, oracle.orc_int4_acc_i32
    old = lib.eif_hip_set_gemv_rowpair(mode)
    try:
        x = synth.activations((73, N, K), 1, K)
        xq, xs, xq_d, xs_d = dev_inputs(gpu, oracle, x, qw.kpad)
        oacc = np.zeros((1, N), np.int32)
        afn(P(w), P(xq), qw.kpad, 1, N, K, P(oacc))
        for bias in (None, synth.rng(74, N).standard_normal(N).astype(np.float32)):
            oy = np.zeros((1, N), np.float32)
            fn(P(w), P(s), P(xq), qw.kpad, P(xs), P(bias), P(oy), N, 1, N, K)
            for m in (mode, -1):
                lib.eif_hip_set_gemv_rowpair(m)
                y = run_linear(gpu, qw, xq_d, xs_d, 1, GEMV, bias)
                assert np.array_equal(y.view(np.uint32), oy.view(np.uint32)), (m, bias is None)
        for m in (mode, -1):
            lib.eif_hip_set_gemv_rowpair(m)
            acc = run_acc(gpu, qw, xq_d, 1, (1, N), GEMV)
            assert np.array_equal(acc, oacc), m
    finally:
        lib.eif_hip_set_gemv_rowpair(old)
    qw.close()
