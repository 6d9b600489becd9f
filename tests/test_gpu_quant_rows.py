"""FP32 weight rows -> INT8 / INT4 row-scaled codes on the GPU (eif_hip_quant_rows) against the oracle's restatement
of the reference's GGUF import quant_rows (src/eif_qwen35_gguf.c:225-258): codes and scales bit for bit, at a
vocabulary head's full size too; then the quantized INT4 head feeds the INT4 GEMV, whose output equals the
oracle's GEMV of the same codes bit for bit.
"""
import numpy as np
import pytest

from conftest import P
import synth

pytestmark = pytest.mark.gpu


def run_gpu(gpu, x, bits, ldx=None):
    import torch
    dev = torch.device("cuda:0")
    rows, cols = x.shape
    ldx = ldx or cols
    xp = np.zeros((rows, ldx), np.float32)
    xp[:, :cols] = x
    xd = torch.from_numpy(xp).to(dev)[:, :cols]
    rb = cols if bits == 8 else (cols + 1) // 2
    dst = torch.full((rows, rb), 0xAB, dtype=torch.uint8, device=dev)
    sc = torch.zeros(rows, dtype=torch.float32, device=dev)
    gpu.quant_rows(xd, bits, dst, sc)
    torch.cuda.synchronize()
    return dst, sc


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rows,cols,ldx", [(7, 64, None), (5, 33, 40), (300, 1024, None), (2, 1, None),
                                           (64, 3584, 3600)])
def test_quant_rows_vs_oracle(gpu, oracle, bits, rows, cols, ldx):
    r = np.random.default_rng(80 + bits + cols)
    x = (r.standard_normal((rows, cols)) * 10.0 ** r.integers(-3, 3, (rows, 1))).astype(np.float32)
    if rows > 2:
        x[2] = 0.0
    dst, sc = run_gpu(gpu, x, bits, ldx)
    rb = cols if bits == 8 else (cols + 1) // 2
    od = np.zeros((rows, rb), np.uint8)
    osc = np.zeros(rows, np.float32)
    oracle.orc_quant_rows(P(x), cols, rows, cols, bits, P(od), P(osc))
    assert np.array_equal(dst.cpu().numpy(), od)
    assert np.array_equal(sc.cpu().numpy().view(np.uint32), osc.view(np.uint32))


def test_quantized_int4_head_feeds_gemv(gpu, oracle):
    # the tied head 151936 x 1024 from FP32 rows: quantized on the GPU, repacked from device memory, GEMV at M = 1
    import torch
    N, K = synth.QWEN35_INT4_HEAD[1:]
    r = np.random.default_rng(90)
    x = (r.standard_normal((N, K)) * 0.05).astype(np.float32)
    dst, sc = run_gpu(gpu, x, 4)
    od = np.zeros((N, K // 2), np.uint8)
    osc = np.zeros(N, np.float32)
    oracle.orc_quant_rows(P(x), K, N, K, 4, P(od), P(osc))
    assert np.array_equal(dst.cpu().numpy(), od) and np.array_equal(sc.cpu().numpy(), osc)
    del x
    qw = gpu.QWeight(gpu.W_INT4, N, K, 0, dst, sc, on_device=True)
    act = synth.activations((91, 1), 1, K)
    xq = np.zeros((1, qw.kpad), np.int8)
    xs = np.zeros(1, np.float32)
    assert oracle.orc_prep_rows(P(act), K, None, 1, K, 0, 1.0, P(xq), qw.kpad, P(xs), None, 0) == 0
    y = torch.full((1, N), float("nan"), dtype=torch.float32, device="cuda:0")
    qw.linear(torch.from_numpy(xq).cuda(), torch.from_numpy(xs).cuda(), y, M=1, path=1)
    torch.cuda.synchronize()
    oy = np.zeros((1, N), np.float32)
    oracle.orc_int4_gemv_i8act(P(od), P(osc), P(xq), qw.kpad, P(xs), None, P(oy), N, 1, N, K)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), oy.view(np.uint32))
    qw.close()
