"""GPU activation prep (sign flip + blockwise WHT + absmax INT8) against the oracle: bit-exact int8 codes, scales
and rotated FP32 rows."""
import ctypes as C

import numpy as np
import pytest

from conftest import P
import synth

pytestmark = pytest.mark.gpu


def run_case(gpu, oracle, x, block, signs=None, with_rot=False, ldq=None):
    import torch
    M, K = x.shape
    ldq = ldq or (K + 255) // 256 * 256
    norm = gpu.wht_norm(block) if block else 1.0
    dev = torch.device("cuda:0")
    xd = torch.from_numpy(x).to(dev)
    sd = torch.from_numpy(signs).to(dev) if signs is not None else None
    xq = torch.full((M, ldq), 77, dtype=torch.int8, device=dev)
    xs = torch.zeros(M, dtype=torch.float32, device=dev)
    xr = torch.zeros((M, K), dtype=torch.float32, device=dev) if with_rot else None
    gpu.prep_rows(xd, xq, xs, block, norm, signs=sd, xrot=xr)
    torch.cuda.synchronize()
    oq = np.zeros((M, ldq), np.int8)
    os_ = np.zeros(M, np.float32)
    orot = np.zeros((M, K), np.float32)
    rc = oracle.orc_prep_rows(P(x), K, P(signs), M, K, block, C.c_float(norm), P(oq), ldq, P(os_), P(orot), K)
    assert rc == 0
    assert np.array_equal(xq.cpu().numpy(), oq)
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), os_.view(np.uint32))
    if with_rot:
        assert np.array_equal(xr.cpu().numpy().view(np.uint32), orot.view(np.uint32))


@pytest.mark.parametrize("M,K,block,signed", [
    (1, 2560, 128, False),      # single BitNet linear input
    (8, 2560, 128, True),
    (64, 6912, 128, False),     # down-projection input
    (3, 896, 0, False),         # INT8 layer input, no rotation
    (5, 1024, 1024, True),
    (2, 4864, 0, False),
    (1, 12288, 4096, True),     # largest row of the fused kernel
    (512, 2560, 128, False),    # prefill batch
    (3, 2560, 512, True),       # largest block of the register path
    (2, 2560, 1, True),         # block 1: signs and norm only
    (2, 996, 4, True),          # K % 8 != 0: LDS path with a small block
    (4, 11264, 256, False),     # six chunks of the register path
])
def test_prep_matches_oracle(gpu, oracle, M, K, block, signed):
    x = synth.activations((31, M, K), M, K)
    signs = np.where(synth.rng(32, K).uniform(size=K) > 0.5, 1.0, -1.0).astype(np.float32) if signed else None
    run_case(gpu, oracle, x, block, signs, with_rot=True)


@pytest.mark.parametrize("K,block", [(16384, 128), (32768, 16384)])
def test_prep_long_rows(gpu, oracle, K, block):
    # rows beyond the fused kernel's LDS: segment rotation (block <= 8192) or one launch per stage
    x = synth.activations((33, K), 2, K)
    signs = np.where(synth.rng(34, K).uniform(size=K) > 0.5, 1.0, -1.0).astype(np.float32)
    run_case(gpu, oracle, x, block, signs, with_rot=True)


def test_prep_edge_rows(gpu, oracle):
    K = 256
    x = np.zeros((6, K), np.float32)
    x[1] = 1e-13                                   # amax < 1e-12: zeros, scale 1
    x[2, :8] = [127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 63.5]  # ties at .5 with amax 127
    x[3] = synth.activations((35,), 1, K)[0] * 1e-30   # tiny but above the threshold
    x[4] = np.linspace(-3, 3, K, dtype=np.float32)
    x[5, 17] = -5.0                                # single negative spike
    run_case(gpu, oracle, x, 0)
    run_case(gpu, oracle, x, 64)


def test_prep_random_scales(gpu, oracle):
    # many amax values: exercises the correctly rounded 127/amax and amax*(1/127)
    r = np.random.default_rng(36)
    x = (r.standard_normal((200, 320)) * r.uniform(1e-6, 1e6, (200, 1))).astype(np.float32)
    run_case(gpu, oracle, x, 32)
