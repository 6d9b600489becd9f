"""The pre-ops of the fused prep (eif_hip_prep_spec: RMSNorm, SiLU-gate + RMSNorm) and the prep on its own.

* eif_hip_prep_spec_rows against the reference's formulas restated in float32 numpy (RMSNorm: sequential
  sum of squares, (x * (1 / sqrtf(ss / K + eps))) * w, src/eif_tinyllm.c:196-330; SiLU gate: (g * (1 / (1 +
  expf(-g)))) * u, :774-780) followed by the oracle's prep (WHT + absmax INT8). The GPU sums the squares in
  another order, so a code that sits on a rounding boundary may take its neighbour: codes agree to +-1 with
  at most 1% of them off by one, and the scales to 1e-5.
* The prep on its own followed by the GEMV == the prep fused into the GEMV, bit for bit (one prep code).
* A vocabulary-sized row-scaled matrix (65536 rows or more) at M = 1 takes a prep launch and then the GEMV:
  the same bits as the prep-then-GEMV pair, and the oracle's INT8 GEMV of those codes bit for bit.
"""
import ctypes as C

import numpy as np
import pytest

from conftest import P
import synth

pytestmark = pytest.mark.gpu


def ref_pre(x, pre, x2, nw, eps):
    """The reference's float32 pre-ops, one row at a time, sums in column order."""
    out = np.empty_like(x)
    for m in range(x.shape[0]):
        v = x[m].astype(np.float32)
        if pre == 2:
            one = np.float32(1.0)
            v = (v * (one / (one + np.exp(-v)))) * x2[m]
        ss = np.float32(0.0)
        for e in v:
            ss = np.float32(ss + np.float32(e * e))
        inv = np.float32(1.0) / np.sqrt(np.float32(ss / np.float32(len(v)) + np.float32(eps)))
        out[m] = (v * inv) * (nw if nw is not None else np.float32(1.0))
    return out


CASES = [
    # pre, K, M, WHT block, signed, norm weight
    (0, 2560, 1, 128, True, False),
    (1, 2560, 1, 128, True, True),
    (1, 2560, 3, 0, False, True),
    (1, 6912, 2, 128, False, False),
    (2, 6912, 1, 128, True, True),
    (2, 1024, 4, 256, False, True),
]


@pytest.mark.parametrize("pre,K,M,block,signed,with_w", CASES)
def test_prep_spec_rows_vs_formula(gpu, oracle, pre, K, M, block, signed, with_w):
    import torch
    dev = torch.device("cuda:0")
    r = synth.rng(60, pre, K, M)
    x = (r.standard_normal((M, K)) * 2.0).astype(np.float32)
    x2 = r.standard_normal((M, K)).astype(np.float32) if pre == 2 else None
    nw = (1.0 + 0.1 * r.standard_normal(K)).astype(np.float32) if with_w else None
    signs = np.where(r.uniform(size=K) > 0.5, 1.0, -1.0).astype(np.float32) if signed else None
    eps = 1e-5
    norm = gpu.wht_norm(block) if block else 1.0
    ldq = (K + 255) // 256 * 256
    xd = torch.from_numpy(x).to(dev)
    x2d = torch.from_numpy(x2).to(dev) if x2 is not None else None
    nwd = torch.from_numpy(nw).to(dev) if nw is not None else None
    sd = torch.from_numpy(signs).to(dev) if signed else None
    xq = torch.full((M, ldq), 99, dtype=torch.int8, device=dev)
    xs = torch.zeros(M, dtype=torch.float32, device=dev)
    sp = gpu.prep_spec(xd, pre=pre, x2=x2d, norm_w=nwd, eps=eps, signs=sd, block=block, norm=norm)
    gpu.prep_spec_rows(sp, K, xq, xs, M)
    torch.cuda.synchronize()
    gq, gs = xq.cpu().numpy(), xs.cpu().numpy()
    assert not gq[:, K:].any()                                   # zeros past K
    v = ref_pre(x, pre, x2, nw, eps) if pre else x
    oq = np.zeros((M, ldq), np.int8)
    os_ = np.zeros(M, np.float32)
    assert oracle.orc_prep_rows(P(np.ascontiguousarray(v)), K, P(signs), M, K, block, C.c_float(norm), P(oq), ldq,
                                P(os_), None, 0) == 0
    d = np.abs(gq.astype(np.int32) - oq.astype(np.int32))
    if pre == 0:
        assert d.max() == 0 and np.array_equal(gs.view(np.uint32), os_.view(np.uint32))
    else:
        assert d.max() <= 1 and (d > 0).mean() <= 0.01, (d.max(), (d > 0).mean())
        assert np.abs(gs - os_).max() <= 1e-5 * np.abs(os_).max()


@pytest.mark.parametrize("fmt,N,K,g,pre,M", [
    ("tern", 3840, 2560, 128, 1, 1),
    ("tern", 2560, 6912, 96, 2, 1),
    ("tern", 13824, 2560, 128, 1, 3),
    ("int8", 4864, 896, 0, 1, 2),
    ("int4", 1024, 3584, 0, 2, 1),
])
def test_prep_spec_rows_then_linear_equals_fused(gpu, fmt, N, K, g, pre, M):
    import torch
    dev = torch.device("cuda:0")
    if fmt == "tern":
        w, s = synth.ternary_weight((61, N, K, g), N, K, g)
        qw = gpu.QWeight(gpu.W_TERNARY, N, K, g, w, s)
    elif fmt == "int8":
        w, s = synth.int8_weight((62, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT8, N, K, 0, w, s)
    else:
        w, s = synth.int4_weight((63, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT4, N, K, 0, w, s)
    r = synth.rng(64, N, K)
    x = torch.from_numpy(r.standard_normal((M, K)).astype(np.float32)).to(dev)
    x2 = torch.from_numpy(r.standard_normal((M, K)).astype(np.float32)).to(dev) if pre == 2 else None
    nw = torch.from_numpy((1.0 + 0.1 * r.standard_normal(K)).astype(np.float32)).to(dev)
    bias = torch.from_numpy(r.standard_normal(N).astype(np.float32)).to(dev)
    block = 128 if fmt == "tern" else 0
    sp = gpu.prep_spec(x, pre=pre, x2=x2, norm_w=nw, eps=1e-5, block=block,
                       norm=gpu.wht_norm(block) if block else 1.0)
    y1 = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    gpu.check(gpu.load().eif_hip_qlinear_prep(qw.h, C.byref(sp), gpu.ptr(bias), gpu.ptr(y1), N, M,
                                              gpu.stream_ptr()), "eif_hip_qlinear_prep")
    xq = torch.zeros((M, qw.kpad), dtype=torch.int8, device=dev)
    xs = torch.zeros(M, dtype=torch.float32, device=dev)
    gpu.prep_spec_rows(sp, K, xq, xs, M)
    y2 = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    qw.linear(xq, xs, y2, M=M, bias=bias, path=1)
    torch.cuda.synchronize()
    assert np.array_equal(y1.cpu().numpy().view(np.uint32), y2.cpu().numpy().view(np.uint32))
    qw.close()


@pytest.mark.parametrize("fmt,N,K", [("int8", 70000, 512), ("int4", 66000, 1024)])
def test_vocab_head_two_step(gpu, oracle, fmt, N, K):
    import torch
    dev = torch.device("cuda:0")
    if fmt == "int8":
        w, s = synth.int8_weight((65, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT8, N, K, 0, w, s)
    else:
        w, s = synth.int4_weight((66, N, K), N, K)
        qw = gpu.QWeight(gpu.W_INT4, N, K, 0, w, s)
    r = synth.rng(67, N, K)
    x = torch.from_numpy(r.standard_normal((1, K)).astype(np.float32)).to(dev)
    nw = torch.from_numpy((1.0 + 0.1 * r.standard_normal(K)).astype(np.float32)).to(dev)
    sp = gpu.prep_spec(x, pre=1, norm_w=nw, eps=1e-6)
    y1 = torch.full((1, N), float("nan"), dtype=torch.float32, device=dev)
    gpu.check(gpu.load().eif_hip_qlinear_prep(qw.h, C.byref(sp), None, gpu.ptr(y1), N, 1, gpu.stream_ptr()),
              "eif_hip_qlinear_prep")
    xq = torch.zeros((1, qw.kpad), dtype=torch.int8, device=dev)
    xs = torch.zeros(1, dtype=torch.float32, device=dev)
    gpu.prep_spec_rows(sp, K, xq, xs, 1)
    y2 = torch.full((1, N), float("nan"), dtype=torch.float32, device=dev)
    qw.linear(xq, xs, y2, M=1, path=1)
    torch.cuda.synchronize()
    y1, y2 = y1.cpu().numpy(), y2.cpu().numpy()
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    hq, hs = xq.cpu().numpy(), xs.cpu().numpy()
    oy = np.zeros((1, N), np.float32)
    fn = oracle.orc_int8_gemv_i8act if fmt == "int8" else oracle.orc_int4_gemv_i8act
    fn(P(w), P(s), P(hq), qw.kpad, P(hs), None, P(oy), N, 1, N, K)
    assert np.array_equal(y1.view(np.uint32), oy.view(np.uint32))
    qw.close()


@pytest.mark.parametrize("N,K,M", [(13824, 2560, 1), (512, 640, 3)])
def test_glu_form(gpu, oracle, N, K, M):
    """eif_hip_qlinear_prep_glu: SiLU(gate) * up of the stacked gate|up matrix in one launch. Fed to the next linear
    with the RMSNorm pre-op, its rows give the bits of the two halves with the SwiGLU pre-op; against the two halves
    it is the SwiGLU of src/eif_tinyllm.c:774-780 to float32 rounding."""
    import torch
    dev = torch.device("cuda:0")
    lib = gpu.load()
    h = N // 2
    w, s = synth.ternary_weight((66, N, K), N, K, 128)
    qw = gpu.QWeight(gpu.W_TERNARY, N, K, 128, w, s)
    wd, sd = synth.ternary_weight((67, K, h), K, h, 128 if h % 128 == 0 else 64)
    gd = 128 if h % 128 == 0 else 64
    qd = gpu.QWeight(gpu.W_TERNARY, K, h, gd, wd, sd)
    r = synth.rng(68, N, K)
    x = torch.from_numpy(r.standard_normal((M, K)).astype(np.float32)).to(dev)
    nw = torch.from_numpy((1.0 + 0.1 * r.standard_normal(K)).astype(np.float32)).to(dev)
    nw2 = torch.from_numpy((1.0 + 0.1 * r.standard_normal(h)).astype(np.float32)).to(dev)
    sp = gpu.prep_spec(x, pre=1, norm_w=nw, eps=1e-5, block=128, norm=gpu.wht_norm(128))
    yg = torch.full((M, h), float("nan"), dtype=torch.float32, device=dev)
    gpu.check(lib.eif_hip_qlinear_prep_glu(qw.h, C.byref(sp), gpu.ptr(yg), h, M, gpu.stream_ptr()),
              "eif_hip_qlinear_prep_glu")
    y2 = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    gpu.check(lib.eif_hip_qlinear_prep(qw.h, C.byref(sp), None, gpu.ptr(y2), N, M, gpu.stream_ptr()),
              "eif_hip_qlinear_prep")
    torch.cuda.synchronize()
    g, u = y2[:, :h].cpu().numpy(), y2[:, h:].cpu().numpy()
    want = (g * (np.float32(1.0) / (np.float32(1.0) + np.exp(-g)))) * u
    got = yg.cpu().numpy()
    assert np.max(np.abs(got - want) / (np.abs(want) + 1e-30 + 1e-6 * np.abs(want).max())) <= 1e-5
    # the down projection: RMSNorm pre-op on the GLU rows == SwiGLU pre-op on the two halves, bit for bit
    blk = 128 if h % 128 == 0 else 64
    ya = torch.full((M, K), float("nan"), dtype=torch.float32, device=dev)
    yb = torch.full((M, K), float("nan"), dtype=torch.float32, device=dev)
    spa = gpu.prep_spec(yg, pre=1, norm_w=nw2, eps=1e-5, block=blk, norm=gpu.wht_norm(blk))
    spb = gpu.prep_spec(y2[:, :h], pre=2, x2=y2[:, h:], norm_w=nw2, eps=1e-5, block=blk, norm=gpu.wht_norm(blk))
    gpu.check(lib.eif_hip_qlinear_prep(qd.h, C.byref(spa), None, gpu.ptr(ya), K, M, gpu.stream_ptr()), "down a")
    gpu.check(lib.eif_hip_qlinear_prep(qd.h, C.byref(spb), None, gpu.ptr(yb), K, M, gpu.stream_ptr()), "down b")
    torch.cuda.synchronize()
    assert np.array_equal(ya.cpu().numpy().view(np.uint32), yb.cpu().numpy().view(np.uint32))
    # a shape outside the form is refused (the caller takes the two-step path)
    w3, s3 = synth.ternary_weight((69, 96, K), 96, K, 128)
    q3 = gpu.QWeight(gpu.W_TERNARY, 96, K, 128, w3, s3)
    assert lib.eif_hip_qlinear_prep_glu(q3.h, C.byref(sp), gpu.ptr(yg), h, M, gpu.stream_ptr()) == -4   # LIMIT
    for q in (qw, qd, q3):
        q.close()
