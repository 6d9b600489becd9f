"""The host-pointer drop-in ABI (the reference's own symbols) on the GPU, against the outputs the reference
produced (tests/golden) and the oracle. Integer / quantization / WHT paths bit for bit, FP32-activation GEMVs to
1e-5 of sum |w*x| (the reference tests' normalisation)."""
import ctypes as C
import os
import threading

import numpy as np
import pytest

from conftest import P, ROOT
import synth

pytestmark = pytest.mark.gpu
GOLD = os.path.join(ROOT, "tests", "golden", "reference_vectors.npz")


@pytest.fixture(scope="module")
def gold():
    # Every array materialized once and kept for the module: the host API keeps device copies of weight buffers
    # keyed by their host address (weights live in stable pools, as in the reference), so a weight array must not
    # be freed and another allocated at its address while its copy is cached. An NpzFile makes a new array on
    # every access.
    with np.load(GOLD) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="module")
def lib(gpu):
    lib = gpu.load()
    lib.eif_hip_forget_host_weights(None)   # no copies left by earlier tests' freed buffers
    yield lib
    lib.eif_hip_forget_host_weights(None)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def within(y, want, mag, tol=1e-5):
    return np.max(np.abs(y.astype(np.float64) - want.astype(np.float64)) / (tol * mag + 1e-30)) <= 1.0


def test_hadamard_rotate(lib, oracle, gold):
    for name in ("wht_2560_128", "wht_4096_1024"):
        n, b, signed = (int(v) for v in gold[name + "_meta"])
        y = gold[name + "_x"].copy()
        signs = gold[name + "_signs"] if signed else None
        lib.eif_hadamard_rotate_f32(P(y), P(signs), n, b)
        # the oracle with the norm this host's build computes: bit for bit
        o = gold[name + "_x"].copy()
        oracle.orc_hadamard_rotate(P(o), P(signs), n, b, C.c_float(lib.eif_hip_wht_norm(b)))
        assert np.array_equal(bits(y), bits(o))
        # the reference's own output: bit for bit when this host's rsqrtss gives the fixture's norm
        if np.float32(lib.eif_hip_wht_norm(b)) == gold["wht_norms"][int(np.log2(b))]:
            assert np.array_equal(bits(y), bits(gold[name + "_y"]))
        else:
            assert np.allclose(y, gold[name + "_y"], rtol=2e-7, atol=0)
    # invalid arguments are a silent no-op, as in the reference
    x = np.ones(96, np.float32)
    lib.eif_hadamard_rotate_f32(P(x), None, 96, 64)
    lib.eif_hadamard_rotate_f32(P(x), None, 96, 96)
    assert np.all(x == 1.0)


def test_quantize_activation(lib, gold):
    for name in ("quant_2560", "quant_6912", "quant_17"):
        x = gold[name + "_x"]
        q, s = np.zeros(x.size, np.int8), np.zeros(1, np.float32)
        lib.eif_quantize_activation_i8(P(x), P(q), P(s), x.size)
        assert np.array_equal(q, gold[name + "_q"]) and bits(s)[0] == bits(gold[name + "_scale"])[0]
    z, q, s = np.zeros(8, np.float32), np.full(8, 5, np.int8), np.zeros(1, np.float32)
    lib.eif_quantize_activation_i8(P(z), P(q), P(s), 8)
    assert np.all(q == 0) and s[0] == 1.0


def test_integer_ternary_paths(lib, gold):
    y = np.zeros(64, np.float32)
    lib.eif_matmul_bitnet_i8xternary_f32(P(gold["i8x_w"]), P(gold["i8x_scales"]), P(gold["i8x_xq"]),
                                         float(gold["i8x_scale_in"][0]), P(gold["i8x_bias"]), P(y), 64, 2560)
    assert np.array_equal(bits(y), bits(gold["i8x_y"]))
    y = np.zeros(64, np.float32)
    lib.eif_matmul_bitnet_act_quant_f32(P(gold["i8x_w"]), P(gold["i8x_scales"]), P(gold["aq_x"]), None, P(y), 64,
                                        2560)
    assert np.array_equal(bits(y), bits(gold["aq_y"]))
    sw, sin, sout = (float(v) for v in gold["i8o_scales"])
    y8 = np.zeros(40, np.int8)
    lib.eif_matmul_bitnet_int8(P(gold["i8o_w"]), sw, P(gold["i8o_x"]), sin, P(gold["i8o_bias"]), P(y8), sout, 40, 256)
    assert np.array_equal(y8, gold["i8o_y"])


def test_fp32_activation_ternary(lib, gold):
    rows, cols = 48, 640
    codes = synth.unpack_ternary(gold["f32_w"], cols).astype(np.float64)
    x = gold["f32_x"].astype(np.float64)
    bias = gold["f32_bias"]
    sc = gold["f32_scales"]
    for g in (128, 64, 4):
        bs = gold[f"blk{g}_scales"]
        y = np.zeros(rows, np.float32)
        lib.eif_matmul_bitnet_block_f32(P(gold["f32_w"]), P(bs), g, P(gold["f32_x"]), P(bias), P(y), rows, cols)
        mag = (np.abs(codes) * np.repeat(bs.reshape(rows, -1), g, axis=1)[:, :cols]) @ np.abs(x) + np.abs(bias)
        assert within(y, gold[f"blk{g}_y"], mag), g
    mag = (np.abs(codes) @ np.abs(x)) * sc + np.abs(bias)
    for fn, w, key in ((lib.eif_matmul_bitnet_f32, gold["f32_w"], "f32_y"),
                       (lib.eif_matmul_bitnet_dense_f32, gold["dense_w"], "dense_y"),
                       (lib.eif_matmul_bitnet_tmac_interleaved_f32, gold["tmac_w"], "tmac_y")):
        y = np.zeros(rows, np.float32)
        fn(P(w), P(sc), P(gold["f32_x"]), P(bias), P(y), rows, cols)
        assert within(y, gold[key], mag), key
    h = rows // 2
    y1, y3 = np.zeros(h, np.float32), np.zeros(h, np.float32)
    w1, w3 = gold["f32_w"][:h].copy(), gold["f32_w"][h:].copy()
    lib.eif_matmul_bitnet_f32_w1w3(P(y1), P(y3), P(w1), P(w3), P(sc[:h].copy()), P(sc[h:].copy()), P(gold["f32_x"]),
                                   h, cols)
    mag = (np.abs(codes) @ np.abs(x)) * sc
    assert within(y1, gold["w1w3_y1"], mag[:h]) and within(y3, gold["w1w3_y3"], mag[h:])


def test_int_row_scaled_fp32(lib, gold):
    w, s, x = gold["int8_w"], gold["int8_scales"], gold["int8_x"]
    mag = (np.abs(w.astype(np.float64)) @ np.abs(x.astype(np.float64))) * s
    for fn, key in ((lambda y: lib.tinyllm_matmul_int8_rowscale(P(y), P(w), P(x), 896, 64, P(s)), "int8_y"),
                    (lambda y: lib.eif_int8_gemv_f32(P(y), P(w), P(s), P(x), 64, 896), "int8q_y")):
        y = np.zeros(64, np.float32)
        fn(y)
        assert within(y, gold[key], mag)
    w4, s4, x4 = gold["int4_w"], gold["int4_scales"], gold["int4_x"]
    mag = (np.abs(synth.unpack_int4(w4, 1024).astype(np.float64)) @ np.abs(x4.astype(np.float64))) * s4
    y = np.zeros(64, np.float32)
    lib.eif_int4_gemv_f32(P(y), P(w4), P(s4), P(x4), 64, 1024)
    assert within(y, gold["int4_y"], mag)


def test_gemm_and_softmax(lib, gold):
    A, W, b = gold["gemm_A"], gold["gemm_W"], gold["gemm_b"]
    Cm = np.zeros((13, 25), np.float32)
    lib.eif_gemm_f32_nt(P(A), P(W), P(b), P(Cm), 13, 25, 257, 1, 0)
    mag = np.abs(A.astype(np.float64)) @ np.abs(W.astype(np.float64)).T + np.abs(b) + 1
    assert np.max(np.abs(Cm - gold["gemm_C"]) / mag) < 1e-5
    # accumulate mode and strided operands against float64 (tests/test_gemm.c:9-34 bounds)
    r = np.random.default_rng(3)
    M, N, K, lda, ldw, ldc = 67, 70, 300, 310, 305, 80
    A = r.uniform(-1, 1, (M, lda)).astype(np.float32)
    W = r.uniform(-1, 1, (N, ldw)).astype(np.float32)
    C0 = r.uniform(-1, 1, (M, ldc)).astype(np.float32)
    Cm = C0.copy()
    lib.eif_gemm_f32_nt_ld(P(A), lda, P(W), ldw, None, P(Cm), ldc, M, N, K, 0, 1)
    want = A[:, :K].astype(np.float64) @ W[:, :K].astype(np.float64).T + C0[:, :N]
    mag = np.abs(A[:, :K].astype(np.float64)) @ np.abs(W[:, :K].astype(np.float64)).T + 1
    assert np.max(np.abs(Cm[:, :N] - want) / mag) < 1e-5
    assert np.array_equal(Cm[:, N:], C0[:, N:])
    S = gold["softmax_in"].copy()
    lib.eif_softmax_rows_f32(P(S), 5, 7, 10, 0.5)
    want = gold["softmax_out"]
    assert np.max(np.abs(S[:, :7] - want[:, :7]) / (want[:, :7] + 1e-30)) < 1e-5
    assert np.array_equal(S[:, 7:], want[:, 7:])


def test_block_f32_full_size(lib, oracle):
    # the decode path of the reference engines at the BitNet-2B shape: 6912 x 2560, g128, FP32 activations
    N, K, g = 6912, 2560, 128
    w, s = synth.ternary_weight((70,), N, K, g)
    x = synth.activations((71,), 1, K)[0]
    y = np.zeros(N, np.float32)
    lib.eif_matmul_bitnet_block_f32(P(w), P(s), g, P(x), None, P(y), N, K)
    o = np.zeros(N, np.float32)
    oracle.orc_matmul_bitnet_block_f32(P(w), P(s), g, P(x), None, P(o), N, K)
    codes = synth.unpack_ternary(w, K).astype(np.float64)
    mag = (np.abs(codes) * np.repeat(s, g, axis=1)) @ np.abs(x.astype(np.float64))
    assert within(y, o, mag)
    lib.eif_hip_forget_host_weights(P(w))
    lib.eif_hip_forget_host_weights(P(s))


def test_resident_weight_cache(lib, oracle):
    rows, cols = 256, 1024
    w, s = synth.ternary_weight((72,), rows, cols, 0)
    xq = np.random.default_rng(5).integers(-127, 128, cols).astype(np.int8)
    y1, y2, o = (np.zeros(rows, np.float32) for _ in range(3))
    lib.eif_matmul_bitnet_i8xternary_f32(P(w), P(s), P(xq), 0.5, None, P(y1), rows, cols)
    lib.eif_matmul_bitnet_i8xternary_f32(P(w), P(s), P(xq), 0.5, None, P(y2), rows, cols)
    assert np.array_equal(bits(y1), bits(y2))
    w[:] = synth.pack_ternary(np.random.default_rng(6).integers(-1, 2, (rows, cols)).astype(np.int8))
    lib.eif_hip_forget_host_weights(P(w))
    lib.eif_matmul_bitnet_i8xternary_f32(P(w), P(s), P(xq), 0.5, None, P(y2), rows, cols)
    oracle.orc_matmul_bitnet_i8xternary_f32(P(w), P(s), P(xq), 0.5, None, P(o), rows, cols)
    assert np.array_equal(bits(y2), bits(o))


def test_concurrent_callers(lib, oracle):
    # the reference engines call these symbols from OpenMP workers: per-thread streams and staging
    rows, cols = 512, 2560
    w, s = synth.ternary_weight((73,), rows, cols, 128)
    xs = [synth.activations((74, t), 1, cols)[0] for t in range(6)]
    outs = [np.zeros(rows, np.float32) for _ in range(6)]
    errs = []

    def work(t):
        try:
            for _ in range(20):
                lib.eif_matmul_bitnet_block_f32(P(w), P(s), 128, P(xs[t]), None, P(outs[t]), rows, cols)
        except Exception as e:  # pragma: no cover
            errs.append(e)

    th = [threading.Thread(target=work, args=(t,)) for t in range(6)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert not errs
    codes = synth.unpack_ternary(w, cols).astype(np.float64)
    for t in range(6):
        o = np.zeros(rows, np.float32)
        oracle.orc_matmul_bitnet_block_f32(P(w), P(s), 128, P(xs[t]), None, P(o), rows, cols)
        mag = (np.abs(codes) * np.repeat(s, 128, axis=1)) @ np.abs(xs[t].astype(np.float64))
        assert within(outs[t], o, mag)
    lib.eif_hip_forget_host_weights(P(w))
    lib.eif_hip_forget_host_weights(P(s))


def with_code3(packed, key):
    """The reference's 2-bit rows may hold code 11 for a zero (read as 0): turn about half the zero codes into 11."""
    p = packed.copy()
    r = np.random.default_rng(key)
    for i in range(4):
        zero = ((p >> (2 * i)) & 3) == 0
        p[zero & (r.uniform(size=p.shape) < 0.5)] |= np.uint8(3 << (2 * i))
    return p


# (rows, cols, block): the row-tile path (K <= 8192, blocks of whole 16-column chunks), ragged rows and columns,
# and the row-major fallbacks (K > 8192, a block of 4 or 40 columns)
TERN_BLOCK_SHAPES = [(6912, 2560, 128), (2560, 6912, 96), (37, 200, 32), (5, 48, 16), (130, 8192, 256),
                     (1001, 1000, 64), (3, 8200, 128), (64, 640, 4), (50, 400, 40)]


@pytest.mark.parametrize("rows,cols,block", TERN_BLOCK_SHAPES)
def test_block_f32_shapes(lib, oracle, rows, cols, block):
    w, s = synth.ternary_weight((80, rows, cols, block), rows, cols, block)
    w = with_code3(w, (81, rows))
    x = synth.activations((82, cols), 1, cols)[0]
    bias = synth.rng(83, rows).standard_normal(rows).astype(np.float32) if rows % 2 else None
    y = np.full(rows, np.nan, np.float32)
    lib.eif_matmul_bitnet_block_f32(P(w), P(s), block, P(x), P(bias), P(y), rows, cols)
    o = np.zeros(rows, np.float32)
    oracle.orc_matmul_bitnet_block_f32(P(w), P(s), block, P(x), P(bias), P(o), rows, cols)
    codes = synth.unpack_ternary(w, cols).astype(np.float64)
    mag = (np.abs(codes) * np.repeat(s, block, axis=1)[:, :cols]) @ np.abs(x.astype(np.float64))
    if bias is not None:
        mag = mag + np.abs(bias)
    assert np.all(np.isfinite(y)) and within(y, o, mag)
    lib.eif_hip_forget_host_weights(P(w))
    lib.eif_hip_forget_host_weights(P(s))


@pytest.mark.parametrize("rows,cols", [(6912, 2560), (2561, 1000), (17, 33), (4099, 4096), (8, 9000)])
def test_row_scaled_f32_layouts(lib, oracle, rows, cols):
    """The same values in the three reference layouts (2-bit rows, 4-row interleaved, base 3) give outputs within
    1e-5 of the oracle's for each."""
    r = synth.rng(84, rows, cols)
    v = r.integers(-1, 2, size=(rows, cols), dtype=np.int8)
    w = with_code3(synth.pack_ternary(v), (85, rows))
    il = np.zeros_like(w)
    oracle.orc_interleave_weights_4rows(P(w), P(il), rows, cols)
    dense = np.zeros((rows, (cols + 4) // 5), np.uint8)
    for i in range(rows):
        oracle.orc_pack_ternary_dense(P(np.ascontiguousarray(v[i])), P(dense[i]), cols)
    s = (np.abs(r.standard_normal(rows)) * 0.02).astype(np.float32)
    x = synth.activations((86, cols), 1, cols)[0]
    bias = r.standard_normal(rows).astype(np.float32)
    mag = (np.abs(v.astype(np.float64)) @ np.abs(x.astype(np.float64))) * s + np.abs(bias)
    for fn, ofn, wt in ((lib.eif_matmul_bitnet_f32, oracle.orc_matmul_bitnet_f32, w),
                        (lib.eif_matmul_bitnet_tmac_interleaved_f32, oracle.orc_matmul_bitnet_tmac_interleaved_f32, il),
                        (lib.eif_matmul_bitnet_dense_f32, oracle.orc_matmul_bitnet_dense_f32, dense)):
        y = np.full(rows, np.nan, np.float32)
        fn(P(wt), P(s), P(x), P(bias), P(y), rows, cols)
        o = np.zeros(rows, np.float32)
        ofn(P(wt), P(s), P(x), P(bias), P(o), rows, cols)
        assert np.all(np.isfinite(y)) and within(y, o, mag), fn
        lib.eif_hip_forget_host_weights(P(wt))


@pytest.mark.parametrize("rows,cols", [(151936, 1024), (4864, 896), (37, 1001), (40, 9000)])
def test_int_f32_shapes(lib, oracle, rows, cols):
    """INT4 (the tied vocabulary head's shape) and INT8 row-scaled GEMVs with FP32 activations against the
    oracle, ragged and past the row-tile path's 8192 columns."""
    w4, s4 = synth.int4_weight((87, rows, cols), rows, cols)
    w8, s8 = synth.int8_weight((88, rows, cols), rows, cols)
    x = synth.activations((89, cols), 1, cols)[0]
    xa = np.abs(x.astype(np.float64))

    def absdot(vals):   # sum_c |w[r][c]| |x[c]| over row blocks (bounded memory)
        return np.concatenate([np.abs(vals(i, i + 8192).astype(np.float64)) @ xa for i in range(0, rows, 8192)])
    y = np.full(rows, np.nan, np.float32)
    lib.eif_int4_gemv_f32(P(y), P(w4), P(s4), P(x), rows, cols)
    o = np.zeros(rows, np.float32)
    oracle.orc_int4_gemv_f32(P(o), P(w4), P(s4), P(x), rows, cols)
    mag = absdot(lambda a, b: synth.unpack_int4(w4[a:b], cols)) * s4
    assert np.all(np.isfinite(y)) and within(y, o, mag)
    y = np.full(rows, np.nan, np.float32)
    lib.tinyllm_matmul_int8_rowscale(P(y), P(w8), P(x), cols, rows, P(s8))
    o = np.zeros(rows, np.float32)
    oracle.orc_int8_rowscale_f32(P(o), P(w8), P(x), cols, rows, P(s8))
    mag = absdot(lambda a, b: w8[a:b]) * s8
    assert np.all(np.isfinite(y)) and within(y, o, mag)
    lib.eif_hip_forget_host_weights(P(w4))
    lib.eif_hip_forget_host_weights(P(w8))


def test_f32_tile_knobs(lib, oracle):
    """Tiles per wave change the launch, never the bits; waves per tile (K split) change only the order of the FP32
    sums: every setting within 1e-5 of the oracle."""
    rows, cols, g = 6912, 2560, 128
    w, s = synth.ternary_weight((90,), rows, cols, g)
    w4, s4 = synth.int4_weight((91,), 20000, 1024)
    x = synth.activations((92,), 1, cols)[0]
    o = np.zeros(rows, np.float32)
    oracle.orc_matmul_bitnet_block_f32(P(w), P(s), g, P(x), None, P(o), rows, cols)
    codes = synth.unpack_ternary(w, cols).astype(np.float64)
    mag = (np.abs(codes) * np.repeat(s, g, axis=1)) @ np.abs(x.astype(np.float64))
    old_tw, old_ks = lib.eif_hip_set_f32_tiles_per_wave(0), lib.eif_hip_set_f32_ksplit(0)
    try:
        for ks in (1, 2, 3, 4, 8):
            lib.eif_hip_set_f32_ksplit(ks)
            outs = []
            for tw in (1, 2):
                lib.eif_hip_set_f32_tiles_per_wave(tw)
                y, y4 = np.zeros(rows, np.float32), np.zeros(20000, np.float32)
                lib.eif_matmul_bitnet_block_f32(P(w), P(s), g, P(x), None, P(y), rows, cols)
                lib.eif_int4_gemv_f32(P(y4), P(w4), P(s4), P(x), 20000, 1024)
                outs.append((bits(y), bits(y4)))
                assert within(y, o, mag), (ks, tw)
            assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1]), ks
    finally:
        lib.eif_hip_set_f32_tiles_per_wave(old_tw)
        lib.eif_hip_set_f32_ksplit(old_ks)
    for a in (w, s, w4):
        lib.eif_hip_forget_host_weights(P(a))


def test_gpu_seat(lib, oracle):
    """The reference's GPU seat (include/eif_gpu.h:55-70) computes on the GPU and says so: the same bits as
    eif_matmul_bitnet_f32, within 1e-5 of the oracle; invalid sizes return false and leave the output alone."""
    rows, cols = 3001, 2560
    w, s = synth.ternary_weight((93,), rows, cols, 0)
    x = synth.activations((94,), 1, cols)[0]
    bias = synth.rng(95).standard_normal(rows).astype(np.float32)
    y, y1, o = np.zeros(rows, np.float32), np.zeros(rows, np.float32), np.zeros(rows, np.float32)
    assert lib.eif_gpu_matmul_bitnet_f32(None, P(w), P(s), P(x), P(bias), P(y), rows, cols)
    lib.eif_matmul_bitnet_f32(P(w), P(s), P(x), P(bias), P(y1), rows, cols)
    assert np.array_equal(bits(y), bits(y1))
    oracle.orc_matmul_bitnet_f32(P(w), P(s), P(x), P(bias), P(o), rows, cols)
    codes = synth.unpack_ternary(w, cols).astype(np.float64)
    assert within(y, o, (np.abs(codes) @ np.abs(x.astype(np.float64))) * s + np.abs(bias))
    z = np.full(4, 7.0, np.float32)
    assert not lib.eif_gpu_matmul_bitnet_f32(None, P(w), P(s), P(x), None, P(z), 0, cols)
    assert np.all(z == 7.0)
    lib.eif_hip_forget_host_weights(P(w))


def test_weight_cache_bound(lib, oracle):
    """With a bound on the resident copies, least recently used copies are evicted and uploaded again when needed:
    the cache stays within the bound and every output matches the oracle."""
    lib.eif_hip_forget_host_weights(None)
    assert lib.eif_hip_host_weight_cache_bytes() == 0
    rows, cols, g = 2048, 2560, 128
    ws = [synth.ternary_weight((96, i), rows, cols, g) for i in range(4)]   # 1.3 MB codes + 160 KB scales each
    x = synth.activations((97,), 1, cols)[0]
    old = lib.eif_hip_set_host_weight_cache_limit(4 << 20)
    try:
        for rep in range(2):
            for i, (w, s) in enumerate(ws):
                y, o = np.zeros(rows, np.float32), np.zeros(rows, np.float32)
                lib.eif_matmul_bitnet_block_f32(P(w), P(s), g, P(x), None, P(y), rows, cols)
                oracle.orc_matmul_bitnet_block_f32(P(w), P(s), g, P(x), None, P(o), rows, cols)
                codes = synth.unpack_ternary(w, cols).astype(np.float64)
                mag = (np.abs(codes) * np.repeat(s, g, axis=1)) @ np.abs(x.astype(np.float64))
                assert within(y, o, mag), (rep, i)
                assert lib.eif_hip_host_weight_cache_bytes() <= 4 << 20, (rep, i)
    finally:
        lib.eif_hip_set_host_weight_cache_limit(old)
        lib.eif_hip_forget_host_weights(None)
    assert lib.eif_hip_host_weight_cache_bytes() == 0


def test_host_api_beyond_pinned_buffers(lib, oracle):
    """Inputs and outputs above the 4 MiB of a thread's pinned bounce buffers are copied from and to the caller's
    memory directly; calls before and after them go through the pinned buffers. Every result against the oracle:
    an INT8 row-scaled GEMV with a 4.4 MB activation row (3 x 1,100,000) and one with a 4.4 MB output
    (1,100,000 x 16), between two small ones."""
    def run(rows, cols, key):
        w = synth.rng(90, key).integers(-127, 128, size=(rows, cols), dtype=np.int8)
        s = (np.abs(synth.rng(91, key).standard_normal(rows)) * 0.01).astype(np.float32)
        x = synth.rng(92, key).standard_normal(cols).astype(np.float32)
        y = np.full(rows, np.nan, np.float32)
        lib.tinyllm_matmul_int8_rowscale(P(y), P(w), P(x), cols, rows, P(s))
        o = np.zeros(rows, np.float32)
        oracle.orc_int8_rowscale_f32(P(o), P(w), P(x), cols, rows, P(s))
        mag = (np.abs(w.astype(np.float64)) @ np.abs(x.astype(np.float64))) * s
        assert np.all(np.isfinite(y)) and within(y, o, mag), (rows, cols)
        lib.eif_hip_forget_host_weights(P(w))
    run(64, 896, 1)
    run(3, 1_100_000, 2)     # x: 4.4 MB
    run(64, 896, 3)
    run(1_100_000, 16, 4)    # y: 4.4 MB
    run(64, 896, 5)
