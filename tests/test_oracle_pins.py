"""Pins the CPU oracle before it is trusted as the checker (CPU only).

Each check is chosen so that a plausible mistake fails it: the reference's known-answer tests
(tests/test_all_features.c, tests/test_bitnet_hadamard.c), closed forms (Sylvester matrix, involution, integer
brute force in int64) and bit-for-bit agreement with the reference compiled from its own sources (oracle/_ref).
"""
import os

import numpy as np
import pytest

from conftest import P
import synth


def rng(seed):
    return np.random.default_rng(seed)


# ---- a1: 2-bit codes ----

def test_pack_unpack_kat(oracle):
    # tests/test_all_features.c:72-89: {0,1,-1,0, 1,1,-1,-1} -> 2 bytes and back.
    v = np.array([0, 1, -1, 0, 1, 1, -1, -1], np.int8)
    out = np.zeros(2, np.uint8)
    assert oracle.orc_pack_ternary(P(v), P(out), 8) == 2
    assert out.tolist() == [0b00100100, 0b10100101]
    assert [oracle.orc_unpack_ternary(int(out[i // 4]), i % 4) for i in range(8)] == v.tolist()
    dense = np.array([-1, 0, 1, -1, 1], np.int8)
    d = np.zeros(1, np.uint8)
    assert oracle.orc_pack_ternary_dense(P(dense), P(d), 5) == 1
    assert int(d[0]) == 2 + 0 * 3 + 1 * 9 + 2 * 27 + 1 * 81


def test_unpack_all_bytes(oracle):
    # every byte, every position; the reserved code 11 decodes to 0
    for b in range(256):
        for p in range(4):
            code = (b >> (2 * p)) & 3
            assert oracle.orc_unpack_ternary(b, p) == {0: 0, 1: 1, 2: -1, 3: 0}[code]


def test_pack_matches_numpy(oracle):
    v = rng(1).integers(-1, 2, 1001).astype(np.int8)
    out = np.zeros((1001 + 3) // 4, np.uint8)
    oracle.orc_pack_ternary(P(v), P(out), 1001)
    assert np.array_equal(out, synth.pack_ternary(v))


# ---- a2: size helpers ----

def test_size_helpers(oracle):
    # tests/test_bitnet_hadamard.c:34-36
    assert oracle.orc_hadamard_block_size(576) == 64 and oracle.orc_hadamard_block_size(1536) == 512
    assert oracle.orc_bitnet_group_size(576, 128) == 96 and oracle.orc_bitnet_group_size(1536, 128) == 128
    assert oracle.orc_bitnet_group_size(576, 0) == 0
    for n in range(1, 5000, 7):
        b = oracle.orc_hadamard_block_size(n)
        assert n % b == 0 and b <= 1024 and (b & (b - 1)) == 0
        assert b == 1024 or n % (2 * b) != 0
        g = oracle.orc_bitnet_group_size(n, 128)
        brute = next((x for x in range(128, 31, -32) if 128 < n and n % x == 0), 0)
        assert g == brute


# ---- a3: Walsh-Hadamard rotation ----

def sylvester(b):
    i = np.arange(b)
    return np.where(np.vectorize(lambda v: bin(v).count("1") & 1)(i[:, None] & i[None, :]), -1.0, 1.0) / np.sqrt(b)


@pytest.mark.parametrize("n,b", [(192, 64), (2560, 128), (512, 512), (6912, 128), (96, 32)])
def test_wht_closed_form(oracle, n, b):
    r = rng(n + b)
    x = r.uniform(-1, 1, n).astype(np.float32)
    signs = np.where(r.uniform(size=n) > 0.5, 1.0, -1.0).astype(np.float32)
    y = x.copy()
    assert oracle.orc_hadamard_rotate(P(y), P(signs), n, b, oracle.orc_wht_norm_exact(b)) == 0
    H = sylvester(b)
    want = ((x * signs).astype(np.float64).reshape(-1, b) @ H).reshape(-1)
    assert np.max(np.abs(y - want)) < 1e-5 * max(1.0, np.sqrt(b) / 8)
    # involution: H(H(x)) = x without signs
    z = x.copy()
    nb = oracle.orc_wht_norm_exact(b)
    oracle.orc_hadamard_rotate(P(z), None, n, b, nb)
    oracle.orc_hadamard_rotate(P(z), None, n, b, nb)
    assert np.max(np.abs(z - x)) < 1e-5


def test_wht_rejects(oracle):
    x = np.ones(96, np.float32)
    assert oracle.orc_hadamard_rotate(P(x), None, 96, 0, 1.0) == -1
    assert oracle.orc_hadamard_rotate(P(x), None, 96, 64, 1.0) == -1     # n % block != 0
    assert oracle.orc_hadamard_rotate(P(x), None, 96, 96, 1.0) == -2     # not a power of two
    assert np.all(x == 1.0)


def test_norm_fastmath_vs_ref(oracle, ref):
    # the compiled reference: rotating e0 with block b writes norm(b) to every element of the block
    for k in range(0, 15):
        b = 1 << k
        x = np.zeros(b, np.float32)
        x[0] = 1.0
        ref.eif_hadamard_rotate_f32(P(x), None, b, b)
        assert np.all(x.view(np.uint32) == np.float32(oracle.orc_wht_norm_fastmath(b)).view(np.uint32)), b


@pytest.mark.parametrize("n,b,signed", [(2560, 128, False), (2560, 128, True), (6912, 128, True), (4096, 1024, False),
                                        (192, 64, True)])
def test_wht_bits_vs_ref(oracle, ref, n, b, signed):
    r = rng(7 * n + b)
    x = synth.activations((9, n, b), 1, n)[0]
    signs = np.where(r.uniform(size=n) > 0.5, 1.0, -1.0).astype(np.float32) if signed else None
    a, o = x.copy(), x.copy()
    ref.eif_hadamard_rotate_f32(P(a), P(signs), n, b)
    oracle.orc_hadamard_rotate(P(o), P(signs), n, b, oracle.orc_wht_norm_fastmath(b))
    assert np.array_equal(a.view(np.uint32), o.view(np.uint32))


# ---- a4: activation quantization ----

def test_quant_closed_form(oracle):
    x = np.array([1, 2, 3, 4, 5, 6, 7, 8], np.float32)            # tests/test_all_features.c:145-149
    q, s = np.zeros(8, np.int8), np.zeros(1, np.float32)
    oracle.orc_quantize_activation_i8(P(x), P(q), P(s), 8)
    assert q[7] == 127 and s[0] > 0
    # amax < 1e-12: zeros and scale 1
    x = np.full(5, 1e-13, np.float32)
    q = np.full(5, 7, np.int8)
    oracle.orc_quantize_activation_i8(P(x), P(q), P(s), 5)
    assert np.all(q == 0) and s[0] == 1.0
    # round half away from zero: amax 127 -> inv 1, q = trunc(v +- 0.5)
    x = np.array([127.0, 0.5, -0.5, 1.5, -1.5, 2.49, -2.51], np.float32)
    q = np.zeros(7, np.int8)
    oracle.orc_quantize_activation_i8(P(x), P(q), P(s), 7)
    assert q.tolist() == [127, 1, -1, 2, -2, 2, -3]
    assert s[0] == np.float32(127.0) * np.float32(1.0 / 127.0)


def test_quant_bits_vs_ref(oracle, ref):
    r = rng(3)
    for t in range(200):
        n = int(r.integers(1, 4000))
        x = (r.standard_normal(n) * r.uniform(1e-3, 1e3)).astype(np.float32)
        if t % 7 == 0:
            x[r.integers(0, n)] *= 50
        qa, qb = np.zeros(n, np.int8), np.zeros(n, np.int8)
        sa, sb = np.zeros(1, np.float32), np.zeros(1, np.float32)
        ref.eif_quantize_activation_i8(P(x), P(qa), P(sa), n)
        oracle.orc_quantize_activation_i8(P(x), P(qb), P(sb), n)
        assert np.array_equal(qa, qb) and sa.view(np.uint32)[0] == sb.view(np.uint32)[0]


# ---- a5 / new contract: exact integer accumulators ----

def brute_acc(codes, xq, group):
    """int64 brute force: acc[m, r, g]"""
    N, K = codes.shape
    g = group if 0 < group < K else K
    ng = -(-K // g)
    prod = xq.astype(np.int64)[:, None, :] * codes.astype(np.int64)[None, :, :]
    pad = ng * g - K
    prod = np.pad(prod, ((0, 0), (0, 0), (0, pad)))
    return prod.reshape(xq.shape[0], N, ng, g).sum(-1)


@pytest.mark.parametrize("N,K,group,M", [(7, 130, 32, 3), (16, 2560, 128, 2), (5, 576, 96, 1), (9, 100, 0, 2),
                                         (4, 8, 4, 1)])
def test_ternary_acc_brute(oracle, N, K, group, M):
    r = rng(N * K + group)
    codes = r.integers(-1, 2, (N, K)).astype(np.int8)
    w = synth.pack_ternary(codes)
    if K % 4 == 0:  # include the reserved code 11 (decodes to 0)
        w[0, 0] |= 0b11
        codes[0, 0] = 0
    xq = r.integers(-128, 128, (M, K)).astype(np.int8)
    g = group if 0 < group < K else K
    ng = -(-K // g)
    acc = np.zeros((M, N, ng), np.int32)
    oracle.orc_ternary_acc_i32(P(w), P(xq), K, M, N, K, group, P(acc))
    assert np.array_equal(acc, brute_acc(codes, xq, group))


def test_int8_int4_acc_brute(oracle):
    r = rng(11)
    N, K, M = 13, 333, 3
    w8 = r.integers(-128, 128, (N, K)).astype(np.int8)
    v4 = r.integers(-8, 8, (N, K)).astype(np.int8)
    w4 = synth.pack_int4(v4)
    xq = r.integers(-128, 128, (M, K)).astype(np.int8)
    a8, a4 = np.zeros((M, N), np.int32), np.zeros((M, N), np.int32)
    oracle.orc_int8_acc_i32(P(w8), P(xq), K, M, N, K, P(a8))
    oracle.orc_int4_acc_i32(P(w4), P(xq), K, M, N, K, P(a4))
    assert np.array_equal(a8, xq.astype(np.int64) @ w8.astype(np.int64).T)
    assert np.array_equal(a4, xq.astype(np.int64) @ v4.astype(np.int64).T)


def test_i8xternary_kat(oracle):
    # the 4x8 KAT of tests/test_all_features.c:104-171 (per-row scales, bias)
    raw = np.array([[1, 0, -1, 1, 0, -1, 1, 0], [-1, 1, 0, 0, 1, -1, -1, 1], [0, 0, 1, 1, -1, -1, 0, 1],
                    [1, 1, -1, -1, 0, 0, 1, -1]], np.int8)
    w = synth.pack_ternary(raw)
    sc = np.array([0.5, 1.0, 2.0, 0.25], np.float32)
    x = np.arange(1, 9, dtype=np.float32)
    bias = np.array([0.1, -0.2, 0.5, 0.0], np.float32)
    want = (raw.astype(np.float64) @ x) * sc + bias
    y = np.zeros(4, np.float32)
    oracle.orc_matmul_bitnet_f32(P(w), P(sc), P(x), P(bias), P(y), 4, 8)
    assert np.max(np.abs(y - want)) < 1e-4
    oracle.orc_matmul_bitnet_block_f32(P(w), P(np.repeat(sc, 2)), 4, P(x), P(bias), P(y), 4, 8)
    assert np.max(np.abs(y - want)) < 1e-4
    oracle.orc_matmul_bitnet_act_quant_f32(P(w), P(sc), P(x), P(bias), P(y), 4, 8)
    assert np.max(np.abs(y - want)) < 0.5
    il = np.zeros(8, np.uint8)
    assert oracle.orc_interleave_weights_4rows(P(w), P(il), 4, 8) == 8
    oracle.orc_matmul_bitnet_tmac_interleaved_f32(P(il), P(sc), P(x), P(bias), P(y), 4, 8)
    assert np.max(np.abs(y - want)) < 1e-4


@pytest.mark.parametrize("rows,cols,with_bias", [(64, 2560, True), (33, 577, False), (1, 3, True)])
def test_i8xternary_bits_vs_ref(oracle, ref, rows, cols, with_bias):
    r = rng(rows + cols)
    w = r.integers(0, 256, rows * ((cols + 3) // 4), dtype=np.uint8)
    xq = r.integers(-128, 128, cols).astype(np.int8)
    sc = r.random(rows, dtype=np.float32)
    bias = r.standard_normal(rows).astype(np.float32) if with_bias else None
    ya, yb = np.zeros(rows, np.float32), np.zeros(rows, np.float32)
    ref.eif_matmul_bitnet_i8xternary_f32(P(w), P(sc), P(xq), 0.0173, P(bias), P(ya), rows, cols)
    oracle.orc_matmul_bitnet_i8xternary_f32(P(w), P(sc), P(xq), 0.0173, P(bias), P(yb), rows, cols)
    assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32))


def test_int8_out_bits_vs_ref(oracle, ref):
    r = rng(5)
    for rows, cols in [(40, 256), (7, 13)]:
        w = r.integers(0, 256, rows * ((cols + 3) // 4), dtype=np.uint8)
        x = r.integers(-128, 128, cols).astype(np.int8)
        bias = r.integers(-500, 500, rows).astype(np.int32)
        ya, yb = np.zeros(rows, np.int8), np.zeros(rows, np.int8)
        for sout in (0.37, 0.0):
            ref.eif_matmul_bitnet_int8(P(w), 0.02, P(x), 0.9, P(bias), P(ya), sout, rows, cols)
            oracle.orc_matmul_bitnet_int8(P(w), 0.02, P(x), 0.9, P(bias), P(yb), sout, rows, cols)
            assert np.array_equal(ya, yb)


def test_act_quant_bits_vs_ref(oracle, ref):
    r = rng(8)
    rows, cols = 50, 2560
    w = r.integers(0, 256, rows * cols // 4, dtype=np.uint8)
    x = synth.activations((8,), 1, cols)[0]
    sc = r.random(rows, dtype=np.float32)
    ya, yb = np.zeros(rows, np.float32), np.zeros(rows, np.float32)
    ref.eif_matmul_bitnet_act_quant_f32(P(w), P(sc), P(x), None, P(ya), rows, cols)
    oracle.orc_matmul_bitnet_act_quant_f32(P(w), P(sc), P(x), None, P(yb), rows, cols)
    assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32))


# ---- FP32-activation GEMVs, against float64 and the compiled reference, with the reference tests' bounds ----

def rel_err(y, want, mag):
    return np.max(np.abs(y.astype(np.float64) - want) / (mag + 1e-30))


def test_fp32_gemvs_vs_ref(oracle, ref):
    r = rng(21)
    rows, cols = 96, 2560
    codes = r.integers(-1, 2, (rows, cols)).astype(np.int8)
    w = synth.pack_ternary(codes)
    x = synth.activations((21,), 1, cols)[0]
    mag = np.abs(codes.astype(np.float64)) @ np.abs(x.astype(np.float64))
    for g in (128, 96, 64):
        nb = -(-cols // g)
        bs = r.random((rows, nb), dtype=np.float32)
        want = ((codes.astype(np.float64) * np.repeat(bs, g, axis=1)[:, :cols]) @ x)
        m = (np.abs(codes) * np.repeat(bs, g, axis=1)[:, :cols]) @ np.abs(x.astype(np.float64))
        for lib, fn in ((ref, ref.eif_matmul_bitnet_block_f32), (oracle, oracle.orc_matmul_bitnet_block_f32)):
            y = np.zeros(rows, np.float32)
            fn(P(w), P(bs), g, P(x), None, P(y), rows, cols)
            assert rel_err(y, want, m) < 1e-5
    sc = r.random(rows, dtype=np.float32)
    want = (codes.astype(np.float64) @ x) * sc
    for fn in (ref.eif_matmul_bitnet_f32, oracle.orc_matmul_bitnet_f32):
        y = np.zeros(rows, np.float32)
        fn(P(w), P(sc), P(x), None, P(y), rows, cols)
        assert rel_err(y, want, mag * sc) < 1e-5


GROUPED_SHAPES = [
    # N, K, group, M: the single BitNet linear (one token and a batch), then the BitNet-2B layer's linears
    (6912, 2560, 128, 1),
    (6912, 2560, 128, 3),
] + [(N, K, g, 2) for _, N, K, g in synth.BITNET_2B_LAYER if _ != "up"] + [
    (130, 200, 32, 2),   # ragged: a short last group and a row count off the tiles
]


@pytest.mark.parametrize("N,K,g,M", GROUPED_SHAPES)
def test_ternary_gemv_grouped_vs_double(oracle, N, K, g, M):
    # orc_ternary_gemv_grouped (the GPU linear's FP32 contract) against the float64 closed form
    #   y[m, r] = xs[m] * sum_g s[r, g] * sum_{k in g} code[r, k] * xq[m, k] + bias[r],
    # built from unpacked codes, per-group slices and a matrix product, to 1e-5 of sum_g |s * acc_g| * xs + |bias|.
    # Planted mistakes it catches (each checked on the CPU): a dropped last group, scales indexed [g, r], xs of
    # token 0 for every token, the bias added before the xs multiply.
    w, s = synth.ternary_weight((60, N, K, g), N, K, g)
    x = synth.activations((61, M, K), M, K)
    kpad = -(-K // 128) * 128
    xq = np.zeros((M, kpad), np.int8)
    xs = np.zeros(M, np.float32)
    assert oracle.orc_prep_rows(P(x), K, None, M, K, 0, 1.0, P(xq), kpad, P(xs), None, 0) == 0
    bias = synth.rng(62, N).standard_normal(N).astype(np.float32)
    codes = synth.unpack_ternary(w, K).astype(np.float64)
    ng = -(-K // g)
    want = np.zeros((M, N))
    mag = np.zeros((M, N))
    for gi in range(ng):
        a = xq[:, gi * g:min(K, (gi + 1) * g)].astype(np.float64) @ codes[:, gi * g:min(K, (gi + 1) * g)].T
        want += a * s[None, :, gi]
        mag += np.abs(a) * s[None, :, gi]
    want = want * xs[:, None].astype(np.float64) + bias[None, :]
    mag = mag * xs[:, None].astype(np.float64) + np.abs(bias)[None, :]
    for b in (None, bias):
        y = np.full((M, N), np.nan, np.float32)
        oracle.orc_ternary_gemv_grouped(P(w), P(s), g, P(xq), kpad, P(xs), P(b), P(y), N, M, N, K)
        wb = want if b is not None else want - bias[None, :]
        assert rel_err(y, wb, mag) <= 1e-5, (N, K, g, M, b is not None)


def test_int8_int4_fp32_bounds_vs_ref(oracle, ref):
    # tests/test_int8_gemv.c:10-56 and tests/test_q35_int4.c:5-51: FP32-activation paths exact to rounding
    r = rng(4)
    for rows, cols in [(7, 579), (9, 6), (4, 13), (64, 896)]:
        w = r.integers(-127, 128, (rows, cols)).astype(np.int8)
        x = (r.uniform(-1, 1, cols) + np.where(np.arange(cols) % 97 == 0, 6.0, 0.0)).astype(np.float32)
        sc = (0.001 * (1 + np.arange(rows) % 5)).astype(np.float32)
        want = w.astype(np.float64) @ x
        mag = np.abs(w.astype(np.float64)) @ np.abs(x.astype(np.float64))
        for fn in (ref.tinyllm_matmul_int8_rowscale, oracle.orc_int8_rowscale_f32):
            y = np.zeros(rows, np.float32)
            fn(P(y), P(w), P(x), cols, rows, P(sc))
            assert np.max(np.abs(want - y / sc) / (1e-5 * mag + 1e-30)) <= 1.0
    for rows, cols in [(37, 3584), (5, 33), (64, 1024)]:
        v = r.integers(-8, 8, (rows, cols)).astype(np.int8)
        w = synth.pack_int4(v)
        x = (r.uniform(-1, 1, cols) + np.where(np.arange(cols) % 61 == 0, 9.0, 0.0)).astype(np.float32)
        sc = (0.01 * (1 + np.arange(rows) % 3)).astype(np.float32)
        want = v.astype(np.float64) @ x
        mag = np.abs(v.astype(np.float64)) @ np.abs(x.astype(np.float64))
        for fn in (ref.ref_q35_int4_gemv, oracle.orc_int4_gemv_f32):
            y = np.zeros(rows, np.float32)
            fn(P(y), P(w), P(sc), P(x), rows, cols)
            assert np.max(np.abs(want - y / sc) / (1e-6 * mag * 4 + 1e-30)) <= 1.0


# ---- a14/a15 on INT8 activations: the row-scaled FP32 epilogue ----

def _int_linear(fmt, key, N, K):
    if fmt == "int8":
        w, s = synth.int8_weight(key, N, K)
        return w, s, w
    w, s = synth.int4_weight(key, N, K)
    return w, s, synth.unpack_int4(w, K)


def _prep(oracle, key, M, K):
    kpad = -(-K // 128) * 128
    x = synth.activations(key, M, K)
    xq = np.zeros((M, kpad), np.int8)
    xs = np.zeros(M, np.float32)
    assert oracle.orc_prep_rows(P(x), K, None, M, K, 0, 1.0, P(xq), kpad, P(xs), None, 0) == 0
    return xq, xs, kpad


INT_I8ACT_SHAPES = [
    # Qwen2.5-0.5B-like INT8 layer: gate/up, down, stacked q|k|v, at one and 128 token rows
    ("int8", 4864, 896, 1), ("int8", 4864, 896, 128), ("int8", 896, 4864, 1), ("int8", 896, 4864, 128),
    ("int8", 1152, 896, 1), ("int8", 1152, 896, 128),
    # INT4 FFN linears and the 151936 x 1024 tied head, at one and 32 token rows
    ("int4", 3584, 1024, 1), ("int4", 3584, 1024, 32), ("int4", 1024, 3584, 1), ("int4", 1024, 3584, 32),
    ("int4", 151936, 1024, 1), ("int4", 151936, 1024, 32),
]


@pytest.mark.parametrize("fmt,N,K,M", INT_I8ACT_SHAPES)
def test_int_i8act_vs_double(oracle, fmt, N, K, M):
    # orc_int8_gemv_i8act / orc_int4_gemv_i8act (the GPU linears' FP32 contract) against the float64 closed form
    # acc * xs[m] * s[r] + bias[r] with acc the exact integer product, per-token xs from the prep, with and
    # without a bias, to 1e-6 of |acc| * xs * s + |bias|.
    import closed_form as cf
    w, s, vals = _int_linear(fmt, (70, N, K), N, K)
    xq, xs, kpad = _prep(oracle, (71, M, K), M, K)
    assert M == 1 or len(set(xs.tolist())) == M       # per-token scales differ, so an xs[0] mistake shows
    bias = synth.rng(72, N).standard_normal(N).astype(np.float32)
    acc = cf.exact_acc(xq, vals)
    fn = oracle.orc_int8_gemv_i8act if fmt == "int8" else oracle.orc_int4_gemv_i8act
    for b in (None, bias):
        y = np.full((M, N), np.nan, np.float32)
        fn(P(w), P(s), P(xq), kpad, P(xs), P(b), P(y), N, M, N, K)
        assert cf.rowscale_error(y, acc, xs, s, b) <= cf.ROWSCALE_TOL, (fmt, N, K, M, b is not None)


@pytest.fixture(scope="module")
def planted_oracles(tmp_path_factory):
    """The oracle built three more times, each with one planted mistake in its row-scaled epilogue
    (ORC_PLANT_ROWSCALE in oracle.c: 1 = xs[0] for every token, 2 = the scale indexed by token, 3 = the bias added
    before the xs multiply)."""
    import shutil
    import subprocess
    import oracle_api
    cc = shutil.which("gcc") or shutil.which("cc")
    if not cc:
        pytest.skip("no C compiler to build the planted oracles")
    src = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle")
    d = tmp_path_factory.mktemp("planted")
    libs = {}
    for k in (1, 2, 3):
        so = str(d / f"liboracle_plant{k}.so")
        subprocess.run([cc, "-std=c99", "-D_GNU_SOURCE", "-O1", "-fno-fast-math", "-ffp-contract=off", "-fPIC",
                        "-shared", f"-DORC_PLANT_ROWSCALE={k}", "-o", so, os.path.join(src, "oracle.c"),
                        os.path.join(src, "decode_oracle.c"), "-lm"], check=True)
        libs[k] = oracle_api.load(so)
    return libs


@pytest.mark.parametrize("fmt", ["int8", "int4"])
def test_int_i8act_planted_mistakes_fail(oracle, planted_oracles, fmt):
    # the closed form above rejects each planted epilogue mistake, at several token rows, with a bias
    import closed_form as cf
    N, K, M = 96, 640, 4
    w, s, vals = _int_linear(fmt, (73, N, K), N, K)
    xq, xs, kpad = _prep(oracle, (74, M, K), M, K)
    bias = synth.rng(75, N).standard_normal(N).astype(np.float32)
    acc = cf.exact_acc(xq, vals)
    name = "orc_int8_gemv_i8act" if fmt == "int8" else "orc_int4_gemv_i8act"
    y = np.zeros((M, N), np.float32)
    getattr(oracle, name)(P(w), P(s), P(xq), kpad, P(xs), P(bias), P(y), N, M, N, K)
    assert cf.rowscale_error(y, acc, xs, s, bias) <= cf.ROWSCALE_TOL
    for k, lib in planted_oracles.items():
        yb = np.zeros((M, N), np.float32)
        getattr(lib, name)(P(w), P(s), P(xq), kpad, P(xs), P(bias), P(yb), N, M, N, K)
        assert cf.rowscale_error(yb, acc, xs, s, bias) > 100 * cf.ROWSCALE_TOL, f"planted mistake {k} not caught"


def test_gemm_softmax_vs_double(oracle):
    # tests/test_gemm.c:9-34 bounds (normalised by sum |a*w| + 1, 1e-5)
    r = rng(9)
    for M, N, K, act, accum in [(13, 25, 257, 1, 0), (9, 11, 5, 0, 1), (1, 1, 1, 0, 0)]:
        A = r.uniform(-1, 1, (M, K)).astype(np.float32)
        W = r.uniform(-1, 1, (N, K)).astype(np.float32)
        b = r.uniform(-1, 1, N).astype(np.float32)
        C0 = r.uniform(-1, 1, (M, N)).astype(np.float32)
        C = C0.copy()
        oracle.orc_gemm_f32_nt_ld(P(A), K, P(W), K, P(b), P(C), N, M, N, K, act, accum)
        v = A.astype(np.float64) @ W.astype(np.float64).T + b
        mag = np.abs(A.astype(np.float64)) @ np.abs(W.astype(np.float64)).T + np.abs(b)
        if accum:
            v = v + C0
        elif act:
            v = 0.5 * v * (1 + np.tanh(0.7978845608028654 * (v + 0.044715 * v ** 3)))
        assert np.max(np.abs(v - C) / (mag + 1)) < 1e-5
    S0 = (r.uniform(-1, 1, (5, 10)) * 40).astype(np.float32)
    S = S0.copy()
    oracle.orc_softmax_rows_f32(P(S), 5, 7, 10, 1.0)
    e = np.exp((S0[:, :7] - S0[:, :7].max(1, keepdims=True)).astype(np.float64))
    ref_sm = e / e.sum(1, keepdims=True)
    assert np.max(np.abs(S[:, :7] - ref_sm) / (ref_sm + 1e-30)) < 1e-5
    assert np.array_equal(S[:, 7:], S0[:, 7:])


def _quant_rows_np(x, bits):
    """The reference's quant_rows (src/eif_qwen35_gguf.c:225-258) in numpy float32 arithmetic, as its -ffast-math
    build computes it: s = amax * (1 / qmax) where the source divides."""
    x = np.asarray(x, np.float32)
    rows, cols = x.shape
    qmax = np.float32(127.0 if bits == 8 else 7.0)
    lo, hi = (-128, 127) if bits == 8 else (-8, 7)
    amax = np.maximum(np.abs(x).max(axis=1), np.float32(1e-8)).astype(np.float32)
    sc = (amax * (np.float32(1.0) / qmax)).astype(np.float32)
    inv = (np.float32(1.0) / sc).astype(np.float32)
    q = np.clip(np.rint((x * inv[:, None]).astype(np.float32)), lo, hi).astype(np.int32)
    if bits == 8:
        return q.astype(np.int8).view(np.uint8), sc
    if cols % 2:
        q = np.concatenate([q, np.zeros((rows, 1), np.int32)], axis=1)
    packed = (((q[:, 0::2] + 8) << 4) | ((q[:, 1::2] + 8) & 0xF)).astype(np.uint8)
    return packed, sc


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("rows,cols", [(7, 64), (5, 33), (3, 1), (2, 1024)])
def test_quant_rows(oracle, bits, rows, cols):
    r = np.random.default_rng(70 + bits + cols)
    x = (r.standard_normal((rows, cols)) * 10.0 ** r.integers(-3, 3, (rows, 1))).astype(np.float32)
    x[0, : min(4, cols)] = 0.0
    if rows > 2:
        x[2] = 0.0                                        # all-zero row: the 1e-8 floor, codes 0
    if rows > 1 and cols > 3:
        amax = np.abs(x[1]).max()
        qmax = 127.0 if bits == 8 else 7.0
        x[1, 1] = np.float32(amax / qmax * 2.5)           # at 2.5 steps: a tie goes to even
    rb = cols if bits == 8 else (cols + 1) // 2
    dst = np.zeros((rows, rb), np.uint8)
    sc = np.zeros(rows, np.float32)
    oracle.orc_quant_rows(P(x), cols, rows, cols, bits, P(dst), P(sc))
    want, wsc = _quant_rows_np(x, bits)
    assert np.array_equal(dst, want) and np.array_equal(sc.view(np.uint32), wsc.view(np.uint32))
    # closed forms: decode (int4 nibble order of tests/test_q35_int4.c:20: even column in the high nibble)
    if bits == 8:
        q = dst.view(np.int8).astype(np.float64)
    else:
        q = np.stack([(dst >> 4).astype(np.int32) - 8, (dst & 0xF).astype(np.int32) - 8], axis=2).reshape(rows, -1)[:, :cols]
    s64 = sc.astype(np.float64)[:, None]
    err = np.abs(x.astype(np.float64) - q * s64)
    assert (err <= s64 * (0.5 + 1e-5)).all()               # within half a step (no value is clamped)
    big = np.abs(x).argmax(axis=1)
    for i in range(rows):
        if np.abs(x[i]).max() > 0:
            assert abs(q[i, big[i]]) == (127 if bits == 8 else 7)


def _gguf_blocks(r, kind, rows, cols):
    """Synthetic GGUF tensor rows: 32-column blocks of a finite fp16 scale and TL codes (10 bytes) or Q8_0 values
    (34 bytes)."""
    blocks = (cols + 31) // 32
    h = r.uniform(0.01, 2.0, (rows, blocks)).astype(np.float16).view(np.uint16)
    if kind == 8:
        body = r.integers(-128, 128, (rows, blocks, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
    else:
        body = r.integers(0, 256, (rows, blocks, 8), dtype=np.int16).astype(np.uint8)
    raw = np.concatenate([h.view(np.uint8).reshape(rows, blocks, 2), body], axis=2)
    return np.ascontiguousarray(raw), h


@pytest.mark.parametrize("kind", [34, 35, 8])
@pytest.mark.parametrize("rows,cols", [(5, 256), (3, 100), (2, 32)])
def test_gguf_ternary_rows(oracle, kind, rows, cols):
    r = np.random.default_rng(95 + kind + cols)
    raw, h = _gguf_blocks(r, kind, rows, cols)
    rb = (cols + 3) // 4
    codes = np.zeros((rows, rb), np.uint8)
    sc = np.zeros(rows, np.float32)
    oracle.orc_gguf_ternary_rows(kind, P(raw), rows, cols, P(codes), P(sc))
    blocks = raw.shape[1]
    want_sc = np.zeros(rows, np.float32)
    for i in range(rows):
        s = np.float32(0.0)
        for b in range(blocks):
            s = np.float32(s + h[i, b].view(np.float16).astype(np.float32))
        want_sc[i] = np.float32(s * (np.float32(1.0) / np.float32(blocks)))   # the reference build's mean
    assert np.array_equal(sc.view(np.uint32), want_sc.view(np.uint32))
    if kind == 8:
        q = raw[:, :, 2:].view(np.int8).reshape(rows, -1)[:, :cols]
        c = np.where(q > 0, 1, np.where(q < 0, 2, 0)).astype(np.uint8)
        c = np.concatenate([c, np.zeros((rows, 4 * rb - cols), np.uint8)], axis=1).reshape(rows, rb, 4)
        want = c[:, :, 0] | (c[:, :, 1] << 2) | (c[:, :, 2] << 4) | (c[:, :, 3] << 6)
    else:
        want = raw[:, :, 2:].reshape(rows, -1)[:, :rb]
    assert np.array_equal(codes, want)
    # the decoded codes of Q8_0 rows are the values' signs
    if kind == 8:
        dec = synth.unpack_ternary(codes, cols)
        assert np.array_equal(dec, np.sign(q))


def test_gguf_fp16_scales_every_value(oracle):
    # one 32-column TL block per row, every fp16 bit pattern as its scale: the row scale is that value exactly
    rows = 65536
    raw = np.zeros((rows, 1, 10), np.uint8)
    raw[:, 0, :2] = np.arange(rows, dtype=np.uint32).astype(np.uint16).view(np.uint8).reshape(rows, 2)
    codes = np.zeros((rows, 8), np.uint8)
    sc = np.zeros(rows, np.float32)
    oracle.orc_gguf_ternary_rows(34, P(raw), rows, 32, P(codes), P(sc))
    want = np.arange(rows, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    want = (np.float32(0.0) + want) * np.float32(1.0)   # the mean's sum starts at +0 (so -0 becomes +0)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(sc), nan)
    assert np.array_equal(sc[~nan].view(np.uint32), want[~nan].view(np.uint32))
