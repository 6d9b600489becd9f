"""The oracle against the vectors the reference itself produced (tests/golden/reference_vectors.npz, written by
tests/golden/make_golden.py from the reference compiled from its sources). CPU only."""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import P, ROOT

GOLD = os.path.join(ROOT, "tests", "golden", "reference_vectors.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLD)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def rel_bound(y, want, mag, tol=1e-5):
    return np.max(np.abs(y.astype(np.float64) - want.astype(np.float64)) / (tol * mag + 1e-30)) <= 1.0


def test_wht_matches_reference_bits(oracle, gold):
    norms = gold["wht_norms"]
    for name in ("wht_2560_128", "wht_4096_1024"):
        n, b, signed = gold[name + "_meta"]
        y = gold[name + "_x"].copy()
        nb = float(norms[int(np.log2(b))])
        assert oracle.orc_hadamard_rotate(P(y), P(gold[name + "_signs"]) if signed else None, n, b, C.c_float(nb)) == 0
        assert np.array_equal(bits(y), bits(gold[name + "_y"]))


def test_norms_are_the_fastmath_sequence(oracle, gold):
    # on the x86 host that produced the fixture the emulated sequence reproduces every stored value
    here = np.array([oracle.orc_wht_norm_fastmath(1 << k) for k in range(15)], np.float32)
    if not np.array_equal(bits(here), bits(gold["wht_norms"])):
        pytest.skip("this host's rsqrtss estimate differs from the fixture host's (vendor-specific instruction)")
    assert np.array_equal(bits(here), bits(gold["wht_norms"]))


def test_quant_matches_reference_bits(oracle, gold):
    for name in ("quant_2560", "quant_6912", "quant_17"):
        x = gold[name + "_x"]
        q, s = np.zeros(x.size, np.int8), np.zeros(1, np.float32)
        oracle.orc_quantize_activation_i8(P(x), P(q), P(s), x.size)
        assert np.array_equal(q, gold[name + "_q"]) and bits(s)[0] == bits(gold[name + "_scale"])[0]


def test_integer_paths_match_reference_bits(oracle, gold):
    y = np.zeros(64, np.float32)
    oracle.orc_matmul_bitnet_i8xternary_f32(P(gold["i8x_w"]), P(gold["i8x_scales"]), P(gold["i8x_xq"]),
                                            float(gold["i8x_scale_in"][0]), P(gold["i8x_bias"]), P(y), 64, 2560)
    assert np.array_equal(bits(y), bits(gold["i8x_y"]))
    y = np.zeros(64, np.float32)
    oracle.orc_matmul_bitnet_act_quant_f32(P(gold["i8x_w"]), P(gold["i8x_scales"]), P(gold["aq_x"]), None, P(y),
                                           64, 2560)
    assert np.array_equal(bits(y), bits(gold["aq_y"]))
    sw, sin, sout = (float(v) for v in gold["i8o_scales"])
    y8 = np.zeros(40, np.int8)
    oracle.orc_matmul_bitnet_int8(P(gold["i8o_w"]), sw, P(gold["i8o_x"]), sin, P(gold["i8o_bias"]), P(y8), sout, 40,
                                  256)
    assert np.array_equal(y8, gold["i8o_y"])


def test_fp32_gemvs_match_reference(oracle, gold):
    import synth
    rows, cols = 48, 640
    codes = synth.unpack_ternary(gold["f32_w"], cols).astype(np.float64)
    x = gold["f32_x"].astype(np.float64)
    bias = gold["f32_bias"]
    for g in (128, 64, 4):
        bs = gold[f"blk{g}_scales"]
        y = np.zeros(rows, np.float32)
        oracle.orc_matmul_bitnet_block_f32(P(gold["f32_w"]), P(bs), g, P(gold["f32_x"]), P(bias), P(y), rows, cols)
        sc = np.repeat(bs.reshape(rows, -1), g, axis=1)[:, :cols]
        mag = (np.abs(codes) * sc) @ np.abs(x) + np.abs(bias)
        assert rel_bound(y, gold[f"blk{g}_y"], mag)
    y = np.zeros(rows, np.float32)
    oracle.orc_matmul_bitnet_f32(P(gold["f32_w"]), P(gold["f32_scales"]), P(gold["f32_x"]), P(bias), P(y), rows, cols)
    mag = (np.abs(codes) @ np.abs(x)) * gold["f32_scales"] + np.abs(bias)
    assert rel_bound(y, gold["f32_y"], mag)
    y = np.zeros(rows, np.float32)
    oracle.orc_matmul_bitnet_dense_f32(P(gold["dense_w"]), P(gold["f32_scales"]), P(gold["f32_x"]), P(bias), P(y),
                                       rows, cols)
    assert rel_bound(y, gold["dense_y"], mag)
    y = np.zeros(rows, np.float32)
    oracle.orc_matmul_bitnet_tmac_interleaved_f32(P(gold["tmac_w"]), P(gold["f32_scales"]), P(gold["f32_x"]), P(bias),
                                                  P(y), rows, cols)
    assert rel_bound(y, gold["tmac_y"], mag)


def test_int_fp32_and_gemm_match_reference(oracle, gold):
    import synth
    w, s, x = gold["int8_w"], gold["int8_scales"], gold["int8_x"]
    mag = (np.abs(w.astype(np.float64)) @ np.abs(x.astype(np.float64))) * s
    y = np.zeros(64, np.float32)
    oracle.orc_int8_rowscale_f32(P(y), P(w), P(x), 896, 64, P(s))
    assert rel_bound(y, gold["int8_y"], mag) and rel_bound(y, gold["int8q_y"], mag)
    w4, s4, x4 = gold["int4_w"], gold["int4_scales"], gold["int4_x"]
    v4 = synth.unpack_int4(w4, 1024).astype(np.float64)
    mag = (np.abs(v4) @ np.abs(x4.astype(np.float64))) * s4
    y = np.zeros(64, np.float32)
    oracle.orc_int4_gemv_f32(P(y), P(w4), P(s4), P(x4), 64, 1024)
    assert rel_bound(y, gold["int4_y"], mag)
    A, W, b = gold["gemm_A"], gold["gemm_W"], gold["gemm_b"]
    Cm = np.zeros((13, 25), np.float32)
    oracle.orc_gemm_f32_nt_ld(P(A), 257, P(W), 257, P(b), P(Cm), 25, 13, 25, 257, 1, 0)
    mag = np.abs(A.astype(np.float64)) @ np.abs(W.astype(np.float64)).T + np.abs(b) + 1
    assert np.max(np.abs(Cm - gold["gemm_C"]) / mag) < 1e-5
    S = gold["softmax_in"].copy()
    oracle.orc_softmax_rows_f32(P(S), 5, 7, 10, 0.5)
    want = gold["softmax_out"]
    assert np.max(np.abs(S[:, :7] - want[:, :7]) / (want[:, :7] + 1e-30)) < 1e-5
    assert np.array_equal(S[:, 7:], want[:, 7:])
