"""The decode oracle (oracle/decode_oracle.c) against the reference's own BitNet tinyllm decode.

* FP32-linear mode against the golden decode of the reference (tests/golden/decode_vectors.npz, written by the
  scalar build of the reference sources, oracle/_ref/libref_scalar.so): logits to 1e-5 of their largest
  magnitude, the same greedy tokens. Where the reference build is present, also against it live.
* INT8-activation mode (the GPU contract) against FP32 mode: the quantization of the linear inputs moves the
  logits a little and keeps the greedy tokens.
* orc_round_f16 (fp16 KV cache) against numpy's IEEE binary16 conversion.
"""
import ctypes as C
import os
import sys

import numpy as np
import pytest

from conftest import P, ROOT

sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
import synth  # noqa: E402
import oracle_api  # noqa: E402
import make_golden  # noqa: E402


def run_oracle(oracle, cfg, w, tokens, mode):
    c, ws = oracle_api.bitnet_structs(cfg, w)
    kv = cfg["n_kv_heads"] * cfg["head_dim"]
    kc = np.zeros((cfg["n_layers"], cfg["seq_len"], kv), np.float32)
    vc = np.zeros_like(kc)
    out = []
    for pos, tok in enumerate(tokens):
        lo = np.zeros(cfg["vocab"], np.float32)
        assert oracle.orc_bitnet_forward(C.byref(c), C.byref(ws), P(kc), P(vc), int(tok), pos, mode, P(lo)) == 0
        out.append(lo)
    return np.stack(out), kc, vc


@pytest.fixture(scope="module")
def tiny():
    cfg = make_golden.decode_config()
    return cfg, synth.bitnet_model(make_golden.DECODE_KEY, cfg)


@pytest.fixture(scope="module")
def golden():
    return np.load(os.path.join(ROOT, "tests", "golden", "decode_vectors.npz"))


def test_f32_mode_matches_reference_golden(oracle, tiny, golden):
    cfg, w = tiny
    tokens = golden["scalar_tokens"]
    lo, _, _ = run_oracle(oracle, cfg, w, tokens[:-1], oracle_api.ORC_LIN_F32)
    ref = golden["scalar_logits"]
    err = np.abs(lo - ref).max(axis=1) / np.abs(ref).max(axis=1)
    assert err.max() <= 1e-5, err
    assert np.array_equal(np.argmax(lo, axis=1), tokens[1:])
    # the reference-flag build (fast-math exp in its SiLU, AVX2 sums) stays close to the scalar one
    x86 = golden["x86_logits"]
    assert (np.abs(x86 - ref).max(axis=1) / np.abs(ref).max(axis=1)).max() <= 1e-3


def test_f32_mode_matches_reference_live(oracle, tiny):
    path = os.path.join(ROOT, "oracle", "_ref", "libref_scalar.so")
    if not os.path.exists(path):
        pytest.skip("oracle/_ref/libref_scalar.so not built (no reference tree)")
    ref = oracle_api.load_ref_tinyllm(path)
    cfg, w = tiny
    # a longer run with another start token
    c, ws = oracle_api.bitnet_structs(cfg, w)
    h = ref.ref_bitnet_create(C.byref(c), C.byref(ws), cfg["g_q"])
    try:
        tokens, rl = [17], []
        for pos in range(24):
            lp = ref.ref_bitnet_forward(h, tokens[-1], pos)
            rl.append(np.ctypeslib.as_array(lp, shape=(cfg["vocab"],)).copy())
            tokens.append(int(np.argmax(rl[-1])))
    finally:
        ref.ref_bitnet_destroy(h)
    lo, _, _ = run_oracle(oracle, cfg, w, tokens[:-1], oracle_api.ORC_LIN_F32)
    rl = np.stack(rl)
    assert (np.abs(lo - rl).max(axis=1) / np.abs(rl).max(axis=1)).max() <= 1e-5
    assert np.array_equal(np.argmax(lo, axis=1), tokens[1:])


def test_int8_mode_close_to_f32(oracle, tiny, golden):
    cfg, w = tiny
    tokens = golden["scalar_tokens"][:-1]
    lf, _, _ = run_oracle(oracle, cfg, w, tokens, oracle_api.ORC_LIN_F32)
    lq, kc, _ = run_oracle(oracle, cfg, w, tokens, oracle_api.ORC_LIN_INT8)
    for a, b in zip(lq, lf):
        assert np.corrcoef(a, b)[0, 1] > 0.9995
    assert np.array_equal(np.argmax(lq, axis=1), np.argmax(lf, axis=1))
    # the INT8 mode keeps its cache in fp16 values
    used = kc[:, :len(tokens)]
    assert np.array_equal(used, used.astype(np.float16).astype(np.float32))


def test_round_f16(oracle):
    r = np.random.default_rng(5)
    v = np.concatenate([r.standard_normal(20000) * 10.0 ** r.integers(-9, 6, 20000),
                        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -70000.0, 6.1035156e-05, 5.96e-08, 2.98e-08,
                                  2.99e-08, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, np.inf, -np.inf])]).astype(np.float32)
    got = np.array([oracle.orc_round_f16(float(x)) for x in v], np.float32)
    with np.errstate(over='ignore'):
        want = v.astype(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
