"""Qwen3.5 GGUF files -> QWN5 images (eif_qwen35_gguf_image, include/eif_hip_qwen35.h), on the CPU.

A llama.cpp-style Qwen3.5 GGUF of the test writer (model_files.qwen35_gguf: 24 blocks, DeltaNet and attention layers,
linears in F32 / F16 / BF16 / Q8_0 / Q4_0 / Q4_K / Q5_K / Q6_K, embeddings in several of them) goes through the
reference's own image builder (qwen35_gguf_build_image, src/eif_qwen35_gguf.c:262-454, compiled into
oracle/_ref/libref.so with the reference's flags) and through eif_qwen35_gguf_image. The images are byte for byte
the same: header, configuration, layer types, every INT4 / INT8 row and scale, conv, dt, norms. The one exception
is A_log = logf(-ssm_a): the reference's -ffast-math build evaluates logf with glibc's vector variants, here the
scalar logf gives it, bit for bit what the reference's scalar build (libref_scalar.so) stores and within 4 ulp of
the vector form. The oracle's orc_quant_rows reproduces the image's INT4 / INT8 rows of F32 tensors bit for bit
(its arithmetic is the reference build's). Files the builder refuses are refused here too.
"""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import ROOT, P
import bitllm_hip as bh
import synth
import model_files

REF = os.path.join(ROOT, "oracle", "_ref", "libref.so")
REF_SCALAR = os.path.join(ROOT, "oracle", "_ref", "libref_scalar.so")


def _builder(path):
    if not os.path.exists(path):
        pytest.skip("oracle/_ref not built (reference tree absent)")
    lib = C.CDLL(path)
    lib.qwen35_gguf_build_image.restype = C.c_int
    lib.qwen35_gguf_build_image.argtypes = [C.c_char_p, C.c_size_t, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)]
    libc = C.CDLL(None)
    libc.free.argtypes = [C.c_void_p]

    def build(gguf):
        out, n = C.c_void_p(), C.c_size_t()
        rc = lib.qwen35_gguf_build_image(gguf, len(gguf), C.byref(out), C.byref(n))
        if rc:
            return rc, None
        img = C.string_at(out, n.value)
        libc.free(out)
        return 0, img
    return build


@pytest.fixture(scope="module")
def ref_build():
    return _builder(REF)


@pytest.fixture(scope="module")
def ref_scalar_build():
    return _builder(REF_SCALAR)


SMALL = dict(dim=64, hidden=128, n_heads=2, n_kv_heads=1, head_dim=32, vocab=100, heads_k=2, k_dim=16, v_dim=32)
CASES = {   # writer options
    "kquants_q6k_emb": dict(),
    "q4k_emb_mixed": dict(emb_type=model_files.GGUF_Q4_K, lin_types=(model_files.GGUF_Q5_K, model_files.GGUF_BF16, model_files.GGUF_Q4_0,
                                                                model_files.GGUF_Q6_K), ctx=1000),
    "small_block32": dict(SMALL, emb_type=model_files.GGUF_F16, lin_types=(model_files.GGUF_Q8_0, model_files.GGUF_Q4_0, model_files.GGUF_F32,
                                                                      model_files.GGUF_BF16, model_files.GGUF_F16)),
    "small_f32_emb_q8": dict(SMALL, emb_type=model_files.GGUF_F32, lin_types=(model_files.GGUF_F32,), ctx=9000),
}
# (a full-attention layer every 4 of the 24 gives the 18 DeltaNet and 6 attention layers the reference's loader
# holds; the builder itself accepts other intervals)


def a_log_slots(img):
    lay = bh.qwen35_parse(img)
    nv = lay.config[12]
    return [(lay.a_log[l], nv) for l in range(lay.n_layers) if lay.a_log[l]]


@pytest.mark.parametrize("case", sorted(CASES))
def test_image_matches_reference_builder(ref_build, ref_scalar_build, case):
    gguf = model_files.qwen35_gguf((2,), **CASES[case])
    rc, ref = ref_build(gguf)
    assert rc == 0
    ours = bh.qwen35_gguf_image(gguf)
    assert len(ours) == len(ref)
    a, b = np.frombuffer(ref, np.uint8).copy(), np.frombuffer(ours, np.uint8).copy()
    _, scalar = ref_scalar_build(gguf)
    s = np.frombuffer(scalar, np.uint8)
    for off, n in a_log_slots(ours):
        ra, oa = (np.frombuffer(x[off:off + 4 * n], np.float32) for x in (ref, ours))
        assert np.array_equal(oa.view(np.uint32), np.frombuffer(scalar[off:off + 4 * n], np.uint32))
        ulp = np.abs(ra.view(np.int32).astype(np.int64) - oa.view(np.int32).astype(np.int64))
        assert ulp.max() <= 4         # the vector logf against the scalar one
        a[off:off + 4 * n] = b[off:off + 4 * n] = 0
    assert np.array_equal(a, b), np.flatnonzero(a != b)[:8]
    assert len(a_log_slots(ours)) > 0


def test_oracle_quant_rows_matches_reference_image(ref_build, oracle):
    """The image's INT4 and INT8 rows of F32 tensors are orc_quant_rows of those rows (the oracle's arithmetic is
    the compiled reference's)."""
    cap = []
    orig = model_files.gguf_dense_tensor

    def spy(r, rows, cols, ty):
        raw = orig(r, rows, cols, ty)
        cap.append((np.frombuffer(raw, np.float32).reshape(rows, cols).copy() if ty == model_files.GGUF_F32 else None))
        return raw
    model_files.gguf_dense_tensor = spy
    try:
        gguf = model_files.qwen35_gguf((3,), emb_type=model_files.GGUF_F32, lin_types=(model_files.GGUF_F32,))
    finally:
        model_files.gguf_dense_tensor = orig
    rc, img = ref_build(gguf)
    assert rc == 0
    lay = bh.qwen35_parse(img)
    checks = [(lay.embed, cap[0], 8), (lay.lin[0][bh.Q35_DN_QKV], cap[1], 4), (lay.lin[0][bh.Q35_DN_OUT], cap[3], 4),
              (lay.lin[0][bh.Q35_FF_DOWN], cap[8], 4)]
    for t, x, bits in checks:
        rows, cols = x.shape
        assert (t.rows, t.cols) == (rows, cols)
        rb = cols if bits == 8 else (cols + 1) // 2
        dst = np.zeros((rows, rb), np.uint8)
        sc = np.zeros(rows, np.float32)
        oracle.orc_quant_rows(P(x), cols, rows, cols, bits, P(dst), P(sc))
        assert dst.tobytes() == img[t.codes:t.codes + rows * rb]
        assert sc.tobytes() == img[t.scales:t.scales + 4 * rows]


def _set(kv, key, t, v):
    return [(k, t, v) if k == key else (k, tt, vv) for k, tt, vv in kv]


def test_gguf_image_rejects(ref_build):
    def edit(**kw):
        return model_files.qwen35_gguf((4,), **dict(SMALL, emb_type=model_files.GGUF_F16, **kw))
    bad = {
        "arch": edit(kv_edit=lambda kv: _set(kv, "general.architecture", model_files.GGUF_STR, "llama")),
        "23 blocks": edit(kv_edit=lambda kv: _set(kv, "qwen35.block_count", model_files.GGUF_U32, 23)),
        "eps 1e-5": edit(kv_edit=lambda kv: _set(kv, "qwen35.attention.layer_norm_rms_epsilon", model_files.GGUF_F32V, 1e-5)),
        "k heads != v heads": edit(kv_edit=lambda kv: _set(kv, "qwen35.ssm.time_step_rank", model_files.GGUF_U32, 4)),
        "untied head": edit(extra_tensors=[("output.weight", model_files.GGUF_F32, (64, 100), bytes(64 * 100 * 4))]),
        "missing tensor": edit(drop=("blk.5.ffn_up.weight",)),
        "Q4_1 linear": edit(lin_types=(model_files.GGUF_Q4_1,)),
    }
    good = edit()
    bad["truncated"] = good[:len(good) - 4096]
    for name, g in bad.items():
        with pytest.raises(bh.HipError):
            bh.qwen35_gguf_image(g)
        if name != "truncated":
            assert ref_build(g)[0] != 0, name      # the reference's builder refuses it too
    assert len(bh.qwen35_gguf_image(good)) > 0
