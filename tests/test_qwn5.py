"""Qwen3.5 model files (QWN5, include/eif_hip_qwen35.h), on the CPU.

The test writer (model_files.qwen35_image) is checked against the reference's own loader, qwen35_load
(src/eif_qwen35.c:1223-1481, compiled from the reference sources into oracle/_ref/libref.so): every pointer the
loader sets lands on the array the writer put there, for INT4, ternary 2-bit (row and group scales, Hadamard
signs), ternary base-3 and FP32 files, with and without SubLN vectors, plain linears, and regions off their
natural alignment. The writer's base-3 packing is checked against the reference's own base-3 GEMV. Then
eif_qwen35_parse, the product's host-side walk, is checked against the same offsets, and against malformed
images that it must refuse.
"""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import P
import bitllm_hip as bh
import synth
import model_files

DN_KINDS = ("qkv", "z", "out", "pb", "pa")
FA_KINDS = ("q", "k", "v", "o")
FF_KINDS = ("gate", "up", "down")
KIND_ID = {"qkv": bh.Q35_DN_QKV, "z": bh.Q35_DN_Z, "out": bh.Q35_DN_OUT, "pb": bh.Q35_DN_B, "pa": bh.Q35_DN_A,
           "q": bh.Q35_FA_Q, "k": bh.Q35_FA_K, "v": bh.Q35_FA_V, "o": bh.Q35_FA_O,
           "gate": bh.Q35_FF_GATE, "up": bh.Q35_FF_UP, "down": bh.Q35_FF_DOWN}

# dim 64 = q_dim = val_dim (what a Hadamard file needs), two DeltaNet and two attention layers
BASE = dict(dim=64, hidden=128, layer_types=[0, 1, 0, 1], n_heads=2, n_kv_heads=1, head_dim=32, vocab=100,
            lin_k_heads=2, lin_k_dim=16, lin_v_heads=2, lin_v_dim=32)
CASES = {
    "int4_int8emb": (dict(quant_lm=model_files.Q35_INT4, quant_embed=model_files.Q35_EMBED_INT8), True, 0),
    "tern_rows_2bitemb": (dict(quant_lm=model_files.Q35_TERN2, quant_embed=model_files.Q35_EMBED_2BIT), True, 0),
    "tern_g32_hadamard": (dict(quant_lm=model_files.Q35_TERN2, quant_embed=model_files.Q35_EMBED_2BIT, group=32, hadamard=32),
                          True, 1),
    "dense_no_subln": (dict(quant_lm=model_files.Q35_TERN3, quant_embed=model_files.Q35_EMBED_DENSE), False, 3),
    "g64_plain_int8emb": (dict(quant_lm=model_files.Q35_TERN2, quant_embed=model_files.Q35_EMBED_INT8, group=64, plain=1),
                          True, 0),
    "fp32": (dict(quant_lm=model_files.Q35_FP32, quant_embed=model_files.Q35_EMBED_FP32), True, 2),
}


def make(case, key=(1,)):
    kw, subs, pad = CASES[case]
    cfg = model_files.qwen35_config(**dict(BASE, **kw))
    img, arrays = model_files.qwen35_image(cfg, key, sub_norms=subs, region_pad=pad)
    return cfg, img, arrays


def writer_order(cfg, arrays):
    """The writer's offsets in the order of ref_q35_layout (-1: absent)."""
    def off(name, field=0):
        a = arrays.get(name)
        return -1 if a is None or (field == 3 and a[3] == 0) else a[field]
    lt = cfg["layer_types"]
    out = [off("embed"), off("embed", 3)]
    for l in [l for l in range(len(lt)) if lt[l] == 0]:
        out += [off(f"L{l}.{k}") for k in DN_KINDS]
        out += [off(f"L{l}.conv"), off(f"L{l}.dt"), off(f"L{l}.alog")]
        out += [off(f"L{l}.{k}", 3) for k in DN_KINDS]
        out += [off(f"L{l}.dnorm")]
    for l in [l for l in range(len(lt)) if lt[l] == 1]:
        out += [off(f"L{l}.{k}") for k in FA_KINDS] + [off(f"L{l}.{k}", 3) for k in FA_KINDS]
        out += [off(f"L{l}.qnorm"), off(f"L{l}.knorm"), off(f"L{l}.sub_att") if not cfg["plain"] else -1]
    for l in range(len(lt)):
        out += [off(f"L{l}.{k}") for k in FF_KINDS] + [off(f"L{l}.{k}", 3) for k in FF_KINDS]
        out += [off(f"L{l}.sub_ffn") if not cfg["plain"] else -1, off(f"L{l}.rms_att"), off(f"L{l}.rms_ffn")]
    out += [off("rms_final"), off("signs_dim"), off("signs_hid")]
    return out


def parse_order(cfg, lay):
    """eif_qwen35_parse's offsets in the same order."""
    z = lambda v: -1 if v == 0 else v   # noqa: E731
    lt = cfg["layer_types"]
    out = [z(lay.embed.codes), z(lay.embed.scales)]
    for l in [l for l in range(len(lt)) if lt[l] == 0]:
        t = lay.lin[l]
        out += [z(t[KIND_ID[k]].codes) for k in DN_KINDS]
        out += [z(lay.conv[l]), z(lay.dt_bias[l]), z(lay.a_log[l])]
        out += [z(t[KIND_ID[k]].scales) for k in DN_KINDS] + [z(lay.delta_norm[l])]
    for l in [l for l in range(len(lt)) if lt[l] == 1]:
        t = lay.lin[l]
        out += [z(t[KIND_ID[k]].codes) for k in FA_KINDS] + [z(t[KIND_ID[k]].scales) for k in FA_KINDS]
        out += [z(lay.q_norm[l]), z(lay.k_norm[l]), z(lay.sub_att[l])]
    for l in range(len(lt)):
        t = lay.lin[l]
        out += [z(t[KIND_ID[k]].codes) for k in FF_KINDS] + [z(t[KIND_ID[k]].scales) for k in FF_KINDS]
        out += [z(lay.sub_ffn[l]), z(lay.rms_att[l]), z(lay.rms_ffn[l])]
    out += [z(lay.rms_final), z(lay.signs_dim), z(lay.signs_hid)]
    return out


def ref_order(ref, path):
    offs = np.zeros(4096, np.int64)
    n = C.c_int()
    rc = ref.ref_q35_layout(os.fsencode(path), P(offs), offs.size, C.byref(n))
    return rc, list(offs[:n.value])


@pytest.mark.parametrize("case", sorted(CASES))
def test_writer_matches_reference_loader(ref, tmp_path, case):
    cfg, img, arrays = make(case)
    path = tmp_path / "m.eifm"
    path.write_bytes(img)
    rc, got = ref_order(ref, str(path))
    assert rc == 0
    assert got == writer_order(cfg, arrays)


@pytest.mark.parametrize("case", sorted(CASES))
def test_parse_matches_writer(case):
    cfg, img, arrays = make(case)
    lay = bh.qwen35_parse(img)
    assert parse_order(cfg, lay) == writer_order(cfg, arrays)
    assert list(lay.layer_types[:lay.n_layers]) == cfg["layer_types"]
    assert lay.hadamard_block == cfg["hadamard"]
    # shapes, storage types and groups of the matrices
    g = cfg["group"]
    qtype = {model_files.Q35_TERN2: bh.Q35_TERN2, model_files.Q35_TERN3: bh.Q35_TERN3, model_files.Q35_INT4: bh.Q35_INT4,
             model_files.Q35_FP32: bh.Q35_FP32}[cfg["quant_lm"]]
    for l, t in enumerate(cfg["layer_types"]):
        for k in (DN_KINDS if t == 0 else FA_KINDS) + FF_KINDS:
            a, m = arrays[f"L{l}.{k}"], lay.lin[l][KIND_ID[k]]
            assert (m.rows, m.cols) == a[1].shape, (l, k)
            small = k in ("pb", "pa")
            want_qt = bh.Q35_FP32 if small and g > 0 else qtype
            assert m.qtype == want_qt, (l, k)
            assert m.group == (g if want_qt == bh.Q35_TERN2 else 0), (l, k)
    emb_qt = {model_files.Q35_EMBED_INT8: bh.Q35_INT8, model_files.Q35_EMBED_INT4: bh.Q35_INT4,
              model_files.Q35_EMBED_2BIT: bh.Q35_TERN2, model_files.Q35_EMBED_DENSE: bh.Q35_TERN3,
              model_files.Q35_EMBED_FP32: bh.Q35_FP32}[cfg["quant_embed"]]
    assert (lay.embed.rows, lay.embed.cols, lay.embed.qtype) == (cfg["vocab"], cfg["dim"], emb_qt)
    if not cfg["plain"]:                    # a plain file's SubLN vectors are ignored, as the reference does
        assert lay.norms_end == len(img)


def test_dense_packing_matches_reference_gemv(ref):
    """The writer's base-3 rows through the reference's own base-3 GEMV equal the ternary values' products."""
    r = np.random.default_rng(5)
    for rows, cols in ((7, 64), (5, 33), (3, 1)):
        v = r.integers(-1, 2, size=(rows, cols)).astype(np.int8)
        sc = (np.abs(r.standard_normal(rows)) + 0.1).astype(np.float32)
        x = r.integers(-4, 5, size=cols).astype(np.float32)   # small integers: the sums are exact
        out = np.zeros(rows, np.float32)
        packed = np.ascontiguousarray(model_files.pack_ternary_dense(v))
        ref.ref_q35_dense_gemv(P(out), P(packed), P(sc), P(x), rows, cols)
        np.testing.assert_array_equal(out, (v.astype(np.float32) @ x) * sc)
    # every byte value: five digits, the first column least significant (bytes above 242 keep five digits)
    allb = np.arange(256, dtype=np.uint8).reshape(256, 1)
    x = np.array([1.0, 10.0, 100.0, 1000.0, 10000.0], np.float32)
    out = np.zeros(256, np.float32)
    ref.ref_q35_dense_gemv(P(out), P(np.ascontiguousarray(allb)), P(np.ones(256, np.float32)), P(x), 256, 5)
    digits = np.stack([(np.arange(256) // 3 ** i) % 3 for i in range(5)], axis=1)
    vals = np.where(digits == 1, 1, np.where(digits == 2, -1, 0)).astype(np.float32)
    np.testing.assert_array_equal(out, vals @ x)


def corrupt(img, at, value, fmt="<I"):
    import struct
    b = bytearray(img)
    struct.pack_into(fmt, b, at, value)
    return bytes(b)


def test_parse_rejects_malformed(ref, tmp_path):
    cfg, img, _ = make("tern_g32_hadamard")
    bad = {
        "magic": corrupt(img, 0, 0x12345678),
        "version": corrupt(img, 4, 2),
        "group 48": corrupt(img, 48 + 4 * 27, 48, "<i"),
        "hadamard 24": corrupt(img, 48 + 4 * 28, 24, "<i"),
        "layers 25": corrupt(img, 48 + 4 * 2, 25, "<i"),
        "delta count": corrupt(img, 48 + 4 * 8, 1, "<i"),
    }
    for name, b in bad.items():
        with pytest.raises(bh.HipError):
            bh.qwen35_parse(b)
        path = tmp_path / "bad.eifm"
        path.write_bytes(b)
        rc, _ = ref_order(ref, str(path))
        assert rc < 0, name                    # the reference's loader refuses them too
    # refused here only (the reference would read past the file or past its arrays)
    cut = img[:len(img) - 100]
    with pytest.raises(bh.HipError):
        bh.qwen35_parse(cut)                   # norms region past the end of the file
    with pytest.raises(bh.HipError):
        bh.qwen35_parse(corrupt(img, 12, len(img) - 10))   # weights region runs past the file
    lt = bytearray(img)
    lt[176] = 2                                # a layer type that is neither DeltaNet nor attention
    with pytest.raises(bh.HipError):
        bh.qwen35_parse(bytes(lt))
    with pytest.raises(bh.HipError):
        bh.qwen35_parse(img[:40])
