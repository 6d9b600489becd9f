"""QWN5 files into resident GPU weights (eif_hip_qwen35_load): every quantized linear and the tied head of a
file read from disk gives, through eif_hip_qlinear (GEMV and GEMM paths), the same output bits as a weight
created directly from the arrays the test writer put in the file (base-3 rows as the 2-bit rows of the same
values); FP32 matrices have no GPU weight; every FP32 vector of the layout is on the device with its file's
values. The writer's layout is pinned against the reference's loader in tests/test_qwn5.py."""
import ctypes as C

import numpy as np
import pytest

import synth
import model_files
from test_qwn5 import CASES, DN_KINDS, FA_KINDS, FF_KINDS, KIND_ID, make

pytestmark = pytest.mark.gpu

VECTORS = ("rms_att", "rms_ffn", "sub_att", "sub_ffn", "conv", "dt_bias", "a_log", "delta_norm", "q_norm", "k_norm")
VEC_NAME = {"rms_att": "rms_att", "rms_ffn": "rms_ffn", "sub_att": "sub_att", "sub_ffn": "sub_ffn", "conv": "conv",
            "dt_bias": "dt", "a_log": "alog", "delta_norm": "dnorm", "q_norm": "qnorm", "k_norm": "knorm"}


def expected_weight(gpu, qt, values, scales, group):
    rows, cols = values.shape
    if qt == model_files.Q35_INT4:
        return gpu.QWeight(gpu.W_INT4, rows, cols, 0, np.ascontiguousarray(synth.pack_int4(values)), scales)
    if qt == 4:
        return gpu.QWeight(gpu.W_INT8, rows, cols, 0, np.ascontiguousarray(values), scales)
    g = group if qt == model_files.Q35_TERN2 else 0
    return gpu.QWeight(gpu.W_TERNARY, rows, cols, g, np.ascontiguousarray(synth.pack_ternary(values)),
                       np.ascontiguousarray(scales.reshape(rows, -1) if g else scales))


def same_outputs(gpu, w, want, key):
    import torch
    dev = torch.device("cuda:0")
    assert (w.rows, w.cols, w.kpad) == (want.rows, want.cols, want.kpad)
    r = np.random.default_rng(key)
    for M in (3, 20):   # GEMV and GEMM paths
        xq = torch.from_numpy(r.integers(-127, 128, size=(M, w.kpad), dtype=np.int8)).to(dev)
        xq[:, w.cols:] = 0
        xs = torch.from_numpy((np.abs(r.standard_normal(M)) + 0.1).astype(np.float32)).to(dev)
        y0 = torch.zeros((M, w.rows), device=dev)
        y1 = torch.zeros((M, w.rows), device=dev)
        w.linear(xq, xs, y0)
        want.linear(xq, xs, y1)
        torch.cuda.synchronize()
        assert torch.equal(y0.view(torch.int32), y1.view(torch.int32)), M


def device_floats(ptr, n):
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    out = np.zeros(n, np.float32)
    assert hip.hipMemcpy(out.ctypes.data, ptr, n * 4, 2) == 0
    return out


@pytest.mark.parametrize("case", sorted(CASES))
def test_qwen35_file_weights(gpu, tmp_path, case):
    cfg, img, arrays = make(case, key=(7,))
    path = tmp_path / "m.eifm"
    path.write_bytes(img)
    m = gpu.Qwen35Model(str(path))
    try:
        lay, g, qlm = m.layout, cfg["group"], cfg["quant_lm"]
        n_checked = 0
        for l, t in enumerate(cfg["layer_types"]):
            for k in (DN_KINDS if t == 0 else FA_KINDS) + FF_KINDS:
                _, values, scales, _ = arrays[f"L{l}.{k}"]
                qt = model_files.Q35_FP32 if k in ("pb", "pa") and g > 0 else qlm
                w = m.linear(l, KIND_ID[k])
                if qt == model_files.Q35_FP32:
                    assert w is None, (l, k)
                    continue
                want = expected_weight(gpu, qt, values, scales, g)
                same_outputs(gpu, w, want, (l, KIND_ID[k]))
                want.close()
                n_checked += 1
            for other in range(gpu.Q35_KINDS):   # kinds the layer does not have
                names = (DN_KINDS if t == 0 else FA_KINDS) + FF_KINDS
                if other not in [KIND_ID[k] for k in names]:
                    assert m.linear(l, other) is None
        assert n_checked == 0 or qlm != model_files.Q35_FP32
        # the tied head
        emb_qt = {model_files.Q35_EMBED_INT8: 4, model_files.Q35_EMBED_INT4: model_files.Q35_INT4, model_files.Q35_EMBED_2BIT: model_files.Q35_TERN2,
                  model_files.Q35_EMBED_DENSE: model_files.Q35_TERN3, model_files.Q35_EMBED_FP32: model_files.Q35_FP32}[cfg["quant_embed"]]
        _, values, scales, _ = arrays["embed"]
        h = m.head()
        if emb_qt == model_files.Q35_FP32:
            assert h is None
        else:
            want = expected_weight(gpu, emb_qt, values, scales, g)
            same_outputs(gpu, h, want, (99,))
            want.close()
        # FP32 vectors on the device
        for l in range(lay.n_layers):
            for field in VECTORS:
                off = getattr(lay, field)[l]
                name = f"L{l}.{VEC_NAME[field]}"
                if off == 0:
                    assert name not in arrays or (cfg["plain"] and field in ("sub_att", "sub_ffn"))
                    continue
                v = arrays[name][1]
                np.testing.assert_array_equal(device_floats(m.vector(off), v.size), v)
        for field, name in (("rms_final", "rms_final"), ("signs_dim", "signs_dim"), ("signs_hid", "signs_hid")):
            off = getattr(lay, field)
            if off:
                v = arrays[name][1]
                ptr = m.vector(off)
                assert ptr % 16 == 0
                np.testing.assert_array_equal(device_floats(ptr, v.size), v)
        assert m.vector(lay.rms_final + 4) == 0    # not the start of a vector
    finally:
        m.close()


def test_qwen35_load_rejects(gpu, tmp_path):
    _, img, _ = make("tern_rows_2bitemb")
    path = tmp_path / "bad.eifm"
    path.write_bytes(img[:len(img) // 2])
    with pytest.raises(gpu.HipError):
        gpu.Qwen35Model(str(path))
    with pytest.raises(gpu.HipError):
        gpu.Qwen35Model(str(tmp_path / "missing.eifm"))


def test_qwen35_gguf_loads_as_its_image(gpu, tmp_path):
    """A Qwen3.5 GGUF path given to eif_hip_qwen35_load loads as the QWN5 image eif_qwen35_gguf_image builds from
    it (the reference's image, tests/test_qwen35_gguf.py): the same layout, every INT4 linear and the INT8 head
    giving the same output bits, the same FP32 vectors."""
    gguf = model_files.qwen35_gguf((6,), dim=256, hidden=512, vocab=500)
    pg, pi = tmp_path / "m.gguf", tmp_path / "m.eifm"
    pg.write_bytes(gguf)
    pi.write_bytes(gpu.qwen35_gguf_image(gguf))
    mg, mi = gpu.Qwen35Model(str(pg)), gpu.Qwen35Model(str(pi))
    try:
        lg, li = mg.layout, mi.layout
        assert lg.n_layers == li.n_layers == 24 and list(lg.layer_types[:24]) == list(li.layer_types[:24])
        n = 0
        for l in range(24):
            for k in range(gpu.Q35_KINDS):
                a, b = mg.linear(l, k), mi.linear(l, k)
                assert (a is None) == (b is None), (l, k)
                if a is not None:
                    same_outputs(gpu, a, b, (l, k))
                    n += 1
        assert n == 18 * 5 + 6 * 4 + 24 * 3
        same_outputs(gpu, mg.head(), mi.head(), (77,))
        # lengths of the writer's defaults: dim 256, hidden 512, 4 value heads of 64, key 4 x 32, head_dim 64
        size = {"rms_att": 256, "rms_ffn": 256, "sub_att": 256, "sub_ffn": 512, "conv": 512 * 4, "dt_bias": 4,
                "a_log": 4, "delta_norm": 64, "q_norm": 64, "k_norm": 64}
        for l in range(24):
            for field in VECTORS:
                off = getattr(lg, field)[l]
                assert off == getattr(li, field)[l]
                if off:
                    np.testing.assert_array_equal(device_floats(mg.vector(off), size[field]),
                                                  device_floats(mi.vector(off), size[field]))
    finally:
        mg.close()
        mi.close()
