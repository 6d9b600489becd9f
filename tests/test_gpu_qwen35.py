"""QWN5 files into resident GPU weights (eif_hip_qwen35_load): every quantized linear and the tied head of a
file read from disk gives, through eif_hip_qlinear (GEMV and GEMM paths), the same output bits as a weight
created directly from the arrays the test writer put in the file (base-3 rows as the 2-bit rows of the same
values); FP32 matrices have no GPU weight; every FP32 vector of the layout is on the device with its file's
values. The writer's layout is pinned against the reference's loader in tests/test_qwn5.py."""
import ctypes as C

import numpy as np
import pytest

from conftest import P
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


# The reference's prefill runs every quantized linear of a layer on n token rows at once (linear_gemm inside
# prefill_chunk, src/eif_qwen35.c:1034-1065, 1067-1153), the rows rotated by had_rows with the layer input's signs
# (signs_dim for inputs of width dim, q_dim and val_dim; signs_hid for the down projection's input).
C3 = model_files.qwen35_config(dim=1024, hidden=3584, layer_types=[0, 1], n_heads=8, n_kv_heads=2, head_dim=128,
                               vocab=2048, lin_k_heads=4, lin_k_dim=128, lin_v_heads=8, lin_v_dim=128,
                               quant_lm=model_files.Q35_INT4, quant_embed=model_files.Q35_EMBED_INT4)
BATCH_KINDS = {0: ("qkv", "out", "gate", "down"), 1: ("q", "o", "up", "down")}
EMB_QT = {model_files.Q35_EMBED_INT8: 4, model_files.Q35_EMBED_INT4: model_files.Q35_INT4,
          model_files.Q35_EMBED_2BIT: model_files.Q35_TERN2, model_files.Q35_EMBED_DENSE: model_files.Q35_TERN3,
          model_files.Q35_EMBED_FP32: model_files.Q35_FP32}


def oracle_batch(oracle, qt, values, scales, group, x, signs, block, norm, kpad, bias):
    """orc_prep_rows of the FP32 rows, then the oracle's linear of the weight's storage type:
    (y [M, rows], |contributions| [M, rows] for the tolerance of a grouped K split, or None)."""
    M, K = x.shape
    rows = values.shape[0]
    xq = np.zeros((M, kpad), np.int8)
    xs = np.zeros(M, np.float32)
    assert oracle.orc_prep_rows(P(np.ascontiguousarray(x)), K, P(signs), M, K, block, C.c_float(norm), P(xq), kpad,
                                P(xs), None, 0) == 0
    y = np.zeros((M, rows), np.float32)
    mag = None
    if qt == model_files.Q35_INT4:
        oracle.orc_int4_gemv_i8act(P(np.ascontiguousarray(synth.pack_int4(values))), P(scales), P(xq), kpad, P(xs),
                                   P(bias), P(y), rows, M, rows, K)
    elif qt == 4:
        oracle.orc_int8_gemv_i8act(P(np.ascontiguousarray(values)), P(scales), P(xq), kpad, P(xs), P(bias), P(y),
                                   rows, M, rows, K)
    else:
        w = np.ascontiguousarray(synth.pack_ternary(values))
        g = group if qt == model_files.Q35_TERN2 else 0
        if g:
            s = np.ascontiguousarray(scales.reshape(rows, -1))
            oracle.orc_ternary_gemv_grouped(P(w), P(s), g, P(xq), kpad, P(xs), P(bias), P(y), rows, M, rows, K)
            acc = np.zeros((M, rows, s.shape[1]), np.int32)
            oracle.orc_ternary_acc_i32(P(w), P(xq), kpad, M, rows, K, g, P(acc))
            mag = np.einsum("mng,ng->mn", np.abs(acc).astype(np.float64), s.astype(np.float64)) * xs[:, None]
            if bias is not None:
                mag = mag + np.abs(bias)[None, :]
        else:
            oracle.orc_ternary_gemv_rowscale(P(w), P(scales), P(xq), kpad, P(xs), P(bias), P(y), rows, M, rows, K)
    return y, mag


def check_batch(gpu, oracle, m, cfg, layer, kind, w, values, scales, qt, M, key):
    """eif_hip_qwen35_linear_batch on M FP32 rows (row stride K + 4) into y (row stride rows + 8): the oracle's
    output bit for bit (row-scaled INT4 / INT8 / ternary; grouped ternary when the GEMM does not split), grouped
    ternary within 1e-5 relative to the sum of |contributions| otherwise; y's padding columns untouched."""
    import torch
    dev = torch.device("cuda:0")
    lay = m.layout
    rows, K = values.shape
    assert (w.rows, w.cols) == (rows, K)
    block = lay.hadamard_block
    sig_off = (lay.signs_hid if kind == KIND_ID["down"] else lay.signs_dim) if block else 0
    signs = device_floats(m.vector(sig_off), K) if sig_off else None
    norm = gpu.wht_norm(block) if block else 1.0
    r = synth.rng(70, *key, M)
    x = r.standard_normal((M, K)).astype(np.float32)
    x[r.uniform(size=(M, K)) < 0.01] *= 20.0
    bias = r.standard_normal(rows).astype(np.float32) if M % 2 else None
    xd = torch.zeros((M, K + 4), device=dev)
    xd[:, :K] = torch.from_numpy(x).to(dev)
    yd = torch.full((M, rows + 8), 7.0, device=dev)
    bd = torch.from_numpy(bias).to(dev) if bias is not None else None
    sp = gpu.PrepSpec(x=gpu.ptr(xd).value, ldx=K + 4, x2=None, norm_w=None, eps=0.0, pre=gpu.PRE_NONE,
                      signs=m.vector(sig_off) if sig_off else None, wht_block=block, wht_norm=norm)
    m.linear_batch(layer, kind, sp, yd, M=M, bias=bd)
    torch.cuda.synchronize()
    yg = yd.cpu().numpy()
    assert np.all(yg[:, rows:] == 7.0), key
    yg = np.ascontiguousarray(yg[:, :rows])
    g = cfg["group"] if qt == model_files.Q35_TERN2 else 0
    want, mag = oracle_batch(oracle, qt, values, scales, g, x, signs, block, norm, w.kpad, bias)
    if mag is None:
        assert np.array_equal(yg.view(np.uint32), want.view(np.uint32)), key
    else:
        err = np.abs(yg.astype(np.float64) - want) / (mag + 1e-30)
        assert np.all(np.isfinite(yg)) and err.max() <= 1e-5, (key, err.max())


BATCH_FILES = ("int4_int8emb", "tern_rows_2bitemb", "tern_g32_hadamard", "dense_no_subln", "g64_plain_int8emb", "c3")


@pytest.mark.parametrize("case", BATCH_FILES)
def test_qwen35_linear_batch(gpu, oracle, tmp_path, case):
    """The prefill's batched linear on a file's resident weights: M = 64 rows take the int8-MFMA GEMM, 20 the
    streaming GEMV; every file's rotation (block and signs) as the file sets it. The c3 file has the layer shapes
    of a 1024-wide INT4 model (FFN 3584) and its INT4 head, unrotated (a QWN5 rotation needs grouped ternary
    linears and a 2-bit embedding, src/eif_qwen35.c:1273-1281). FP32 linears and bad indices are refused."""
    import torch
    if case == "c3":
        cfg = C3
        img, arrays = model_files.qwen35_image(cfg, (8,))
    else:
        cfg, img, arrays = make(case, key=(9,))
    path = tmp_path / "m.eifm"
    path.write_bytes(img)
    m = gpu.Qwen35Model(str(path))
    try:
        g, qlm = cfg["group"], cfg["quant_lm"]
        qt = EMB_QT[cfg["quant_embed"]]
        for M in (64, 20):
            for l, t in enumerate(cfg["layer_types"]):
                for k in BATCH_KINDS[t]:
                    _, values, scales, _ = arrays[f"L{l}.{k}"]
                    check_batch(gpu, oracle, m, cfg, l, KIND_ID[k], m.linear(l, KIND_ID[k]), values, scales, qlm, M,
                                (l, KIND_ID[k]))
            _, values, scales, _ = arrays["embed"]
            check_batch(gpu, oracle, m, cfg, 0, gpu.Q35_HEAD, m.head(), values, scales, qt, M, (99,))
        M = 64
        x = torch.zeros((M, cfg["dim"]), device="cuda:0")
        y = torch.zeros((M, cfg["hidden"]), device="cuda:0")
        sp = gpu.prep_spec(x)
        if g:   # a grouped file's beta projection is FP32: no GPU weight
            with pytest.raises(gpu.HipError):
                m.linear_batch(0, KIND_ID["pb"], sp, y, M=M)
        with pytest.raises(gpu.HipError):
            m.linear_batch(len(cfg["layer_types"]), KIND_ID["gate"], sp, y, M=M)
    finally:
        m.close()
