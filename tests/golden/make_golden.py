"""Writes tests/golden/reference_vectors.npz: inputs and outputs of the reference's own hot-path functions.

The outputs come from oracle/_ref/libref.so, which oracle/Makefile (`make ref`) compiles from the reference's
sources with its own flags (-O3 -mavx2 -mfma -ffast-math -fopenmp); the reference ships no golden vectors for this
path. Run from the repository root in the container that has the reference tree:  python tests/golden/make_golden.py
The fixture is data only (seeded inputs and the outputs the reference computed for them).

The reference runs single-threaded here: its T-MAC GEMV keeps the activation LUT in a __thread buffer filled by
the calling thread only (src/eif_quantize_bitnet.c:608-610, :780-796), so under OpenMP the rows computed by worker
threads read an unfilled table and come out wrong. With one thread every function computes its documented result.
"""
import os
import sys

os.environ["OMP_NUM_THREADS"] = "1"

import numpy as np  # noqa: E402

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "bitllm.c_amd"))
import oracle_api  # noqa: E402
import synth  # noqa: E402

P = oracle_api.P


def main():
    ref = oracle_api.load_ref(os.path.join(ROOT, "oracle", "_ref", "libref.so"))
    r = np.random.default_rng(20261201)
    out = {}

    # WHT norm the reference build uses, for blocks 1 .. 2^14 (e0 rotated: every element = norm)
    norms = []
    for k in range(15):
        b = 1 << k
        e = np.zeros(b, np.float32)
        e[0] = 1.0
        ref.eif_hadamard_rotate_f32(P(e), None, b, b)
        norms.append(e[0])
    out["wht_norms"] = np.array(norms, np.float32)

    # a3: rotation, K = 2560 block 128 with signs, K = 4096 block 1024 without
    for name, n, b, signed in (("wht_2560_128", 2560, 128, True), ("wht_4096_1024", 4096, 1024, False)):
        x = synth.activations((7000, n), 1, n)[0]
        s = np.where(r.uniform(size=n) > 0.5, 1.0, -1.0).astype(np.float32) if signed else np.ones(n, np.float32)
        y = x.copy()
        ref.eif_hadamard_rotate_f32(P(y), P(s) if signed else None, n, b)
        out[name + "_x"], out[name + "_signs"], out[name + "_y"] = x, s, y
        out[name + "_meta"] = np.array([n, b, int(signed)], np.int32)

    # a4: activation quantization
    for name, n in (("quant_2560", 2560), ("quant_6912", 6912), ("quant_17", 17)):
        x = (synth.activations((7001, n), 1, n)[0] * r.uniform(0.01, 50)).astype(np.float32)
        q, sc = np.zeros(n, np.int8), np.zeros(1, np.float32)
        ref.eif_quantize_activation_i8(P(x), P(q), P(sc), n)
        out[name + "_x"], out[name + "_q"], out[name + "_scale"] = x, q, sc

    # a5 / a6 / a10: integer paths
    rows, cols = 64, 2560
    w = r.integers(0, 256, rows * cols // 4, dtype=np.uint8)
    xq = r.integers(-127, 128, cols).astype(np.int8)
    sc = (np.abs(r.standard_normal(rows)) * 0.02).astype(np.float32)
    bias = r.standard_normal(rows).astype(np.float32)
    y = np.zeros(rows, np.float32)
    ref.eif_matmul_bitnet_i8xternary_f32(P(w), P(sc), P(xq), 0.0173, P(bias), P(y), rows, cols)
    out.update(i8x_w=w, i8x_xq=xq, i8x_scales=sc, i8x_bias=bias, i8x_scale_in=np.float32([0.0173]), i8x_y=y)
    x = synth.activations((7002,), 1, cols)[0]
    y = np.zeros(rows, np.float32)
    ref.eif_matmul_bitnet_act_quant_f32(P(w), P(sc), P(x), None, P(y), rows, cols)
    out.update(aq_x=x, aq_y=y)
    r8, c8 = 40, 256
    w8 = r.integers(0, 256, r8 * c8 // 4, dtype=np.uint8)
    x8 = r.integers(-128, 128, c8).astype(np.int8)
    b8 = r.integers(-500, 500, r8).astype(np.int32)
    y8 = np.zeros(r8, np.int8)
    ref.eif_matmul_bitnet_int8(P(w8), 0.02, P(x8), 0.9, P(b8), P(y8), 0.37, r8, c8)
    out.update(i8o_w=w8, i8o_x=x8, i8o_bias=b8, i8o_y=y8, i8o_scales=np.float32([0.02, 0.9, 0.37]))

    # a7 / a8 / a9 / a11 / a12: FP32-activation GEMVs (rows 48, cols 640)
    rows, cols = 48, 640
    codes = r.integers(-1, 2, (rows, cols)).astype(np.int8)
    wt = synth.pack_ternary(codes)
    x = synth.activations((7003,), 1, cols)[0]
    rsc = (np.abs(r.standard_normal(rows)) * 0.02).astype(np.float32)
    bias = r.standard_normal(rows).astype(np.float32)
    out.update(f32_w=wt, f32_x=x, f32_scales=rsc, f32_bias=bias)
    for g in (128, 64, 4):
        nb = -(-cols // g)
        bs = (np.abs(r.standard_normal(rows * nb)) * 0.02).astype(np.float32)
        y = np.zeros(rows, np.float32)
        ref.eif_matmul_bitnet_block_f32(P(wt), P(bs), g, P(x), P(bias), P(y), rows, cols)
        out[f"blk{g}_scales"], out[f"blk{g}_y"] = bs, y
    y = np.zeros(rows, np.float32)
    ref.eif_matmul_bitnet_f32(P(wt), P(rsc), P(x), P(bias), P(y), rows, cols)
    out["f32_y"] = y
    y1, y3 = np.zeros(rows // 2, np.float32), np.zeros(rows // 2, np.float32)
    w1, w3 = wt[: rows // 2].copy(), wt[rows // 2:].copy()
    ref.eif_matmul_bitnet_f32_w1w3(P(y1), P(y3), P(w1), P(w3), P(rsc[: rows // 2].copy()),
                                   P(rsc[rows // 2:].copy()), P(x), rows // 2, cols)
    out.update(w1w3_y1=y1, w1w3_y3=y3)
    dense = np.zeros(rows * ((cols + 4) // 5), np.uint8)
    for i in range(rows):
        ref.eif_pack_ternary_dense(P(np.ascontiguousarray(codes[i])), P(dense[i * ((cols + 4) // 5):]), cols)
    y = np.zeros(rows, np.float32)
    ref.eif_matmul_bitnet_dense_f32(P(dense), P(rsc), P(x), P(bias), P(y), rows, cols)
    out.update(dense_w=dense, dense_y=y)
    il = np.zeros_like(wt.reshape(-1))
    ref.eif_interleave_weights_4rows(P(wt), P(il), rows, cols)
    y = np.zeros(rows, np.float32)
    ref.eif_matmul_bitnet_tmac_interleaved_f32(P(il), P(rsc), P(x), P(bias), P(y), rows, cols)
    out.update(tmac_w=il, tmac_y=y)

    # a14 / a15 / a16: INT8 and INT4 row-scaled, FP32 activations
    w, s = synth.int8_weight((7004,), 64, 896)
    x = synth.activations((7005,), 1, 896)[0]
    y = np.zeros(64, np.float32)
    ref.tinyllm_matmul_int8_rowscale(P(y), P(w), P(x), 896, 64, P(s))
    out.update(int8_w=w, int8_scales=s, int8_x=x, int8_y=y)
    y = np.zeros(64, np.float32)
    ref.ref_q35_int8_gemv(P(y), P(w), P(s), P(x), 64, 896)
    out["int8q_y"] = y
    w, s = synth.int4_weight((7006,), 64, 1024)
    x = synth.activations((7007,), 1, 1024)[0]
    y = np.zeros(64, np.float32)
    ref.ref_q35_int4_gemv(P(y), P(w), P(s), P(x), 64, 1024)
    out.update(int4_w=w, int4_scales=s, int4_x=x, int4_y=y)

    # a18: FP32 GEMM (bias + GELU) and softmax
    M, N, K = 13, 25, 257
    A = r.uniform(-1, 1, (M, K)).astype(np.float32)
    W = r.uniform(-1, 1, (N, K)).astype(np.float32)
    b = r.uniform(-1, 1, N).astype(np.float32)
    C = np.zeros((M, N), np.float32)
    ref.eif_gemm_f32_nt_ld(P(A), K, P(W), K, P(b), P(C), N, M, N, K, 1, 0)
    out.update(gemm_A=A, gemm_W=W, gemm_b=b, gemm_C=C)
    S = (r.uniform(-1, 1, (5, 10)) * 40).astype(np.float32)
    S_out = S.copy()
    ref.eif_softmax_rows_f32(P(S_out), 5, 7, 10, 0.5)
    out.update(softmax_in=S, softmax_out=S_out)

    path = os.path.join(ROOT, "tests", "golden", "reference_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes")


# the decode fixture: a tiny BitNet model regenerated from its seed by synth.bitnet_model (weights are not stored)
DECODE_KEY = (7,)
DECODE_CFG = dict(dim=128, hidden=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=32, vocab=300, seq_len=32,
                  group_in=32, group_down=32, wht_dim=128, wht_q=128, wht_hidden=256)
DECODE_STEPS = 16


def decode_config():
    c = dict(DECODE_CFG)
    return synth.bitnet_config(c.pop("dim"), c.pop("hidden"), c.pop("n_layers"), c.pop("n_heads"), c.pop("n_kv_heads"),
                               c.pop("head_dim"), c.pop("vocab"), c.pop("seq_len"), c.pop("group_in"),
                               c.pop("group_down"), c.pop("wht_dim"), c.pop("wht_q"), c.pop("wht_hidden"))


def decode_main():
    """Writes tests/golden/decode_vectors.npz: greedy decode of the reference's own tinyllm BitNet model
    (oracle/ref_tinyllm_wrap.c) built from synth.bitnet_model(DECODE_KEY, ...), by the scalar build
    (_ref/libref_scalar.so) and by the reference-flag build (_ref/libref.so)."""
    import ctypes as C
    cfg = decode_config()
    w = synth.bitnet_model(DECODE_KEY, cfg)
    c, ws = oracle_api.bitnet_structs(cfg, w)
    out = {}
    for tag, lib in (("scalar", "libref_scalar.so"), ("x86", "libref.so")):
        ref = oracle_api.load_ref_tinyllm(os.path.join(ROOT, "oracle", "_ref", lib))
        h = ref.ref_bitnet_create(C.byref(c), C.byref(ws), cfg["g_q"])
        tokens, logits = [5], []
        for pos in range(DECODE_STEPS):
            lp = ref.ref_bitnet_forward(h, tokens[-1], pos)
            lo = np.ctypeslib.as_array(lp, shape=(cfg["vocab"],)).copy()
            logits.append(lo)
            tokens.append(int(np.argmax(lo)))
        ref.ref_bitnet_destroy(h)
        out[tag + "_tokens"] = np.array(tokens, np.int32)
        out[tag + "_logits"] = np.stack(logits)
    path = os.path.join(ROOT, "tests", "golden", "decode_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
    decode_main()
