"""Writers of model files for the tests: BitNet SVLM and TTML files, Qwen3.5 QWN5 images, GGUF containers (BitNet and
Qwen3.5), each in the reference's layout, from the seeded arrays of synth.py. Test infrastructure only: the product
library reads such files, and these writers make the inputs its file tests feed it."""
import struct

import numpy as np

from synth import bitnet_model, pack_int4, pack_ternary, rng


def write_svlm(path, cfg, w, group_bound, hadamard=True):
    """Write a BitNet model (bitnet_model's arrays) as a file in the reference's SVLM layout, the one
    tinyllm_load_quantized_model reads (src/eif_tinyllm.c:2442-2556, pointers as tinyllm_setup_quantized_pointers
    sets them, :2690-2731; configuration words as src/eif_llm.c:321-342 reads them). cfg's groups must be the
    ones the reader derives: eif_bitnet_group_size(input width, group_bound), or 0 (one scale per row) when that is
    0 or the width itself."""
    d, h, L = cfg["dim"], cfg["hidden"], cfg["n_layers"]
    weights = b"".join(np.ascontiguousarray(w[k]).tobytes()
                       for k in ("emb", "wq", "wk", "wv", "wo", "w1", "w2", "w3", "wcls"))
    skeys = ["emb_scale", "gq", "gk", "gv", "go", "g1", "g3", "g2", "wcls_scale"]
    if hadamard:
        skeys += ["signs_dim", "signs_q", "signs_hidden"]
    scales = b"".join(np.ascontiguousarray(w[k], dtype=np.float32).tobytes() for k in skeys)
    norms = b"".join(np.ascontiguousarray(w[k], dtype=np.float32).tobytes()
                     for k in ("rms_att", "rms_ffn", "rms_final", "rms_sub_att", "rms_sub_ffn"))
    w_off = 48 + 128
    s_off = w_off + len(weights)
    r_off = s_off + len(scales)
    hdr = np.zeros(12, np.uint32)
    hdr[0], hdr[1] = 0x53564C4D, 1
    hdr[3], hdr[4], hdr[5] = w_off, s_off, r_off
    hdr[7], hdr[8], hdr[9] = len(weights), len(scales), len(norms)
    ci = np.zeros(32, np.int32)
    ci[:8] = [d, h, L, cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["vocab"], cfg["seq_len"]]
    ci[12], ci[14], ci[15] = 3, group_bound, 1 if hadamard else 0
    with open(path, "wb") as f:
        f.write(hdr.tobytes())
        f.write(ci.tobytes())
        f.write(weights)
        f.write(scales)
        f.write(norms)


# ---- Qwen3.5 (QWN5) model files ----
Q35_FP32, Q35_INT4, Q35_TERN2, Q35_TERN3 = 0, 1, 2, 3
Q35_EMBED_INT8, Q35_EMBED_INT4, Q35_EMBED_2BIT, Q35_EMBED_DENSE, Q35_EMBED_FP32 = 0, 1, 2, 3, 4


def qwen35_config(dim, hidden, layer_types, n_heads, n_kv_heads, head_dim, vocab, lin_k_heads, lin_k_dim,
                  lin_v_heads, lin_v_dim, conv_k=4, seq_len=64, quant_lm=Q35_TERN2, quant_embed=Q35_EMBED_INT8,
                  group=0, hadamard=0, plain=0):
    """A Qwen3.5 hybrid configuration (qwen35_config_t, include/eif_qwen35.h:56-110): layer_types is a list of
    0 (DeltaNet) / 1 (full attention)."""
    lt = list(layer_types)
    return dict(dim=dim, hidden=hidden, layer_types=lt, n_heads=n_heads, n_kv_heads=n_kv_heads, head_dim=head_dim,
                vocab=vocab, lin_k_heads=lin_k_heads, lin_k_dim=lin_k_dim, lin_v_heads=lin_v_heads,
                lin_v_dim=lin_v_dim, conv_k=conv_k, seq_len=seq_len, quant_lm=quant_lm, quant_embed=quant_embed,
                group=group, hadamard=hadamard, plain=plain)


def pack_ternary_dense(v):
    """int8 values in {-1,0,1}, shape [..., K] -> uint8 [..., (K+4)//5]: five base-3 digits per byte, the first
    column least significant, digit 1 = +1, 2 = -1 (the reference's dense LUT, src/eif_qwen35.c:78-92)."""
    v = np.asarray(v)
    K = v.shape[-1]
    Kp = (K + 4) // 5 * 5
    d = np.zeros(v.shape[:-1] + (Kp,), np.int32)
    d[..., :K] = np.where(v > 0, 1, np.where(v < 0, 2, 0))
    d = d.reshape(v.shape[:-1] + (Kp // 5, 5))
    return (d[..., 0] + 3 * d[..., 1] + 9 * d[..., 2] + 27 * d[..., 3] + 81 * d[..., 4]).astype(np.uint8)


def _q35_matrix(r, rows, cols, qt):
    """Random rows of one storage type: (bytes, values) with values the ternary / int4 ints or FP32 floats."""
    if qt == Q35_FP32:
        v = r.standard_normal((rows, cols)).astype(np.float32)
        return v.tobytes(), v
    if qt == Q35_INT4:
        v = r.integers(-8, 8, size=(rows, cols), dtype=np.int8)
        return pack_int4(v).tobytes(), v
    if qt == 4:   # int8 embedding
        v = r.integers(-127, 128, size=(rows, cols), dtype=np.int8)
        return v.tobytes(), v
    v = r.integers(-1, 2, size=(rows, cols), dtype=np.int8)
    return (pack_ternary(v) if qt == Q35_TERN2 else pack_ternary_dense(v)).tobytes(), v


def qwen35_image(cfg, key, sub_norms=True, region_pad=0):
    """A QWN5 image in the layout qwen35_load walks (src/eif_qwen35.c:1223-1430), random contents: returns
    (image bytes, arrays) where arrays maps a name to (byte offset, values, scales or None, scales' byte offset or
    0). Names: "embed";
    "L{l}.{kind}" for kinds qkv, z, out, pb, pa (DeltaNet), q, k, v, o (attention), gate, up, down; FP32 vectors
    "L{l}.rms_att", "L{l}.rms_ffn", "rms_final", "L{l}.conv", "L{l}.dt", "L{l}.alog", "L{l}.dnorm", "L{l}.qnorm",
    "L{l}.knorm", "L{l}.sub_att", "L{l}.sub_ffn", "signs_dim", "signs_hid". region_pad bytes go before each region
    (an odd count puts every array off its natural alignment)."""
    r = rng(*key, 40)
    d, h, lt, V = cfg["dim"], cfg["hidden"], cfg["layer_types"], cfg["vocab"]
    L = len(lt)
    nh, nkv, hd = cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    nk, kd, nv, vd, ck = cfg["lin_k_heads"], cfg["lin_k_dim"], cfg["lin_v_heads"], cfg["lin_v_dim"], cfg["conv_k"]
    qlm, qe, g, had = cfg["quant_lm"], cfg["quant_embed"], cfg["group"], cfg["hadamard"]
    key_dim, val_dim = nk * kd, nv * vd
    conv_dim, q_dim, kv_dim = 2 * key_dim + val_dim, nh * hd, nkv * hd
    small = Q35_FP32 if g > 0 else qlm
    dn = [l for l in range(L) if lt[l] == 0]
    fa = [l for l in range(L) if lt[l] == 1]
    arrays = {}
    regions = {"w": bytearray(), "s": bytearray(), "n": bytearray()}
    pending = []   # (region, name, field, position in region)

    def put(region, name, data, field=0):
        pending.append((region, name, field, len(regions[region])))
        regions[region] += data

    def scales_of(rows, cols, grouped):
        n = rows * (cols // g) if grouped else rows
        return (np.abs(r.standard_normal(n)) * 0.02 + 1e-3).astype(np.float32)

    emb_qt = {Q35_EMBED_INT8: 4, Q35_EMBED_INT4: Q35_INT4, Q35_EMBED_2BIT: Q35_TERN2,
              Q35_EMBED_DENSE: Q35_TERN3, Q35_EMBED_FP32: Q35_FP32}[qe]
    b, v = _q35_matrix(r, V, d, emb_qt)
    arrays["embed"] = [0, v, None, 0]
    put("w", "embed", b)
    shapes = {"qkv": (conv_dim, d), "z": (val_dim, d), "out": (d, val_dim), "pb": (nv, d), "pa": (nv, d),
              "q": (2 * q_dim, d), "k": (kv_dim, d), "v": (kv_dim, d), "o": (d, q_dim),
              "gate": (h, d), "up": (h, d), "down": (d, h)}

    def mats(kinds, layers, qt=None, slots=None):
        for kind in kinds:
            rows, cols = shapes[kind]
            for i in range(slots if slots is not None else len(layers)):
                b, v = _q35_matrix(r, rows, cols, qt if qt is not None else qlm)
                if i < len(layers):
                    arrays[f"L{layers[i]}.{kind}"] = [0, v, None, 0]
                    put("w", f"L{layers[i]}.{kind}", b)
                else:
                    regions["w"] += b     # an unused FFN slot
    mats(("qkv", "z", "out"), dn)
    mats(("pb", "pa"), dn, qt=small)
    mats(("q", "k", "v", "o"), fa)
    mats(("gate", "up", "down"), list(range(L)), slots=24)
    for name, n in (("conv", conv_dim * ck), ("dt", nv), ("alog", nv)):
        for l in dn:
            v = r.standard_normal(n).astype(np.float32)
            arrays[f"L{l}.{name}"] = [0, v, None, 0]
            put("w", f"L{l}.{name}", v.tobytes())
    # scales
    ge = qe == Q35_EMBED_2BIT and g > 0
    s = scales_of(V, d, ge)
    arrays["embed"][2] = s
    put("s", "embed", s.tobytes(), 3)
    grouped = g > 0
    for l in dn:
        for kind in ("qkv", "z", "out"):
            s = scales_of(*shapes[kind], grouped)
            arrays[f"L{l}.{kind}"][2] = s
            put("s", f"L{l}.{kind}", s.tobytes(), 3)
        if not grouped:
            for kind in ("pb", "pa"):
                s = scales_of(nv, d, False)
                arrays[f"L{l}.{kind}"][2] = s
                put("s", f"L{l}.{kind}", s.tobytes(), 3)
    for l in fa:
        for kind in ("q", "k", "v", "o"):
            s = scales_of(*shapes[kind], grouped)
            arrays[f"L{l}.{kind}"][2] = s
            put("s", f"L{l}.{kind}", s.tobytes(), 3)
    for slot in range(24):
        for kind in ("gate", "up", "down"):
            s = scales_of(*shapes[kind], grouped)
            if slot < L:
                arrays[f"L{slot}.{kind}"][2] = s
                put("s", f"L{slot}.{kind}", s.tobytes(), 3)
            else:
                regions["s"] += s.tobytes()

    def vec(name, n, signs=False):
        v = (np.where(r.random(n) < 0.5, -1.0, 1.0) if signs else 1.0 + 0.1 * r.standard_normal(n)).astype(np.float32)
        if name is not None:
            arrays[name] = [0, v, None, 0]
            put("n", name, v.tobytes())
        else:
            regions["n"] += v.tobytes()
    for which in ("rms_att", "rms_ffn"):
        for slot in range(24):
            vec(f"L{slot}.{which}" if slot < L else None, d)
    vec("rms_final", d)
    for l in range(L):
        if lt[l] == 0:
            vec(f"L{l}.dnorm", vd)
        else:
            vec(f"L{l}.qnorm", hd)
            vec(f"L{l}.knorm", hd)
    if had:
        vec("signs_dim", d, True)
        vec("signs_hid", h, True)
    if sub_norms:
        for l in range(L):
            if lt[l] == 1:
                vec(f"L{l}.sub_att", q_dim)
            vec(f"L{l}.sub_ffn", h)
    # place: header, config, layer types, then the weights, scales and norms regions
    head = 48 + 128 + L
    offs = {}
    pos = head
    for key_ in ("w", "s", "n"):
        pos += region_pad
        offs[key_] = pos
        pos += len(regions[key_])
    img = bytearray(pos)
    hdr = np.zeros(12, np.uint32)
    hdr[0], hdr[1], hdr[2] = 0x51574E35, 1, 48
    hdr[3], hdr[4], hdr[5] = offs["w"], offs["s"], offs["n"]
    hdr[7], hdr[8], hdr[9] = len(regions["w"]), len(regions["s"]), len(regions["n"])
    ci = np.zeros(32, np.int32)
    ci[:15] = [d, h, L, nh, nkv, hd, V, cfg["seq_len"], len(dn), len(fa), nk, kd, nv, vd, ck]
    ci[22], ci[23], ci[25], ci[26], ci[27], ci[28] = 1, qlm, qe, cfg["plain"], g, had
    img[:48] = hdr.tobytes()
    img[48:176] = ci.tobytes()
    img[176:176 + L] = bytes(lt)
    for key_ in ("w", "s", "n"):
        img[offs[key_]:offs[key_] + len(regions[key_])] = regions[key_]
    for region, name, field, at in pending:
        arrays[name][field] = offs[region] + at
    return bytes(img), {k: tuple(v) for k, v in arrays.items()}


def write_ttml(path, cfg, w, rope_theta=None, magic=0x54544D4C, interleaved=0):
    """Write a BitNet model with one scale per row (bitnet_model's arrays with every group 0) as a TTML / TLLM file:
    the 36-byte header and the tinyllm_config_t that tinyllm_save_quantized_model writes (src/eif_tinyllm.c:2305-2313,
    :2319-2400; read back by src/eif_llm.c:341-351 up to the BitNet group fields), then the weights in SVLM's order
    and the per-row scale layout of tinyllm_setup_quantized_pointers (src/eif_tinyllm.c:2694-2702) as the decode
    indexes it (src/eif_tinyllm.c:383-385, :420-422, :713-787): embedding scales [vocab]; per layer the attention
    scales at q 0, k wk, v wv, o wo within a stride (q_dim + 2 kv_dim + dim when head_dim is set apart from dim /
    n_heads, else 4 dim + 2 kv_dim with k at dim, v at 2 dim, o at 2 dim + kv_dim); per layer w1, w3, w2; head
    scales [vocab]. Norms: attention, FFN, final, then the sub-norms. interleaved: the rope_interleaved word."""
    d, h, L, V = cfg["dim"], cfg["hidden"], cfg["n_layers"], cfg["vocab"]
    nh, nkv, hd = cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    qd, kvd = nh * hd, nkv * hd
    assert all(cfg[k] == 0 for k in ("g_q", "g_o", "g_13", "g_2"))
    weights = b"".join(np.ascontiguousarray(w[k]).tobytes()
                       for k in ("emb", "wq", "wk", "wv", "wo", "w1", "w2", "w3", "wcls"))
    explicit = hd != d // nh
    stride = qd + 2 * kvd + d if explicit else 4 * d + 2 * kvd
    offs = (0, qd, qd + kvd, qd + 2 * kvd) if explicit else (0, d, 2 * d, 2 * d + kvd)
    att = np.zeros((L, stride), np.float32)
    for name, off, rows in (("gq", offs[0], qd), ("gk", offs[1], kvd), ("gv", offs[2], kvd), ("go", offs[3], d)):
        att[:, off:off + rows] = w[name].reshape(L, rows)
    ffn = np.concatenate([w["g1"].reshape(L, h), w["g3"].reshape(L, h), w["g2"].reshape(L, d)], axis=1)
    scales = b"".join(np.ascontiguousarray(a, dtype=np.float32).tobytes()
                      for a in (w["emb_scale"], att, ffn, w["wcls_scale"]))
    norms = b"".join(np.ascontiguousarray(w[k], dtype=np.float32).tobytes()
                     for k in ("rms_att", "rms_ffn", "rms_final", "rms_sub_att", "rms_sub_ffn"))
    theta = cfg["rope_theta"] if rope_theta is None else rope_theta
    config = (np.array([d, h, L, nh, nkv, V, cfg["seq_len"], 3, hd, interleaved], np.int32).tobytes() +
              np.array([theta], np.float32).tobytes() + np.array([0, 0, 0], np.int32).tobytes())
    hdr = np.array([magic, 2, len(config), len(weights), len(scales), len(norms), 0, 0, 0], np.uint32)
    with open(path, "wb") as f:
        f.write(hdr.tobytes())
        f.write(config)
        f.write(weights)
        f.write(scales)
        f.write(norms)


# ---- GGUF containers (the reference's GGUF causal-model reader, src/eif_tinyllm.c:2843-3009, :3529-3838) ----
GGUF_F32, GGUF_F16, GGUF_Q4_0, GGUF_Q4_1, GGUF_Q8_0, GGUF_Q4_K, GGUF_Q5_K, GGUF_Q6_K, GGUF_BF16, GGUF_TL1, \
    GGUF_TL2 = 0, 1, 2, 3, 8, 12, 13, 14, 30, 34, 35
# bytes per block and values per block of the block types (ggml's published layouts)
GGUF_BLOCK = {GGUF_Q4_0: (18, 32), GGUF_Q4_1: (20, 32), GGUF_Q8_0: (34, 32), GGUF_Q4_K: (144, 256),
              GGUF_Q5_K: (176, 256), GGUF_Q6_K: (210, 256)}
GGUF_U8, GGUF_I8, GGUF_U16, GGUF_I16, GGUF_U32, GGUF_I32, GGUF_F32V, GGUF_BOOL, GGUF_STR, GGUF_ARR, GGUF_U64, \
    GGUF_I64, GGUF_F64 = range(13)
_GGUF_FMT = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


def gguf_image(kv, tensors, alignment=32, version=3):
    """A GGUF container: 'GGUF', version, tensor count, metadata count; the metadata [(key, value type, value)]
    (an array's value: (element type, [elements])); the tensor table [(name, ggml type, dims with the row length
    first, raw bytes)] with offsets from the data start, each tensor at a multiple of alignment; the data start
    at the header's end rounded up to alignment."""
    import struct

    def string(x):
        b = x.encode()
        return struct.pack("<Q", len(b)) + b

    def value(t, v):
        if t in _GGUF_FMT:
            return struct.pack(_GGUF_FMT[t], v)
        if t == GGUF_STR:
            return string(v)
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(value(et, x) for x in items)

    head = [b"GGUF", struct.pack("<IQQ", version, len(tensors), len(kv))]
    for k, t, v in kv:
        head += [string(k), struct.pack("<I", t), value(t, v)]
    data, off = [], 0
    for name, ty, dims, raw in tensors:
        pad = -off % alignment
        data.append(b"\0" * pad)
        off += pad
        head += [string(name), struct.pack("<I", len(dims)), struct.pack(f"<{len(dims)}Q", *dims),
                 struct.pack("<IQ", ty, off)]
        data.append(bytes(raw))
        off += len(raw)
    h = b"".join(head)
    return h + b"\0" * (-len(h) % alignment) + b"".join(data)


def _fp16_scales(r, n):
    return (np.abs(r.standard_normal(n)) * 0.02 + 0.004).astype(np.float16)


def gguf_ternary_tensor(r, rows, cols, ty):
    """A BitNet projection as a GGUF tensor: (raw bytes, ternary values [rows, cols], fp16 block scales [rows,
    cols / 32]). TL1 / TL2: per 32-column
    block an fp16 scale then the block's 8 bytes of 2-bit codes (the reference's packing, copied by its loader,
    src/eif_tinyllm.c:3366-3379); Q8_0: an fp16 scale then 32 int8 values, taken by sign (:3380-3402)."""
    assert cols % 32 == 0
    nb = cols // 32
    sc = _fp16_scales(r, rows * nb).reshape(rows, nb)
    if ty in (GGUF_TL1, GGUF_TL2):
        v = r.integers(-1, 2, size=(rows, cols), dtype=np.int8)
        codes = pack_ternary(v).reshape(rows, nb, 8)
        blk = np.concatenate([sc.view(np.uint8).reshape(rows, nb, 2), codes], axis=2)
        return blk.tobytes(), v, sc
    q = r.integers(-127, 128, size=(rows, cols), dtype=np.int8)
    q[r.uniform(size=q.shape) < 0.2] = 0
    blk = np.concatenate([sc.view(np.uint8).reshape(rows, nb, 2), q.view(np.uint8).reshape(rows, nb, 32)], axis=2)
    return blk.tobytes(), np.sign(q).astype(np.int8), sc


def gguf_dense_tensor(r, rows, cols, ty):
    """An embedding / output matrix as a GGUF tensor (raw bytes): F32, F16, or blocks of Q4_0 (fp16 d, 16 bytes of
    nibbles: the block's first 16 values low, last 16 high), Q4_1 (fp16 d, fp16 m, 16 bytes), Q8_0 (fp16 d, 32
    int8), Q4_K (fp16 d, fp16 dmin, 12 bytes of 6-bit scales and mins, 128 bytes of nibbles), Q6_K (128 bytes of
    low nibbles, 64 of high 2-bit pairs, 16 int8 scales, fp16 d), Q5_K (fp16 d, fp16 dmin, 12 bytes of scales and
    mins, 32 bytes of fifth bits, 128 bytes of nibbles), BF16; the codes uniform, the fp16 fields drawn in a range
    that keeps every value finite."""
    if ty == GGUF_BF16:
        x = (r.standard_normal((rows, cols)) * 0.05).astype(np.float32)
        return (x.view(np.uint32) >> 16).astype(np.uint16).tobytes()
    if ty in (GGUF_Q4_0, GGUF_Q4_1, GGUF_Q4_K, GGUF_Q5_K, GGUF_Q6_K):
        bb, bv = GGUF_BLOCK[ty]
        assert cols % bv == 0
        nb = rows * (cols // bv)
        blk = r.integers(0, 256, size=(nb, bb), dtype=np.uint16).astype(np.uint8)

        def f16(lo, hi):
            return (r.uniform(lo, hi, size=nb) * np.where(r.uniform(size=nb) < 0.5, -1, 1)).astype(
                np.float16).view(np.uint8).reshape(nb, 2)
        if ty == GGUF_Q4_0:
            blk[:, 0:2] = f16(0.001, 0.02)
        elif ty == GGUF_Q4_1:
            blk[:, 0:2], blk[:, 2:4] = f16(0.001, 0.02), f16(0.0, 0.1)
        elif ty in (GGUF_Q4_K, GGUF_Q5_K):
            blk[:, 0:2], blk[:, 2:4] = f16(0.0001, 0.002), f16(0.0001, 0.002)
        else:
            blk[:, 208:210] = f16(0.0001, 0.002)
        return blk.tobytes()
    x = (r.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    x[r.uniform(size=rows) < 0.05] *= 0.0          # some all-zero rows (scale 1)
    if ty == GGUF_F32:
        return x.tobytes()
    if ty == GGUF_F16:
        return x.astype(np.float16).tobytes()
    assert cols % 32 == 0
    nb = cols // 32
    sc = _fp16_scales(r, rows * nb).reshape(rows, nb)
    q = r.integers(-127, 128, size=(rows, cols), dtype=np.int8)
    return np.concatenate([sc.view(np.uint8).reshape(rows, nb, 2), q.view(np.uint8).reshape(rows, nb, 32)],
                          axis=2).tobytes()


def bitnet_gguf(cfg, key, arch="bitnet", proj_types=(GGUF_TL1,), emb_type=GGUF_F16, head_type=None,
                norm_type=GGUF_F32, alignment=32, rope_theta=None, key_length=False, int_type=GGUF_U32,
                permute=None, nested=False, kv_edit=None, drop=(), extra_tensors=()):
    """A BitNet model as a GGUF file image: the metadata the reference reads (<arch>.embedding_length, ...,
    tokenizer.ggml.tokens) among keys of every value type that it skips, then per layer attn_norm, attn_q/k/v,
    attn_output, ffn_norm, ffn_gate/up/down, then token_embd, output_norm and, unless head_type is None (tied),
    output. Projection types cycle through proj_types (the first, blk.0.attn_q, decides BitNet). permute(kind, rows)
    -> a row order, applied to the q / k tensors (block scales move with their rows): the same draws as another
    file with its rows reordered. kv_edit(metadata list) -> metadata list; drop: tensor names left out; extra_tensors:
    more (name, type, dims, raw) at the end. Returns
    (image, {'L<l>.<kind>': ternary values as written, 'L<l>.<kind>.scales': their fp16 block scales})."""
    d, h, L, V = cfg["dim"], cfg["hidden"], cfg["n_layers"], cfg["vocab"]
    nh, nkv, hd = cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    qd, kvd = nh * hd, nkv * hd
    a = arch + "."
    kv = [("general.name", GGUF_STR, "synthetic"), ("general.architecture", GGUF_STR, arch),
          ("general.alignment", GGUF_U32, alignment), ("general.file_type", GGUF_U32, 1),
          (a + "embedding_length", int_type, d), ("misc.u8", GGUF_U8, 7), ("misc.i16", GGUF_I16, -3),
          (a + "feed_forward_length", int_type, h), (a + "block_count", int_type, L),
          ("misc.bool", GGUF_BOOL, True), ("misc.f64", GGUF_F64, 2.5), ("misc.i64", GGUF_I64, -9),
          (a + "attention.head_count", int_type, nh), (a + "attention.head_count_kv", int_type, nkv),
          (a + "context_length", int_type, cfg["seq_len"]),
          (a + "rope.freq_base", GGUF_F32V, cfg["rope_theta"] if rope_theta is None else rope_theta),
          ("misc.arr_i32", GGUF_ARR, (GGUF_I32, [1, -2, 3])),
          ("tokenizer.ggml.model", GGUF_STR, "gpt2"),
          ("tokenizer.ggml.tokens", GGUF_ARR, (GGUF_STR, [f"t{i}" for i in range(V)])),
          ("tokenizer.ggml.scores", GGUF_ARR, (GGUF_F32V, [0.0] * 4))]
    if key_length:
        kv.append((a + "attention.key_length", int_type, hd))
    if nested:      # an array of arrays (the reference's metadata walk cannot skip one, src/eif_tinyllm.c:3595-3606)
        kv.insert(3, ("misc.arr_arr", GGUF_ARR, (GGUF_ARR, [(GGUF_U16, [1, 2]), (GGUF_STR, ["x", "yz"])])))
    if kv_edit is not None:
        kv = kv_edit(kv)
    r = rng(*key, 70)
    tensors, vals = [], {}
    shapes = (("attn_q", qd, d), ("attn_k", kvd, d), ("attn_v", kvd, d), ("attn_output", d, qd),
              ("ffn_gate", h, d), ("ffn_up", h, d), ("ffn_down", d, h))
    i = 0
    for l in range(L):
        tensors.append((f"blk.{l}.attn_norm.weight", GGUF_F32, (d,), _norm_bytes(r, d, norm_type)))
        for kind, rows, cols in shapes:
            ty = proj_types[i % len(proj_types)]
            i += 1
            if ty in (GGUF_TL1, GGUF_TL2, GGUF_Q8_0):
                raw, v, sc = gguf_ternary_tensor(r, rows, cols, ty)
            else:               # a dense tensor the reference ternarizes by its absolute mean
                raw, v, sc = gguf_dense_tensor(r, rows, cols, ty), None, None
            if permute is not None and kind in ("attn_q", "attn_k"):
                assert v is not None
                order = permute(kind, rows)            # new row i = written row order[i]
                raw = np.frombuffer(raw, np.uint8).reshape(rows, -1)[order].tobytes()
                v, sc = v[order], sc[order]
            vals[f"L{l}.{kind}"] = v
            vals[f"L{l}.{kind}.scales"] = sc
            tensors.append((f"blk.{l}.{kind}.weight", ty, (cols, rows), raw))
            if kind == "attn_v":
                tensors.append((f"blk.{l}.ffn_norm.weight", GGUF_F32, (d,), _norm_bytes(r, d, norm_type)))
    for nm, ty in (("token_embd.weight", emb_type), ("output.weight", head_type)):
        if ty is not None:
            tensors.append((nm, ty, (d, V), gguf_dense_tensor(r, V, d, ty)))
    tensors.append(("output_norm.weight", GGUF_F32, (d,), _norm_bytes(r, d, norm_type)))
    tensors = [(n, (norm_type if n.endswith("norm.weight") else t), dims, raw) for n, t, dims, raw in tensors
               if n not in drop] + list(extra_tensors)
    return gguf_image(kv, tensors, alignment=alignment), vals


def _norm_bytes(r, n, ty):
    x = (1.0 + 0.1 * r.standard_normal(n)).astype(np.float32)
    return x.astype(np.float16).tobytes() if ty == GGUF_F16 else x.tobytes()


def qwen35_gguf(key, dim=256, hidden=512, n_heads=4, n_kv_heads=2, head_dim=64, vocab=300, heads_k=4, k_dim=32,
                v_dim=64, conv_k=4, interval=4, ctx=2048, lin_types=(GGUF_Q4_K, GGUF_Q6_K, GGUF_Q8_0, GGUF_Q5_K,
                                                                        GGUF_Q4_0, GGUF_F16, GGUF_BF16, GGUF_F32),
                emb_type=GGUF_Q6_K, kv_edit=None, drop=(), extra_tensors=()):
    """A Qwen3.5 text model as a llama.cpp-style GGUF image (what qwen35_gguf_build_image reads,
    src/eif_qwen35_gguf.c:262-454): qwen35.* metadata (24 blocks, a full-attention layer every `interval`), the
    tied token_embd, per DeltaNet layer attn_qkv / attn_gate / ssm_out / ssm_beta / ssm_alpha, ssm_conv1d, ssm_dt.bias,
    ssm_a (negative), ssm_norm; per attention layer attn_q (with its gate rows) / attn_k / attn_v / attn_output,
    attn_q_norm / attn_k_norm; per layer ffn_gate / ffn_up / ffn_down, attn_norm, post_attention_norm; output_norm.
    Linear types cycle through lin_types."""
    L = 24
    nv = heads_k
    key_dim, val_dim = heads_k * k_dim, nv * v_dim
    conv_dim, q_dim, kv_dim = 2 * key_dim + val_dim, n_heads * head_dim, n_kv_heads * head_dim
    a = "qwen35."
    kv = [("general.architecture", GGUF_STR, "qwen35"), ("general.alignment", GGUF_U32, 32),
          (a + "block_count", GGUF_U32, L), (a + "embedding_length", GGUF_U32, dim),
          (a + "feed_forward_length", GGUF_U32, hidden), (a + "attention.head_count", GGUF_U32, n_heads),
          (a + "attention.head_count_kv", GGUF_U32, n_kv_heads), (a + "attention.key_length", GGUF_U32, head_dim),
          (a + "context_length", GGUF_U64, ctx), (a + "full_attention_interval", GGUF_U32, interval),
          (a + "attention.layer_norm_rms_epsilon", GGUF_F32V, 1e-6), (a + "ssm.conv_kernel", GGUF_U32, conv_k),
          (a + "ssm.state_size", GGUF_U32, k_dim), (a + "ssm.group_count", GGUF_U32, heads_k),
          (a + "ssm.time_step_rank", GGUF_U32, nv), (a + "ssm.inner_size", GGUF_U32, val_dim),
          ("misc.note", GGUF_STR, "synthetic"), ("tokenizer.ggml.tokens", GGUF_ARR, (GGUF_STR, ["a"] * 4))]
    if kv_edit is not None:
        kv = kv_edit(kv)
    r = rng(*key, 80)
    tensors = [("token_embd.weight", emb_type, (dim, vocab), gguf_dense_tensor(r, vocab, dim, emb_type))]
    it = [0]

    def lin(name, rows, cols):
        ty = lin_types[it[0] % len(lin_types)]
        it[0] += 1
        blk = GGUF_BLOCK.get(ty, (0, 1))[1]
        if cols % blk:
            ty = GGUF_F16
        tensors.append((name, ty, (cols, rows), gguf_dense_tensor(r, rows, cols, ty)))

    def vec(name, n, lo=0.5, hi=1.5, dims=None):
        x = r.uniform(lo, hi, size=n).astype(np.float32)
        tensors.append((name, GGUF_F32, dims or (n,), x.tobytes()))
    for l in range(L):
        b = f"blk.{l}."
        vec(b + "attn_norm.weight", dim)
        if (l + 1) % interval:
            lin(b + "attn_qkv.weight", conv_dim, dim)
            lin(b + "attn_gate.weight", val_dim, dim)
            lin(b + "ssm_out.weight", dim, val_dim)
            lin(b + "ssm_beta.weight", nv, dim)
            lin(b + "ssm_alpha.weight", nv, dim)
            vec(b + "ssm_conv1d.weight", conv_dim * conv_k, -0.5, 0.5, dims=(conv_k, conv_dim))
            vec(b + "ssm_dt.bias", nv, -1.0, 1.0)
            vec(b + "ssm_a", nv, -8.0, -0.01)
            vec(b + "ssm_norm.weight", v_dim)
        else:
            lin(b + "attn_q.weight", 2 * q_dim, dim)
            lin(b + "attn_k.weight", kv_dim, dim)
            lin(b + "attn_v.weight", kv_dim, dim)
            lin(b + "attn_output.weight", dim, q_dim)
            vec(b + "attn_q_norm.weight", head_dim)
            vec(b + "attn_k_norm.weight", head_dim)
        lin(b + "ffn_gate.weight", hidden, dim)
        lin(b + "ffn_up.weight", hidden, dim)
        lin(b + "ffn_down.weight", dim, hidden)
        vec(b + "post_attention_norm.weight", dim)
    vec("output_norm.weight", dim)
    tensors = [t for t in tensors if t[0] not in drop] + list(extra_tensors)
    return gguf_image(kv, tensors)
