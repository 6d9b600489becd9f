"""BitNet models in GGUF files (include/eif_hip_gguf.h), on the CPU.

A GGUF file of the test writer (model_files.bitnet_gguf) is read both by the reference itself, as its engine reads one
(tinyllm_read_gguf_config, tinyllm_init, tinyllm_load_gguf: src/eif_tinyllm.c:2843-3838, compiled with the
reference's own flags into oracle/_ref/libref.so), and by eif_gguf_bitnet_open. The configuration and every
converted array agree bit for bit: 2-bit rows and row scales of TL1 / TL2 / Q8_0 projections and of F32 / F16 / Q4_0
/ Q4_1 / Q4_K / Q6_K projections ternarized by their absolute mean (odd column counts make the mean's 1 / cols
inexact; the block types' sum runs over eight lanes as the reference's build forms it), the INT8 embedding
and head with their row scales from F32, F16, Q8_0, Q4_0, Q4_1, Q4_K and Q6_K tensors (a vocabulary of 1200 rows
for the block types, whose fp16 block fields leave each dequantised value one rounding), the norm weights; over
odd block counts, data
alignments, integer value types of the metadata and a head_dim set apart from dim / heads. The codes the reference
decodes are the writer's ternary values, so the writer lays out what the reference reads. The configuration rules
(context length default and clamp, RoPE theta defaults, interleaved architectures, the key prefix before
general.architecture) agree with the reference's. Files the reference cannot read safely are refused here. A
model whose RoPE pairs are interleaved decodes in the reference as the same model with its q / k rows reordered for
half-split pairs, the reordering eif_hip_bitnet_load_gguf applies, to 1e-5 of the logits.
"""
import ctypes as C
import os

import numpy as np
import pytest

from conftest import ROOT, P
import bitllm_hip as bh
import oracle_api
import synth
import model_files

REF = os.path.join(ROOT, "oracle", "_ref", "libref.so")
TL1, TL2, Q8, F16, F32 = model_files.GGUF_TL1, model_files.GGUF_TL2, model_files.GGUF_Q8_0, model_files.GGUF_F16, model_files.GGUF_F32


@pytest.fixture(scope="module")
def reft():
    if not os.path.exists(REF):
        pytest.skip("oracle/_ref/libref.so not built (reference tree absent)")
    return oracle_api.load_ref_tinyllm(REF)


SHAPES = {   # dim, hidden, layers, heads, kv heads, head_dim (key_length written when set apart from dim / heads)
    "d128": (128, 256, 2, 4, 2, 32),
    "odd_blocks": (96, 224, 2, 3, 1, 32),        # 3 and 7 blocks of 32 per row: the mean's 1 / blocks is inexact
    "hd_apart": (128, 256, 2, 4, 2, 64),
    "d256": (256, 256, 1, 4, 2, 64),            # rows of whole 256-value K-quant blocks
}
CASES = {
    "tl1_f16emb": dict(proj_types=(TL1,), emb_type=F16),
    "mixed_f32emb_q8head": dict(proj_types=(TL1, Q8, TL2), emb_type=F32, head_type=Q8, alignment=64,
                                int_type=model_files.GGUF_U64),
    "tl2_q8emb_f16head_f16norms": dict(proj_types=(TL2, TL1), emb_type=Q8, head_type=F16, norm_type=F16,
                                       int_type=model_files.GGUF_I32),
    "q4k_emb_q6k_head": dict(proj_types=(TL1,), emb_type=model_files.GGUF_Q4_K, head_type=model_files.GGUF_Q6_K),
    "q4_0_emb_q4_1_head": dict(proj_types=(TL2,), emb_type=model_files.GGUF_Q4_0, head_type=model_files.GGUF_Q4_1),
    # projections the reference ternarizes by their absolute mean (the probe stays TL1 / TL2)
    "absmean_block32": dict(proj_types=(TL1, F32, F16, model_files.GGUF_Q4_0, model_files.GGUF_Q4_1, Q8, TL2)),
    "absmean_kquants": dict(proj_types=(TL2, model_files.GGUF_Q4_K, model_files.GGUF_Q6_K, TL1)),
}


def config(shape, vocab=300, seq_len=64):
    vocab = 1200 if shape == "d256" else vocab
    d, h, L, nh, nkv, hd = SHAPES[shape]
    return synth.bitnet_config(d, h, L, nh, nkv, hd, vocab, seq_len, 0, 0, 0, 0, 0, rope_theta=10000.0)


def write(tmp_path, cfg, name="m.gguf", key=(3,), **kw):
    kw.setdefault("key_length", cfg["head_dim"] != cfg["dim"] // cfg["n_heads"])
    img, vals = model_files.bitnet_gguf(cfg, key, **kw)
    path = tmp_path / name
    path.write_bytes(img)
    return str(path), vals


def ref_model(reft, path):
    """The reference's configuration and converted arrays, indexed as its decode indexes them."""
    h = reft.ref_gguf_create(os.fsencode(path))
    assert h
    cfg = np.zeros(10, np.int32)
    th = C.c_float()
    p = (C.c_void_p * 19)()
    reft.ref_tinyllm_view(h, P(cfg), C.byref(th), p)
    d, hid, L, nh, nkv, hd, V = (int(v) for v in cfg[:7])
    qd, kvd = nh * hd, nkv * hd
    explicit = hd != d // nh
    stride = qd + 2 * kvd + d if explicit else 4 * d + 2 * kvd
    offs = (0, qd, qd + kvd, qd + 2 * kvd) if explicit else (0, d, 2 * d, 2 * d + kvd)

    def get(ptr, dt, n, off=0):
        sz = np.dtype(dt).itemsize
        return np.frombuffer(C.string_at(ptr + off * sz, n * sz), dt).copy()

    shapes = {"q": (qd, d, p[2]), "k": (kvd, d, p[3]), "v": (kvd, d, p[4]), "o": (d, qd, p[5]), "1": (hid, d, p[6]),
              "3": (hid, d, p[8]), "2": (d, hid, p[7])}
    layers = []
    for l in range(L):
        lay = {}
        for k, (rows, cols, ptr) in shapes.items():
            rb = (cols + 3) // 4
            lay["w" + k] = get(ptr, np.uint8, rows * rb, l * rows * rb).reshape(rows, rb)
        for k, off, rows in zip("qkvo", offs, (qd, kvd, kvd, d)):
            lay["g" + k] = get(p[9], np.float32, rows, l * stride + off)
        for k, off, rows in (("1", 0, hid), ("3", hid, hid), ("2", 2 * hid, d)):
            lay["g" + k] = get(p[10], np.float32, rows, l * (2 * hid + d) + off)
        lay["rms_att"] = get(p[11], np.float32, d, l * d)
        lay["rms_ffn"] = get(p[12], np.float32, d, l * d)
        layers.append(lay)
    glob = {"emb": get(p[0], np.int8, V * d).reshape(V, d), "emb_scale": get(p[1], np.float32, V),
            "rms_final": get(p[13], np.float32, d), "wcls": get(p[14], np.int8, V * d).reshape(V, d),
            "wcls_scale": get(p[15], np.float32, V)}
    return h, cfg, th.value, layers, glob, (p[16], p[17], p[18])


def same_bits(a, b):
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


@pytest.mark.parametrize("shape,case", [("d128", "tl1_f16emb"), ("odd_blocks", "mixed_f32emb_q8head"),
                                        ("hd_apart", "tl2_q8emb_f16head_f16norms"), ("odd_blocks", "tl1_f16emb"),
                                        ("d256", "q4k_emb_q6k_head"), ("d256", "q4_0_emb_q4_1_head"),
                                        ("odd_blocks", "absmean_block32"), ("d256", "absmean_kquants")])
def test_gguf_matches_reference_loader(reft, tmp_path, shape, case):
    cfg = config(shape)
    path, vals = write(tmp_path, cfg, **CASES[case])
    h, rc, theta, rlayers, rglob, nulls = ref_model(reft, path)
    g = bh.GgufBitnet(path)
    try:
        i = g.info
        assert [i.dim, i.hidden, i.n_layers, i.n_heads, i.n_kv_heads, i.head_dim, i.vocab, i.seq_len] == list(rc[:8])
        assert rc[8] == 3 and i.rope_interleaved == rc[9] == 0      # BitNet, half-split
        assert np.float32(i.rope_theta) == np.float32(theta) == np.float32(10000.0)
        assert i.arch == b"bitnet" and i.proj_type == CASES[case]["proj_types"][0]
        assert nulls == (None, None, None)                          # no sub-norms, no biases in the reference either
        kinds = {"q": "attn_q", "k": "attn_k", "v": "attn_v", "o": "attn_output", "1": "ffn_gate", "3": "ffn_up",
                 "2": "ffn_down"}
        for l in range(cfg["n_layers"]):
            ours = g.layer(l)
            for k, a in rlayers[l].items():
                assert same_bits(ours[k], a), (l, k)
            for k, kind in kinds.items():    # the reference decodes the writer's values
                cols = ours["w" + k].shape[1] * 4
                if vals[f"L{l}.{kind}"] is not None:
                    assert np.array_equal(synth.unpack_ternary(rlayers[l]["w" + k], cols), vals[f"L{l}.{kind}"]), (l, k)
        ours = g.globals()
        for k, a in rglob.items():
            assert same_bits(ours[k], a), k
        if CASES[case].get("head_type") is None:
            assert same_bits(ours["wcls"], ours["emb"])
    finally:
        g.close()
        reft.ref_bitnet_destroy(h)


def _set(kv, key, t, v):
    return [(k, t, v) if k == key else (k, tt, vv) for k, tt, vv in kv]


def _drop(kv, *keys):
    return [e for e in kv if e[0] not in keys]


RULES = {   # name: (arch, kv_edit, file name, n_kv_heads): the reference's defaults and clamps
    "no_context": ("bitnet", lambda kv: _drop(kv, "bitnet.context_length"), "m.gguf", 2),
    "long_context": ("bitnet", lambda kv: _set(kv, "bitnet.context_length", model_files.GGUF_U32, 10000), "m.gguf", 2),
    "qwen_theta": ("qwen2", lambda kv: _drop(kv, "qwen2.rope.freq_base"), "m.gguf", 2),
    "qwen_in_path": ("bitnet", lambda kv: _drop(kv, "bitnet.rope.freq_base"), "my_qwen_model.gguf", 2),
    "plain_theta": ("bitnet", lambda kv: _drop(kv, "bitnet.rope.freq_base"), "m.gguf", 2),
    "theta_f64_alt_key": ("bitnet", lambda kv: _drop(kv, "bitnet.rope.freq_base") +
                          [("foo.rope_freq_base", model_files.GGUF_F64, 250000.0)], "m.gguf", 2),
    "llama_interleaved": ("llama", None, "m.gguf", 2),
    "no_arch_llama_keys": ("llama", lambda kv: _drop(kv, "general.architecture"), "m.gguf", 2),
    "kv_heads_default": ("bitnet", lambda kv: _drop(kv, "bitnet.attention.head_count_kv"), "m.gguf", 4),
}


@pytest.mark.parametrize("rule", sorted(RULES))
def test_gguf_config_rules(reft, tmp_path, rule):
    arch, edit, name, nkv = RULES[rule]
    cfg = synth.bitnet_config(128, 256, 1, 4, nkv, 32, 300, 64, 0, 0, 0, 0, 0, rope_theta=10000.0)
    path, _ = write(tmp_path, cfg, name=name, arch=arch, kv_edit=edit)
    h, rc, theta, _, _, _ = ref_model(reft, path)
    g = bh.GgufBitnet(path)
    try:
        i = g.info
        assert [i.dim, i.hidden, i.n_layers, i.n_heads, i.n_kv_heads, i.head_dim, i.vocab, i.seq_len] == list(rc[:8])
        assert i.rope_interleaved == rc[9]
        assert np.float32(i.rope_theta) == np.float32(theta)
        want = {"no_context": ("seq_len", 2048), "long_context": ("seq_len", 4096), "qwen_theta": ("theta", 1e6),
                "qwen_in_path": ("theta", 1e6), "plain_theta": ("theta", 1e4), "theta_f64_alt_key": ("theta", 2.5e5),
                "llama_interleaved": ("interleaved", 1), "no_arch_llama_keys": ("interleaved", 0),
                "kv_heads_default": ("n_kv_heads", 4)}[rule]
        got = {"seq_len": i.seq_len, "theta": i.rope_theta, "interleaved": i.rope_interleaved,
               "n_kv_heads": i.n_kv_heads}[want[0]]
        assert got == want[1]
        assert i.arch == (b"" if rule == "no_arch_llama_keys" else arch.encode())
    finally:
        g.close()
        reft.ref_bitnet_destroy(h)


def test_gguf_nested_metadata(tmp_path):
    """An array of arrays among the skipped metadata (valid GGUF, which the reference's walk cannot skip) reads as
    the same model."""
    cfg = config("d128")
    a, _ = write(tmp_path, cfg, name="a.gguf")
    b, _ = write(tmp_path, cfg, name="b.gguf", nested=True)
    ga, gb = bh.GgufBitnet(a), bh.GgufBitnet(b)
    try:
        for l in range(cfg["n_layers"]):
            la, lb = ga.layer(l), gb.layer(l)
            assert all(same_bits(la[k], lb[k]) for k in la)
        assert all(same_bits(v, gb.globals()[k]) for k, v in ga.globals().items())
    finally:
        ga.close()
        gb.close()


def corrupt(img, at, value, fmt="<I"):
    import struct
    b = bytearray(img)
    struct.pack_into(fmt, b, at, value)
    return bytes(b)


def test_gguf_rejects(reft, tmp_path):
    cfg = config("d128")
    good, _ = write(tmp_path, cfg)
    img = open(good, "rb").read()
    bad = {
        "magic": corrupt(img, 0, 0x12345678),
        "truncated data": img[:len(img) // 2],
        "truncated metadata": img[:200],
    }

    def variant(**kw):
        return model_files.bitnet_gguf(cfg, (3,), **kw)[0]
    bad["probe Q8_0 (an INT8 model for the reference)"] = variant(proj_types=(Q8, TL1))
    bad["missing projection"] = variant(drop=("blk.1.ffn_up.weight",))
    bad["missing embedding"] = variant(drop=("token_embd.weight",))
    bad["q bias"] = variant(extra_tensors=[("blk.0.attn_q.bias", F32, (128,), np.zeros(128, np.float32).tobytes())])
    bad["no token list"] = variant(kv_edit=lambda kv: _drop(kv, "tokenizer.ggml.tokens"))
    bad["vocabulary != embedding rows"] = variant(
        kv_edit=lambda kv: _set(kv, "tokenizer.ggml.tokens", model_files.GGUF_ARR, (model_files.GGUF_STR, ["t"] * 301)))
    bad["alignment 24"] = variant(kv_edit=lambda kv: _set(kv, "general.alignment", model_files.GGUF_U32, 24))
    bad["block_count as f32"] = variant(kv_edit=lambda kv: _set(kv, "bitnet.block_count", model_files.GGUF_F32V, 2.0))
    bad["BF16 projection (a type tinyllm's loader does not read)"] = variant(drop=("blk.0.attn_v.weight",), extra_tensors=[
        ("blk.0.attn_v.weight", model_files.GGUF_BF16, (128, 64), np.zeros(64 * 128, np.uint16).tobytes())])
    bad["Q4_K embedding of part blocks"] = model_files.bitnet_gguf(config("odd_blocks"), (3,), drop=("token_embd.weight",),
                                                           extra_tensors=[("token_embd.weight", model_files.GGUF_Q4_K,
                                                                           (96, 300), bytes(300 * 144))])[0]
    bad["misshapen projection"] = variant(drop=("blk.0.attn_v.weight",), extra_tensors=[
        ("blk.0.attn_v.weight", TL1, (128, 32), bytes(32 * 4 * 10))])
    for name, b in bad.items():
        path = tmp_path / "bad.gguf"
        path.write_bytes(b)
        with pytest.raises(bh.HipError):
            bh.GgufBitnet(str(path))
        if name == "magic":
            assert not reft.ref_gguf_create(os.fsencode(str(path)))   # the reference refuses it too
    with pytest.raises(bh.HipError):
        bh.GgufBitnet(str(tmp_path / "missing.gguf"))


def half_split_order(n_heads, head_dim):
    """Rows of an interleaved-RoPE projection in half-split order: per head 0, 2, 4, ..., then 1, 3, 5, ..."""
    h = np.arange(n_heads)[:, None] * head_dim
    return np.concatenate([h + np.arange(0, head_dim, 2), h + np.arange(1, head_dim, 2)], axis=1).ravel()


def interleaved_files(tmp_path, cfg, key=(5,)):
    """The same draws as a llama file (interleaved RoPE), a bitnet file with q / k rows reordered for half-split
    pairs, and a bitnet file with the rows as drawn."""
    nh, nkv, hd = cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]

    def order(kind, rows):
        return half_split_order(nh if kind == "attn_q" else nkv, hd)
    a, _ = write(tmp_path, cfg, name="inter.gguf", key=key, arch="llama")
    b, _ = write(tmp_path, cfg, name="split.gguf", key=key, arch="bitnet", permute=order)
    c, _ = write(tmp_path, cfg, name="plain.gguf", key=key, arch="bitnet")
    return a, b, c


def test_gguf_interleaved_rope_is_reordered_rows(reft, tmp_path):
    cfg = config("d128")
    a, b, c = interleaved_files(tmp_path, cfg)
    hs = [ref_model(reft, p)[0] for p in (a, b, c)]
    V = cfg["vocab"]
    try:
        tok, worst, apart = 17, 0.0, 0.0
        for pos in range(10):
            la, lb, lc = (np.ctypeslib.as_array(reft.ref_bitnet_forward(h, tok, pos), shape=(V,)).copy() for h in hs)
            worst = max(worst, np.abs(la - lb).max() / np.abs(la).max())
            apart = max(apart, np.abs(la - lc).max() / np.abs(la).max())
            assert int(np.argmax(la)) == int(np.argmax(lb)), pos
            tok = int(np.argmax(la))
        assert worst <= 1e-5
        assert apart > 1e-3      # the pairing matters: the rows as drawn, rotated half-split, are another model
    finally:
        for h in hs:
            reft.ref_bitnet_destroy(h)
