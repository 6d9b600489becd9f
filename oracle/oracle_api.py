"""ctypes declarations for the CPU oracle (liboracle.so / liboracle_port.so) and the compiled reference subset
(_ref/libref.so). TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg."""
import ctypes as C

_vp, _i, _f, _sz = C.c_void_p, C.c_int, C.c_float, C.c_size_t

ORACLE_SIGS = {
    "orc_unpack_ternary": (C.c_int8, [C.c_uint8, _i]),
    "orc_pack_ternary": (_sz, [_vp, _vp, _sz]),
    "orc_pack_ternary_dense": (_sz, [_vp, _vp, _sz]),
    "orc_hadamard_block_size": (_i, [_i]),
    "orc_bitnet_group_size": (_i, [_i, _i]),
    "orc_wht_norm_exact": (_f, [_i]),
    "orc_wht_norm_fastmath": (_f, [_i]),
    "orc_hadamard_rotate": (_i, [_vp, _vp, _i, _i, _f]),
    "orc_quantize_activation_i8": (None, [_vp, _vp, _vp, _i]),
    "orc_prep_rows": (_i, [_vp, _i, _vp, _i, _i, _i, _f, _vp, _i, _vp, _vp, _i]),
    "orc_ternary_acc_i32": (None, [_vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "orc_ternary_gemv_grouped": (None, [_vp, _vp, _i, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _i]),
    "orc_matmul_bitnet_i8xternary_f32": (None, [_vp, _vp, _vp, _f, _vp, _vp, _i, _i]),
    "orc_ternary_gemv_rowscale": (None, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _i]),
    "orc_matmul_bitnet_act_quant_f32": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "orc_matmul_bitnet_int8": (None, [_vp, _f, _vp, _f, _vp, _vp, _f, _i, _i]),
    "orc_int8_acc_i32": (None, [_vp, _vp, _i, _i, _i, _i, _vp]),
    "orc_int4_acc_i32": (None, [_vp, _vp, _i, _i, _i, _i, _vp]),
    "orc_int8_gemv_i8act": (None, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _i]),
    "orc_int4_gemv_i8act": (None, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _i]),
    "orc_matmul_bitnet_f32": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "orc_matmul_bitnet_block_f32": (None, [_vp, _vp, _i, _vp, _vp, _vp, _i, _i]),
    "orc_matmul_bitnet_f32_w1w3": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i]),
    "orc_matmul_bitnet_dense_f32": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "orc_interleave_weights_4rows": (_sz, [_vp, _vp, _i, _i]),
    "orc_matmul_bitnet_tmac_interleaved_f32": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "orc_int8_rowscale_f32": (None, [_vp, _vp, _vp, _i, _i, _vp]),
    "orc_int4_gemv_f32": (None, [_vp, _vp, _vp, _vp, _i, _i]),
    "orc_gemm_f32_nt_ld": (None, [_vp, _i, _vp, _i, _vp, _vp, _i, _i, _i, _i, _i, _i]),
    "orc_softmax_rows_f32": (None, [_vp, _i, _i, _i, _f]),
    "orc_num_threads": (_i, []),
    "orc_round_f16": (_f, [_f]),
    "orc_quant_rows": (None, [_vp, _i, _i, _i, _i, _vp, _vp]),
    "orc_gguf_ternary_rows": (None, [_i, _vp, _i, _i, _vp, _vp]),
    "orc_bitnet_forward": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
}

# The reference's own symbols (same signatures as the product's drop-in ABI) plus the two wrapped statics.
REF_SIGS = {
    "eif_unpack_ternary": (C.c_int8, [C.c_uint8, _i]),
    "eif_pack_ternary": (_sz, [_vp, _vp, _sz]),
    "eif_pack_ternary_dense": (_sz, [_vp, _vp, _sz]),
    "eif_hadamard_block_size": (_i, [_i]),
    "eif_bitnet_group_size": (_i, [_i, _i]),
    "eif_hadamard_rotate_f32": (None, [_vp, _vp, _i, _i]),
    "eif_quantize_activation_i8": (None, [_vp, _vp, _vp, _i]),
    "eif_matmul_bitnet_i8xternary_f32": (None, [_vp, _vp, _vp, _f, _vp, _vp, _i, _i]),
    "eif_matmul_bitnet_act_quant_f32": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "eif_matmul_bitnet_int8": (None, [_vp, _f, _vp, _f, _vp, _vp, _f, _i, _i]),
    "eif_matmul_bitnet_f32": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "eif_matmul_bitnet_block_f32": (None, [_vp, _vp, _i, _vp, _vp, _vp, _i, _i]),
    "eif_matmul_bitnet_f32_w1w3": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i]),
    "eif_matmul_bitnet_dense_f32": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "eif_interleave_weights_4rows": (_sz, [_vp, _vp, _i, _i]),
    "eif_matmul_bitnet_tmac_interleaved_f32": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "tinyllm_matmul_int8_rowscale": (None, [_vp, _vp, _vp, _i, _i, _vp]),
    "ref_q35_int4_gemv": (None, [_vp, _vp, _vp, _vp, _i, _i]),
    "ref_q35_int8_gemv": (None, [_vp, _vp, _vp, _vp, _i, _i]),
    "ref_q35_layout": (_i, [C.c_char_p, _vp, _i, _vp]),
    "ref_q35_dense_gemv": (None, [_vp, _vp, _vp, _vp, _i, _i]),
    "eif_gemm_f32_nt_ld": (None, [_vp, _i, _vp, _i, _vp, _vp, _i, _i, _i, _i, _i, _i]),
    "eif_softmax_rows_f32": (None, [_vp, _i, _i, _i, _f]),
}


def _bind(path, sigs):
    lib = C.CDLL(path)
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    return lib


def load(path):
    return _bind(path, ORACLE_SIGS)


def load_ref(path):
    return _bind(path, REF_SIGS)


def load_ref_tinyllm(path):
    """The reference's tinyllm decode wrapper (_ref/libref.so or _ref/libref_scalar.so)."""
    return _bind(path, REF_TINYLLM_SIGS)


def P(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


ORC_LIN_INT8, ORC_LIN_F32 = 0, 1


class OrcBitnetCfg(C.Structure):
    _fields_ = [(n, _i) for n in ("dim", "hidden", "n_layers", "n_heads", "n_kv_heads", "head_dim", "vocab", "seq_len")] + \
               [(n, _f) for n in ("rope_theta", "rms_eps", "sub_eps")] + \
               [(n, _i) for n in ("wht_dim", "wht_q", "wht_hidden")] + \
               [(n, _f) for n in ("wht_norm_dim", "wht_norm_q", "wht_norm_hidden")] + \
               [(n, _i) for n in ("g_q", "g_o", "g_13", "g_2")]


BITNET_WEIGHT_FIELDS = ("emb", "emb_scale", "wq", "wk", "wv", "wo", "w1", "w3", "w2", "gq", "gk", "gv", "go", "g1", "g3",
                        "g2", "rms_att", "rms_ffn", "rms_sub_att", "rms_sub_ffn", "rms_final", "signs_dim", "signs_q",
                        "signs_hidden", "wcls", "wcls_scale")


class OrcBitnetWeights(C.Structure):
    _fields_ = [(n, _vp) for n in BITNET_WEIGHT_FIELDS]


def bitnet_structs(cfg, w):
    """ctypes (config, weights) for a model from synth.bitnet_model; the numpy arrays must outlive them."""
    c = OrcBitnetCfg(**{k: cfg[k] for k, _ in OrcBitnetCfg._fields_})
    ws = OrcBitnetWeights(**{k: (w[k].ctypes.data if w.get(k) is not None else None) for k in BITNET_WEIGHT_FIELDS})
    return c, ws


REF_TINYLLM_SIGS = {
    "ref_bitnet_create": (_vp, [_vp, _vp, _i]),
    "ref_bitnet_forward": (C.POINTER(_f), [_vp, _i, _i]),
    "ref_bitnet_destroy": (None, [_vp]),
    "ref_bitnet_fill_cache": (C.c_int, [_vp, _i]),
    "ref_svlm_create": (_vp, [C.c_char_p]),
    "ref_ttml_create": (_vp, [C.c_char_p]),
    "ref_gguf_create": (_vp, [C.c_char_p]),
    "ref_tinyllm_view": (C.c_int, [_vp, _vp, _vp, _vp]),
}
