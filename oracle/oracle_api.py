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


def P(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)
