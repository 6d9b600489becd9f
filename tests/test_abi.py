"""The C-ABI library loads without a GPU and exports every function declared in include/*.h (CPU only)."""
import ctypes as C
import glob
import os
import re
import subprocess

from conftest import ROOT

LIB = os.path.join(ROOT, "bitllm.c_amd", "libbitllm_hip.so")


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M):
            if not m.group(0).lstrip().startswith(("#", "typedef", "return")):
                names.add(m.group(1))
    return names


def test_headers_declare_the_reference_api():
    names = declared_functions()
    # include/eif_quantize_bitnet.h:32-272 and include/eif_gemm.h:22-30 of the reference, one by one
    ref_api = {
        "eif_unpack_ternary", "eif_pack_ternary", "eif_pack_ternary_dense", "eif_matmul_bitnet_f32",
        "eif_matmul_bitnet_dense_f32", "eif_matmul_bitnet_int8", "eif_matmul_bitnet_f32_w1w3",
        "eif_quantize_activation_i8", "eif_matmul_bitnet_i8xternary_f32", "eif_matmul_bitnet_act_quant_f32",
        "eif_matmul_bitnet_block_f32", "eif_interleave_weights_4rows", "eif_matmul_bitnet_tmac_interleaved_f32",
        "eif_hadamard_block_size", "eif_bitnet_group_size", "eif_hadamard_rotate_f32", "eif_gemm_f32_nt",
        "eif_gemm_f32_nt_ld", "eif_softmax_rows_f32", "tinyllm_matmul_int8_rowscale",
    }
    assert ref_api <= names, ref_api - names


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB), "libbitllm_hip.so not built"
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = declared_functions() - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"


def test_library_loads_without_gpu():
    lib = C.CDLL(LIB)
    lib.eif_hadamard_block_size.restype = C.c_int
    assert lib.eif_hadamard_block_size(1536) == 512
    lib.eif_bitnet_group_size.restype = C.c_int
    assert lib.eif_bitnet_group_size(576, 128) == 96
    lib.eif_hip_wht_norm.restype = C.c_float
    lib.eif_hip_wht_norm.argtypes = [C.c_int]
    assert abs(lib.eif_hip_wht_norm(128) - 128 ** -0.5) < 1e-6


def test_host_pack_helpers_match_oracle(oracle):
    import numpy as np
    from conftest import P
    lib = C.CDLL(LIB)
    lib.eif_pack_ternary.restype = C.c_size_t
    lib.eif_pack_ternary.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
    lib.eif_pack_ternary_dense.restype = C.c_size_t
    lib.eif_pack_ternary_dense.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
    lib.eif_interleave_weights_4rows.restype = C.c_size_t
    lib.eif_interleave_weights_4rows.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int]
    r = np.random.default_rng(0)
    v = r.integers(-1, 2, 999).astype(np.int8)
    a, b = np.zeros(250, np.uint8), np.zeros(250, np.uint8)
    assert lib.eif_pack_ternary(P(v), P(a), 999) == oracle.orc_pack_ternary(P(v), P(b), 999) == 250
    assert np.array_equal(a, b)
    a, b = np.zeros(200, np.uint8), np.zeros(200, np.uint8)
    assert lib.eif_pack_ternary_dense(P(v), P(a), 999) == oracle.orc_pack_ternary_dense(P(v), P(b), 999) == 200
    assert np.array_equal(a, b)
    w = r.integers(0, 256, 7 * 5, dtype=np.uint8)
    a, b = np.zeros(35, np.uint8), np.zeros(35, np.uint8)
    assert lib.eif_interleave_weights_4rows(P(w), P(a), 7, 17) == oracle.orc_interleave_weights_4rows(P(w), P(b), 7, 17)
    assert np.array_equal(a, b)
