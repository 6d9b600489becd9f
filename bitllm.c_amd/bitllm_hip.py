"""ctypes binding of libbitllm_hip.so for tests, the benchmark and the smoke check.

The library is the product: a C ABI over hand-written gfx950 kernels (csrc/). This module only passes device
pointers of torch tensors (PyTorch is used for device memory and streams) or host numpy buffers through. It
never computes anything itself, and it raises if the library has not been built -- there is no fallback.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbitllm_hip.so")

W_TERNARY, W_INT8, W_INT4 = 1, 2, 3
PATH_AUTO, PATH_GEMV, PATH_GEMM = 0, 1, 2

_vp, _i, _f, _sz = C.c_void_p, C.c_int, C.c_float, C.c_size_t

# name: (restype, argtypes) for every exported symbol this module binds.
_SIGS = {
    "eif_hip_init": (_i, [_i]),
    "eif_hip_strerror": (C.c_char_p, [_i]),
    "eif_hip_wht_norm": (_f, [_i]),
    "eif_hip_wht_norm_exact": (_f, [_i]),
    "eif_hip_prep_rows": (_i, [_vp, _i, _vp, _i, _i, _i, _f, _vp, _i, _vp, _vp, _i, _vp]),
    "eif_hip_qweight_create": (_i, [C.POINTER(_vp), _i, _i, _i, _i, _vp, _vp, _i, _vp]),
    "eif_hip_qweight_destroy": (None, [_vp]),
    "eif_hip_qweight_info": (_i, [_vp, C.POINTER(_i), C.POINTER(_i), C.POINTER(_i), C.POINTER(_i),
                                  C.POINTER(_sz)]),
    "eif_hip_qlinear": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _i, _vp]),
    "eif_hip_qlinear_ex": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "eif_hip_qlinear_acc": (_i, [_vp, _vp, _i, _vp, _i, _i, _vp]),
    "eif_hip_qlinear_f32": (_i, [_vp, _vp, _i, _vp, _i, _f, _vp, _vp, _i, _i, _vp]),
    "eif_hip_qlinear_f32_acc": (_i, [_vp, _vp, _i, _vp, _i, _f, _vp, _i, _vp]),
    "eif_hip_set_gemm_min_tokens": (_i, [_i]),
    "eif_hip_gemm_min_tokens": (_i, []),
    "eif_hip_set_gemv_ksplit": (_i, [_i]),
    "eif_hip_set_gemv_row_tiles": (_i, [_i]),
    "eif_hip_set_gemm_split": (_i, [_i]),
    "eif_hip_forget_host_weights": (None, [_vp]),
    # host-pointer drop-in ABI
    "eif_unpack_ternary": (C.c_int8, [C.c_uint8, _i]),
    "eif_pack_ternary": (_sz, [_vp, _vp, _sz]),
    "eif_pack_ternary_dense": (_sz, [_vp, _vp, _sz]),
    "eif_matmul_bitnet_f32": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "eif_matmul_bitnet_dense_f32": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "eif_matmul_bitnet_int8": (None, [_vp, _f, _vp, _f, _vp, _vp, _f, _i, _i]),
    "eif_matmul_bitnet_f32_w1w3": (None, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i]),
    "eif_quantize_activation_i8": (None, [_vp, _vp, _vp, _i]),
    "eif_matmul_bitnet_i8xternary_f32": (None, [_vp, _vp, _vp, _f, _vp, _vp, _i, _i]),
    "eif_matmul_bitnet_act_quant_f32": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "eif_matmul_bitnet_block_f32": (None, [_vp, _vp, _i, _vp, _vp, _vp, _i, _i]),
    "eif_interleave_weights_4rows": (_sz, [_vp, _vp, _i, _i]),
    "eif_matmul_bitnet_tmac_interleaved_f32": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "eif_hadamard_block_size": (_i, [_i]),
    "eif_bitnet_group_size": (_i, [_i, _i]),
    "eif_hadamard_rotate_f32": (None, [_vp, _vp, _i, _i]),
    "eif_gemm_f32_nt": (None, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i]),
    "eif_gemm_f32_nt_ld": (None, [_vp, _i, _vp, _i, _vp, _vp, _i, _i, _i, _i, _i, _i]),
    "eif_softmax_rows_f32": (None, [_vp, _i, _i, _i, _f]),
    "tinyllm_matmul_int8_rowscale": (None, [_vp, _vp, _vp, _i, _i, _vp]),
    "eif_int4_gemv_f32": (None, [_vp, _vp, _vp, _vp, _i, _i]),
    "eif_int8_gemv_f32": (None, [_vp, _vp, _vp, _vp, _i, _i]),
}

_lib = None


class HipError(RuntimeError):
    pass


def load():
    """Load the built library (raises if it is missing: build it with __graft_entry__.build())."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise HipError(f"{LIB_PATH} is not built; run __graft_entry__.build() first")
        lib = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        _lib = lib
    return _lib


def check(rc, what):
    if rc != 0:
        raise HipError(f"{what}: {load().eif_hip_strerror(rc).decode()} ({rc})")


def ptr(t):
    """Device pointer of a torch tensor, host pointer of a numpy array, None for None."""
    if t is None:
        return None
    if hasattr(t, "data_ptr"):
        return C.c_void_p(t.data_ptr())
    return t.ctypes.data_as(C.c_void_p)


def stream_ptr(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def wht_norm(block):
    return load().eif_hip_wht_norm(block)


def prep_rows(x, xq, xs, block, norm, signs=None, xrot=None, stream=None):
    """x [M, K] float32 -> xq [M, ldq] int8 (+ xs [M], optional xrot [M, ldr]) on the GPU."""
    M, K = x.shape
    check(load().eif_hip_prep_rows(ptr(x), x.stride(0), ptr(signs), M, K, block, norm, ptr(xq),
                                   xq.stride(0) if xq is not None else 0, ptr(xs), ptr(xrot),
                                   xrot.stride(0) if xrot is not None else 0, stream_ptr(stream)),
          "eif_hip_prep_rows")


class QWeight:
    """A weight matrix resident in HBM in the GPU layout (created from reference-format codes)."""

    def __init__(self, fmt, rows, cols, group, codes, scales, on_device=False, stream=None):
        h = C.c_void_p()
        check(load().eif_hip_qweight_create(C.byref(h), fmt, rows, cols, group, ptr(codes), ptr(scales),
                                            1 if on_device else 0, stream_ptr(stream) if on_device else None),
              "eif_hip_qweight_create")
        self.h, self.fmt, self.rows, self.cols, self.group = h, fmt, rows, cols, group
        r, c, kp, g, b = C.c_int(), C.c_int(), C.c_int(), C.c_int(), C.c_size_t()
        check(load().eif_hip_qweight_info(h, C.byref(r), C.byref(c), C.byref(kp), C.byref(g), C.byref(b)),
              "eif_hip_qweight_info")
        self.kpad, self.bytes = kp.value, b.value

    def close(self):
        if self.h:
            load().eif_hip_qweight_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def linear(self, xq, xs, y, M=None, bias=None, path=PATH_AUTO, stream=None):
        M = xq.shape[0] if M is None else M
        check(load().eif_hip_qlinear_ex(self.h, ptr(xq), xq.stride(0), ptr(xs), ptr(bias), ptr(y), y.stride(0),
                                        M, path, stream_ptr(stream)), "eif_hip_qlinear_ex")

    def acc(self, xq, acc, M=None, path=PATH_AUTO, stream=None):
        M = xq.shape[0] if M is None else M
        check(load().eif_hip_qlinear_acc(self.h, ptr(xq), xq.stride(0), ptr(acc), M, path, stream_ptr(stream)),
              "eif_hip_qlinear_acc")

    def linear_f32(self, x, y, block, norm, signs=None, bias=None, stream=None):
        """prep(x) fused into the GEMV: x [M, K] FP32 on the device, M <= 8."""
        check(load().eif_hip_qlinear_f32(self.h, ptr(x), x.stride(0), ptr(signs), block, norm, ptr(bias), ptr(y),
                                         y.stride(0), x.shape[0], stream_ptr(stream)), "eif_hip_qlinear_f32")

    def acc_f32(self, x, acc, block, norm, signs=None, stream=None):
        check(load().eif_hip_qlinear_f32_acc(self.h, ptr(x), x.stride(0), ptr(signs), block, norm, ptr(acc),
                                             x.shape[0], stream_ptr(stream)), "eif_hip_qlinear_f32_acc")
