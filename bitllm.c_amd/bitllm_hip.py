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

PRE_NONE, PRE_RMS, PRE_SWIGLU_RMS = 0, 1, 2


class PrepSpec(C.Structure):
    """eif_hip_prep_spec (include/eif_hip.h)."""
    _fields_ = [("x", _vp), ("ldx", _i), ("x2", _vp), ("norm_w", _vp), ("eps", _f), ("pre", _i), ("signs", _vp),
                ("wht_block", _i), ("wht_norm", _f)]


class BitnetConfig(C.Structure):
    """eif_hip_bitnet_config (include/eif_hip_decode.h)."""
    _fields_ = [(n, _i) for n in ("dim", "hidden", "n_layers", "n_heads", "n_kv_heads", "head_dim", "vocab", "seq_len")] + \
               [(n, _f) for n in ("rope_theta", "rms_eps", "sub_eps")] + \
               [(n, _i) for n in ("wht_dim", "wht_q", "wht_hidden")] + \
               [(n, _f) for n in ("wht_norm_dim", "wht_norm_q", "wht_norm_hidden")] + \
               [(n, _i) for n in ("g_q", "g_o", "g_13", "g_2")]


class BitnetLayer(C.Structure):
    _fields_ = [(n, _vp) for n in ("wq", "wk", "wv", "wo", "w1", "w3", "w2", "gq", "gk", "gv", "go", "g1", "g3", "g2",
                                    "rms_att", "rms_ffn", "rms_sub_att", "rms_sub_ffn")]


class BitnetGlobals(C.Structure):
    _fields_ = [(n, _vp) for n in ("emb", "emb_scale", "rms_final", "signs_dim", "signs_q", "signs_hidden", "wcls",
                                    "wcls_scale")]


class GgufInfo(C.Structure):
    """eif_gguf_bitnet_info (include/eif_hip_gguf.h)."""
    _fields_ = [("arch", C.c_char * 64), ("version", C.c_uint32), ("alignment", C.c_uint32)] + \
               [(n, _i) for n in ("dim", "hidden", "n_layers", "n_heads", "n_kv_heads", "head_dim", "vocab", "seq_len")] + \
               [("rope_theta", _f)] + [(n, _i) for n in ("rope_interleaved", "proj_type", "emb_type", "head_type")]


# name: (restype, argtypes) for every exported symbol this module binds.
_SIGS = {
    "eif_gguf_bitnet_open": (_i, [C.POINTER(_vp), C.c_char_p]),
    "eif_gguf_bitnet_close": (None, [_vp]),
    "eif_gguf_bitnet_get_info": (_i, [_vp, C.POINTER(GgufInfo)]),
    "eif_gguf_bitnet_get_layer": (_i, [_vp, _i, C.POINTER(BitnetLayer)]),
    "eif_gguf_bitnet_get_globals": (_i, [_vp, C.POINTER(BitnetGlobals)]),
    "eif_hip_bitnet_load_gguf": (_i, [_vp, C.c_char_p, _i]),
    "eif_hip_qlinear_prep": (_i, [_vp, C.POINTER(PrepSpec), _vp, _vp, _i, _i, _vp]),
    "eif_hip_qlinear_prep_glu": (_i, [_vp, C.POINTER(PrepSpec), _vp, _i, _i, _vp]),
    "eif_hip_qlinear_prep_acc": (_i, [_vp, C.POINTER(PrepSpec), _vp, _i, _vp]),
    "eif_hip_prep_spec_rows": (_i, [C.POINTER(PrepSpec), _i, _vp, _i, _vp, _i, _vp]),
    "eif_hip_quant_rows": (_i, [_vp, _i, _i, _i, _i, _vp, _vp, _vp]),
    "eif_gguf_ternary_rows": (_i, [_i, _vp, _i, _i, _vp, _vp]),
    "eif_hip_qweight_from_gguf_ternary": (_i, [_vp, _i, _vp, _i, _i, _vp]),
    "eif_hip_bitnet_create": (_i, [C.POINTER(_vp), C.POINTER(BitnetConfig)]),
    "eif_hip_bitnet_set_layer": (_i, [_vp, _i, C.POINTER(BitnetLayer)]),
    "eif_hip_bitnet_set_globals": (_i, [_vp, C.POINTER(BitnetGlobals)]),
    "eif_hip_bitnet_reset": (_i, [_vp, _vp, _i, _vp]),
    "eif_hip_bitnet_steps": (_i, [_vp, _i, _i, _vp]),
    "eif_hip_bitnet_set_persistent": (_i, [_vp, _i]),
    "eif_hip_bitnet_prefill": (_i, [_vp, _i, _vp]),
    "eif_hip_bitnet_load_svlm": (_i, [_vp, C.c_char_p, _i]),
    "eif_qwen35_parse": (_i, [_vp, _sz, _vp]),
    "eif_hip_qwen35_load": (_i, [_vp, C.c_char_p, _vp]),
    "eif_qwen35_gguf_image": (_i, [C.c_char_p, _sz, C.POINTER(_vp), C.POINTER(_sz)]),
    "eif_qwen35_image_free": (None, [_vp]),
    "eif_hip_qwen35_destroy": (None, [_vp]),
    "eif_hip_qwen35_get_layout": (_vp, [_vp]),
    "eif_hip_qwen35_linear": (_vp, [_vp, _i, _i]),
    "eif_hip_qwen35_head": (_vp, [_vp]),
    "eif_hip_qwen35_linear_batch": (_i, [_vp, _i, _i, C.POINTER(PrepSpec), _vp, _vp, _i, _i, _vp]),
    "eif_hip_qwen35_vector": (_vp, [_vp, _sz]),
    "eif_hip_bitnet_get_config": (_i, [_vp, _vp]),
    "eif_hip_bitnet_tokens": (_i, [_vp, _vp, _i, _vp]),
    "eif_hip_bitnet_logits": (_i, [_vp, _vp, _vp]),
    "eif_hip_bitnet_position": (_i, [_vp, _vp]),
    "eif_hip_bitnet_kv_cache": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp]),
    "eif_hip_bitnet_weight_bytes": (_sz, [_vp]),
    "eif_hip_bitnet_kv_bytes": (_sz, [_vp, _i]),
    "eif_hip_bitnet_destroy": (None, [_vp]),
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
    "eif_hip_qlinear_ex_noalloc": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "eif_hip_qlinear_noalloc_max_bytes": (C.c_size_t, []),
    "eif_hip_qlinear_acc": (_i, [_vp, _vp, _i, _vp, _i, _i, _vp]),
    "eif_hip_qlinear_f32": (_i, [_vp, _vp, _i, _vp, _i, _f, _vp, _vp, _i, _i, _vp]),
    "eif_hip_qlinear_f32_acc": (_i, [_vp, _vp, _i, _vp, _i, _f, _vp, _i, _vp]),
    "eif_hip_set_gemm_min_tokens": (_i, [_i]),
    "eif_hip_gemm_min_tokens": (_i, []),
    "eif_hip_set_gemv_ksplit": (_i, [_i]),
    "eif_hip_set_gemv_row_tiles": (_i, [_i]),
    "eif_hip_set_gemv_token_chunk": (_i, [_i]),
    "eif_hip_set_gemv_stream": (_i, [_i]),
    "eif_hip_set_gemv_rowpair": (_i, [_i]),
    "eif_hip_set_f32_tiles_per_wave": (_i, [_i]),
    "eif_hip_set_f32_ksplit": (_i, [_i]),
    "eif_hip_set_gemv_prep_cols": (_i, [_i]),
    "eif_hip_set_gemm_split": (_i, [_i]),
    "eif_hip_set_gemm_token_tiles": (_i, [_i]),
    "eif_hip_set_gemm_prefetch": (_i, [_i]),
    "eif_hip_set_gemm_panel": (_i, [_i]),
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
    "eif_hip_set_host_weight_cache_limit": (_sz, [_sz]),
    "eif_hip_host_weight_cache_bytes": (_sz, []),
    "eif_hip_set_host_error_mode": (_i, [_i]),
    "eif_hip_host_last_error": (_i, [_vp, _sz]),
    "eif_gpu_matmul_bitnet_f32": (C.c_bool, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i]),
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


# return codes of include/eif_hip.h
OK, E_ARG, E_DEVICE, E_NOMEM, E_LIMIT = 0, -1, -2, -3, -4


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

    @classmethod
    def wrap(cls, h):
        """A QWeight around a handle made by another constructor of the library (it takes ownership)."""
        self = cls.__new__(cls)
        r, c, kp, g, b = C.c_int(), C.c_int(), C.c_int(), C.c_int(), C.c_size_t()
        check(load().eif_hip_qweight_info(h, C.byref(r), C.byref(c), C.byref(kp), C.byref(g), C.byref(b)),
              "eif_hip_qweight_info")
        self.h, self.fmt, self.rows, self.cols, self.group = h, None, r.value, c.value, g.value
        self.kpad, self.bytes = kp.value, b.value
        return self

    @classmethod
    def view(cls, h, owner):
        """A QWeight around a handle that `owner` keeps (and destroys); holds a reference to the owner."""
        self = cls.wrap(h)
        self._owner = owner
        return self

    def close(self):
        if self.h and getattr(self, "_owner", None) is None:
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


def prep_spec(x, pre=PRE_NONE, x2=None, norm_w=None, eps=0.0, signs=None, block=0, norm=1.0):
    """An eif_hip_prep_spec over device tensors (kept alive by the caller)."""
    return PrepSpec(x=ptr(x).value, ldx=x.stride(0) if x.dim() > 1 else x.shape[-1], x2=ptr(x2).value if x2 is not None else None,
                    norm_w=ptr(norm_w).value if norm_w is not None else None, eps=eps, pre=pre,
                    signs=ptr(signs).value if signs is not None else None, wht_block=block, wht_norm=norm)


def prep_spec_rows(spec, K, xq, xs, M, stream=None):
    """The prep of a spec on its own: M rows of K columns -> xq [M, ldq] int8 + xs [M] (device tensors)."""
    check(load().eif_hip_prep_spec_rows(C.byref(spec), K, ptr(xq), xq.stride(0), ptr(xs), M, stream_ptr(stream)),
          "eif_hip_prep_spec_rows")


def quant_rows(x, bits, dst, scales, stream=None):
    """FP32 rows x [rows, cols] (device) -> INT8 / INT4 row-scaled codes dst and scales (device)."""
    rows, cols = x.shape
    check(load().eif_hip_quant_rows(ptr(x), x.stride(0), rows, cols, bits, ptr(dst), ptr(scales), stream_ptr(stream)),
          "eif_hip_quant_rows")


class BitnetModel:
    """The GPU BitNet decoder (include/eif_hip_decode.h) loaded from a configuration and reference-format
    weights as synth.bitnet_model builds them (per-layer arrays concatenated over layers)."""

    def __init__(self, cfg, w):
        import numpy as np
        lib = load()
        self.cfg = cfg
        self.c = BitnetConfig(**{k: cfg[k] for k, _ in BitnetConfig._fields_})
        h = C.c_void_p()
        check(lib.eif_hip_bitnet_create(C.byref(h), C.byref(self.c)), "eif_hip_bitnet_create")
        self.h = h
        d, hid, L = cfg["dim"], cfg["hidden"], cfg["n_layers"]
        qd, kvd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
        rows = {"q": qd, "k": kvd, "v": kvd, "o": d, "1": hid, "3": hid, "2": d}
        norms = {"rms_att": d, "rms_ffn": d, "rms_sub_att": qd, "rms_sub_ffn": hid}

        def at(a, l, n):
            a = np.ascontiguousarray(a).reshape(L, -1) if a.ndim == 1 else np.ascontiguousarray(a).reshape(L, n, -1)
            return a[l].ctypes.data, a

        keep = []
        for l in range(L):
            f = {}
            for k, n in rows.items():
                pw, a = at(w["w" + k], l, n)
                pg, b = at(w["g" + k], l, n)
                keep += [a, b]
                f["w" + k], f["g" + k] = pw, pg
            for k, n in norms.items():
                pn, a = at(w[k], l, n)
                keep.append(a)
                f[k] = pn
            check(lib.eif_hip_bitnet_set_layer(h, l, C.byref(BitnetLayer(**f))), "eif_hip_bitnet_set_layer")
        g = BitnetGlobals(**{k: (w[k].ctypes.data if w.get(k) is not None else None)
                             for k, _ in BitnetGlobals._fields_})
        check(lib.eif_hip_bitnet_set_globals(h, C.byref(g)), "eif_hip_bitnet_set_globals")

    @classmethod
    def from_svlm(cls, path, seq_len=0):
        """A model read from a BitNet SVLM file (eif_hip_bitnet_load_svlm)."""
        lib = load()
        h = C.c_void_p()
        check(lib.eif_hip_bitnet_load_svlm(C.byref(h), os.fsencode(path), seq_len), "eif_hip_bitnet_load_svlm")
        self = cls.__new__(cls)
        self.h = h
        self.c = BitnetConfig()
        check(lib.eif_hip_bitnet_get_config(h, C.byref(self.c)), "eif_hip_bitnet_get_config")
        self.cfg = {k: getattr(self.c, k) for k, _ in BitnetConfig._fields_}
        return self

    @classmethod
    def from_gguf(cls, path, seq_len=0):
        """A model read from a BitNet GGUF file (eif_hip_bitnet_load_gguf)."""
        lib = load()
        h = C.c_void_p()
        check(lib.eif_hip_bitnet_load_gguf(C.byref(h), os.fsencode(path), seq_len), "eif_hip_bitnet_load_gguf")
        self = cls.__new__(cls)
        self.h = h
        self.c = BitnetConfig()
        check(lib.eif_hip_bitnet_get_config(h, C.byref(self.c)), "eif_hip_bitnet_get_config")
        self.cfg = {k: getattr(self.c, k) for k, _ in BitnetConfig._fields_}
        return self

    def reset(self, prompt, stream=None):
        import numpy as np
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        check(load().eif_hip_bitnet_reset(self.h, p.ctypes.data, len(p), stream_ptr(stream)), "eif_hip_bitnet_reset")

    def steps(self, n, graph=False, stream=None):
        check(load().eif_hip_bitnet_steps(self.h, n, 1 if graph else 0, stream_ptr(stream)), "eif_hip_bitnet_steps")

    def prefill(self, n, stream=None):
        check(load().eif_hip_bitnet_prefill(self.h, n, stream_ptr(stream)), "eif_hip_bitnet_prefill")

    def tokens(self, n, stream=None):
        import numpy as np
        out = np.zeros(n, np.int32)
        check(load().eif_hip_bitnet_tokens(self.h, out.ctypes.data, n, stream_ptr(stream)), "eif_hip_bitnet_tokens")
        return out

    def logits(self, stream=None):
        import numpy as np
        out = np.zeros(self.cfg["vocab"], np.float32)
        check(load().eif_hip_bitnet_logits(self.h, out.ctypes.data, stream_ptr(stream)), "eif_hip_bitnet_logits")
        return out

    def position(self, stream=None):
        p = load().eif_hip_bitnet_position(self.h, stream_ptr(stream))
        if p < 0:
            check(p, "eif_hip_bitnet_position")
        return p

    def set_persistent(self, on):
        """Token steps as one persistent kernel (on=True) or as separate launches; returns whether steps run
        persistent (False when the model's shapes are outside the persistent kernel). on=None only queries."""
        rc = load().eif_hip_bitnet_set_persistent(self.h, -1 if on is None else int(bool(on)))
        if rc < 0:
            check(rc, "eif_hip_bitnet_set_persistent")
        return rc == 1

    def kv_cache(self, layer, pos0, n, stream=None):
        """Keys and values of one layer at positions [pos0, pos0 + n), float [n, kv_dim] each."""
        import numpy as np
        kvd = self.cfg["n_kv_heads"] * self.cfg["head_dim"]
        k, v = np.zeros((n, kvd), np.float32), np.zeros((n, kvd), np.float32)
        check(load().eif_hip_bitnet_kv_cache(self.h, layer, pos0, n, k.ctypes.data, v.ctypes.data, stream_ptr(stream)),
              "eif_hip_bitnet_kv_cache")
        return k, v

    def weight_bytes(self):
        return load().eif_hip_bitnet_weight_bytes(self.h)

    def kv_bytes(self, pos):
        return load().eif_hip_bitnet_kv_bytes(self.h, pos)

    def close(self):
        if self.h:
            load().eif_hip_bitnet_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GgufBitnet:
    """A BitNet GGUF file read and converted on the host (eif_gguf_bitnet_open; no GPU): its configuration and
    the reference-format arrays, one scale per row, rows as the file holds them."""

    def __init__(self, path):
        lib = load()
        h = C.c_void_p()
        check(lib.eif_gguf_bitnet_open(C.byref(h), os.fsencode(path)), "eif_gguf_bitnet_open")
        self.h = h
        self.info = GgufInfo()
        check(lib.eif_gguf_bitnet_get_info(h, C.byref(self.info)), "eif_gguf_bitnet_get_info")

    def layer(self, l):
        """Copies of layer l's arrays: w* uint8 [rows, cols / 4], g* float32 [rows], rms_att / rms_ffn [dim]."""
        import numpy as np
        lw = BitnetLayer()
        check(load().eif_gguf_bitnet_get_layer(self.h, l, C.byref(lw)), "eif_gguf_bitnet_get_layer")
        i = self.info
        qd, kvd = i.n_heads * i.head_dim, i.n_kv_heads * i.head_dim
        shapes = {"q": (qd, i.dim), "k": (kvd, i.dim), "v": (kvd, i.dim), "o": (i.dim, qd), "1": (i.hidden, i.dim),
                  "3": (i.hidden, i.dim), "2": (i.dim, i.hidden)}
        out = {}
        for k, (rows, cols) in shapes.items():
            out["w" + k] = _host_array(getattr(lw, "w" + k), np.uint8, (rows, (cols + 3) // 4))
            out["g" + k] = _host_array(getattr(lw, "g" + k), np.float32, (rows,))
        out["rms_att"] = _host_array(lw.rms_att, np.float32, (i.dim,))
        out["rms_ffn"] = _host_array(lw.rms_ffn, np.float32, (i.dim,))
        return out

    def globals(self):
        import numpy as np
        g = BitnetGlobals()
        check(load().eif_gguf_bitnet_get_globals(self.h, C.byref(g)), "eif_gguf_bitnet_get_globals")
        i = self.info
        return {"emb": _host_array(g.emb, np.int8, (i.vocab, i.dim)),
                "emb_scale": _host_array(g.emb_scale, np.float32, (i.vocab,)),
                "rms_final": _host_array(g.rms_final, np.float32, (i.dim,)),
                "wcls": _host_array(g.wcls, np.int8, (i.vocab, i.dim)),
                "wcls_scale": _host_array(g.wcls_scale, np.float32, (i.vocab,))}

    def model(self, seq_len=0):
        """(cfg, w) for BitnetModel(cfg, w): the converted arrays with the decoder configuration
        eif_hip_bitnet_load_gguf gives them (rows as the file holds them, sub-norms 1)."""
        import numpy as np
        i = self.info
        qd = i.n_heads * i.head_dim
        cfg = dict(dim=i.dim, hidden=i.hidden, n_layers=i.n_layers, n_heads=i.n_heads, n_kv_heads=i.n_kv_heads,
                   head_dim=i.head_dim, vocab=i.vocab, seq_len=seq_len if seq_len > 0 else i.seq_len,
                   rope_theta=i.rope_theta, rms_eps=1e-6 if i.vocab > 120000 else 1e-5, sub_eps=1e-5, wht_dim=0,
                   wht_q=0, wht_hidden=0, wht_norm_dim=0.0, wht_norm_q=0.0, wht_norm_hidden=0.0, g_q=0, g_o=0,
                   g_13=0, g_2=0)
        layers = [self.layer(l) for l in range(i.n_layers)]
        w = {k: np.concatenate([lay[k] for lay in layers]) for k in layers[0]}
        w["rms_sub_att"] = np.ones(i.n_layers * qd, np.float32)
        w["rms_sub_ffn"] = np.ones(i.n_layers * i.hidden, np.float32)
        w.update(self.globals())
        return cfg, w

    def close(self):
        if self.h:
            load().eif_gguf_bitnet_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _host_array(ptr, dtype, shape):
    import numpy as np
    n = int(np.prod(shape)) * np.dtype(dtype).itemsize
    return np.frombuffer(C.string_at(ptr, n), dtype=dtype).reshape(shape).copy()


# ---- Qwen3.5 model files (include/eif_hip_qwen35.h) ----
Q35_DN_QKV, Q35_DN_Z, Q35_DN_OUT, Q35_DN_B, Q35_DN_A, Q35_FA_Q, Q35_FA_K, Q35_FA_V, Q35_FA_O, Q35_FF_GATE, \
    Q35_FF_UP, Q35_FF_DOWN = range(12)
Q35_KINDS = 12
Q35_HEAD = -1   # the tied head's kind for Qwen35Model.linear_batch
Q35_FP32, Q35_INT4, Q35_TERN2, Q35_TERN3, Q35_INT8 = range(5)


class Q35Tensor(C.Structure):
    _fields_ = [("codes", C.c_size_t), ("scales", C.c_size_t), ("rows", C.c_int), ("cols", C.c_int),
                ("qtype", C.c_int), ("group", C.c_int)]


class Q35Layout(C.Structure):
    _fields_ = [("config", C.c_int32 * 32), ("layer_types", C.c_uint8 * 24), ("n_layers", C.c_int),
                ("embed", Q35Tensor), ("lin", (Q35Tensor * Q35_KINDS) * 24),
                ("rms_att", C.c_size_t * 24), ("rms_ffn", C.c_size_t * 24), ("rms_final", C.c_size_t),
                ("sub_att", C.c_size_t * 24), ("sub_ffn", C.c_size_t * 24),
                ("conv", C.c_size_t * 24), ("dt_bias", C.c_size_t * 24), ("a_log", C.c_size_t * 24),
                ("delta_norm", C.c_size_t * 24), ("q_norm", C.c_size_t * 24), ("k_norm", C.c_size_t * 24),
                ("signs_dim", C.c_size_t), ("signs_hid", C.c_size_t), ("hadamard_block", C.c_int),
                ("weights_end", C.c_size_t), ("scales_end", C.c_size_t), ("norms_end", C.c_size_t)]


def qwen35_parse(image):
    """The layout of a QWN5 image (bytes) as eif_qwen35_parse walks it (host code, no GPU)."""
    buf = (C.c_uint8 * len(image)).from_buffer_copy(image)
    lay = Q35Layout()
    check(load().eif_qwen35_parse(C.cast(buf, _vp), len(image), C.byref(lay)), "eif_qwen35_parse")
    return lay


def qwen35_gguf_image(gguf_bytes):
    """The QWN5 image (bytes) of a Qwen3.5 GGUF file's bytes (eif_qwen35_gguf_image; host code, no GPU)."""
    lib = load()
    out, n = C.c_void_p(), C.c_size_t()
    check(lib.eif_qwen35_gguf_image(gguf_bytes, len(gguf_bytes), C.byref(out), C.byref(n)), "eif_qwen35_gguf_image")
    try:
        return C.string_at(out, n.value)
    finally:
        lib.eif_qwen35_image_free(out)


class Qwen35Model:
    """A QWN5 file's quantized linears and tied head resident on the GPU (eif_hip_qwen35_load)."""

    def __init__(self, path, stream=None):
        h = C.c_void_p()
        check(load().eif_hip_qwen35_load(C.byref(h), os.fsencode(path), stream_ptr(stream)), "eif_hip_qwen35_load")
        self.h = h
        self.layout = Q35Layout.from_address(load().eif_hip_qwen35_get_layout(h))

    def linear(self, layer, kind):
        """The resident weight (a QWeight view) or None (absent or FP32)."""
        w = load().eif_hip_qwen35_linear(self.h, layer, kind)
        return QWeight.view(w, self) if w else None

    def head(self):
        w = load().eif_hip_qwen35_head(self.h)
        return QWeight.view(w, self) if w else None

    def vector(self, offset):
        """Device address of an FP32 vector of the layout (0 if absent)."""
        return load().eif_hip_qwen35_vector(self.h, offset) or 0

    def linear_batch(self, layer, kind, spec, y, M=None, bias=None, stream=None):
        """The prefill's batched linear (eif_hip_qwen35_linear_batch): y [M, N] from the rows of spec; kind
        Q35_HEAD for the tied head."""
        M = y.shape[0] if M is None else M
        check(load().eif_hip_qwen35_linear_batch(self.h, layer, kind, C.byref(spec), ptr(bias), ptr(y), y.stride(0), M,
                                                 stream_ptr(stream)), "eif_hip_qwen35_linear_batch")

    def close(self):
        if self.h:
            load().eif_hip_qwen35_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
