"""Seeded synthetic inputs of the benchmark workloads, in the reference's storage formats.

Every tensor draws from its own numpy PCG64 stream keyed by (workload id, tensor id, copy), so the CPU baseline,
the GPU runs and the parity tests see identical bytes on any machine.

Formats (reference):
  ternary  2-bit codes, column c in byte c>>2 at bits 2*(c&3); 01 = +1, 10 = -1   include/eif_quantize_bitnet.h:4-11
  int8     row-major int8                                                     src/eif_tinyllm.c:1651-1721
  int4     (cols+1)/2 bytes per row, even column in the high nibble, v = n-8   src/eif_qwen35_gguf.c:249-253
Distributions: ternary codes uniform over {-1, 0, +1}; group scales |N(0,1)|*0.02; row scales |N(0,1)|*0.01;
activations N(0,1) float32 with exactly floor(0.01*K) distinct entries per row multiplied by 20; int8 codes
uniform in [-127, 127]; int4 codes uniform in [-8, 7].
"""
import numpy as np


def rng(*key):
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence([0xB17, *[int(k) for k in key]])))


def pack_ternary(v):
    """int8 values in {-1,0,1}, shape [..., K] -> uint8 [..., (K+3)//4] in the reference 2-bit format."""
    v = np.asarray(v)
    K = v.shape[-1]
    Kp = (K + 3) // 4 * 4
    codes = np.zeros(v.shape[:-1] + (Kp,), np.uint8)
    codes[..., :K] = np.where(v > 0, 1, np.where(v < 0, 2, 0))
    c = codes.reshape(v.shape[:-1] + (Kp // 4, 4))
    return (c[..., 0] | (c[..., 1] << 2) | (c[..., 2] << 4) | (c[..., 3] << 6)).astype(np.uint8)


def unpack_ternary(packed, K):
    p = np.asarray(packed, np.uint8)
    codes = np.stack([(p >> (2 * i)) & 3 for i in range(4)], axis=-1).reshape(p.shape[:-1] + (-1,))[..., :K]
    return np.where(codes == 1, 1, np.where(codes == 2, -1, 0)).astype(np.int8)


def pack_int4(v):
    """int values in [-8,7], shape [..., K] -> uint8 [..., (K+1)//2], even column in the high nibble."""
    v = np.asarray(v)
    K = v.shape[-1]
    Kp = (K + 1) // 2 * 2
    n = np.full(v.shape[:-1] + (Kp,), 8, np.uint8)
    n[..., :K] = (v + 8).astype(np.uint8)
    return ((n[..., 0::2] << 4) | n[..., 1::2]).astype(np.uint8)


def unpack_int4(packed, K):
    p = np.asarray(packed, np.uint8).astype(np.int16)
    v = np.stack([(p >> 4) - 8, (p & 15) - 8], axis=-1).reshape(p.shape[:-1] + (-1,))[..., :K]
    return v.astype(np.int8)


def ternary_weight(key, N, K, group):
    """(packed [N,(K+3)//4] uint8, scales) with group scales [N, ceil(K/group)] or row scales [N]."""
    r = rng(*key, 1)
    codes = r.integers(-1, 2, size=(N, K), dtype=np.int8)
    ns = N * ((K + group - 1) // group) if group > 0 else N
    scales = (np.abs(rng(*key, 2).standard_normal(ns)) * 0.02).astype(np.float32)
    return pack_ternary(codes), scales.reshape(N, -1) if group > 0 else scales


def int8_weight(key, N, K):
    w = rng(*key, 1).integers(-127, 128, size=(N, K), dtype=np.int8)
    scales = (np.abs(rng(*key, 2).standard_normal(N)) * 0.01).astype(np.float32)
    return w, scales


def int4_weight(key, N, K):
    v = rng(*key, 1).integers(-8, 8, size=(N, K), dtype=np.int8)
    scales = (np.abs(rng(*key, 2).standard_normal(N)) * 0.01).astype(np.float32)
    return pack_int4(v), scales


def activations(key, M, K, outliers=True):
    r = rng(*key, 3)
    x = r.standard_normal((M, K)).astype(np.float32)
    if outliers:
        n = int(0.01 * K)
        for m in range(M):
            idx = r.choice(K, size=n, replace=False)
            x[m, idx] *= np.float32(20.0)
    return x


# Decoder layer of a BitNet-b1.58-2B-shaped model: hidden 2560, 20 query / 5 KV heads of dim 128, FFN 6912.
BITNET_2B_LAYER = [
    # name, rows (N), cols (K), group
    ("qkv", 3840, 2560, 128),
    ("o", 2560, 2560, 128),
    ("gate", 6912, 2560, 128),
    ("up", 6912, 2560, 128),
    ("down", 2560, 6912, 96),
]

# Qwen2.5-0.5B-like layer: hidden 896, 14 query / 2 KV heads of dim 64, FFN 4864 (INT8 weights).
QWEN25_05B_LAYER = [
    ("q", 896, 896), ("k", 128, 896), ("v", 128, 896), ("o", 896, 896),
    ("gate", 4864, 896), ("up", 4864, 896), ("down", 896, 4864),
]

# Qwen3.5-style INT4 layer linears and the tied vocab head.
QWEN35_INT4_LAYER = [("gate", 3584, 1024), ("up", 3584, 1024), ("down", 1024, 3584)]
QWEN35_INT4_HEAD = ("head", 151936, 1024)


def ternary_linear_bytes(N, K, group, M):
    """Algorithmic bytes of one int8-activation ternary linear: codes + fp32 scales + xq and its fp32 scale in
    + fp32 y out."""
    ns = N * ((K + group - 1) // group) if group > 0 else N
    return N * ((K + 3) // 4) + 4 * ns + M * (K + 4) + 4 * M * N


def int_linear_bytes(N, K, bits, M):
    return N * ((K * bits + 7) // 8) + 4 * N + M * (K + 4) + 4 * M * N


# byte value of 4 ternary codes (t0 + 3 t1 + 9 t2 + 27 t3, digit d = value + 1) in the 2-bit packing
_TERN4 = np.array([sum({0: 2, 1: 0, 2: 1}[(v // 3 ** p) % 3] << (2 * p) for p in range(4)) for v in range(81)], np.uint8)


def ternary_packed(key, rows, cols):
    """Packed 2-bit rows [rows, cols/4] of codes uniform over {-1, 0, +1} (cols a multiple of 4): one uniform
    draw in [0, 81) per byte, mapped through the 81 four-code combinations."""
    assert cols % 4 == 0
    return _TERN4[rng(*key).integers(0, 81, size=(rows, cols // 4), dtype=np.uint8)]


def bitnet_config(dim, hidden, n_layers, n_heads, n_kv_heads, head_dim, vocab, seq_len, group_in, group_down,
                  wht_dim, wht_q, wht_hidden, rope_theta=500000.0, rms_eps=None, sub_eps=1e-5):
    """A BitNet-b1.58 decoder configuration (the reference's tinyllm BitNet model, src/eif_tinyllm.c:371-857).

    group_in: ternary group of every matrix whose input is dim or q_dim wide; group_down: of the down projection.
    rms_eps defaults to the reference's choice (1e-6 for vocabularies above 120000, else 1e-5)."""
    def norm(b):
        return float(np.float32(1.0) / np.sqrt(np.float32(b))) if b else 1.0
    return dict(dim=dim, hidden=hidden, n_layers=n_layers, n_heads=n_heads, n_kv_heads=n_kv_heads, head_dim=head_dim,
                vocab=vocab, seq_len=seq_len, rope_theta=rope_theta,
                rms_eps=(1e-6 if vocab > 120000 else 1e-5) if rms_eps is None else rms_eps, sub_eps=sub_eps,
                wht_dim=wht_dim, wht_q=wht_q, wht_hidden=wht_hidden, wht_norm_dim=norm(wht_dim),
                wht_norm_q=norm(wht_q), wht_norm_hidden=norm(wht_hidden),
                g_q=group_in, g_o=group_in, g_13=group_in, g_2=group_down)


# The BitNet-b1.58-2B-shaped decode model: 30 layers of the layer shapes above, WHT-128, g128 (g96 down),
# INT8 vocabulary head 128256 x 2560, context 2048.
BITNET_2B_DECODE = dict(dim=2560, hidden=6912, n_layers=30, n_heads=20, n_kv_heads=5, head_dim=128, vocab=128256,
                        seq_len=2048, group_in=128, group_down=96, wht_dim=128, wht_q=128, wht_hidden=128)


def bitnet_model(key, cfg):
    """Random-init weights of a BitNet decoder in the reference's formats, per-layer arrays concatenated over layers:
    INT8 embedding with per-token scales, 2-bit ternary matrices with grouped FP32 scales, RMSNorm weights, +-1
    rotation signs, INT8 head with per-row scales."""
    d, h, L = cfg["dim"], cfg["hidden"], cfg["n_layers"]
    qd, kvd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    V = cfg["vocab"]
    w = {}
    r = rng(*key, 10)
    w["emb"] = r.integers(-127, 128, size=(V, d), dtype=np.int8)
    w["emb_scale"] = (np.abs(rng(*key, 11).standard_normal(V)) * 0.01 + 0.01).astype(np.float32)
    shapes = {"q": (qd, d, cfg["g_q"]), "k": (kvd, d, cfg["g_q"]), "v": (kvd, d, cfg["g_q"]), "o": (d, qd, cfg["g_o"]),
              "1": (h, d, cfg["g_13"]), "3": (h, d, cfg["g_13"]), "2": (d, h, cfg["g_2"])}
    for i, (name, (N, K, g)) in enumerate(shapes.items()):
        w["w" + name] = ternary_packed((*key, 20 + i), L * N, K)
        ng = -(-K // g) if g else 1   # g = 0: one scale per row
        w["g" + name] = (np.abs(rng(*key, 30 + i).standard_normal((L * N, ng))) * 0.02 + 0.005).astype(np.float32)
    for i, (name, n) in enumerate((("rms_att", d), ("rms_ffn", d), ("rms_sub_att", qd), ("rms_sub_ffn", h))):
        w[name] = (1.0 + 0.1 * rng(*key, 40 + i).standard_normal(L * n)).astype(np.float32)
    w["rms_final"] = (1.0 + 0.1 * rng(*key, 45).standard_normal(d)).astype(np.float32)
    for i, (name, n) in enumerate((("signs_dim", d), ("signs_q", qd), ("signs_hidden", h))):
        w[name] = np.where(rng(*key, 50 + i).uniform(size=n) < 0.5, -1.0, 1.0).astype(np.float32)
    w["wcls"] = rng(*key, 60).integers(-127, 128, size=(V, d), dtype=np.int8)
    w["wcls_scale"] = (np.abs(rng(*key, 61).standard_normal(V)) * 0.01 + 0.002).astype(np.float32)
    return w
