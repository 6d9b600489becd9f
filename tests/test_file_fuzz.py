"""The host-side model-file readers on corrupted inputs (CPU, no GPU): bytes of the header, metadata and tensor
table overwritten at random and files cut at random lengths must each end in a clean refusal (HipError) or a
successful read, never a crash or an unbounded allocation. eif_gguf_bitnet_open (BitNet GGUF),
eif_qwen35_gguf_image (Qwen3.5 GGUF) and eif_qwen35_parse (QWN5 images); seeded, a few hundred cases each."""
import numpy as np
import pytest

import bitllm_hip as bh
import synth
import model_files


def mutations(img, seed, n, span):
    r = np.random.default_rng(seed)
    for _ in range(n):
        b = bytearray(img)
        if r.uniform() < 0.2:
            yield bytes(b[:int(r.integers(0, len(b)))])
            continue
        for _ in range(int(r.integers(1, 4))):
            at = int(r.integers(0, min(span, len(b))))
            b[at] = int(r.integers(0, 256)) if r.uniform() < 0.7 else (0xFF if r.uniform() < 0.5 else 0)
        yield bytes(b)


def test_bitnet_gguf_fuzz(tmp_path):
    cfg = synth.bitnet_config(128, 256, 1, 4, 2, 32, 64, 64, 0, 0, 0, 0, 0, rope_theta=10000.0)
    img, _ = model_files.bitnet_gguf(cfg, (9,), proj_types=(model_files.GGUF_TL1, model_files.GGUF_F16, model_files.GGUF_Q4_0))
    path = tmp_path / "f.gguf"
    ok = 0
    for b in mutations(img, 1, 300, 2600):
        path.write_bytes(b)
        try:
            g = bh.GgufBitnet(str(path))
            ok += 1
            g.close()
        except bh.HipError:
            pass
    assert ok > 0           # some corruptions leave a readable file (e.g. in skipped metadata)


def test_qwen35_gguf_fuzz():
    img = model_files.qwen35_gguf((9,), dim=64, hidden=128, n_heads=2, n_kv_heads=1, head_dim=32, vocab=64, heads_k=2,
                            k_dim=16, v_dim=32, emb_type=model_files.GGUF_F16,
                            lin_types=(model_files.GGUF_Q8_0, model_files.GGUF_F16, model_files.GGUF_Q4_0))
    ok = 0
    for b in mutations(img, 2, 300, 12000):
        try:
            bh.qwen35_gguf_image(b)
            ok += 1
        except bh.HipError:
            pass
    assert ok > 0


def test_qwn5_parse_fuzz():
    from test_qwn5 import make
    _, img, _ = make("tern_g32_hadamard")
    for b in mutations(img, 3, 400, 400):
        try:
            bh.qwen35_parse(b)
        except bh.HipError:
            pass
