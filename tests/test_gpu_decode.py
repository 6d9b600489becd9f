"""The GPU BitNet decoder (include/eif_hip_decode.h) against the decode oracle's INT8-activation form.

Before each step the oracle is given the token and the KV cache the GPU holds (teacher forcing), so each
comparison covers one step. The GPU sums RMSNorm, attention and softmax in another order than the oracle, so
now and then an activation that sits on an int8 rounding boundary takes the neighbouring code: on these models
the oracle's own logits move by up to 2.3% of their largest magnitude for a 3e-7 relative change of one norm
weight. Per step the logits agree to 3e-2 of their largest magnitude with a correlation above 0.9995; over a
run, the median step agrees to 2e-3. The greedy token agrees wherever the oracle's top-two margin exceeds the
step's bound. A captured step replayed as a HIP graph gives the eager step's bits.
"""
import ctypes as C
import os
import sys

import numpy as np
import pytest

from conftest import ROOT, P

sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
import synth  # noqa: E402
import model_files  # noqa: E402
import oracle_api  # noqa: E402
import make_golden  # noqa: E402

pytestmark = pytest.mark.gpu
REL, REL_MEDIAN = 3e-2, 2e-3


class OracleRun:
    def __init__(self, oracle, cfg, w):
        self.oracle, self.cfg = oracle, cfg
        self.c, self.ws = oracle_api.bitnet_structs(cfg, w)
        kv = cfg["n_kv_heads"] * cfg["head_dim"]
        self.kc = np.zeros((cfg["n_layers"], cfg["seq_len"], kv), np.float32)
        self.vc = np.zeros_like(self.kc)

    def step(self, tok, pos):
        lo = np.zeros(self.cfg["vocab"], np.float32)
        assert self.oracle.orc_bitnet_forward(C.byref(self.c), C.byref(self.ws), P(self.kc), P(self.vc), int(tok), pos,
                                              oracle_api.ORC_LIN_INT8, P(lo)) == 0
        return lo


def compare_steps(gpu, oracle, cfg, w, prompt, n_steps, graph, prefill=0, oracle_cfg=None):
    m = gpu.BitnetModel(cfg, w)
    orc = OracleRun(oracle, oracle_cfg or cfg, w)
    try:
        m.reset(prompt)
        if prefill:
            m.prefill(prefill)
        errs = []
        for pos in range(prefill, n_steps):
            for layer in range(cfg["n_layers"]):       # the GPU's cache for the positions before this step
                if pos > 0:
                    orc.kc[layer, :pos], orc.vc[layer, :pos] = m.kv_cache(layer, 0, pos)
            m.steps(1, graph=graph)
            lg = m.logits()
            seq = m.tokens(pos + 2)
            lo = orc.step(seq[pos], pos)
            err = np.abs(lg - lo).max() / np.abs(lo).max()
            errs.append(err)
            assert err <= REL and np.corrcoef(lg, lo)[0, 1] > 0.9995, (pos, err)
            if pos + 1 >= len(prompt):
                assert seq[pos + 1] == int(np.argmax(lg))
                top2 = np.sort(lo)[-2:]
                if top2[1] - top2[0] > 2 * err * np.abs(lo).max() + 1e-6:   # a clear winner: the same token
                    assert seq[pos + 1] == int(np.argmax(lo)), pos
            else:
                assert seq[pos + 1] == prompt[pos + 1]
        assert np.median(errs) <= REL_MEDIAN, errs
        assert m.position() == n_steps
        return m.tokens(n_steps + 1), m.logits()
    finally:
        m.close()


def tiny():
    cfg = make_golden.decode_config()
    return cfg, synth.bitnet_model(make_golden.DECODE_KEY, cfg)


def test_decode_tiny_vs_oracle(gpu, oracle):
    cfg, w = tiny()
    compare_steps(gpu, oracle, cfg, w, [5], 16, graph=False)


def test_decode_prompt_then_greedy(gpu, oracle):
    cfg, w = tiny()
    prompt = list(np.random.default_rng(3).integers(0, cfg["vocab"], 10))
    toks, _ = compare_steps(gpu, oracle, cfg, w, prompt, 20, graph=False)
    assert list(toks[:10]) == prompt


def test_decode_head128_gqa(gpu, oracle):
    # head_dim 128, 4 query heads per kv head, g128 inputs / g96 down, WHT-128 everywhere, two 64-token prompts
    cfg = synth.bitnet_config(512, 768, 3, 8, 2, 128, 1000, 96, 128, 96, 128, 128, 128)
    w = synth.bitnet_model((8,), cfg)
    prompt = list(np.random.default_rng(4).integers(0, cfg["vocab"], 64))
    compare_steps(gpu, oracle, cfg, w, prompt, 80, graph=False)


def test_decode_long_context_shares(gpu, oracle):
    # head_dim 128: attention chunks of 128 positions up to position 1023 (eight shares at 1016..1023), then of
    # 256 (position 1024 alone in the fifth chunk); graph replays across the change of chunk length
    cfg = synth.bitnet_config(512, 768, 2, 8, 2, 128, 1000, 1280, 128, 96, 128, 128, 128)
    w = synth.bitnet_model((21,), cfg)
    prompt = list(np.random.default_rng(22).integers(0, cfg["vocab"], 1040))
    compare_steps(gpu, oracle, cfg, w, prompt, 1030, graph=True, prefill=1016)


def test_decode_shares_head64(gpu, oracle):
    # head_dim 64: chunks of 256 positions, the second chunk starting at position 256
    cfg = synth.bitnet_config(256, 512, 2, 4, 2, 64, 500, 320, 64, 64, 64, 64, 128)
    w = synth.bitnet_model((23,), cfg)
    prompt = list(np.random.default_rng(24).integers(0, cfg["vocab"], 270))
    compare_steps(gpu, oracle, cfg, w, prompt, 262, graph=False, prefill=250)


def test_decode_big_vocab_head(gpu, oracle):
    # a 70000-token INT8 head (4375 row tiles): the vocabulary-sized head path (one prep launch, then the GEMV
    # with per-tile maxima over 4375 tiles) against the oracle
    cfg = synth.bitnet_config(128, 256, 1, 4, 2, 32, 70000, 32, 32, 32, 128, 128, 256)
    w = synth.bitnet_model((25,), cfg)
    prompt = [11, 69999, 123]
    compare_steps(gpu, oracle, cfg, w, prompt, 10, graph=False)


def test_decode_row_scales(gpu, oracle):
    # one scale per ternary row (group 0 on the GPU, one group spanning the input in the oracle)
    cfg = make_golden.decode_config()
    for k in ("g_q", "g_o", "g_13", "g_2"):
        cfg[k] = 0
    w = synth.bitnet_model((13,), cfg)
    ocfg = dict(cfg, g_q=cfg["dim"], g_o=cfg["n_heads"] * cfg["head_dim"], g_13=cfg["dim"], g_2=cfg["hidden"])
    prompt = list(np.random.default_rng(9).integers(0, cfg["vocab"], 6))
    compare_steps(gpu, oracle, cfg, w, prompt, 16, graph=False, prefill=4, oracle_cfg=ocfg)


def test_decode_graph_equals_eager(gpu, oracle):
    cfg, w = tiny()
    prompt = [7, 11, 13]
    m = gpu.BitnetModel(cfg, w)
    try:
        m.reset(prompt)
        m.steps(20, graph=False)
        eager_t, eager_l = m.tokens(21), m.logits()
        m.reset(prompt)
        m.steps(5, graph=True)
        m.steps(15, graph=True)
        graph_t, graph_l = m.tokens(21), m.logits()
    finally:
        m.close()
    assert np.array_equal(eager_t, graph_t)
    assert np.array_equal(eager_l.view(np.uint32), graph_l.view(np.uint32))


def test_decode_limits(gpu):
    cfg, w = tiny()
    m = gpu.BitnetModel(cfg, w)
    try:
        with pytest.raises(gpu.HipError):
            m.reset([cfg["vocab"]])            # token out of range
        m.reset([1])
        m.steps(cfg["seq_len"])
        with pytest.raises(gpu.HipError):
            m.steps(1)                         # past the context
    finally:
        m.close()


def test_decode_api_order(gpu):
    """Steps before the first reset have no position or token and are refused before any launch; a layer's
    weights are set once."""
    cfg, w = tiny()
    m = gpu.BitnetModel(cfg, w)
    try:
        with pytest.raises(gpu.HipError):
            m.steps(1)
        lib = gpu.load()
        d, L = cfg["dim"], cfg["n_layers"]
        qd, kvd, hid = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"], cfg["hidden"]
        rows = {"q": qd, "k": kvd, "v": kvd, "o": d, "1": hid, "3": hid, "2": d}
        f = {}
        for k, n in rows.items():
            f["w" + k] = np.ascontiguousarray(w["w" + k]).reshape(L, n, -1)[0].ctypes.data
            f["g" + k] = np.ascontiguousarray(w["g" + k]).reshape(L, n, -1)[0].ctypes.data
        assert lib.eif_hip_bitnet_set_layer(m.h, 0, C.byref(gpu.BitnetLayer(**f))) == gpu.E_ARG
        m.reset([3])
        m.steps(2)
        assert m.position() == 2
    finally:
        m.close()


def test_decode_bitnet2b_width(gpu, oracle):
    """Two layers at the full width of the BitNet-b1.58-2B-shaped model (dim 2560, FFN 6912, 20 query and 5 KV
    heads of 128, g128 / g96 down, WHT-128, the 128256-row INT8 head, context 2048) under the tight bounds of the
    small models: a 513-token prompt, 512 positions prefilled as one batch, then teacher-forced steps at positions
    512..519 (the 20-head shares-combining O projection over five-chunk attention, the 6912-wide SiLU-gate prep,
    the argmax over 8016 head tiles), greedy tokens against the oracle's, graph replays against eager."""
    c = dict(synth.BITNET_2B_DECODE, n_layers=2)
    cfg = synth.bitnet_config(**c)
    w = synth.bitnet_model((33,), cfg)
    prompt = [int(t) for t in np.random.default_rng(34).integers(0, cfg["vocab"], 513)]
    toks, _ = compare_steps(gpu, oracle, cfg, w, prompt, 520, graph=True, prefill=512)
    assert list(toks[:513]) == prompt


def _rrms(a, b):
    return float(np.sqrt(np.mean((a - b) ** 2)) / np.sqrt(np.mean(b ** 2)))


def _rmax(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


class Sensitivity:
    """The oracle's own spread under perturbations the size of a summation-order change: every RMSNorm weight
    times (1 + 2^-23), every RMSNorm weight times (1 - 2^-24), every embedding scale times (1 + 2^-23). Through a
    deep INT8-activation stack such a change flips activations that sit on an int8 rounding boundary, and the
    flips compound layer by layer; the GPU, which sums norms and softmaxes in another order, is held to a small
    multiple of that spread, per layer, pooled over the checked positions."""

    FACTORS = ((("rms_att", "rms_ffn", "rms_sub_att", "rms_sub_ffn", "rms_final"), 1 + 2.0 ** -23),
               (("rms_att", "rms_ffn", "rms_sub_att", "rms_sub_ffn", "rms_final"), 1 - 2.0 ** -24),
               (("emb_scale",), 1 + 2.0 ** -23))

    def __init__(self, oracle, cfg, w):
        self.runs = []
        for keys, f in self.FACTORS:
            wp = dict(w)
            for k in keys:
                wp[k] = (w[k] * np.float32(f)).astype(np.float32)
            self.runs.append((OracleRun(oracle, cfg, wp), wp))
        L = cfg["n_layers"]
        self.kv_rms, self.kv_max = np.zeros(L), np.zeros(L)
        self.lg_rms, self.lg_max = 0.0, 0.0

    def add(self, orc, token, pos, lo):
        """One position: each perturbed oracle run from the cache orc holds; the spread against orc's outputs."""
        L = len(self.kv_rms)
        for run, _ in self.runs:
            run.kc[:, :pos], run.vc[:, :pos] = orc.kc[:, :pos], orc.vc[:, :pos]
            lp = run.step(token, pos)
            for layer in range(L):
                for got, want in ((run.kc[layer, pos], orc.kc[layer, pos]), (run.vc[layer, pos], orc.vc[layer, pos])):
                    self.kv_rms[layer] = max(self.kv_rms[layer], _rrms(got, want))
                    self.kv_max[layer] = max(self.kv_max[layer], _rmax(got, want))
            self.lg_rms = max(self.lg_rms, _rrms(lp, lo))
            self.lg_max = max(self.lg_max, _rmax(lp, lo))


# GPU deviation <= K_SPREAD x the oracle's own spread at that layer, or the floor where the spread is smaller
K_SPREAD, FLOOR_RMS, FLOOR_MAX = 2.5, 0.02, 0.05


def test_decode_bitnet2b_full_size(gpu, oracle):
    """The 30-layer BitNet-b1.58-2B-shaped decode model at its own shape: dim 2560, FFN 6912, 20 query and 5 KV
    heads of 128, g128 scales (g96 down), WHT-128 before every linear, 128256-row INT8 head, context 2048.

    A 513-token prompt; positions 0..511 prefilled as one batch; then teacher-forced token steps at positions
    512..514 (the prompt's last token, then two greedy tokens). At sampled prefill positions and at every step the
    oracle runs one step from the GPU's cache of the positions before:
      - layer 0's keys and values (before any int8 flip can compound) agree to 1e-3 of their largest magnitude
        (fp16 rounding of the cache);
      - every layer's keys and values, and the logits, deviate from the oracle's by at most K_SPREAD times the
        oracle's own spread under 1-ulp perturbations at that layer (Sensitivity), or a floor (2% rms, 5% max);
        a mistake planted in the oracle (two KV heads' key rows swapped in one layer) must exceed that bound;
      - each greedy token is the first maximum of the returned logits, and the oracle's where its top-two margin
        exceeds the step's deviation;
    the same steps replayed as a HIP graph after a second prefill give the eager bits."""
    cfg = synth.bitnet_config(**synth.BITNET_2B_DECODE)
    w = synth.bitnet_model((31,), cfg)
    prompt = [int(t) for t in np.random.default_rng(32).integers(0, cfg["vocab"], 513)]
    L, n = cfg["n_layers"], 512
    m = gpu.BitnetModel(cfg, w)
    orc = OracleRun(oracle, cfg, w)
    sens = Sensitivity(oracle, cfg, w)
    dev = []   # (pos, layer, K or V, rms, max) of the GPU against the oracle

    def record(pos, kv_at):
        for layer in range(L):
            for name, got, want in (("K", kv_at[layer][0], orc.kc[layer, pos]), ("V", kv_at[layer][1], orc.vc[layer, pos])):
                dev.append((pos, layer, name, _rrms(got, want), _rmax(got, want)))
                if layer == 0:
                    assert _rmax(got, want) <= 1e-3, (pos, name, _rmax(got, want))

    try:
        m.reset(prompt)
        m.prefill(n)
        assert m.position() == n
        kv = [m.kv_cache(layer, 0, n) for layer in range(L)]
        pre_lg = m.logits()
        lg_dev = []
        for p in (0, 255, 511):
            for layer in range(L):
                orc.kc[layer, :p], orc.vc[layer, :p] = kv[layer][0][:p], kv[layer][1][:p]
            lo = orc.step(prompt[p], p)
            sens.add(orc, prompt[p], p, lo)
            record(p, [(kv[layer][0][p], kv[layer][1][p]) for layer in range(L)])
        lg_dev.append((_rrms(pre_lg, lo), _rmax(pre_lg, lo)))
        # a planted mistake: the oracle with the key rows of layer 7's first two KV heads swapped (a wrong head
        # index; every other array the same)
        wbad = dict(w)
        kvd, hd = cfg["n_kv_heads"] * cfg["head_dim"], cfg["head_dim"]
        wk = np.ascontiguousarray(w["wk"]).reshape(L * kvd, -1).copy()
        gk = np.ascontiguousarray(w["gk"]).reshape(L * kvd, -1).copy()
        r0 = 7 * kvd
        for a in (wk, gk):
            a[r0:r0 + 2 * hd] = np.concatenate([a[r0 + hd:r0 + 2 * hd], a[r0:r0 + hd]])
        wbad["wk"], wbad["gk"] = wk.reshape(w["wk"].shape), gk.reshape(w["gk"].shape)
        bad = OracleRun(oracle, cfg, wbad)
        bad.kc[:, :255], bad.vc[:, :255] = orc.kc[:, :255], orc.vc[:, :255]
        bad.step(prompt[255], 255)
        for pos in (512, 513, 514):
            for layer in range(L):
                orc.kc[layer, :pos], orc.vc[layer, :pos] = m.kv_cache(layer, 0, pos)
            m.steps(1, graph=False)
            lg = m.logits()
            seq = m.tokens(pos + 2)
            lo = orc.step(seq[pos], pos)
            sens.add(orc, seq[pos], pos, lo)
            record(pos, [tuple(a[0] for a in m.kv_cache(layer, pos, 1)) for layer in range(L)])
            lg_dev.append((_rrms(lg, lo), _rmax(lg, lo)))
            assert seq[pos + 1] == int(np.argmax(lg)), pos          # greedy = first maximum of the logits
            top2 = np.sort(lo)[-2:]
            if top2[1] - top2[0] > 2 * _rmax(lg, lo) * np.abs(lo).max() + 1e-6:
                assert seq[pos + 1] == int(np.argmax(lo)), pos
        for pos, layer, name, r, mx in dev:
            assert r <= max(K_SPREAD * sens.kv_rms[layer], FLOOR_RMS), (pos, layer, name, r, sens.kv_rms[layer])
            assert mx <= max(K_SPREAD * sens.kv_max[layer], FLOOR_MAX), (pos, layer, name, mx, sens.kv_max[layer])
        for r, mx in lg_dev:
            assert r <= max(K_SPREAD * sens.lg_rms, FLOOR_RMS), (r, sens.lg_rms)
            assert mx <= max(K_SPREAD * sens.lg_max, FLOOR_MAX), (mx, sens.lg_max)
        # the bound separates a real mistake from rounding: the planted one exceeds it at layer 7
        over = _rrms(bad.kc[7, 255], kv[7][0][255]) / max(K_SPREAD * sens.kv_rms[7], FLOOR_RMS)
        assert over > 1.0, over
        eager_t, eager_l = m.tokens(n + 4), m.logits()
        m.reset(prompt)
        m.prefill(n)
        m.steps(3, graph=True)
        graph_t, graph_l = m.tokens(n + 4), m.logits()
        assert np.array_equal(eager_t, graph_t)
        assert np.array_equal(eager_l.view(np.uint32), graph_l.view(np.uint32))
    finally:
        m.close()


def run_path(m, prompt, prefill, n_steps, persistent, graph):
    """Prefill, then n_steps token steps on one path; the sequence, last logits and every layer's KV cache."""
    L = m.cfg["n_layers"]
    m.set_persistent(persistent)
    m.reset(prompt)
    if prefill:
        m.prefill(prefill)
    m.steps(n_steps, graph=graph)
    n = prefill + n_steps
    return m.tokens(n + 1), m.logits(), [m.kv_cache(layer, 0, n) for layer in range(L)]


def assert_same_bits(a, b):
    ta, la, kva = a
    tb, lb, kvb = b
    assert np.array_equal(ta, tb)
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    for (ka, va), (kb, vb) in zip(kva, kvb):
        assert np.array_equal(ka.view(np.uint32), kb.view(np.uint32))
        assert np.array_equal(va.view(np.uint32), vb.view(np.uint32))


def test_persistent_step_same_bits(gpu):
    """The persistent token step (one launch for the layer stack) against the separate launches: the same tokens,
    logits and KV cache bits, eagerly and replayed as a graph, over attention chunks of 128 positions and across
    the change to 256 at position 1024 (head_dim 128, g128 inputs, g96 down, WHT-128, 8/2 heads)."""
    cfg = synth.bitnet_config(512, 768, 3, 8, 2, 128, 1000, 1280, 128, 96, 128, 128, 128)
    w = synth.bitnet_model((41,), cfg)
    prompt = list(np.random.default_rng(42).integers(0, cfg["vocab"], 1020))
    m = gpu.BitnetModel(cfg, w)
    try:
        assert m.set_persistent(True)
        sep = run_path(m, prompt, 1000, 40, False, graph=False)
        per = run_path(m, prompt, 1000, 40, True, graph=False)
        assert_same_bits(sep, per)
        per_g = run_path(m, prompt, 1000, 40, True, graph=True)
        assert_same_bits(sep, per_g)
        short = run_path(m, prompt[:5], 0, 30, True, graph=True)   # from position 0, one chunk
        assert_same_bits(run_path(m, prompt[:5], 0, 30, False, graph=False), short)
    finally:
        m.close()


def test_persistent_step_bitnet2b_same_bits(gpu):
    """The persistent step of the 30-layer BitNet-b1.58-2B-shaped model (dim 2560, FFN 6912, 20/5 heads x 128,
    g128 / g96 down, 128256-row INT8 head, context 2048) gives the separate launches' bits after a 512-token
    prefill: 16 greedy tokens, the last logits and all 30 layers' KV caches."""
    cfg = synth.bitnet_config(**synth.BITNET_2B_DECODE)
    w = synth.bitnet_model((31,), cfg)
    prompt = [int(t) for t in np.random.default_rng(32).integers(0, cfg["vocab"], 513)]
    m = gpu.BitnetModel(cfg, w)
    try:
        assert m.set_persistent(True)
        sep = run_path(m, prompt, 512, 16, False, graph=True)
        per = run_path(m, prompt, 512, 16, True, graph=True)
        assert_same_bits(sep, per)
    finally:
        m.close()


def test_persistent_unsupported_shapes_fall_back(gpu):
    """Shapes outside the persistent kernel (head_dim 32, g32) keep the separate launches."""
    cfg, w = tiny()
    m = gpu.BitnetModel(cfg, w)
    try:
        assert not m.set_persistent(True)
        m.reset([3])
        m.steps(3)
        assert m.position() == 3
    finally:
        m.close()


def check_prefill(gpu, oracle, cfg, w, prompt, chunks):
    """Prefill in the given chunks; every prompt position checked one step at a time against the oracle given
    the GPU's cache of the positions before it: that position's keys and values in every layer and, at the
    last position, the logits and the next token."""
    m = gpu.BitnetModel(cfg, w)
    orc = OracleRun(oracle, cfg, w)
    L, n = cfg["n_layers"], sum(chunks)
    try:
        m.reset(prompt)
        for c in chunks:
            m.prefill(c)
        assert m.position() == n
        seq = m.tokens(n + 1)
        assert list(seq[:n]) == list(prompt[:n])
        kv = [m.kv_cache(layer, 0, n) for layer in range(L)]
        lg = m.logits()
        kv_errs = []
        for p in range(n):
            for layer in range(L):
                orc.kc[layer, :p], orc.vc[layer, :p] = kv[layer][0][:p], kv[layer][1][:p]
            lo = orc.step(prompt[p], p)
            for layer in range(L):
                for got, want in ((kv[layer][0][p], orc.kc[layer, p]), (kv[layer][1][p], orc.vc[layer, p])):
                    e = np.abs(got - want).max() / np.abs(want).max()
                    kv_errs.append(e)
                    assert e <= REL, (p, layer, e)
        assert np.median(kv_errs) <= REL_MEDIAN, kv_errs
        err = np.abs(lg - lo).max() / np.abs(lo).max()
        assert err <= REL and np.corrcoef(lg, lo)[0, 1] > 0.9995, err
        if n < len(prompt):
            assert seq[n] == prompt[n]
        else:
            assert seq[n] == int(np.argmax(lg))
        return m.logits()
    finally:
        m.close()


def test_prefill_tiny(gpu, oracle):
    cfg, w = tiny()
    prompt = list(np.random.default_rng(5).integers(0, cfg["vocab"], 20))
    check_prefill(gpu, oracle, cfg, w, prompt, [20])          # the whole prompt, GEMM path (M >= 16)
    check_prefill(gpu, oracle, cfg, w, prompt, [5, 3, 9])     # chunks below the GEMM threshold, stops early


def test_prefill_head128_gqa(gpu, oracle):
    cfg = synth.bitnet_config(512, 768, 3, 8, 2, 128, 1000, 96, 128, 96, 128, 128, 128)
    w = synth.bitnet_model((8,), cfg)
    prompt = list(np.random.default_rng(6).integers(0, cfg["vocab"], 70))
    check_prefill(gpu, oracle, cfg, w, prompt, [64, 6])


def test_prefill_long_split(gpu, oracle):
    # causal ranges longer than one attention workgroup's (8 tiles of 16 keys) are split and combined: 200 tokens
    # in one batch, then as two batches of 100 (the second starting mid-tile, where a share may hold no key a
    # query sees)
    cfg = synth.bitnet_config(512, 768, 2, 8, 2, 128, 1000, 300, 128, 96, 128, 128, 128)
    w = synth.bitnet_model((26,), cfg)
    prompt = list(np.random.default_rng(27).integers(0, cfg["vocab"], 201))
    check_prefill(gpu, oracle, cfg, w, prompt, [200])
    check_prefill(gpu, oracle, cfg, w, prompt, [100, 100])


def test_prefill_then_greedy(gpu, oracle):
    cfg, w = tiny()
    prompt = list(np.random.default_rng(7).integers(0, cfg["vocab"], 12))
    toks, _ = compare_steps(gpu, oracle, cfg, w, prompt, 24, graph=True, prefill=12)
    assert list(toks[:12]) == prompt


def test_prefill_limits(gpu):
    cfg, w = tiny()
    m = gpu.BitnetModel(cfg, w)
    try:
        m.reset([1, 2, 3])
        with pytest.raises(gpu.HipError):
            m.prefill(4)                       # past the prompt
        with pytest.raises(gpu.HipError):
            m.prefill(0)
        m.prefill(3)
        assert m.position() == 3
        with pytest.raises(gpu.HipError):
            m.prefill(1)                       # the prompt is consumed
    finally:
        m.close()


@pytest.mark.parametrize("bound,group", [(32, 32), (0, 0)])
def test_svlm_file_equals_in_memory(gpu, tmp_path, bound, group):
    """A model read from an SVLM file (eif_hip_bitnet_load_svlm) decodes bit for bit as the same arrays set in
    memory with the configuration the reader derives (theta 100000, tinyllm's rotation blocks and groups)."""
    cfg = make_golden.decode_config()
    cfg["rope_theta"] = 100000.0
    for k in ("g_q", "g_o", "g_13", "g_2"):
        cfg[k] = group
    for k, b in (("wht_norm_dim", "wht_dim"), ("wht_norm_q", "wht_q"), ("wht_norm_hidden", "wht_hidden")):
        cfg[k] = gpu.wht_norm(cfg[b])
    w = synth.bitnet_model((12, group), cfg)
    path = str(tmp_path / "model.svlm")
    model_files.write_svlm(path, cfg, w, bound)
    mf = gpu.BitnetModel.from_svlm(path)
    mm = gpu.BitnetModel(cfg, w)
    try:
        for k in ("dim", "hidden", "n_layers", "n_heads", "n_kv_heads", "head_dim", "vocab", "seq_len", "wht_dim",
                  "wht_q", "wht_hidden", "g_q", "g_o", "g_13", "g_2"):
            assert mf.cfg[k] == cfg[k], k
        assert mf.weight_bytes() == mm.weight_bytes()
        prompt = [3, 141, 59, 26]
        out = []
        for m in (mf, mm):
            m.reset(prompt)
            m.prefill(3)
            m.steps(9, graph=True)
            out.append((m.tokens(13), m.logits()))
        assert np.array_equal(out[0][0], out[1][0])
        assert np.array_equal(out[0][1].view(np.uint32), out[1][1].view(np.uint32))
    finally:
        mf.close()
        mm.close()


@pytest.mark.parametrize("head_dim", [32, 64])
def test_ttml_file_equals_in_memory(gpu, tmp_path, head_dim):
    """A TTML file (one scale per row, no rotation; head_dim 64 is set apart from dim / heads, which packs the
    per-layer attention scales) read by eif_hip_bitnet_load_svlm decodes bit for bit as the same arrays set in
    memory, with the RoPE theta the file carries."""
    cfg = synth.bitnet_config(128, 256, 2, 4, 2, head_dim, 300, 32, 0, 0, 0, 0, 0, rope_theta=10000.0)
    w = synth.bitnet_model((14, head_dim), cfg)
    path = str(tmp_path / "model.ttml")
    model_files.write_ttml(path, cfg, w)
    mf = gpu.BitnetModel.from_svlm(path)
    mm = gpu.BitnetModel(cfg, w)
    try:
        for k in ("dim", "hidden", "n_layers", "n_heads", "n_kv_heads", "head_dim", "vocab", "seq_len", "wht_dim",
                  "wht_q", "wht_hidden", "g_q", "g_o", "g_13", "g_2"):
            assert mf.cfg[k] == cfg[k], k
        prompt = [3, 141, 59, 26]
        out = []
        for m in (mf, mm):
            m.reset(prompt)
            m.prefill(3)
            m.steps(9, graph=True)
            out.append((m.tokens(13), m.logits()))
        assert np.array_equal(out[0][0], out[1][0])
        assert np.array_equal(out[0][1].view(np.uint32), out[1][1].view(np.uint32))
    finally:
        mf.close()
        mm.close()


def test_svlm_rejects(gpu, tmp_path):
    cfg, w = tiny()
    path = tmp_path / "m.svlm"
    model_files.write_svlm(str(path), cfg, w, 32)
    raw = bytearray(path.read_bytes())
    bad = tmp_path / "bad.svlm"
    raw[48 + 12 * 4] = 1                      # qtype INT8: not a BitNet file
    bad.write_bytes(bytes(raw))
    with pytest.raises(gpu.HipError):
        gpu.BitnetModel.from_svlm(str(bad))
    bad.write_bytes(path.read_bytes()[:1000])  # truncated
    with pytest.raises(gpu.HipError):
        gpu.BitnetModel.from_svlm(str(bad))
    with pytest.raises(gpu.HipError):
        gpu.BitnetModel.from_svlm(str(tmp_path / "missing.svlm"))


def _same_decode(models):
    prompt = [3, 141, 59, 26]
    out = []
    for m in models:
        m.reset(prompt)
        m.prefill(3)
        m.steps(9, graph=True)
        out.append((m.tokens(13), m.logits()))
    return out


GGUF_CASES = {   # (dim, hidden, layers, heads, kv heads, head_dim), writer options
    "tl1_f16emb_tied": ((128, 256, 2, 4, 2, 32), dict(proj_types=(model_files.GGUF_TL1,), emb_type=model_files.GGUF_F16)),
    "mixed_q8head": ((96, 224, 2, 3, 1, 32), dict(proj_types=(model_files.GGUF_TL1, model_files.GGUF_Q8_0, model_files.GGUF_TL2),
                                                  emb_type=model_files.GGUF_F32, head_type=model_files.GGUF_Q8_0, alignment=64)),
    "hd_apart_f16head": ((128, 256, 2, 4, 2, 64), dict(proj_types=(model_files.GGUF_TL2,), emb_type=model_files.GGUF_Q8_0,
                                                       head_type=model_files.GGUF_F16, key_length=True)),
    "q4k_emb_q6k_head": ((256, 512, 1, 4, 2, 64), dict(proj_types=(model_files.GGUF_TL1,), emb_type=model_files.GGUF_Q4_K,
                                                       head_type=model_files.GGUF_Q6_K, key_length=True)),
    "absmean_projections": ((128, 256, 2, 4, 2, 32), dict(proj_types=(model_files.GGUF_TL1, model_files.GGUF_F32, model_files.GGUF_F16,
                                                                      model_files.GGUF_Q4_0, model_files.GGUF_Q4_1))),
}


@pytest.mark.parametrize("case", sorted(GGUF_CASES))
def test_gguf_file_equals_in_memory(gpu, tmp_path, case):
    """A BitNet GGUF file read by eif_hip_bitnet_load_gguf decodes bit for bit as the arrays eif_gguf_bitnet_open
    converts from it (those are the reference loader's own, tests/test_gguf_model.py) set in memory."""
    shape, kw = GGUF_CASES[case]
    cfg = synth.bitnet_config(*shape, 300, 64, 0, 0, 0, 0, 0, rope_theta=10000.0)
    img, _ = model_files.bitnet_gguf(cfg, (8,), **kw)
    path = tmp_path / "m.gguf"
    path.write_bytes(img)
    g = gpu.GgufBitnet(str(path))
    mcfg, w = g.model()
    g.close()
    mf = gpu.BitnetModel.from_gguf(str(path))
    mm = gpu.BitnetModel(mcfg, w)
    try:
        for k in ("dim", "hidden", "n_layers", "n_heads", "n_kv_heads", "head_dim", "vocab", "seq_len", "g_q",
                  "g_o", "g_13", "g_2", "wht_dim", "wht_q", "wht_hidden"):
            assert mf.cfg[k] == mcfg[k] == (cfg[k] if k in cfg else 0), k
        assert np.float32(mf.cfg["rope_theta"]) == np.float32(10000.0)
        out = _same_decode((mf, mm))
        assert np.array_equal(out[0][0], out[1][0])
        assert np.array_equal(out[0][1].view(np.uint32), out[1][1].view(np.uint32))
    finally:
        mf.close()
        mm.close()


def test_gguf_interleaved_equals_reordered(gpu, tmp_path):
    """A llama-architecture GGUF file (RoPE on interleaved pairs) loads as the bitnet-architecture file of the
    same draws with its q / k rows reordered for half-split pairs, bit for bit (the reference decodes the two as
    one model, tests/test_gguf_model.py); the rows as drawn, half-split, give other logits."""
    from test_gguf_model import interleaved_files
    cfg = synth.bitnet_config(128, 256, 2, 4, 2, 32, 300, 64, 0, 0, 0, 0, 0, rope_theta=10000.0)
    ms = [gpu.BitnetModel.from_gguf(p) for p in interleaved_files(tmp_path, cfg)]
    try:
        out = _same_decode(ms)
        assert np.array_equal(out[0][0], out[1][0])
        assert np.array_equal(out[0][1].view(np.uint32), out[1][1].view(np.uint32))
        assert not np.array_equal(out[0][1], out[2][1])
    finally:
        for m in ms:
            m.close()


def test_ttml_interleaved_equals_reordered(gpu, tmp_path):
    """A TTML file with rope_interleaved set loads as the half-split file whose wq / wk rows (and scales) are
    reordered within each head, bit for bit."""
    cfg = synth.bitnet_config(128, 256, 2, 4, 2, 32, 300, 32, 0, 0, 0, 0, 0, rope_theta=10000.0)
    w = synth.bitnet_model((14, 32), cfg)
    L, hd = cfg["n_layers"], cfg["head_dim"]
    w2 = dict(w)
    for name, heads in (("q", cfg["n_heads"]), ("k", cfg["n_kv_heads"])):
        h = np.arange(L * heads)[:, None] * hd
        order = np.concatenate([h + np.arange(0, hd, 2), h + np.arange(1, hd, 2)], axis=1).ravel()
        w2["w" + name], w2["g" + name] = w["w" + name][order], w["g" + name][order]
    pa, pb = str(tmp_path / "inter.ttml"), str(tmp_path / "split.ttml")
    model_files.write_ttml(pa, cfg, w, interleaved=1)
    model_files.write_ttml(pb, cfg, w2)
    ms = [gpu.BitnetModel.from_svlm(p) for p in (pa, pb)]
    try:
        out = _same_decode(ms)
        assert np.array_equal(out[0][0], out[1][0])
        assert np.array_equal(out[0][1].view(np.uint32), out[1][1].view(np.uint32))
    finally:
        for m in ms:
            m.close()


def test_gguf_load_rejects(gpu, tmp_path):
    cfg = synth.bitnet_config(128, 256, 2, 4, 2, 32, 300, 64, 0, 0, 0, 0, 0, rope_theta=10000.0)
    img, _ = model_files.bitnet_gguf(cfg, (8,))
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(img[:len(img) - 1000])
    with pytest.raises(gpu.HipError):
        gpu.BitnetModel.from_gguf(str(bad))
    with pytest.raises(gpu.HipError):
        gpu.BitnetModel.from_gguf(str(tmp_path / "missing.gguf"))


def test_ttml_rejects(gpu, tmp_path):
    cfg = synth.bitnet_config(128, 256, 2, 4, 2, 32, 300, 32, 0, 0, 0, 0, 0, rope_theta=10000.0)
    w = synth.bitnet_model((14, 32), cfg)
    path = tmp_path / "m.ttml"
    model_files.write_ttml(str(path), cfg, w)
    raw = bytearray(path.read_bytes())
    raw[36 + 4 * 7] = 1                       # qtype INT8: not a BitNet model
    bad = tmp_path / "bad.ttml"
    bad.write_bytes(bytes(raw))
    with pytest.raises(gpu.HipError):
        gpu.BitnetModel.from_svlm(str(bad))
    bad.write_bytes(path.read_bytes()[:2000])  # truncated
    with pytest.raises(gpu.HipError):
        gpu.BitnetModel.from_svlm(str(bad))
