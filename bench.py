"""Benchmark of the quantized-linear hot path on one MI355X.

Workload (the headline): the five ternary linears of one BitNet-b1.58-2B-shaped decoder layer at M = 1 token
(QKV 3840x2560, O 2560x2560, gate and up 6912x2560 with g128 scales, down 2560x6912 with g96 scales). One step =
the four activation preps (WHT-128 + INT8) and the five int8-MFMA GEMVs of that layer, all inputs resident in
HBM. Weights rotate over enough copies (> 2x the 256 MB Infinity Cache) that every step streams from HBM.

value = algorithmic bytes of a step / step time (GB/s). The roofline object covers the dominant kernel, the
ternary GEMV: its algorithmic bytes per launch / its average launch duration, timed with HIP events on the stream
the kernels run on. cpu_baseline times the reference's own x86 path for the same layer (WHT + the FP32-activation
grouped GEMV that its engine runs), compiled from its sources into oracle/_ref, on the host cores.

Extra keys report the other workloads: the single 6912x2560 linear, token batches 8/64/512, the INT4 tied head,
the INT8 layer, and a measured device-to-device copy ceiling.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "bitllm.c_amd"))

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="bound on the CPU-baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="headline workload only")
    ap.add_argument("--no-decode", action="store_true", help="skip the 30-layer decode")
    ap.add_argument("--decode-tokens", type=int, default=128)
    ap.add_argument("--decode-prompt", type=int, default=512)
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="also run one device-to-device copy of this many MiB (known bytes for counter calibration)")
    return ap.parse_args()


def measured_traffic():
    """HBM bytes of one layer step from the committed counter runs of this workload (None if absent)."""
    path = os.path.join(ROOT, "profiles", "qgemv_bitnet2b_layer_m1_hbm_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
        return sum(v["read"] + v["write"] for v in rec["per_launch_bytes"].values())
    except (OSError, ValueError, KeyError):
        return None


class Timer:
    """Seconds per call of fn(i), i = 0..n-1, launched back to back.

    The n calls are captured once into a HIP graph and the graph is replayed; HIP events recorded on the stream
    the graph runs on bracket the replays, so host-side enqueue cost is excluded and the figure is the device time
    of the launches including the gaps between them. eager=True times plain launches from Python instead."""

    def __init__(self, torch):
        self.torch = torch
        self.cs = None   # the capture stream, one for all timings (its workspaces are reused)

    def __call__(self, fn, n, replays=5, eager=False):
        t = self.torch
        s = t.cuda.current_stream()
        a, b = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        if eager:
            t.cuda.synchronize()
            a.record(s)
            for i in range(n):
                fn(i)
            b.record(s)
            b.synchronize()
            return a.elapsed_time(b) / n * 1e-3
        # one eager call on the capture stream first: per-stream workspaces are allocated outside capture
        if self.cs is None:
            self.cs = t.cuda.Stream()
        cs = self.cs
        cs.wait_stream(s)
        with t.cuda.stream(cs):
            fn(0)
        cs.synchronize()
        g = t.cuda.CUDAGraph()
        with t.cuda.graph(g, stream=cs):
            for i in range(n):
                fn(i)
        g.replay()
        t.cuda.synchronize()
        a.record(s)
        for _ in range(replays):
            g.replay()
        b.record(s)
        b.synchronize()
        del g
        return a.elapsed_time(b) / (n * replays) * 1e-3


def copies_for(nbytes):
    return max(3, -(-2 * MALL_BYTES // nbytes) + 1)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU; --gpus {args.gpus} is not supported (the path shards by output rows, "
              f"see the design notes, but no multi-GPU run exists)", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    import bitllm_hip as bh
    import synth

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    lib = bh.load()
    bh.check(lib.eif_hip_init(0), "eif_hip_init")
    dev = torch.device("cuda:0")
    timer = Timer(torch)

    # ---------------- headline: BitNet-2B layer, M = 1 ----------------
    # gate and up share their input, so their rows are stacked into one 13824-row weight (one launch), as the
    # reference's fused w1w3 entry point does (src/eif_quantize_bitnet.c:894-942).
    base = {name: synth.ternary_weight((100, i), N, K, g) for i, (name, N, K, g) in enumerate(synth.BITNET_2B_LAYER)}
    base["gateup"] = (np.concatenate([base["gate"][0], base["up"][0]]), np.concatenate([base["gate"][1], base["up"][1]]))
    layer = [("qkv", 3840, 2560, 128), ("o", 2560, 2560, 128), ("gateup", 13824, 2560, 128), ("down", 2560, 6912, 96)]
    layer_w_bytes = sum(synth.ternary_linear_bytes(N, K, g, 0) for _, N, K, g in layer)
    ncopy = copies_for(layer_w_bytes)
    copies = [{name: bh.QWeight(bh.W_TERNARY, N, K, g, *base[name]) for name, N, K, g in layer}
              for _ in range(ncopy)]
    shapes = {name: (N, K, g) for name, N, K, g in layer}

    M = 1
    x_in = {K: torch.from_numpy(synth.activations((101, K), M, K)).to(dev) for K in (2560, 6912)}
    kp = {K: (K + 255) // 256 * 256 for K in (2560, 6912)}
    xq = {K: torch.zeros((M, kp[K]), dtype=torch.int8, device=dev) for K in (2560, 6912)}
    xs = {K: torch.zeros(M, dtype=torch.float32, device=dev) for K in (2560, 6912)}
    y = {name: torch.zeros((M, N), dtype=torch.float32, device=dev) for name, N, K, g in layer}
    norm = bh.wht_norm(128)

    def prep(K):
        bh.prep_rows(x_in[K], xq[K], xs[K], 128, norm)

    def fused(i, name):
        K = shapes[name][1]
        copies[i % ncopy][name].linear_f32(x_in[K], y[name], 128, norm)

    def layer_step(i):
        # FP32 activations in: each launch rotates + quantizes its input row and runs the ternary GEMV
        for name in ("qkv", "o", "gateup", "down"):
            fused(i, name)

    def layer_step_unfused(i):
        w = copies[i % ncopy]
        for name in ("qkv", "o", "gateup", "down"):
            K = shapes[name][1]
            prep(K)
            w[name].linear(xq[K], xs[K], y[name], path=bh.PATH_GEMV)

    def fused_bytes(N, K, g):
        # codes + fp32 group scales + the fp32 activation row in + fp32 outputs
        return N * (K // 4) + 4 * N * (-(-K // g)) + 4 * M * K + 4 * M * N

    step_bytes = sum(fused_bytes(N, K, g) for _, N, K, g in layer)

    for i in range(args.warmup):
        layer_step(i)
    torch.cuda.synchronize()
    eager_sec = timer(layer_step, min(args.steps, 100), eager=True)
    t0 = time.perf_counter()
    sec = timer(layer_step, args.steps, replays=1)
    wall = time.perf_counter() - t0
    value = step_bytes / sec / 1e9
    unfused_sec = timer(layer_step_unfused, args.steps, replays=1)

    # dominant kernel: the fused prep + ternary GEMV, per-linear launch duration over back-to-back launches
    reps = max(50, args.steps)
    per_linear = {}
    for name, (N, K, g) in shapes.items():
        t = timer(lambda i, name=name: fused(i, name), reps)
        per_linear[name] = {"us": t * 1e6, "GBps": fused_bytes(N, K, g) / t / 1e9}
    gemv_time = sum(v["us"] for v in per_linear.values()) * 1e-6
    gemv_gbs = step_bytes / gemv_time / 1e9
    prep_t = timer(lambda i: prep(2560), reps)

    out = {
        "metric": "Ternary/INT4 GEMV HBM GB/s (% of peak); BitNet-2B-shape decode tok/s",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 x ternary -> int32 acc, fp32 scale",
        "data": "synthetic (seeded; random-init weights of the BitNet-b1.58-2B layer shapes)",
        "config": {"workload": "bitnet2b_layer_linears_m1", "tokens": M, "hidden": 2560, "ffn": 6912,
                   "launches": "qkv 3840x2560, o 2560x2560, gate+up 13824x2560 (g128), down 2560x6912 (g96), "
                               "each with its WHT-128 + INT8 prep fused",
                   "weight_copies": ncopy, "step_bytes": step_bytes},
        "roofline": {"bound": "hbm", "achieved": round(gemv_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gemv_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "traffic_unit": "HBM bytes read + written by the 4 launches of one layer step "
                                     "(FETCH_SIZE x2, WRITE_SIZE x1, calibrated on a device copy)",
                     "algorithmic_bytes": step_bytes,
                     "kernel": "qgemv_kernel (prep fused, ternary int8-MFMA GEMV), the 4 launches of a layer",
                     "per_launch": {k: {"us": round(v["us"], 3), "GBps": round(v["GBps"], 1)}
                                    for k, v in per_linear.items()}},
        "prep_us": round(prep_t * 1e6, 3),
        "step_us_unfused_prep_kernel": round(unfused_sec * 1e6, 2),
        "step_us_eager_python_launch": round(eager_sec * 1e6, 2),
        "timing": "HIP graph of the timed steps, replayed; HIP events on its stream",
        "wall_s_timed": round(wall, 3),
    }

    if not args.no_extra:
        out["extra"] = extra_workloads(args, torch, bh, synth, timer, dev, copies, xq, xs, y, x_in, norm)
    if args.calib_copy_mib > 0:
        src = torch.ones(args.calib_copy_mib << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        out["calib_copy_bytes"] = src.numel() * 4
        del src, dst

    for cs in copies:
        for w in cs.values():
            w.close()

    if not args.no_decode:
        out["decode"] = decode_workload(args, torch, bh, synth, np)

    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args, np, synth, step_bytes)
        if out["cpu_baseline"].get("value"):
            out["gpu_over_cpu"] = round(value / out["cpu_baseline"]["value"], 1)
    print(json.dumps(out))


def extra_workloads(args, torch, bh, synth, timer, dev, copies, xq, xs, y, x_in, norm):
    ex = {}
    reps = max(50, args.steps // 2)
    ncopy = len(copies)
    # the single 6912x2560 g128 linear, M = 1: from prepped int8 activations, and with the prep fused
    gw, gs = synth.ternary_weight((100, 2), 6912, 2560, 128)
    single = [bh.QWeight(bh.W_TERNARY, 6912, 2560, 128, gw, gs)
              for _ in range(copies_for(synth.ternary_linear_bytes(6912, 2560, 128, 0)))]
    ys = torch.zeros((1, 6912), dtype=torch.float32, device=dev)
    bh.prep_rows(x_in[2560], xq[2560], xs[2560], 128, norm)
    t = timer(lambda i: single[i % len(single)].linear(xq[2560], xs[2560], ys, path=bh.PATH_GEMV), reps)
    b = synth.ternary_linear_bytes(6912, 2560, 128, 1)
    ex["ternary_6912x2560_g128_m1"] = {"us": round(t * 1e6, 3), "GBps": round(b / t / 1e9, 1)}
    t = timer(lambda i: single[i % len(single)].linear_f32(x_in[2560], ys, 128, norm), reps)
    b = 6912 * 640 + 4 * 6912 * 20 + 4 * 2560 + 4 * 6912
    ex["ternary_6912x2560_g128_m1_prep_fused"] = {"us": round(t * 1e6, 3), "GBps": round(b / t / 1e9, 1)}
    for q in single:
        q.close()

    # token batches through the layer linears (GEMV for M = 8, MFMA GEMM for M >= 64)
    for M in (8, 64, 512):
        xm = {K: torch.from_numpy(synth.activations((102, K, M), M, K)).to(dev) for K in (2560, 6912)}
        qm = {K: torch.zeros((M, (K + 255) // 256 * 256), dtype=torch.int8, device=dev) for K in (2560, 6912)}
        sm = {K: torch.zeros(M, dtype=torch.float32, device=dev) for K in (2560, 6912)}
        for K in (2560, 6912):
            bh.prep_rows(xm[K], qm[K], sm[K], 128, norm)
        ym = {name: torch.zeros((M, w.rows), dtype=torch.float32, device=dev) for name, w in copies[0].items()}

        def lin(i):
            w = copies[i % ncopy]
            for name, q in w.items():
                K = q.cols
                q.linear(qm[K], sm[K], ym[name])
        t = timer(lin, max(20, reps // 4))
        nbytes = sum(synth.ternary_linear_bytes(q.rows, q.cols, q.group, M) for q in copies[0].values())
        ops = sum(2 * q.rows * q.cols * M for q in copies[0].values())
        ex[f"bitnet2b_layer_linears_m{M}"] = {"us": round(t * 1e6, 2), "GBps": round(nbytes / t / 1e9, 1),
                                              "TOPS": round(ops / t / 1e12, 2),
                                              "path": "gemm" if M >= bh.load().eif_hip_gemm_min_tokens() else "gemv"}
        del xm, qm, sm, ym

    # INT4 tied head 151936x1024 (M = 1 and 32) and INT4 FFN linears
    N, K = synth.QWEN35_INT4_HEAD[1:]
    hw, hs = synth.int4_weight((103,), N, K)
    nb = synth.int_linear_bytes(N, K, 4, 1)
    heads = [bh.QWeight(bh.W_INT4, N, K, 0, hw, hs) for _ in range(copies_for(nb))]
    for M in (1, 32):
        xh = torch.from_numpy(synth.activations((104, M), M, K)).to(dev)
        qh = torch.zeros((M, heads[0].kpad), dtype=torch.int8, device=dev)
        sh = torch.zeros(M, dtype=torch.float32, device=dev)
        bh.prep_rows(xh, qh, sh, 0, 1.0)
        yh = torch.zeros((M, N), dtype=torch.float32, device=dev)
        t = timer(lambda i: heads[i % len(heads)].linear(qh, sh, yh), max(20, reps // 2))
        b = synth.int_linear_bytes(N, K, 4, M)
        ex[f"int4_head_151936x1024_m{M}"] = {"us": round(t * 1e6, 2), "GBps": round(b / t / 1e9, 1),
                                              "frac_hbm": round(b / t / 1e9 / HBM_PEAK_GBS, 4)}
    for h in heads:
        h.close()

    # INT8 Qwen2.5-0.5B-like layer, M = 1 and 128
    l8 = synth.QWEN25_05B_LAYER
    base8 = {name: synth.int8_weight((105, i), N, K) for i, (name, N, K) in enumerate(l8)}
    wb8 = sum(synth.int_linear_bytes(N, K, 8, 0) for _, N, K in l8)
    c8 = [{name: bh.QWeight(bh.W_INT8, N, K, 0, *base8[name]) for name, N, K in l8} for _ in range(copies_for(wb8))]
    for M in (1, 128):
        xk = {K: torch.from_numpy(synth.activations((106, K, M), M, K)).to(dev) for K in (896, 4864)}
        qk = {K: torch.zeros((M, (K + 63) // 64 * 64), dtype=torch.int8, device=dev) for K in (896, 4864)}
        sk = {K: torch.zeros(M, dtype=torch.float32, device=dev) for K in (896, 4864)}
        for K in (896, 4864):
            bh.prep_rows(xk[K], qk[K], sk[K], 0, 1.0)
        yk = {name: torch.zeros((M, N), dtype=torch.float32, device=dev) for name, N, K in l8}

        def lin8(i):
            for name, q in c8[i % len(c8)].items():
                q.linear(qk[q.cols], sk[q.cols], yk[name])
        t = timer(lin8, max(20, reps // 4))
        b = sum(synth.int_linear_bytes(N, K, 8, M) for _, N, K in l8)
        ex[f"int8_qwen05b_layer_m{M}"] = {"us": round(t * 1e6, 2), "GBps": round(b / t / 1e9, 1)}
    for cs in c8:
        for q in cs.values():
            q.close()

    # the drop-in host API (host x in, host y out over PCIe; weights resident after the first call), M = 1
    import numpy as np
    lib = bh.load()
    N, K, g = 6912, 2560, 128
    hw, hsc = synth.ternary_weight((107,), N, K, g)
    hx = synth.activations((108,), 1, K)[0]
    hy = np.zeros(N, np.float32)
    call = lambda: lib.eif_matmul_bitnet_block_f32(hw.ctypes.data, hsc.ctypes.data, g, hx.ctypes.data, None,
                                                   hy.ctypes.data, N, K)
    call()
    n = 200
    t0 = time.perf_counter()
    for _ in range(n):
        call()
    t = (time.perf_counter() - t0) / n
    b = N * (K // 4) + 4 * N * (K // g) + 4 * K + 4 * N
    ex["host_api_block_f32_6912x2560_g128_m1"] = {"us": round(t * 1e6, 2), "GBps": round(b / t / 1e9, 1),
                                                  "note": "synchronous call incl. PCIe copies of x and y"}
    lib.eif_hip_forget_host_weights(None)

    # measured copy ceiling: 1 GiB device-to-device copy (read + write bytes)
    src = torch.empty(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    t = timer(lambda i: dst.copy_(src), 10)
    ex["d2d_copy_GBps"] = round(2 * src.numel() * 4 / t / 1e9, 1)
    del src, dst
    return ex


def decode_workload(args, torch, bh, synth, np):
    """Greedy decode on the 30-layer BitNet-b1.58-2B-shaped model (random init): a random-id prompt of
    --decode-prompt tokens, all but the last as one prefill batch (timed on its own), the last prompt token's
    step (the first greedy token; it captures the step graph), then --decode-tokens greedy token steps timed as
    HIP graph replays of the token step. Bytes per token = the resident weights the step reads (ternary codes, group scales, norms, INT8 head)
    + the fp16 KV cache read at that position."""
    c = dict(synth.BITNET_2B_DECODE)
    cfg = synth.bitnet_config(c.pop("dim"), c.pop("hidden"), c.pop("n_layers"), c.pop("n_heads"), c.pop("n_kv_heads"),
                              c.pop("head_dim"), c.pop("vocab"), c.pop("seq_len"), c.pop("group_in"),
                              c.pop("group_down"), c.pop("wht_dim"), c.pop("wht_q"), c.pop("wht_hidden"))
    t0 = time.perf_counter()
    w = synth.bitnet_model((300,), cfg)
    gen_s = time.perf_counter() - t0
    m = bh.BitnetModel(cfg, w)
    npr, ntok = args.decode_prompt, args.decode_tokens
    prompt = synth.rng(301).integers(0, cfg["vocab"], npr).astype(np.int32)
    s = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    m.reset(prompt)
    m.prefill(npr - 1)             # allocates the batch buffers
    m.reset(prompt)
    torch.cuda.synchronize()
    a.record(s)
    m.prefill(npr - 1)             # the prompt but its last token, one batch
    b.record(s)
    b.synchronize()
    pre_sec = a.elapsed_time(b) * 1e-3
    m.steps(1, graph=True)         # the last prompt token (captures the step graph), not timed
    torch.cuda.synchronize()
    a.record(s)
    m.steps(ntok, graph=True)
    b.record(s)
    b.synchronize()
    sec = a.elapsed_time(b) * 1e-3
    toks = m.tokens(npr + ntok + 1)
    assert list(toks[:npr]) == list(prompt)
    wb = m.weight_bytes()
    kv = float(np.mean([m.kv_bytes(p) for p in range(npr, npr + ntok)]))
    per_tok = wb + kv
    res = {"model": "bitnet-b1.58-2B-shaped, 30 layers, dim 2560, ffn 6912, 20/5 heads x 128, vocab 128256 (INT8 head)",
           "prompt": npr, "tokens": ntok, "context": cfg["seq_len"], "kv": "fp16",
           "ms_per_token": round(sec / ntok * 1e3, 4), "tok_per_s": round(ntok / sec, 1),
           "bytes_per_token": int(per_tok), "weight_bytes": int(wb), "GBps": round(per_tok * ntok / sec / 1e9, 1),
           "frac_hbm": round(per_tok * ntok / sec / 1e9 / HBM_PEAK_GBS, 4),
           "launches_per_token": 5 * cfg["n_layers"] + 3, "timing": "HIP graph of one token step, replayed; HIP events",
           "prefill": {"tokens": npr - 1, "ms": round(pre_sec * 1e3, 3), "tok_per_s": round((npr - 1) / pre_sec, 1),
                       "path": "prep + int8-MFMA GEMM per linear over the batch, causal attention on fp32 MFMAs per (kv head, 16-token block)"},
           "weights_generated_s": round(gen_s, 1), "greedy_tail": [int(t) for t in toks[-8:]]}
    m.close()
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_decode_baseline(args, np, synth, cfg, w)
        if res["cpu_baseline"].get("ms_per_token"):
            res["gpu_over_cpu"] = round(res["cpu_baseline"]["ms_per_token"] / res["ms_per_token"], 1)
    return res


def cpu_decode_baseline(args, np, synth, cfg, w):
    """The reference's own tinyllm BitNet decode (oracle/ref_tinyllm_wrap.c over its sources, reference flags) of
    the same weights on the host cores: g128 scales for every matrix (its one group bound cannot give the down
    projection g96 alone; it reads 54 of the 72 scales of each down row), its own WHT blocks (512 / 256),
    fp32 KV cache. A short prompt, then greedy steps for about --cpu-seconds."""
    import ctypes as C
    nthreads = min(16, os.cpu_count() or 1)
    for k, v in (("OMP_NUM_THREADS", str(nthreads)), ("OMP_PROC_BIND", "close"), ("OMP_WAIT_POLICY", "ACTIVE"),
                 ("GOMP_SPINCOUNT", "100000")):
        os.environ.setdefault(k, v)
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle_api
    path = os.path.join(ROOT, "oracle", "_ref", "libref.so")
    if not os.path.exists(path):
        return {"ms_per_token": None, "kind": "none", "sample": "oracle/_ref/libref.so not built"}
    ref = oracle_api.load_ref_tinyllm(path)
    c, ws = oracle_api.bitnet_structs(cfg, w)
    h = ref.ref_bitnet_create(C.byref(c), C.byref(ws), 128)
    if not h:
        return {"ms_per_token": None, "kind": "reference", "sample": "model construction failed"}
    try:
        tok, times, pos = 1, [], 0
        t_end = time.perf_counter() + args.cpu_seconds
        while pos < 64 and (time.perf_counter() < t_end or len(times) < 3):
            t0 = time.perf_counter()
            lp = ref.ref_bitnet_forward(h, tok, pos)
            lo = np.ctypeslib.as_array(lp, shape=(cfg["vocab"],))
            tok = int(np.argmax(lo))
            if pos >= 2:
                times.append(time.perf_counter() - t0)
            pos += 1
    finally:
        ref.ref_bitnet_destroy(h)
    med = float(np.median(times))
    return {"ms_per_token": round(med * 1e3, 2), "tok_per_s": round(1.0 / med, 2), "cores": nthreads,
            "kind": "reference",
            "sample": f"{len(times)} greedy steps at positions 2..{pos - 1}, median; OMP_NUM_THREADS={os.environ['OMP_NUM_THREADS']}"}


def cpu_baseline(args, np, synth, step_bytes):
    """The reference's own x86 path for the same layer step, on the host cores, over a bounded sample."""
    nthreads = min(16, os.cpu_count() or 1)
    os.environ.setdefault("OMP_NUM_THREADS", str(nthreads))
    os.environ.setdefault("OMP_PROC_BIND", "close")
    os.environ.setdefault("OMP_WAIT_POLICY", "ACTIVE")
    os.environ.setdefault("GOMP_SPINCOUNT", "100000")
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ctypes as C
    import oracle_api
    P = oracle_api.P
    ref_so = os.path.join(ROOT, "oracle", "_ref", "libref.so")
    port_so = os.path.join(ROOT, "oracle", "liboracle_port.so")
    if os.path.exists(ref_so):
        lib, kind = oracle_api.load_ref(ref_so), "reference"
        rot = lambda x, n: lib.eif_hadamard_rotate_f32(P(x), None, n, 128)
        gemv = lambda w, s, g, x, yv, N, K: lib.eif_matmul_bitnet_block_f32(P(w), P(s), g, P(x), None, P(yv), N, K)
    elif os.path.exists(port_so):
        lib, kind = oracle_api.load(port_so), "port"
        nrm = lib.orc_wht_norm_fastmath(128)
        rot = lambda x, n: lib.orc_hadamard_rotate(P(x), None, n, 128, C.c_float(nrm))
        gemv = lambda w, s, g, x, yv, N, K: lib.orc_matmul_bitnet_block_f32(P(w), P(s), g, P(x), None, P(yv), N, K)
    else:
        return {"value": None, "unit": "GB/s", "cores": 0, "kind": "none", "sample": "no CPU library built"}
    layer = synth.BITNET_2B_LAYER
    ncp = 6  # ~120 MB of weights, past the host's last-level cache
    ws = [{name: synth.ternary_weight((100, i), N, K, g) for i, (name, N, K, g) in enumerate(layer)}]
    for c in range(1, ncp):
        ws.append({k: (v[0].copy(), v[1].copy()) for k, v in ws[0].items()})
    x0 = {K: synth.activations((101, K), 1, K)[0] for K in (2560, 6912)}
    yv = {name: np.zeros(N, np.float32) for name, N, K, g in layer}

    def step(i):
        w = ws[i % ncp]
        for name, N, K, g in layer:
            if name in ("qkv", "o", "gate", "down"):
                x = x0[K].copy()
                rot(x, K)
            gemv(w[name][0], w[name][1], g, x, yv[name], N, K)

    step(0)
    times = []
    t_end = time.perf_counter() + args.cpu_seconds
    i = 1
    while time.perf_counter() < t_end or len(times) < 5:
        t0 = time.perf_counter()
        step(i)
        times.append(time.perf_counter() - t0)
        i += 1
    med = float(np.median(times))
    return {"value": round(step_bytes / med / 1e9, 2), "unit": "GB/s", "cores": nthreads, "kind": kind,
            "ms_per_step": round(med * 1e3, 3),
            "sample": f"{len(times)} layer steps (WHT-128 + FP32-activation grouped GEMV, the reference x86 path) "
                      f"over {ncp} weight copies, median; OMP_NUM_THREADS={os.environ['OMP_NUM_THREADS']}"}


if __name__ == "__main__":
    main()
