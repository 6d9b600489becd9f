"""Benchmark of the quantized-linear hot path on one MI355X.

Workload (the headline): the five ternary linears of one BitNet-b1.58-2B-shaped decoder layer at M = 1 token
(QKV 3840x2560, O 2560x2560, gate and up 6912x2560 with g128 scales, down 2560x6912 with g96 scales). One step =
the four activation preps (WHT-128 + INT8) and the five int8-MFMA GEMVs of that layer, all inputs resident in
HBM. Weights rotate over enough copies (> 2x the 256 MB Infinity Cache) that every step streams from HBM.

value = algorithmic bytes of a step / step time (GB/s): the K timed steps are captured in one HIP graph (4 launches
per step, 800 at the default K = 200) and the graph is replayed at least 5 times, each replay bracketed by HIP
events on its stream; the step time is the median replay / K. The roofline object covers the dominant kernel, the
ternary GEMV: its algorithmic bytes per launch / its average launch duration, each linear timed over its own weight
copies (> 512 MiB of them, past the 256 MB Infinity Cache). cpu_baseline times the reference's own x86 path for the
same layer (WHT + the FP32-activation grouped GEMV that its engine runs), compiled from its sources into
oracle/_ref, on the host cores (nproc threads, and min(8, nproc)); cpu_legs time the reference functions of the
other configurations the same way.

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

# CPUs this process may run on, read before any OpenMP runtime starts (with OMP_PROC_BIND set, one pins the
# calling thread to a single CPU when it starts).
NPROC = len(os.sched_getaffinity(0))
# The CPU legs run in a child process that imports no torch (torch's OpenMP runtime has the soname the reference
# library binds, and would already be running with the GPU process's settings), with the reference CLI's OpenMP
# settings (cli/main.c:119-125); thread counts are set per leg at run time.
CPU_CHILD_ENV = {"OMP_PROC_BIND": "close", "OMP_WAIT_POLICY": "ACTIVE", "GOMP_SPINCOUNT": "100000"}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--replays", type=int, default=5, help="graph replays of the K timed steps (median taken)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="bound on the CPU-baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="headline workload only")
    ap.add_argument("--no-decode", action="store_true", help="skip the 30-layer decode")
    ap.add_argument("--decode-tokens", type=int, default=128)
    ap.add_argument("--decode-prompt", type=int, default=512)
    ap.add_argument("--cpu-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_DB", "WRITE_DB"),
                    help="no run: write the layer step's HBM traffic file (profiles/) from two rocprofv3 --pmc "
                         "result databases of this script (FETCH_SIZE, then WRITE_SIZE, with --calib-copy-mib)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="also run one device-to-device copy of this many MiB (known bytes for counter calibration)")
    return ap.parse_args()


def source_hash():
    """First 16 hex digits of the sha256 of the library's sources (bitllm.c_amd/csrc/*, its Makefile), names
    and contents in name order: the build a counter file was measured on."""
    import hashlib
    d = os.path.join(ROOT, "bitllm.c_amd")
    names = sorted(os.path.join("csrc", f) for f in os.listdir(os.path.join(d, "csrc"))) + ["Makefile"]
    h = hashlib.sha256()
    for n in names:
        h.update(n.encode())
        with open(os.path.join(d, n), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


TRAFFIC_JSON = os.path.join(ROOT, "profiles", "qgemv_bitnet2b_layer_m1_hbm_traffic.json")


def traffic_from_dbs(fetch_db, write_db):
    """The headline launches' HBM bytes from two rocprofv3 --pmc runs of this script (FETCH_SIZE, WRITE_SIZE; KiB
    per dispatch), each scaled by what the counter reads for the calibration copy (--calib-copy-mib, the largest
    __amd_rocclr_copyBuffer dispatch), written to TRAFFIC_JSON with these sources' hash. The four fused launches of
    the layer step are told apart by workgroup count (rows / (16 x row tiles)) and, for o and down (both 160), by
    the weight layout argument of qgemv_kernel (4 for g128, 3 for g96)."""
    import sqlite3

    def rows(path, counter):
        db = sqlite3.connect(path)
        q = ("select kernel_name, grid_size, workgroup_size, avg(value), count(*) from counters_collection "
             "where counter_name = ? group by kernel_name, grid_size, workgroup_size")
        out = db.execute(q, (counter,)).fetchall()
        db.close()
        return out

    res = {}
    for path, counter in ((fetch_db, "FETCH_SIZE"), (write_db, "WRITE_SIZE")):
        rr = rows(path, counter)
        copies = [r for r in rr if "copyBuffer" in r[0]]
        if not copies:
            sys.exit(f"{path}: no calibration copy (run with --calib-copy-mib)")
        copy = max(copies, key=lambda r: r[3])
        launches = {}
        for name, grid, wg, kib, n in rr:
            if "qgemv_kernel<" not in name:
                continue
            targs = [t.strip() for t in name.split("qgemv_kernel<", 1)[1].split(">", 1)[0].split(",")]
            if targs[4] == "0" or targs[-1] == "true":   # activations prepped elsewhere / the shares form
                continue
            wgs, ud = grid // wg, targs[1]
            key = {240: "qkv", 216: "gateup"}.get(wgs) or ("o" if wgs == 160 and ud == "4" else
                                                           "down" if wgs == 160 and ud == "3" else None)
            if key:
                launches[key] = {"kib": kib, "dispatches": n,
                                 "kernel": "qgemv_kernel<" + ", ".join(targs) + f">, {wgs} x {wg}"}
        res[counter] = {"copy_kib": copy[3], "launches": launches}
    missing = {"qkv", "o", "gateup", "down"} - set(res["FETCH_SIZE"]["launches"]) - set()
    if missing:
        sys.exit(f"launches not found: {sorted(missing)}")
    # the copy moves copy_bytes in each direction; its size in KiB is what WRITE_SIZE reads for it
    copy_kib = res["WRITE_SIZE"]["copy_kib"]
    ff, wf = copy_kib / res["FETCH_SIZE"]["copy_kib"], copy_kib / res["WRITE_SIZE"]["copy_kib"]
    per = {}
    for name, N, K, g in HEADLINE_LAYER:
        f, w = res["FETCH_SIZE"]["launches"][name], res["WRITE_SIZE"]["launches"][name]
        per[name] = {"read": int(round(f["kib"] * 1024 * ff)), "write": int(round(w["kib"] * 1024 * wf)),
                     "algorithmic": linear_f32_bytes(N, K, g, 1), "fetch_kib": round(f["kib"], 1),
                     "write_kib": round(w["kib"], 1), "kernel": f["kernel"], "dispatches": f["dispatches"]}
    rec = {"workload": "bitnet2b_layer_linears_m1", "kernel": "qgemv_kernel (prep fused, ternary int8-MFMA GEMV)",
           "source_sha256": source_hash(),
           "commands": [f"rocprofv3 --pmc {c} -d prof_{c.lower()} -o run -- python3 bench.py --no-cpu "
                        f"--no-extra --no-decode --steps 20 --warmup 2 --calib-copy-mib 256" for c in
                        ("FETCH_SIZE", "WRITE_SIZE")] +
                       [f"python3 bench.py --traffic-from {fetch_db} {write_db}"],
           "calibration": {"copy_kib_each_way": copy_kib, "fetch_kib": round(res["FETCH_SIZE"]["copy_kib"], 1),
                           "write_kib": round(res["WRITE_SIZE"]["copy_kib"], 1), "fetch_factor": round(ff, 4),
                           "write_factor": round(wf, 4)},
           "per_launch_bytes": per}
    with open(TRAFFIC_JSON, "w") as fh:
        json.dump(rec, fh, indent=1)
    tot = sum(v["read"] + v["write"] for v in per.values())
    alg = sum(v["algorithmic"] for v in per.values())
    print(json.dumps({"traffic": tot, "algorithmic": alg, "ratio": round(tot / alg, 4), "file": TRAFFIC_JSON}))


def measured_traffic():
    """(HBM bytes of one layer step, note) from the committed counter runs of this workload. The bytes are None
    when the file is absent or was measured on sources other than these (its source_sha256)."""
    try:
        with open(TRAFFIC_JSON) as f:
            rec = json.load(f)
        total = sum(v["read"] + v["write"] for v in rec["per_launch_bytes"].values())
    except (OSError, ValueError, KeyError):
        return None, "no counter file"
    if rec.get("source_sha256") != source_hash():
        return None, f"counter file measured on sources {rec.get('source_sha256')}, not these ({source_hash()})"
    return total, f"rocprofv3 counter runs on these sources ({source_hash()})"


class Timer:
    """Seconds per call of fn(i), i = 0..n-1, launched back to back.

    The n calls are captured once into a HIP graph; after one untimed replay the graph is replayed `replays` times,
    each replay bracketed by its own pair of HIP events on the stream the graph runs on, and the median replay / n
    is returned (the replay times in ms stay in .last). Host-side enqueue cost is excluded; the figure is the device
    time of the launches including the gaps between them. eager=True times plain launches from Python instead."""

    def __init__(self, torch):
        self.torch = torch
        self.cs = None   # the capture stream, one for all timings (its workspaces are reused)
        self.last = []

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
        times = []
        for _ in range(replays):
            a.record(s)
            g.replay()
            b.record(s)
            b.synchronize()
            times.append(a.elapsed_time(b))
        del g
        self.last = times
        return sorted(times)[len(times) // 2] / n * 1e-3


HEADLINE_LAYER = [("qkv", 3840, 2560, 128), ("o", 2560, 2560, 128), ("gateup", 13824, 2560, 128),
                  ("down", 2560, 6912, 96)]


def linear_f32_bytes(N, K, g, M):
    """Algorithmic bytes of a linear with FP32 activations in and out: codes + FP32 group scales + the FP32
    activation rows in + the FP32 outputs."""
    return N * (K // 4) + 4 * N * (-(-K // g)) + 4 * M * K + 4 * M * N


def headline_step_bytes(synth):
    return sum(linear_f32_bytes(N, K, g, 1) for _, N, K, g in HEADLINE_LAYER)


def bitnet2b_cfg(synth):
    c = dict(synth.BITNET_2B_DECODE)
    return synth.bitnet_config(c.pop("dim"), c.pop("hidden"), c.pop("n_layers"), c.pop("n_heads"),
                               c.pop("n_kv_heads"), c.pop("head_dim"), c.pop("vocab"), c.pop("seq_len"),
                               c.pop("group_in"), c.pop("group_down"), c.pop("wht_dim"), c.pop("wht_q"),
                               c.pop("wht_hidden"))


def copies_for(nbytes):
    """Weight copies to rotate over so that they total more than 2x the Infinity Cache (512 MiB)."""
    return max(3, -(-2 * MALL_BYTES // nbytes) + 1)


def main():
    args = parse()
    if args.cpu_child:
        return cpu_child(args)
    if args.traffic_from:
        return traffic_from_dbs(*args.traffic_from)
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
    layer = HEADLINE_LAYER
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

    fused_bytes = lambda N, K, g: linear_f32_bytes(N, K, g, M)
    step_bytes = headline_step_bytes(synth)

    for i in range(args.warmup):
        layer_step(i)
    torch.cuda.synchronize()
    eager_sec = timer(layer_step, min(args.steps, 100), eager=True)
    replays = max(5, args.replays)
    t0 = time.perf_counter()
    sec = timer(layer_step, args.steps, replays=replays)
    wall = time.perf_counter() - t0
    replay_ms = [round(v, 4) for v in timer.last]
    value = step_bytes / sec / 1e9
    unfused_sec = timer(layer_step_unfused, args.steps, replays=replays)

    # dominant kernel: the fused prep + ternary GEMV, per-linear launch duration over back-to-back launches, each
    # linear rotating over its own copies (> 512 MiB of them)
    reps = max(100, args.steps)
    per_linear = {}
    for name, (N, K, g) in shapes.items():
        lb = synth.ternary_linear_bytes(N, K, g, 0)
        own = [copies[0][name]] + [bh.QWeight(bh.W_TERNARY, N, K, g, *base[name]) for _ in range(copies_for(lb) - 1)]
        x = x_in[K]
        t = timer(lambda i, own=own, x=x: own[i % len(own)].linear_f32(x, y[name], 128, norm), reps)
        per_linear[name] = {"us": t * 1e6, "GBps": fused_bytes(N, K, g) / t / 1e9, "copies": len(own),
                            "rotated_MiB": round(len(own) * lb / 2**20, 1)}
        for q in own[1:]:
            q.close()
        del own
    gemv_time = sum(v["us"] for v in per_linear.values()) * 1e-6
    gemv_gbs = step_bytes / gemv_time / 1e9
    prep_t = timer(lambda i: prep(2560), reps)
    traffic, traffic_note = measured_traffic()

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
                     "frac": round(gemv_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_unit": "HBM bytes read + written by the 4 launches of one layer step "
                                     "(FETCH_SIZE x2, WRITE_SIZE x1, calibrated on a device copy)",
                     "traffic_source": traffic_note,
                     "algorithmic_bytes": step_bytes,
                     "kernel": "qgemv_kernel (prep fused, ternary int8-MFMA GEMV), the 4 launches of a layer",
                     "per_launch": {k: {"us": round(v["us"], 3), "GBps": round(v["GBps"], 1), "copies": v["copies"],
                                        "rotated_MiB": v["rotated_MiB"]} for k, v in per_linear.items()}},
        "prep_us": round(prep_t * 1e6, 3),
        "step_us_unfused_prep_kernel": round(unfused_sec * 1e6, 2),
        "step_us_eager_python_launch": round(eager_sec * 1e6, 2),
        "timing": f"one HIP graph of the {args.steps} timed steps ({4 * args.steps} launches), replayed {replays} "
                  f"times, each replay between HIP events on its stream; median replay / steps",
        "replay_ms": replay_ms,
        "wall_s_timed": round(wall, 3),
        "source_sha256": source_hash(),
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
        cpu = run_cpu_child(args)
        out["cpu_baseline"] = cpu.get("baseline", {"value": None, "kind": "none", "sample": cpu.get("error")})
        if out["cpu_baseline"].get("value"):
            out["gpu_over_cpu"] = round(value / out["cpu_baseline"]["value"], 1)
        out["cpu_legs"] = cpu.get("legs")
        if "decode" in out:
            d = out["decode"]
            d["cpu_baseline"] = cpu.get("decode")
            if d["cpu_baseline"] and d["cpu_baseline"].get("ms_per_token"):
                d["gpu_over_cpu"] = round(d["cpu_baseline"]["ms_per_token"] / d["ms_per_token"], 1)
    print(json.dumps(out))


def run_cpu_child(args):
    """The CPU legs in a child process (see CPU_CHILD_ENV): its last stdout line is their JSON."""
    import subprocess
    env = dict(os.environ)
    env.update(CPU_CHILD_ENV)
    env["OMP_NUM_THREADS"] = str(NPROC)
    cmd = [sys.executable, os.path.abspath(__file__), "--cpu-child", "--cpu-seconds", str(args.cpu_seconds),
           "--decode-prompt", str(args.decode_prompt), "--decode-tokens", str(args.decode_tokens)]
    if args.no_decode:
        cmd.append("--no-decode")
    try:
        r = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=60 + 8 * args.cpu_seconds)
    except subprocess.TimeoutExpired:
        return {"error": "CPU legs timed out"}
    lines = [l for l in r.stdout.splitlines() if l.startswith("{")]
    if r.returncode != 0 or not lines:
        return {"error": f"CPU legs failed (exit {r.returncode}): {r.stderr[-400:]}"}
    return json.loads(lines[-1])


def cpu_child(args):
    """Entry of the CPU-leg child process: no torch, no GPU."""
    import numpy as np
    import synth
    res = {"baseline": cpu_baseline(args, np, synth, headline_step_bytes(synth)), "legs": cpu_legs(args, np, synth)}
    if not args.no_decode:
        cfg = bitnet2b_cfg(synth)
        res["decode"] = cpu_decode_baseline(args, np, synth, cfg, synth.bitnet_model((300,), cfg))
    print(json.dumps(res), flush=True)


def extra_workloads(args, torch, bh, synth, timer, dev, copies, xq, xs, y, x_in, norm):
    import numpy as np
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

    # INT4 Qwen3.5-style FFN linears (hidden 1024, FFN 3584), M = 1 and 32: gate|up stacked (7168x1024), down
    # 1024x3584
    l4 = synth.QWEN35_INT4_LAYER
    base4 = {name: synth.int4_weight((109, i), N, K) for i, (name, N, K) in enumerate(l4)}
    f4 = {"gateup": (np.concatenate([base4["gate"][0], base4["up"][0]]),
                     np.concatenate([base4["gate"][1], base4["up"][1]])), "down": base4["down"]}
    s4 = [("gateup", 7168, 1024), ("down", 1024, 3584)]
    wb4 = sum(synth.int_linear_bytes(N, K, 4, 0) for _, N, K in s4)
    c4w = [{name: bh.QWeight(bh.W_INT4, N, K, 0, *f4[name]) for name, N, K in s4} for _ in range(copies_for(wb4))]
    for M in (1, 32):
        xk = {K: torch.from_numpy(synth.activations((110, K, M), M, K)).to(dev) for K in (1024, 3584)}
        qk = {K: torch.zeros((M, c4w[0][name].kpad), dtype=torch.int8, device=dev) for name, _, K in s4}
        sk = {K: torch.zeros(M, dtype=torch.float32, device=dev) for K in (1024, 3584)}
        for K in (1024, 3584):
            bh.prep_rows(xk[K], qk[K], sk[K], 0, 1.0)
        yk = {name: torch.zeros((M, N), dtype=torch.float32, device=dev) for name, N, K in s4}

        def lin4(i):
            for name, q in c4w[i % len(c4w)].items():
                q.linear(qk[q.cols], sk[q.cols], yk[name])
        t = timer(lin4, max(20, reps // 4))
        b = sum(synth.int_linear_bytes(N, K, 4, M) for _, N, K in s4)
        ex[f"int4_qwen35_ffn_m{M}"] = {"us": round(t * 1e6, 2), "GBps": round(b / t / 1e9, 1),
                                       "launches": "gate|up 7168x1024, down 1024x3584"}
    for cs in c4w:
        for q in cs.values():
            q.close()

    # INT8 Qwen2.5-0.5B-like layer, M = 1 and 128: q|k|v and gate|up share their input and are stacked into one
    # weight each (1152x896, 9728x896), as the BitNet layer above stacks them, so a layer is four launches
    l8 = synth.QWEN25_05B_LAYER
    base8 = {name: synth.int8_weight((105, i), N, K) for i, (name, N, K) in enumerate(l8)}
    stack = {"qkv": ("q", "k", "v"), "o": ("o",), "gateup": ("gate", "up"), "down": ("down",)}
    s8 = [(name, sum(base8[p][0].shape[0] for p in parts), base8[parts[0]][0].shape[1]) for name, parts in stack.items()]
    sbase = {name: (np.concatenate([base8[p][0] for p in parts]), np.concatenate([base8[p][1] for p in parts]))
             for name, parts in stack.items()}
    wb8 = sum(synth.int_linear_bytes(N, K, 8, 0) for _, N, K in s8)
    c8 = [{name: bh.QWeight(bh.W_INT8, N, K, 0, *sbase[name]) for name, N, K in s8} for _ in range(copies_for(wb8))]
    for M in (1, 128):
        xk = {K: torch.from_numpy(synth.activations((106, K, M), M, K)).to(dev) for K in (896, 4864)}
        qk = {K: torch.zeros((M, c8[0][name].kpad), dtype=torch.int8, device=dev) for name, _, K in s8}
        sk = {K: torch.zeros(M, dtype=torch.float32, device=dev) for K in (896, 4864)}
        for K in (896, 4864):
            bh.prep_rows(xk[K], qk[K], sk[K], 0, 1.0)
        yk = {name: torch.zeros((M, N), dtype=torch.float32, device=dev) for name, N, K in s8}

        def lin8(i):
            for name, q in c8[i % len(c8)].items():
                q.linear(qk[q.cols], sk[q.cols], yk[name])
        t = timer(lin8, max(20, reps // 4))
        b = sum(synth.int_linear_bytes(N, K, 8, M) for _, N, K in s8)
        ex[f"int8_qwen05b_layer_m{M}"] = {"us": round(t * 1e6, 2), "GBps": round(b / t / 1e9, 1),
                                          "launches": "qkv 1152x896, o 896x896, gate|up 9728x896, down 896x4864",
                                          "path": "gemm" if M >= bh.load().eif_hip_gemm_min_tokens() else "gemv"}
    for cs in c8:
        for q in cs.values():
            q.close()

    # the drop-in host API (host x in, host y out over PCIe; weights resident after the first call), M = 1
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
    cfg = bitnet2b_cfg(synth)
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
    return res


def host_info():
    """nproc (CPUs this process may run on), the lscpu model name and the cgroup's CPU quota."""
    import subprocess
    info = {"nproc": NPROC, "lscpu_model": None, "cgroup_cpus": None}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                info["lscpu_model"] = line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, per = f.read().split()
        if q != "max":
            info["cgroup_cpus"] = round(int(q) / int(per), 2)
    except (OSError, ValueError):
        pass
    return info


def cpu_threads():
    """The thread counts of the CPU legs: nproc and min(8, nproc) (the reference CLI's default)."""
    return sorted({NPROC, min(8, NPROC)}, reverse=True)


def set_omp_threads(lib, n):
    """OpenMP threads of the parallel regions the reference library starts from this thread from now on."""
    lib.omp_set_num_threads(n)


def median_time(fn, seconds, min_reps=30, max_reps=100000):
    """Median seconds of fn(i) over at least min_reps calls and about `seconds` (after one untimed call)."""
    fn(0)
    times = []
    t_end = time.perf_counter() + seconds
    i = 1
    while (time.perf_counter() < t_end or len(times) < min_reps) and len(times) < max_reps:
        t0 = time.perf_counter()
        fn(i)
        times.append(time.perf_counter() - t0)
        i += 1
    times.sort()
    return times[len(times) // 2], len(times)


def load_ref_lib():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ctypes as C
    import oracle_api
    path = os.path.join(ROOT, "oracle", "_ref", "libref.so")
    if not os.path.exists(path):
        return None, oracle_api
    lib = oracle_api.load_ref(path)
    lib.omp_set_num_threads.restype, lib.omp_set_num_threads.argtypes = None, [C.c_int]
    return lib, oracle_api


def cpu_decode_baseline(args, np, synth, cfg, w):
    """The reference's own tinyllm BitNet decode (oracle/ref_tinyllm_wrap.c over its sources, reference flags) of
    the same weights on the host cores: g128 scales for every matrix (its one group bound cannot give the down
    projection g96 alone; it reads 54 of the 72 scales of each down row), its own WHT blocks (512 / 256), fp32 KV
    cache. The cache of positions 0 .. prompt - 1 is filled with synthetic values (ref_bitnet_fill_cache), then
    greedy steps are timed at positions prompt, prompt + 1, ... (the GPU's positions), at nproc and min(8, nproc)
    threads, about --cpu-seconds / 2 each."""
    import ctypes as C
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle_api
    path = os.path.join(ROOT, "oracle", "_ref", "libref.so")
    if not os.path.exists(path):
        return {"ms_per_token": None, "kind": "none", "sample": "oracle/_ref/libref.so not built"}
    ref = oracle_api.load_ref_tinyllm(path)
    ref.omp_set_num_threads.restype, ref.omp_set_num_threads.argtypes = None, [C.c_int]
    c, ws = oracle_api.bitnet_structs(cfg, w)
    h = ref.ref_bitnet_create(C.byref(c), C.byref(ws), 128)
    if not h:
        return {"ms_per_token": None, "kind": "reference", "sample": "model construction failed"}
    p0 = args.decode_prompt
    res = {"kind": "reference", "by_threads": {}}
    try:
        if ref.ref_bitnet_fill_cache(h, p0) != 0:
            return {"ms_per_token": None, "kind": "reference", "sample": "cache fill refused"}
        for nt in cpu_threads():
            set_omp_threads(ref, nt)
            tok, times, pos = 1, [], p0
            t_end = time.perf_counter() + args.cpu_seconds / 2
            while pos < p0 + args.decode_tokens and (time.perf_counter() < t_end or len(times) < 5):
                t0 = time.perf_counter()
                lp = ref.ref_bitnet_forward(h, tok, pos)
                lo = np.ctypeslib.as_array(lp, shape=(cfg["vocab"],))
                tok = int(np.argmax(lo))
                if pos > p0:
                    times.append(time.perf_counter() - t0)
                pos += 1
            med = float(np.median(times))
            res["by_threads"][str(nt)] = {"ms_per_token": round(med * 1e3, 2), "tok_per_s": round(1.0 / med, 2),
                                          "steps": len(times), "positions": f"{p0 + 1}..{pos - 1}"}
    finally:
        ref.ref_bitnet_destroy(h)
    first = res["by_threads"][str(cpu_threads()[0])]
    res.update({"ms_per_token": first["ms_per_token"], "tok_per_s": first["tok_per_s"], "cores": cpu_threads()[0],
                "sample": f"greedy steps at positions {first['positions']} after a synthetic-filled cache of "
                          f"{p0} positions, median; threads {cpu_threads()} (OpenMP, OMP_PROC_BIND=close, "
                          f"OMP_WAIT_POLICY=ACTIVE)"})
    return res


def cpu_baseline(args, np, synth, step_bytes):
    """The reference's own x86 path for the headline layer step, on the host cores, over a bounded sample: at
    nproc threads (value) and at min(8, nproc)."""
    import ctypes as C
    lib, oracle_api = load_ref_lib()
    P = oracle_api.P
    port_so = os.path.join(ROOT, "oracle", "liboracle_port.so")
    if lib is not None:
        kind = "reference"
        rot = lambda x, n: lib.eif_hadamard_rotate_f32(P(x), None, n, 128)
        gemv = lambda w, s, g, x, yv, N, K: lib.eif_matmul_bitnet_block_f32(P(w), P(s), g, P(x), None, P(yv), N, K)
    elif os.path.exists(port_so):
        lib, kind = oracle_api.load(port_so), "port"
        lib.omp_set_num_threads.restype, lib.omp_set_num_threads.argtypes = None, [C.c_int]
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

    by = {}
    for nt in cpu_threads():
        set_omp_threads(lib, nt)
        med, n = median_time(step, args.cpu_seconds / 2)
        by[str(nt)] = {"GBps": round(step_bytes / med / 1e9, 2), "ms_per_step": round(med * 1e3, 3), "steps": n}
    nt0 = str(cpu_threads()[0])
    return {"value": by[nt0]["GBps"], "unit": "GB/s", "cores": int(nt0), "kind": kind,
            "ms_per_step": by[nt0]["ms_per_step"], "by_threads": by, "host": host_info(),
            "sample": f"{by[nt0]['steps']} layer steps (WHT-128 + FP32-activation grouped GEMV, the reference x86 "
                      f"path) over {ncp} weight copies, median; threads {cpu_threads()}"}


def cpu_legs(args, np, synth):
    """The reference functions of the other configurations (BASELINE's CPU plan), each over inputs rotated past the
    host's last-level cache, median of >= 30 calls, at nproc and min(8, nproc) threads:
      c0 integer path  eif_hadamard_rotate_f32 + eif_quantize_activation_i8 + eif_matmul_bitnet_i8xternary_f32
      c0 act-quant     eif_matmul_bitnet_act_quant_f32 (FP32 in, INT8 on the fly, row scales)
      c0 FP32 grouped  eif_hadamard_rotate_f32 + eif_matmul_bitnet_block_f32 (g128)
      c2               tinyllm_matmul_int8_rowscale over the 7 linears of the Qwen2.5-0.5B-like layer
      c3               int4_gemv (src/eif_qwen35.c, via ref_q35_int4_gemv) on the 151936 x 1024 tied head and the
                       3584 x 1024 / 1024 x 3584 layer linears"""
    lib, oracle_api = load_ref_lib()
    if lib is None:
        return {"kind": "none", "note": "oracle/_ref/libref.so not built"}
    P = oracle_api.P
    llc = 64 << 20   # rotate past twice the 32 MiB L3 of the hosts measured
    legs = {}

    def copies(nbytes):
        return max(2, -(-llc // nbytes) + 1)

    def run(name, fn, nbytes, shape):
        by = {}
        for nt in cpu_threads():
            set_omp_threads(lib, nt)
            med, n = median_time(fn, args.cpu_seconds / 12)
            by[str(nt)] = {"us": round(med * 1e6, 2), "GBps": round(nbytes / med / 1e9, 2), "calls": n}
        legs[name] = {"shape": shape, "bytes": nbytes, "by_threads": by}

    # c0: the single 6912 x 2560 ternary linear, batch 1
    N, K, g = 6912, 2560, 128
    w, sg = synth.ternary_weight((100, 2), N, K, g)
    rs = (np.abs(synth.rng(110).standard_normal(N)) * 0.02).astype(np.float32)
    nc = copies(w.nbytes)
    wc = [w] + [w.copy() for _ in range(nc - 1)]
    x = synth.activations((101, K), 1, K)[0]
    xb, xq, xsc, yv = x.copy(), np.zeros(K, np.int8), np.zeros(1, np.float32), np.zeros(N, np.float32)

    def c0_int(i):
        xb[:] = x
        lib.eif_hadamard_rotate_f32(P(xb), None, K, 128)
        lib.eif_quantize_activation_i8(P(xb), P(xq), P(xsc), K)
        lib.eif_matmul_bitnet_i8xternary_f32(P(wc[i % nc]), P(rs), P(xq), float(xsc[0]), None, P(yv), N, K)
    run("c0_int8_path_6912x2560", c0_int, w.nbytes + 4 * N + 4 * K + 4 * N, "6912x2560 ternary, row scales, M=1")

    def c0_aq(i):
        lib.eif_matmul_bitnet_act_quant_f32(P(wc[i % nc]), P(rs), P(x), None, P(yv), N, K)
    run("c0_act_quant_f32_6912x2560", c0_aq, w.nbytes + 4 * N + 4 * K + 4 * N, "6912x2560 ternary, row scales, M=1")

    def c0_blk(i):
        xb[:] = x
        lib.eif_hadamard_rotate_f32(P(xb), None, K, 128)
        lib.eif_matmul_bitnet_block_f32(P(wc[i % nc]), P(sg), g, P(xb), None, P(yv), N, K)
    run("c0_block_f32_6912x2560_g128", c0_blk, w.nbytes + sg.nbytes + 4 * K + 4 * N,
        "6912x2560 ternary, g128 scales, M=1")
    del wc

    # c2: the INT8 Qwen2.5-0.5B-like layer, batch 1
    l8 = synth.QWEN25_05B_LAYER
    base8 = {name: synth.int8_weight((105, i), N8, K8) for i, (name, N8, K8) in enumerate(l8)}
    b8 = sum(v[0].nbytes + v[1].nbytes for v in base8.values())
    n8 = copies(b8)
    c8 = [base8] + [{k: (v[0].copy(), v[1].copy()) for k, v in base8.items()} for _ in range(n8 - 1)]
    x8 = {K8: synth.activations((106, K8, 1), 1, K8)[0] for K8 in (896, 4864)}
    y8 = {name: np.zeros(N8, np.float32) for name, N8, K8 in l8}

    def c2(i):
        cw = c8[i % n8]
        for name, N8, K8 in l8:
            lib.tinyllm_matmul_int8_rowscale(P(y8[name]), P(cw[name][0]), P(x8[K8]), K8, N8, P(cw[name][1]))
    run("c2_int8_rowscale_qwen05b_layer", c2, b8 + sum(4 * (K8 + N8) for _, N8, K8 in l8),
        "7 linears (q 896x896, k/v 128x896, o 896x896, gate/up 4864x896, down 896x4864), M=1")
    del c8

    # c3: the INT4 tied head and the INT4 layer linears, batch 1
    Nh, Kh = synth.QWEN35_INT4_HEAD[1:]
    hw, hs = synth.int4_weight((103,), Nh, Kh)
    xh = synth.activations((104, 1), 1, Kh)[0]
    yh = np.zeros(Nh, np.float32)
    nh = copies(hw.nbytes)
    hc = [hw] + [hw.copy() for _ in range(nh - 1)]
    run("c3_int4_gemv_head_151936x1024", lambda i: lib.ref_q35_int4_gemv(P(yh), P(hc[i % nh]), P(hs), P(xh), Nh, Kh),
        hw.nbytes + hs.nbytes + 4 * Kh + 4 * Nh, "151936x1024 int4, row scales, M=1")
    del hc
    l4 = [("gate", 3584, 1024), ("up", 3584, 1024), ("down", 1024, 3584)]
    base4 = {name: synth.int4_weight((47, N4, K4), N4, K4) for name, N4, K4 in l4}
    b4 = sum(v[0].nbytes + v[1].nbytes for v in base4.values())
    n4 = copies(b4)
    c4 = [base4] + [{k: (v[0].copy(), v[1].copy()) for k, v in base4.items()} for _ in range(n4 - 1)]
    x4 = {K4: synth.activations((48, K4, 1), 1, K4)[0] for K4 in (1024, 3584)}
    y4 = {name: np.zeros(N4, np.float32) for name, N4, K4 in l4}

    def c3_layer(i):
        cw = c4[i % n4]
        for name, N4, K4 in l4:
            lib.ref_q35_int4_gemv(P(y4[name]), P(cw[name][0]), P(cw[name][1]), P(x4[K4]), N4, K4)
    run("c3_int4_gemv_ffn_layer", c3_layer, b4 + sum(4 * (K4 + N4) for _, N4, K4 in l4),
        "gate/up 3584x1024 + down 1024x3584 int4, row scales, M=1")
    return {"kind": "reference", "threads": cpu_threads(), "host": host_info(),
            "sample": "median of >= 30 calls per leg and thread count, inputs rotated past 64 MiB", "legs": legs}


if __name__ == "__main__":
    main()
