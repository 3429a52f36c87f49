#!/usr/bin/env python3
"""Benchmark of the batch-1 fused decode-matvec on one MI355X (BASELINE.json metric: per-token matvec us + effective
HBM GB/s, Qwen3-4B shapes, batch 1, vs a BF16 hipBLASLt matvec).

Workload: a Qwen3-4B-shaped stack of 36 layers, each with the fused qkv 6144x2560,
o_proj 2560x4096, fused gate_up 19456x2560 and down 2560x9728 matrices, BF16, layout 0 (--layout 1 for the other
layout of that config).  One step = one token: the 144 token-path matvecs of the stack, captured once as a HIP graph
and replayed.  Weights are N(0, 0.02^2) from fixed seeds; each of the four matrices is encoded once and copied to
36 distinct device buffers (the sweep reads 36 x 4 different buffers, far beyond the 256 MB Infinity Cache).

Reported: value = algorithmic bytes per token / GPU time per token (GB/s), with the per-launch medians (HIP events),
the same sweep with hipBLASLt BF16 matvecs (F.linear), the roofline of the dominant kernel (the gate_up launch:
algorithmic bytes / average launch time; HBM traffic from the committed counter summary profiles/traffic_gate_up.json)
and the CPU baseline (the C oracle's decode + fp32 matvec of configs[0], on the host cores).
usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--layout 0] [--cpu-seconds 10]
       python bench.py --profile-launches 20     (counter target for rocprofv3 --pmc: copies + gate_up launches)
"""
import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "per-token matvec µs + effective HBM GB/s, Qwen3-4B shapes batch 1 vs BF16 matvec"
PEAK_HBM_GBS = 8000.0
LAYERS = 36
SHAPES = [("qkv", 6144, 2560), ("o", 2560, 4096), ("gate_up", 19456, 2560), ("down", 2560, 9728)]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_weight(M, K, seed):
    import torch
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(M, K, generator=g) * 0.02).to(torch.bfloat16)


def clone_weight(c):
    """A second NWCWeight over distinct device buffers with the same content."""
    from nwc_amd.nwc_torch import NWCWeight
    d = NWCWeight.__new__(NWCWeight)
    d.__dict__.update(c.__dict__)
    for k in ("data", "bases", "hdr", "lut", "low", "_row_index"):
        if getattr(c, k, None) is not None:
            setattr(d, k, getattr(c, k).clone())
    return d


class Launch:
    """One prepared nwc_linear_xbf16 call (ctypes arguments built once)."""

    def __init__(self, c, x, y):
        from nwc_amd.nwc_torch import _lib, _ptr
        self.fn = _lib.nwc_linear_xbf16
        ri = c.row_index()
        self.args = [_ptr(c.data), _ptr(c.bases), _ptr(c.hdr), _ptr(c.lut), _ptr(c.low),
                     _ptr(ri) if ri is not None else None, _ptr(x), None,
                     _ptr(c.scale) if c.scale is not None else None, _ptr(y), ctypes.c_uint64(c.n),
                     ctypes.c_uint32(c.in_features), ctypes.c_int(c.code)]

    def __call__(self, stream):
        rc = self.fn(stream, *self.args)
        if rc:
            raise RuntimeError(f"nwc_linear_xbf16 error {rc}")


def event_ms(fn, runs, rotate):
    """Median GPU time of single launches (HIP events on the launch stream), rotating over `rotate` copies."""
    import torch
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(runs)]
    for i in range(runs):
        ev[i][0].record()
        fn(i % rotate)
        ev[i][1].record()
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) for a, b in ev), [a.elapsed_time(b) for a, b in ev]


def avg_launch_ms(fn, rotate, replays):
    """Average GPU time per launch: `rotate` back-to-back launches captured as one HIP graph, replayed `replays` times
    between two HIP events on the launch stream (a graph leaves no launch gaps, so this is the kernel's own time)."""
    import torch
    for i in range(rotate):
        fn(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(rotate):
            fn(i)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (rotate * replays)


DOMINANT = "gate_up"            # the roofline's kernel: the largest matrix, k_layout0<BF16, token, BF16 x, pipelined>
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_gate_up.json")


def run_gpu(args):
    import torch
    from nwc_amd.nwc_torch import NWCWeight
    torch.backends.cuda.preferred_blas_library("hipblaslt")
    dev = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(dev)
    log(f"device: {props.name} ({props.gcnArchName}), {props.multi_processor_count} CUs, {props.total_memory/2**30:.0f} GiB")
    stream = torch.cuda.current_stream()

    # ---- compressed stack ----
    t0 = time.time()
    base = []
    for si, (name, M, K) in enumerate(SHAPES):
        w = make_weight(M, K, 1000 + si)
        c = NWCWeight(w, device=dev, layout=args.layout)
        x = torch.randn(K, generator=torch.Generator().manual_seed(2000 + si)).to(torch.bfloat16).to(dev)
        base.append((name, M, K, c, x, w))
    copies = {name: [c] + [clone_weight(c) for _ in range(LAYERS - 1)] for name, M, K, c, x, w in base}
    ys = {name: [torch.empty(M, dtype=torch.bfloat16, device=dev) for _ in range(LAYERS)] for name, M, K, *_ in base}
    launches = {name: [Launch(copies[name][l], x, ys[name][l]) for l in range(LAYERS)] for name, M, K, c, x, w in base}
    torch.cuda.synchronize()
    log(f"encoded + placed {len(SHAPES)}x{LAYERS} compressed matrices in {time.time()-t0:.1f} s")

    # correctness spot check of the copies against a torch fp32 matvec
    for name, M, K, c, x, w in base:
        y = copies[name][LAYERS - 1].linear_bf16(x, None).float()
        ref = (w.to(dev).float() @ x.float())
        err = ((y - ref).abs() - (2 ** -8) * ref.abs()).max().item()
        if err > 1e-5:
            raise SystemExit(f"{name}: token path outside tolerance ({err:.3e})")

    sh = ctypes.c_void_p(stream.cuda_stream)
    bytes_tok = sum(c.token_bytes() + 2 * K + 2 * M for name, M, K, c, x, w in base) * LAYERS
    bf16_tok = sum(2 * M * K + 2 * K + 2 * M for name, M, K, *_ in base) * LAYERS

    # ---- per-launch medians (the reference kernbench's method) ----
    per = []
    for name, M, K, c, x, w in base:
        L = launches[name]
        for i in range(10):
            L[i % LAYERS](sh)
        ms, _ = event_ms(lambda j: L[j](sh), args.runs, LAYERS)
        per.append({"layer": name, "M": M, "K": K, "nwc_bytes": c.token_bytes(), "nwc_us": ms * 1e3,
                    "nwc_GBps": (c.token_bytes() + 2 * K + 2 * M) / (ms * 1e-3) / 1e9})

    # ---- the timed sweep: one token = 144 launches, captured as a HIP graph ----
    def sweep():
        for l in range(LAYERS):
            for name, *_ in base:
                launches[name][l](ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))

    graph = None
    try:
        sweep()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            sweep()
        torch.cuda.synchronize()
    except Exception as e:  # capture refused: time the eager sweep instead
        log(f"graph capture failed ({e}); timing the eager sweep")
        graph = None
    step = graph.replay if graph is not None else sweep
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / args.steps

    # ---- hipBLASLt BF16 baseline: the same stack uncompressed ----
    blas = None
    if not args.no_baseline:
        import torch.nn.functional as F
        wcopy = {name: [w.to(dev) for _ in range(LAYERS)] for name, M, K, c, x, w in base}
        xs = {name: x.view(1, K) for name, M, K, c, x, w in base}
        blas_per = []
        for name, M, K, *_ in base:
            W = wcopy[name]
            for i in range(10):
                F.linear(xs[name], W[i % LAYERS])
            ms, _ = event_ms(lambda j: F.linear(xs[name], W[j]), args.runs, LAYERS)
            blas_per.append({"layer": name, "us": ms * 1e3, "GBps": (2 * M * K + 2 * K + 2 * M) / (ms * 1e-3) / 1e9})

        def bsweep():
            for l in range(LAYERS):
                for name, *_ in base:
                    F.linear(xs[name], wcopy[name][l])
        bgraph = None
        try:
            bsweep()
            torch.cuda.synchronize()
            bgraph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(bgraph):
                bsweep()
            torch.cuda.synchronize()
        except Exception as e:
            log(f"hipBLASLt graph capture failed ({e}); eager sweep")
            bgraph = None
        bstep = bgraph.replay if bgraph is not None else bsweep
        for _ in range(args.warmup):
            bstep()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(args.steps):
            bstep()
        e1.record()
        torch.cuda.synchronize()
        bms = e0.elapsed_time(e1) / args.steps
        blas = {"us_per_token_graph": bms * 1e3, "us_per_token_sum_of_launches": LAYERS * sum(p["us"] for p in blas_per),
                "GBps": bf16_tok / (bms * 1e-3) / 1e9, "per_layer": blas_per, "bytes_per_token": bf16_tok,
                "library": "torch F.linear, preferred_blas_library=hipblaslt"}
        del wcopy
        torch.cuda.empty_cache()

    # ---- roofline of the dominant kernel: average launch time of back-to-back gate_up launches ----
    name, M, K, c, x, w = next(b for b in base if b[0] == DOMINANT)
    L = launches[name]
    dom_bytes = c.token_bytes() + 2 * K + 2 * M
    dom_ms = avg_launch_ms(lambda j: L[j](ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)), LAYERS, 4)
    sum_launch_us = LAYERS * sum(p["nwc_us"] for p in per)
    return {
        "ms_step": ms_step, "graph": graph is not None, "bytes_tok": bytes_tok, "bf16_tok": bf16_tok, "per": per,
        "sum_launch_us": sum_launch_us, "dom_bytes": dom_bytes, "dom_us": dom_ms * 1e3,
        "achieved": dom_bytes / (dom_ms * 1e-3) / 1e9, "blas": blas,
        "device": {"name": props.name, "arch": props.gcnArchName, "cus": props.multi_processor_count},
    }


def run_cpu(args):
    """CPU baseline: the C oracle's decode + fp32 matvec of BASELINE configs[0] (9728 x 2560, layout 0, BF16) on all
    host cores, repeated for about --cpu-seconds."""
    import numpy as np
    import torch
    from oracle import oracle as O
    cores = len(os.sched_getaffinity(0))
    w = make_weight(9728, 2560, 7).view(torch.int16).numpy().view(np.uint16)
    enc = O.encode(w, 0, 0)
    x = torch.randn(2560, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16).float().numpy()
    nbytes = enc["dl"] + enc["bases"].size * 4 + enc["hdr"].size + 4096 * 4 + enc["n_low"]
    y = O.linear(enc, x, threads=cores)                        # warm-up and check against the float64 closed form
    y64 = O.bf16_to_f64(w) @ x.astype(np.float64)
    assert np.all(np.abs(y - y64) <= 1e-3 * np.abs(y64) + 1e-5), "oracle CPU path outside tolerance"
    reps, t0 = 0, time.perf_counter()
    while True:
        O.linear(enc, x, threads=cores)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= args.cpu_seconds:
            break
    gbs = nbytes * reps / dt / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"configs[0]: 9728x2560 BF16 layout 0 ({nbytes/1e6:.1f} MB compressed), C oracle decode + fp32 matvec "
                      f"(OpenMP over row groups), {reps} reps in {dt:.1f} s",
            "us_per_matvec": round(dt / reps * 1e6, 1)}


def traffic_bytes():
    """HBM bytes per gate_up launch from the committed rocprofv3 counter summary (FETCH_SIZE + WRITE_SIZE, each scaled
    by the factor a plain copy of known size gives), or None when there is none."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)["bytes_per_launch"]
    except (OSError, ValueError, KeyError):
        return None


def run_profile(args):
    """Counter target: --profile-launches gate_up launches, after three device copies of 256 MiB (the calibration
    kernel of known size).  Run under rocprofv3 --pmc; prints one line per phase."""
    import torch
    from nwc_amd.nwc_torch import NWCWeight
    dev = torch.device("cuda:0")
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("calibration: 3 copies of 268435456 bytes", flush=True)
    del src, dst
    name, M, K = next(s for s in SHAPES if s[0] == DOMINANT)
    c = NWCWeight(make_weight(M, K, 1000 + [s[0] for s in SHAPES].index(DOMINANT)), device=dev, layout=args.layout)
    cs = [c] + [clone_weight(c) for _ in range(7)]
    x = torch.randn(K, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(dev)
    ys = [torch.empty(M, dtype=torch.bfloat16, device=dev) for _ in cs]
    L = [Launch(cc, x, y) for cc, y in zip(cs, ys)]
    sh = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for i in range(args.profile_launches):
        L[i % len(L)](sh)
    torch.cuda.synchronize()
    print(f"{DOMINANT}: {args.profile_launches} launches, {c.token_bytes() + 2 * K + 2 * M} algorithmic bytes each", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layout", type=int, default=0, choices=[0, 1])
    ap.add_argument("--runs", type=int, default=60, help="launches per shape for the per-launch medians")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-baseline", action="store_true")
    ap.add_argument("--profile-launches", type=int, default=0,
                    help="only run the counter target (copies + this many gate_up launches), for rocprofv3 --pmc")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this path (a batch-1 decode-matvec) is not run across GPUs in this build; "
              "use --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.profile_launches:
        run_profile(args)
        return

    g = run_gpu(args)
    cpu = None if args.no_cpu else run_cpu(args)
    us_tok = g["ms_step"] * 1e3
    value = g["bytes_tok"] / (g["ms_step"] * 1e-3) / 1e9
    blas = g["blas"]
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(g["ms_step"], 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: N(0,0.02^2) BF16 weights and N(0,1) activations from fixed seeds; 4 matrices encoded once, "
                "36 device copies each",
        "config": {"workload": f"Qwen3-4B-shaped 36-layer batch-1 token sweep (BASELINE configs[2]), layout {args.layout} BF16",
                   "layers": LAYERS, "shapes": {n: [M, K] for n, M, K in SHAPES}, "layout": args.layout, "batch": 1,
                   "step": "one token = 144 fused decode-matvecs replayed as one HIP graph" if g["graph"] else
                           "one token = 144 fused decode-matvecs (eager)"},
        "us_per_token": round(us_tok, 1),
        "us_per_token_sum_of_launches": round(g["sum_launch_us"], 1),
        "bytes_per_token": g["bytes_tok"], "bytes_per_token_bf16": g["bf16_tok"],
        "hbm_frac": round(value / PEAK_HBM_GBS, 4),
        "per_layer": [{k: (round(v, 2) if isinstance(v, float) else v) for k, v in p.items()} for p in g["per"]],
        "hipblaslt": None if blas is None else {k: (round(v, 2) if isinstance(v, float) else v) for k, v in blas.items()},
        "speedup_vs_hipblaslt": None if blas is None else round(blas["us_per_token_graph"] / us_tok, 3),
        "roofline": {"bound": "hbm", "achieved": round(g["achieved"], 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(g["achieved"] / PEAK_HBM_GBS, 4), "traffic": traffic_bytes(),
                     "kernel": "k_layout0<0, 0, true, true> (BF16, token, BF16 x, pipelined): gate_up 19456x2560",
                     "bytes_per_launch": g["dom_bytes"], "avg_launch_us": round(g["dom_us"], 2),
                     "achieved_basis": "NWCWeight.bytes + x + y of one gate_up launch / average time of "
                                       f"{4 * LAYERS} launches (a HIP graph of {LAYERS} back-to-back launches replayed 4 "
                                       "times between HIP events on the launch stream)",
                     "sweep_achieved": round(g["bytes_tok"] / (g["sum_launch_us"] * 1e-6) / 1e9, 1)},
        "cpu_baseline": cpu,
        "device": g["device"],
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
