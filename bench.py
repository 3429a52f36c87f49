#!/usr/bin/env python3
"""Benchmark of the batch-1 fused decode-matvec on one MI355X (BASELINE.json metric: per-token matvec us + effective
HBM GB/s, Qwen3-4B shapes, batch 1, vs a BF16 hipBLASLt matvec).

Default workload: a Qwen3-4B-shaped stack of 36 layers, each with the fused qkv 6144x2560,
o_proj 2560x4096, fused gate_up 19456x2560 and down 2560x9728 matrices, BF16, layout 0 (--layout 1 for the other
layout of that config; --layout 2 for the fixed-width format on the same stack, outside BASELINE's configs).  One
step = one token: the 144 token-path matvecs of the stack, captured once as a HIP graph and replayed.  Weights are N(0, 0.02^2) from fixed seeds; each of the four matrices is encoded once and copied to
36 distinct device buffers (the sweep reads 36 x 4 different buffers, far beyond the 256 MB Infinity Cache).

Reported: value = algorithmic bytes per token / GPU time per token (GB/s), with per-launch times (a HIP graph of the
36 copies' launches of one shape, and single launches between HIP events as the reference's kernbench does), the same
sweep with hipBLASLt BF16 matvecs (F.linear), the roofline of the dominant kernel (the gate_up launch: algorithmic
bytes / average launch time; HBM traffic from the committed counter summary profiles/traffic_gate_up.json) and the
CPU baseline (the C oracle's decode + fp32 matvec of configs[0], on the host cores).  Beside the sweep, and not in
`value`: the vocabulary matrix that ends every token (Qwen3-4B: the tied 151936x2560 embedding used as lm_head), its
launch time, and the per-token time of the sweep followed by it in one graph, as the reference's kernbench sums a
token (36 layers x 4 + lm_head); --no-lm-head skips it.

The other BASELINE configs, each printed as one JSON line of its own (not the driver's line):
  --config qwen3-0.6b      configs[1]: 28 layers of 4096x1024 / 1024x2048 / 6144x1024 / 1024x3072, BF16 layout 0
  --config qwen3-4b-fp8    configs[3]: the 4B stack as weight-only fp8 e4m3 (per-row scale), layout 0 or 1, against
                           the library's uncompressed fp8 matvec (nwc_ref_fp8) and hipBLASLt BF16
  --config qwen2.5-7b-l2   configs[4]: 28 layers of 4608x3584 / 3584x3584 / 37888x3584 / 3584x18944, BF16 layout 2
  --prefill 512            configs[2] prefill: per matrix, dequantization to a BF16 buffer + hipBLASLt GEMM of 512
                           tokens, against the GEMM on resident BF16 weights
  --gather 64              configs[4] embedding: 64 seeded ids from the 152064x3584 table, layouts 0, 1 and 2
  --batch 4                configs[2] at 2..8 tokens: the batched fused kernel (no temporary buffer) against
                           single-token launches, dequantization + hipBLASLt GEMM, and resident BF16
  --decode 128             model level: greedy decode of a random-init Qwen3 (--config qwen3-4b or qwen3-0.6b), one
                           HIP graph per token, BF16 (hipBLASLt) against NWC (--decode-elem bf16 or fp8)
  --encode                 the host encoder on configs[0] against the single-threaded oracle restatement (no GPU)
usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--layout 0] [--cpu-seconds 10] [--config NAME]
       python bench.py --profile-launches 20     (counter target for rocprofv3 --pmc: copies + gate_up launches;
                                                 --profile-shape qkv|o|gate_up|down picks the matrix)
"""
import argparse
import contextlib
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
# BASELINE configs by name: (layers, shapes, element type, default layout, workload text)
CONFIGS = {
    "qwen3-4b": (36, SHAPES, "bf16", 0, "Qwen3-4B-shaped 36-layer batch-1 token sweep (BASELINE configs[2])"),
    "qwen3-0.6b": (28, [("qkv", 4096, 1024), ("o", 1024, 2048), ("gate_up", 6144, 1024), ("down", 1024, 3072)], "bf16", 0,
                   "Qwen3-0.6B-shaped 28-layer batch-1 token sweep (BASELINE configs[1])"),
    "qwen3-4b-fp8": (36, SHAPES, "fp8", 0, "Qwen3-4B-shaped 36-layer batch-1 token sweep, weight-only fp8 e4m3 with "
                                           "per-row scale (BASELINE configs[3])"),
    "qwen2.5-7b-l2": (28, [("qkv", 4608, 3584), ("o", 3584, 3584), ("gate_up", 37888, 3584), ("down", 3584, 18944)],
                      "bf16", 2, "Qwen2.5-7B-shaped 28-layer batch-1 token sweep, layout 2 (BASELINE configs[4])"),
}
# the vocabulary matrix each config's token ends with (Qwen3: the tied embedding; Qwen2.5-7B: the untied lm_head),
# timed beside the sweep as the reference's per-token sum counts it (36 layers x 4 + lm_head)
HEADS = {"qwen3-4b": (151936, 2560), "qwen3-0.6b": (151936, 1024), "qwen3-4b-fp8": (151936, 2560),
         "qwen2.5-7b-l2": (152064, 3584)}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_weight(M, K, seed):
    import torch
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(M, K, generator=g) * 0.02).to(torch.bfloat16)


def clone_weight(c):
    """A second NWCWeight over distinct device buffers with the same content."""
    import torch
    from nwc_amd.nwc_torch import NWCWeight
    d = NWCWeight.__new__(NWCWeight)
    d.__dict__.update(c.__dict__)
    for k in ("data", "bases", "hdr", "lut", "low", "_row_index"):
        if isinstance(getattr(c, k, None), torch.Tensor):
            setattr(d, k, getattr(c, k).clone())
    return d


class Launch:
    """One prepared nwc_linear_xbf16 call (ctypes arguments built once)."""

    def __init__(self, c, x, y):
        from nwc_amd._abi import lib as _lib, ptr as _ptr
        self.fn = _lib.nwc_linear_xbf16
        ri, st = c.row_index(), c.seq_table()
        self.args = [_ptr(c.data), _ptr(c.bases), _ptr(c.hdr), _ptr(c.lut), _ptr(c.low),
                     _ptr(ri) if ri is not None else None, _ptr(st) if st is not None else None, _ptr(x), None,
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


DOMINANT = "gate_up"            # the roofline's kernel: the largest matrix (k_layout0p<BF16, 8 rows>: one round, 13-bit table)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_gate_up.json")


def graph_stack(fns):
    """Capture fns (one callable per launch) as one HIP graph; None if capture is refused."""
    import torch
    for f in fns:
        f()
    torch.cuda.synchronize()
    try:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for f in fns:
                f()
        torch.cuda.synchronize()
        return g
    except Exception as e:
        log(f"graph capture failed ({e}); timing eagerly")
        return None


def timed_steps(step, steps, warmup):
    """GPU ms per step between two HIP events on the current stream."""
    import torch
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def run_gpu(args, cfg, head=None):
    import torch
    from nwc_amd.nwc_torch import NWCWeight, quantize_fp8, ref_bf16_matvec, ref_fp8_matvec
    layers, shapes, elem, layout = cfg
    light = getattr(args, "light", False)    # extra configs: sweep and per-shape graph times only
    torch.backends.cuda.preferred_blas_library("hipblaslt")
    dev = torch.device("cuda:0")
    props = torch.cuda.get_device_properties(dev)
    log(f"device: {props.name} ({props.gcnArchName}), {props.multi_processor_count} CUs, {props.total_memory/2**30:.0f} GiB")
    cur = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    # ---- compressed stack ----
    t0 = time.time()
    base = []
    for si, (name, M, K) in enumerate(shapes):
        w = make_weight(M, K, 1000 + si)
        c = NWCWeight(w, device=dev, layout=layout, elem=elem)
        x = torch.randn(K, generator=torch.Generator().manual_seed(2000 + si)).to(torch.bfloat16).to(dev)
        base.append((name, M, K, c, x, w))
    copies = {name: [c] + [clone_weight(c) for _ in range(layers - 1)] for name, M, K, c, x, w in base}
    ys = {name: [torch.empty(M, dtype=torch.bfloat16, device=dev) for _ in range(layers)] for name, M, K, *_ in base}
    launches = {name: [Launch(copies[name][l], x, ys[name][l]) for l in range(layers)] for name, M, K, c, x, w in base}
    torch.cuda.synchronize()
    log(f"encoded + placed {len(shapes)}x{layers} compressed matrices in {time.time()-t0:.1f} s")

    # the vocabulary matrix (one per token): two device copies alternate in the timings
    if head is not None:
        hM, hK = head
        hw = make_weight(hM, hK, 1100)
        hc = NWCWeight(hw, device=dev, layout=layout, elem=elem)
        hx = torch.randn(hK, generator=torch.Generator().manual_seed(2100)).to(torch.bfloat16).to(dev)
        base_head = ("lm_head", hM, hK, hc, hx, hw)
        hcopies = [hc, clone_weight(hc)]
        hys = [torch.empty(hM, dtype=torch.bfloat16, device=dev) for _ in hcopies]
        hlaunch = [Launch(cc, hx, y) for cc, y in zip(hcopies, hys)]
        torch.cuda.synchronize()
        log(f"encoded + placed the {hM}x{hK} vocabulary matrix ({hc.bytes / 1e6:.1f} MB)")

    # correctness spot check of the last copies against a torch fp32 matvec on the decoded weights
    checks = [(name, M, K, copies[name][layers - 1], x) for name, M, K, c, x, w in base]
    if head is not None:
        checks.append(("lm_head", hM, hK, hcopies[1], hx))
    for name, M, K, c, x in checks:
        y = c.linear_bf16(x, None).float()
        wd = c.dequant().float()[:, :K]
        if c.scale is not None:
            wd = wd * c.scale[:, None]
        ref = wd @ x.float()
        err = ((y - ref).abs() - (2 ** -8) * ref.abs()).max().item()
        if err > 1e-5:
            raise SystemExit(f"{name}: token path outside tolerance ({err:.3e})")
    del wd, ref
    torch.cuda.empty_cache()

    bytes_tok = sum(c.token_bytes() + 2 * K + 2 * M for name, M, K, c, x, w in base) * layers
    bf16_tok = sum(2 * M * K + 2 * K + 2 * M for name, M, K, *_ in base) * layers

    # ---- per-launch times: a graph of the `layers` copies of one shape (kernel time) and single launches between
    #      events (the reference kernbench's method, which includes the host's launch overhead for small kernels) ----
    per = []
    for name, M, K, c, x, w in base:
        L = launches[name]
        g = graph_stack([(lambda j=j: L[j](cur())) for j in range(layers)])
        us = timed_steps(g.replay, 4, 1) / layers * 1e3 if g is not None else None
        ev = None if light else event_ms(lambda j: L[j](cur()), args.runs, layers)[0]
        nb = c.token_bytes() + 2 * K + 2 * M
        per.append({"layer": name, "M": M, "K": K, "nwc_bytes": c.token_bytes(), "nwc_us": us,
                    "nwc_us_event": None if ev is None else ev * 1e3, "nwc_GBps": nb / (us * 1e-6) / 1e9 if us else None,
                    "hbm_frac": nb / (us * 1e-6) / 1e9 / PEAK_HBM_GBS if us else None})
        del g

    # ---- roofline of the dominant kernel: average launch time of back-to-back gate_up launches (measured here,
    #      next to the per-launch times, before the baselines' allocations) ----
    name, M, K, c, x, w = next(b for b in base if b[0] == DOMINANT)
    L = launches[name]
    dom_bytes = c.token_bytes() + 2 * K + 2 * M
    dom_ms = statistics.median(avg_launch_ms(lambda j: L[j](cur()), layers, 4) for _ in range(5))

    # ---- the timed sweep: one token = all launches of the stack, captured as one HIP graph ----
    def sweep():
        for l in range(layers):
            for name, *_ in base:
                launches[name][l](cur())
    graph = graph_stack([sweep])
    ms_step = timed_steps(graph.replay if graph is not None else sweep, args.steps, args.warmup)

    # ---- the vocabulary matrix: its own launch time, and the sweep followed by it as one graph per token ----
    lm = None
    if head is not None:
        nb = hc.token_bytes() + 2 * hK + 2 * hM
        h_ms = statistics.median(avg_launch_ms(lambda j: hlaunch[j % 2](cur()), 2, 4) for _ in range(5))

        def sweep_head():
            sweep()
            hlaunch[0](cur())
        hgraph = graph_stack([sweep_head])
        ms_head = timed_steps(hgraph.replay if hgraph is not None else sweep_head, args.steps, args.warmup)
        lm = {"M": hM, "K": hK, "nwc_bytes": hc.token_bytes(), "nwc_us": h_ms * 1e3, "nwc_GBps": nb / (h_ms * 1e-3) / 1e9,
              "nwc_hbm_frac": nb / (h_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, "bytes": nb, "us_per_token_with_lm_head": ms_head * 1e3}
        del hgraph

    # ---- hipBLASLt BF16 baseline: the same stack uncompressed ----
    blas = fp8 = bf16rows = None
    if not args.no_baseline and not getattr(args, "no_blas", False):
        import torch.nn.functional as F
        wcopy = {name: [w.to(dev) for _ in range(layers)] for name, M, K, c, x, w in base}
        xs = {name: x.view(1, K) for name, M, K, c, x, w in base}
        blas_per = []
        for name, M, K, *_ in base:
            W = wcopy[name]
            g = graph_stack([(lambda j=j: F.linear(xs[name], W[j])) for j in range(layers)])
            us = timed_steps(g.replay, 4, 1) / layers * 1e3 if g is not None else None
            ev = None if light else event_ms(lambda j: F.linear(xs[name], W[j]), args.runs, layers)[0] * 1e3
            blas_per.append({"layer": name, "us": us, "us_event": ev,
                             "GBps": (2 * M * K + 2 * K + 2 * M) / (us * 1e-6) / 1e9 if us else None})
            del g

        def bsweep():
            for l in range(layers):
                for name, *_ in base:
                    F.linear(xs[name], wcopy[name][l])
        bgraph = graph_stack([bsweep])
        bms = timed_steps(bgraph.replay if bgraph is not None else bsweep, args.steps, args.warmup)
        if elem == "bf16":
            bf16rows = _bf16_rows_baseline(args, base, wcopy, layers, bf16_tok)
        blas = {"us_per_token_graph": bms * 1e3, "us_per_token_sum_of_launches": layers * sum(p["us"] for p in blas_per),
                "GBps": bf16_tok / (bms * 1e-3) / 1e9, "per_layer": blas_per, "bytes_per_token": bf16_tok,
                "library": "torch F.linear, preferred_blas_library=hipblaslt"}
        del wcopy, bgraph
        torch.cuda.empty_cache()
        if head is not None:
            hW = [hw.to(dev) for _ in range(2)]
            hxs = hx.view(1, hK)
            g = graph_stack([(lambda j=j: F.linear(hxs, hW[j])) for j in range(2)])
            h_us = timed_steps(g.replay, 4, 1) / 2 * 1e3

            def bsweep_head():
                bsweep()
                F.linear(hxs, hW[0])
            wcopy = {name: [w.to(dev) for _ in range(layers)] for name, M, K, c, x, w in base}
            bhgraph = graph_stack([bsweep_head])
            bhms = timed_steps(bhgraph.replay if bhgraph is not None else bsweep_head, args.steps, args.warmup)
            blas["lm_head_us"] = h_us
            blas["lm_head_GBps"] = (2 * hM * hK + 2 * hK + 2 * hM) / (h_us * 1e-6) / 1e9
            blas["us_per_token_with_lm_head"] = bhms * 1e3
            del g, bhgraph, hW, wcopy
        torch.cuda.empty_cache()
    if not args.no_baseline:
        if elem == "fp8":
            # the library's uncompressed fp8 weight-only matvec on the same quantized weights (1 byte per weight)
            q8 = {}
            for name, M, K, c, x, w in base:
                q, sc = quantize_fp8(w)
                q8[name] = ([q.to(dev) for _ in range(layers)], sc.to(dev), x.float().to(dev))
            fp8_tok = sum(M * K + 4 * M + 4 * K + 2 * M for name, M, K, *_ in base) * layers
            fp8_per = []
            for name, M, K, *_ in base:
                qs, sc, xf = q8[name]
                us = avg_launch_ms(lambda j: ref_fp8_matvec(qs[j], sc, xf), layers, 4) * 1e3
                fp8_per.append({"layer": name, "us": us, "GBps": (M * K + 4 * M + 4 * K + 2 * M) / (us * 1e-6) / 1e9,
                                "hbm_frac": (M * K + 4 * M + 4 * K + 2 * M) / (us * 1e-6) / 1e9 / PEAK_HBM_GBS})

            def fsweep():
                for l in range(layers):
                    for name, *_ in base:
                        qs, sc, xf = q8[name]
                        ref_fp8_matvec(qs[l], sc, xf)
            fgraph = graph_stack([fsweep])
            fms = timed_steps(fgraph.replay if fgraph is not None else fsweep, args.steps, args.warmup)
            fp8 = {"us_per_token_graph": fms * 1e3, "GBps": fp8_tok / (fms * 1e-3) / 1e9, "bytes_per_token": fp8_tok,
                   "per_layer": fp8_per,
                   "library": "nwc_ref_fp8 (uncompressed fp8 e4m3 + fp32 row scale, 1 byte per weight; bandwidth-tuned "
                              "k_fp8_rows: every load of a wave's rows in flight at once)"}
            if head is not None:                     # the vocabulary matrix through the same kernel, two copies
                hq, hsc = quantize_fp8(hw)
                hqs = [hq.to(dev) for _ in range(2)]
                hsc, hxf = hsc.to(dev), hx.float()
                h_us = avg_launch_ms(lambda j: ref_fp8_matvec(hqs[j % 2], hsc, hxf), 2, 8) * 1e3
                hb = hM * hK + 4 * hM + 4 * hK + 2 * hM
                fp8["lm_head_us"] = h_us
                fp8["lm_head_GBps"] = hb / (h_us * 1e-6) / 1e9
                fp8["lm_head_hbm_frac"] = fp8["lm_head_GBps"] / PEAK_HBM_GBS

                def fsweep_head():
                    fsweep()
                    ref_fp8_matvec(hqs[0], hsc, hxf)
                fhgraph = graph_stack([fsweep_head])
                fp8["us_per_token_with_lm_head"] = timed_steps(fhgraph.replay if fhgraph is not None else fsweep_head,
                                                               args.steps, args.warmup) * 1e3
                del hqs, fhgraph
            del q8, fgraph
            torch.cuda.empty_cache()

    sum_launch_us = layers * sum(p["nwc_us"] for p in per)
    return {
        "ms_step": ms_step, "graph": graph is not None, "bytes_tok": bytes_tok, "bf16_tok": bf16_tok, "per": per,
        "sum_launch_us": sum_launch_us, "dom_bytes": dom_bytes, "dom_us": dom_ms * 1e3,
        "achieved": dom_bytes / (dom_ms * 1e-3) / 1e9, "blas": blas, "fp8": fp8, "lm_head": lm, "bf16rows": bf16rows,
        "device": {"name": props.name, "arch": props.gcnArchName, "cus": props.multi_processor_count},
    }


def _bf16_rows_baseline(args, base, wcopy, layers, bf16_tok):
    """The library's bandwidth-tuned uncompressed BF16 matvec (nwc_ref_bf16: the fp8 baseline's pattern at two bytes
    per weight) over the same stack: per-shape graph times and the per-token sweep."""
    from nwc_amd.nwc_torch import ref_bf16_matvec
    per = []
    for name, M, K, c, x, w in base:
        W = wcopy[name]
        us = avg_launch_ms(lambda j: ref_bf16_matvec(W[j], x), layers, 4) * 1e3
        nb = 2 * M * K + 2 * K + 2 * M
        per.append({"layer": name, "us": us, "GBps": nb / (us * 1e-6) / 1e9, "hbm_frac": nb / (us * 1e-6) / 1e9 / PEAK_HBM_GBS})

    def sweep():
        for l in range(layers):
            for name, M, K, c, x, w in base:
                ref_bf16_matvec(wcopy[name][l], x)
    g = graph_stack([sweep])
    ms = timed_steps(g.replay if g is not None else sweep, args.steps, args.warmup)
    del g
    return {"us_per_token_graph": ms * 1e3, "GBps": bf16_tok / (ms * 1e-3) / 1e9,
            "hbm_frac": bf16_tok / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, "per_layer": per,
            "library": "nwc_ref_bf16 (uncompressed BF16, 2 bytes per weight; k_bf16_rows: every load of a wave's rows in "
                       "flight at once, v_dot2_f32_bf16, fp32 accumulation)"}


def run_stream_ceiling(args, sizes_mb=(14.5, 21.8, 34.1, 68.0), copies=36):
    """The read bandwidth a single launch of a given size reaches on this GPU: nwc_stream_read (every byte read once
    with 16-byte non-temporal loads, one residency round of 256-thread workgroups) over `copies` distinct buffers per
    size, graph-timed like the matvecs.  The sizes are the algorithmic bytes of the four Qwen3-4B matrices (o, qkv,
    down, gate_up)."""
    import torch
    from nwc_amd._abi import call, ptr, stream
    dev = torch.device("cuda:0")
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    grids = (cus, 2 * cus, 4 * cus, 8 * cus)
    out = torch.empty(max(grids), dtype=torch.int32, device=dev)
    rows = []
    for mb in sizes_mb:
        nbytes = int(mb * 1e6) // 16 * 16
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(i) for i in range(copies)]
        per_grid = {}
        for grid in grids:
            per_grid[grid] = avg_launch_ms(lambda j: call("nwc_stream_read", stream(), ptr(bufs[j]), nbytes, ptr(out), grid),
                                           copies, 4) * 1e3
        grid, us = min(per_grid.items(), key=lambda kv: kv[1])
        rows.append({"MB": mb, "us": round(us, 2), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "hbm_frac": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4), "grid": grid,
                     "us_per_grid": {str(k): round(v, 2) for k, v in per_grid.items()}})
        del bufs
        torch.cuda.empty_cache()
    return {"kernel": "k_stream_read (256-thread workgroups, 16-byte non-temporal loads, 8 in flight per thread; the "
                      "fastest of 1, 2, 4 and 8 workgroups per CU)", "copies": copies, "per_size": rows}


def run_prefill(args):
    """configs[2] prefill: per 4B matrix, dequantization into a BF16 buffer + the GEMM of --prefill tokens that
    NWCLinear runs (linear_dequantized: hipBLASLt, or the library's split-K GEMM on the shapes where that measured
    faster), against hipBLASLt on resident BF16 weights (the uncompressed model) and the same GEMM choice on them,
    and (layout 0) the fused prefill kernel without the buffer (nwc_prefill_xbf16, checked against float64 to the
    fp32-accumulation bound); 8 copies rotate so every launch reads HBM."""
    import torch
    import torch.nn.functional as F
    from nwc_amd.nwc_torch import NWCWeight, linear_dequantized
    torch.backends.cuda.preferred_blas_library("hipblaslt")
    dev = torch.device("cuda:0")
    T, R = args.prefill, 8
    rows = []
    for si, (name, M, K) in enumerate(SHAPES):
        w = make_weight(M, K, 1000 + si)
        c = NWCWeight(w, device=dev, layout=args.layout)
        cs = [c] + [clone_weight(c) for _ in range(R - 1)]
        wb = [w.to(dev) for _ in range(R)]
        tmp = torch.empty(M, c.K16, dtype=torch.bfloat16, device=dev)
        x = torch.randn(T, K, generator=torch.Generator().manual_seed(3000 + si)).to(torch.bfloat16).to(dev)
        y = linear_dequantized(x, cs[R - 1].dequant(tmp)[:, :K])
        ref = linear_dequantized(x, wb[0])
        if not torch.equal(y, ref):                 # same BF16 weights, same GEMM: identical outputs
            raise SystemExit(f"{name}: prefill through the compressed weights differs from the resident GEMM")
        refd = x.double() @ wb[0].double().t()
        bound = 2.0 ** -8 * refd.abs() + 2.0 ** -20 * (x.double().abs() @ wb[0].double().abs().t()) + 1e-6
        if ((y.double() - refd).abs() > bound).any():
            raise SystemExit(f"{name}: prefill GEMM outside the fp32-accumulation bound of float64")
        del refd, bound
        modes = [("dequant", [(lambda j=j: cs[j].dequant(tmp)) for j in range(R)]),
                 ("gemm", [(lambda j=j: linear_dequantized(x, tmp[:, :K])) for j in range(R)]),
                 ("dequant_gemm", [(lambda j=j: linear_dequantized(x, cs[j].dequant(tmp)[:, :K])) for j in range(R)]),
                 ("dequant_hipblaslt", [(lambda j=j: F.linear(x, cs[j].dequant(tmp)[:, :K])) for j in range(R)]),
                 ("resident_bf16", [(lambda j=j: F.linear(x, wb[j])) for j in range(R)]),
                 ("resident_same_gemm", [(lambda j=j: linear_dequantized(x, wb[j])) for j in range(R)])]
        if args.layout == 0:
            yf = cs[R - 1].prefill(x, None).double()
            refd = x.double() @ w.to(dev).double().t()
            bound = 2.0 ** -8 * refd.abs() + 2.0 ** -20 * (x.double().abs() @ w.to(dev).double().abs().t()) + 1e-6
            if ((yf - refd).abs() > bound).any():
                raise SystemExit(f"{name}: fused prefill outside the fp32-accumulation bound of float64")
            del yf, refd, bound
            modes.append(("fused", [(lambda j=j: cs[j].prefill(x, None)) for j in range(R)]))
        t = {}
        for key, fns in modes:
            g = graph_stack(fns)
            t[key] = timed_steps(g.replay if g is not None else (lambda: [f() for f in fns]), 5, 2) / R * 1e3
            del g
        dq_bytes = c.bytes + 2 * M * c.K16
        rows.append({"layer": name, "M": M, "K": K, "tokens": T, **{k + "_us": round(v, 2) for k, v in t.items()},
                     "dequant_GBps": round(dq_bytes / (t["dequant"] * 1e-6) / 1e9, 1),
                     "gemm_TFLOPs": round(2 * T * M * K / (t["gemm"] * 1e-6) / 1e12, 1)})
        del cs, wb, tmp
        torch.cuda.empty_cache()
    keys = ("dequant_us", "gemm_us", "dequant_gemm_us", "dequant_hipblaslt_us", "resident_bf16_us",
            "resident_same_gemm_us") + (("fused_us",) if args.layout == 0 else ())
    tot = {k: round(LAYERS * sum(r[k] for r in rows), 1) for k in keys}
    return {"metric": f"{args.prefill}-token prefill per Qwen3-4B stack: dequant to BF16 + GEMM vs resident BF16 GEMM",
            "value": tot["dequant_gemm_us"], "unit": "us", "higher_is_better": False, "dtype": "bf16",
            "config": {"workload": "Qwen3-4B-shaped prefill (BASELINE configs[2]), 36 layers", "layout": args.layout,
                       "tokens": T},
            "per_stack": tot, "overhead_vs_resident": round(tot["dequant_gemm_us"] / tot["resident_bf16_us"], 3),
            "per_layer": rows, "data": "synthetic N(0,0.02^2) BF16 weights, N(0,1) activations"}


def run_batch(args):
    """configs[2] at small batch: --batch T tokens through each 4B matrix (layout 0), the batched fused kernel (the
    matrix decoded once per four tokens, no temporary buffer) against T single-token launches, the reference's path
    for T > 1 (dequantization into a BF16 buffer + hipBLASLt GEMM) and the GEMM on resident BF16 weights; 8 copies
    rotate so every launch reads HBM."""
    import torch
    import torch.nn.functional as F
    from nwc_amd._abi import lib as _lib, ptr as _ptr
    from nwc_amd.nwc_torch import NWCWeight
    torch.backends.cuda.preferred_blas_library("hipblaslt")
    dev = torch.device("cuda:0")
    T, R = args.batch, 8
    cur = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rows = []
    for si, (name, M, K) in enumerate(SHAPES):
        w = make_weight(M, K, 1000 + si)
        c = NWCWeight(w, device=dev, layout=0)
        cs = [c] + [clone_weight(c) for _ in range(R - 1)]
        wb = [w.to(dev) for _ in range(R)]
        tmp = torch.empty(M, c.K16, dtype=torch.bfloat16, device=dev)
        X = torch.randn(T, K, generator=torch.Generator().manual_seed(3000 + si)).to(torch.bfloat16).to(dev)
        Y = torch.empty(T, M, dtype=torch.bfloat16, device=dev)
        ys = [torch.empty(M, dtype=torch.bfloat16, device=dev) for _ in range(T)]
        singles = [[Launch(cc, X[t], ys[t]) for t in range(T)] for cc in cs]
        got = cs[R - 1].linear_batch(X, None)
        ref = torch.stack([cs[R - 1].linear_bf16(X[t], None) for t in range(T)])
        if not torch.equal(got, ref):
            raise SystemExit(f"{name}: batched token path differs from the single-token kernel")
        args_b = []
        for cc in cs:
            st = cc.seq_table()
            args_b.append([(_ptr(cc.data), _ptr(cc.bases), _ptr(cc.hdr), _ptr(cc.lut), _ptr(cc.low),
                            _ptr(st) if st is not None else None, _ptr(X[t0]), None, None, _ptr(Y[t0]),
                            ctypes.c_uint64(cc.n), ctypes.c_uint32(K), ctypes.c_int(cc.code), ctypes.c_uint32(min(4, T - t0)))
                           for t0 in range(0, T, 4)])

        def fused(j):
            for a in args_b[j]:
                if _lib.nwc_linear_xbf16_batch(cur(), *a):
                    raise RuntimeError("nwc_linear_xbf16_batch failed")
        t = {}
        for key, fns in (("fused", [(lambda j=j: fused(j)) for j in range(R)]),
                         ("single_token_launches", [(lambda j=j: [L(cur()) for L in singles[j]]) for j in range(R)]),
                         ("dequant_gemm", [(lambda j=j: F.linear(X, cs[j].dequant(tmp)[:, :K])) for j in range(R)]),
                         ("resident_bf16", [(lambda j=j: F.linear(X, wb[j])) for j in range(R)])):
            g = graph_stack(fns)
            t[key] = timed_steps(g.replay if g is not None else (lambda: [f() for f in fns]), 5, 2) / R * 1e3
            del g
        rows.append({"layer": name, "M": M, "K": K, "tokens": T, **{k + "_us": round(v, 2) for k, v in t.items()},
                     "fused_GBps": round((c.token_bytes() + 2 * T * (K + M)) / (t["fused"] * 1e-6) / 1e9, 1)})
        del cs, wb, tmp, singles
        torch.cuda.empty_cache()
    keys = ("fused_us", "single_token_launches_us", "dequant_gemm_us", "resident_bf16_us")
    tot = {k: round(LAYERS * sum(r[k] for r in rows), 1) for k in keys}
    return {"metric": f"{T}-token batch per Qwen3-4B stack: batched fused decode-matvec vs dequant + hipBLASLt GEMM",
            "value": tot["fused_us"], "unit": "us", "higher_is_better": False, "dtype": "bf16",
            "config": {"workload": "Qwen3-4B-shaped small batch (BASELINE configs[2]), 36 layers", "layout": 0,
                       "tokens": T},
            "per_stack": tot, "speedup_vs_dequant_gemm": round(tot["dequant_gemm_us"] / tot["fused_us"], 3),
            "speedup_vs_single_token_launches": round(tot["single_token_launches_us"] / tot["fused_us"], 3),
            "per_layer": rows, "data": "synthetic N(0,0.02^2) BF16 weights, N(0,1) activations"}


# Qwen3 architectures of the BASELINE configs (config.json of Qwen/Qwen3-0.6B and Qwen/Qwen3-4B), built with random
# N(0, 0.02^2) weights (transformers' default init) since no checkpoint can be fetched here
QWEN3_ARCH = {
    "qwen3-0.6b": dict(hidden_size=1024, intermediate_size=3072, num_hidden_layers=28, num_attention_heads=16),
    "qwen3-4b": dict(hidden_size=2560, intermediate_size=9728, num_hidden_layers=36, num_attention_heads=32),
}


def contiguous_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """Attention for the decode benchmark, with the precision of transformers' eager path (BF16 products with fp32
    accumulation, fp32 softmax) under its boolean SDPA mask (None: SDPA's top-left causal).  The query heads that
    share a KV head are stacked as rows of one product, so the cache is not repeated; every batched product's right
    operand is contiguous (the keys are transposed into a copy), which the BF16 batched GEMMs of this ROCm build need,
    and no tensor is created from host data, so a token step can be captured as a HIP graph."""
    import torch
    B, H, q_len, D = query.shape
    hkv = key.shape[1]
    qg = query.contiguous().view(B, hkv, (H // hkv) * q_len, D)
    s = torch.matmul(qg, key.transpose(2, 3).contiguous()).float().view(B, H, q_len, -1) * scaling
    kv_len = s.shape[-1]
    if attention_mask is not None:
        m = attention_mask[:, :, :, :kv_len]
        s = s.masked_fill(~m, float("-inf")) if m.dtype == torch.bool else s + m.float()
    elif q_len > 1:                                # SDPA's is_causal: query i sees keys 0..i (top-left aligned)
        s = s.masked_fill(torch.ones(q_len, kv_len, dtype=torch.bool, device=s.device).triu(1), float("-inf"))
    p = torch.softmax(s, dim=-1).to(value.dtype).view(B, hkv, -1, kv_len)
    o = torch.matmul(p, value.contiguous()).view(B, H, q_len, D)
    return o.transpose(1, 2).contiguous(), None


def register_attention():
    from transformers import AttentionInterface
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS
    AttentionInterface.register("nwc_contiguous", contiguous_attention)
    ALL_MASK_ATTENTION_FUNCTIONS.register("nwc_contiguous", ALL_MASK_ATTENTION_FUNCTIONS["sdpa"])
    return "nwc_contiguous"


def qwen3_model(cfg_kw, seed=0, device="cuda"):
    """A random-init Qwen3ForCausalLM in BF16 on `device` (tied embeddings, head_dim 128, 8 KV heads, 151936 tokens
    unless cfg_kw says otherwise)."""
    import torch
    from transformers import Qwen3Config, Qwen3ForCausalLM
    kw = dict(vocab_size=151936, head_dim=128, num_key_value_heads=8, tie_word_embeddings=True, rms_norm_eps=1e-6,
              rope_theta=1000000.0, max_position_embeddings=40960)
    kw.update(cfg_kw)
    cfg = Qwen3Config(**kw)
    cfg._attn_implementation = register_attention()
    torch.manual_seed(seed)
    with torch.device(device):
        model = Qwen3ForCausalLM(cfg).to(torch.bfloat16)
    return model.eval()


def greedy_token(lg, width=128):
    """First index of the maximum of a 1-D tensor, as torch.argmax, through per-row maxima over rows of `width`
    elements and an argmax over those: every reduction stays inside one workgroup.  A single argmax over a 151936-entry
    vocabulary is a multi-workgroup reduction whose zero-initialised counters a captured HIP graph does not reset
    correctly on later replays."""
    import torch.nn.functional as F
    n = lg.numel()
    rows = F.pad(lg, (0, (-n) % width), value=float("-inf")).view(-1, width)
    vals, idx = rows.max(dim=1)                         # first maximum of each row
    r = vals.argmax(dim=0, keepdim=True)                # first row holding the overall maximum
    return r * width + idx.gather(0, r)


class GraphDecoder:
    """Batch-1 greedy decode with a static KV cache, one token step captured as a HIP graph and replayed (the
    reference's scripts/graph_decode.py:33-67).  `logits` holds the last step's logits (fp32)."""

    def __init__(self, model, ids, max_new):
        import torch
        from transformers import StaticCache
        self.model, self.ids, self.L = model, ids, ids.shape[1]
        dev = ids.device
        self.cache = StaticCache(config=model.config, max_cache_len=self.L + max_new + 8)
        self.cur = torch.zeros(1, 1, dtype=torch.long, device=dev)
        self.pos = torch.zeros(1, dtype=torch.long, device=dev)
        self.res = torch.zeros(max_new + 1, dtype=torch.long, device=dev)
        self.logits = torch.zeros(model.config.vocab_size, dtype=torch.float32, device=dev)
        self.graph = None

    def prefill(self):
        import torch
        with torch.no_grad():
            self.cache.reset()
            out = self.model(input_ids=self.ids, past_key_values=self.cache, use_cache=True,
                             cache_position=torch.arange(self.L, device=self.ids.device))
            lg = out.logits[0, -1].float()
        self.logits.copy_(lg)
        self.cur.copy_(lg.argmax(-1).view(1, 1))
        self.pos.fill_(self.L)
        self.res.zero_()
        self.res[0] = self.cur[0, 0]

    def step(self):
        import torch
        with torch.no_grad():
            o = self.model(input_ids=self.cur, past_key_values=self.cache, cache_position=self.pos, use_cache=True)
            lg = o.logits[0, -1].float()
            self.logits.copy_(lg)
            nxt = greedy_token(lg)
            self.pos.add_(1)
            self.res.index_copy_(0, self.pos - self.L, nxt)
            self.cur.copy_(nxt.view(1, 1))

    def capture(self):
        """Warm-up steps on a side stream (lazy per-matrix set-up runs there), then the capture; the cache is left
        partly written, so call prefill() before replaying."""
        import torch
        self.prefill()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(3):
                self.step()
        torch.cuda.current_stream().wait_stream(s)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.step()


def compressed_weights_equal(model, orig):
    """(matrices checked, matrices whose decompressed weights differ from `orig` in any bit): every NWCLinear,
    NWCEmbedding and fused-projection slice of a converted model against the BF16 state dict taken before conversion
    (fp8 matrices: against quantize_fp8 of it)."""
    import torch
    from nwc_amd.nwc_torch import NWCEmbedding, NWCLinear, _FusedSlice
    checked = bad = 0
    last = (None, None)
    for name, m in model.named_modules():
        if isinstance(m, _FusedSlice):
            lin = m.group.lin
            if last[0] is not lin:
                last = (lin, lin.w.dequant()[:, :lin.in_features])
            start = m.group.starts[m.index]
            w = last[1][start:start + m.group.sizes[m.index]]
        elif isinstance(m, (NWCLinear, NWCEmbedding)):
            w = m.w.dequant()[:, :m.w.in_features]
        else:
            continue
        ref = orig.get(name + ".weight")
        if ref is None:
            continue
        ref = ref.to(w.device)
        if m_elem(m) == "fp8":                          # the stored values are quantize_fp8's codes, unscaled
            from nwc_amd.nwc_torch import quantize_fp8
            ref = quantize_fp8(ref)[0].to(torch.bfloat16)
        checked += 1
        bad += int(not torch.equal(w.view(torch.int16), ref.view(torch.int16)))
    return checked, bad


def m_elem(m):
    w = m.group.lin.w if hasattr(m, "group") else m.w
    return "fp8" if w.scale is not None else "bf16"


def run_decode(args):
    """Model-level batch-1 decode (the caller above the path): a random-init Qwen3 of the config, greedy tokens from a
    seeded prompt, each token step replayed as one HIP graph; BF16 (hipBLASLt linears) first, then the same model after
    fuse + convert (NWC lossless, layout 0).  Also checks that graph replays reproduce eager steps bit for bit."""
    import torch
    from nwc_amd.nwc_torch import convert, fuse
    torch.backends.cuda.preferred_blas_library("hipblaslt")
    name = args.config if args.config in QWEN3_ARCH else "qwen3-4b"
    dev = torch.device("cuda:0")
    T, C = args.decode, 16
    t0 = time.time()
    model = qwen3_model(QWEN3_ARCH[name], seed=0, device=dev)
    log(f"decode: random-init {name} built in {time.time() - t0:.1f} s")
    ids = torch.randint(0, model.config.vocab_size, (1, 16), generator=torch.Generator().manual_seed(7)).to(dev)
    res = {}
    for mode in ("bf16", "nwc"):
        if mode == "nwc":
            orig = {k: v.detach().cpu().clone() for k, v in model.state_dict().items()
                    if v.dtype == torch.bfloat16 and v.dim() == 2}
            t0 = time.time()
            with contextlib.redirect_stdout(sys.stderr):        # stdout carries the one JSON line only
                fuse(model, device=dev, elem=args.decode_elem)
            nwc_bytes, bf16_bytes = convert(model, device=dev, verbose=False, elem=args.decode_elem)
            torch.cuda.synchronize()
            log(f"decode: fuse + convert in {time.time() - t0:.1f} s, {nwc_bytes / 1e9:.2f} GB compressed of "
                f"{bf16_bytes / 1e9:.2f} GB BF16")
            checked, bad = compressed_weights_equal(model, orig)
            del orig
            log(f"decode: {checked} decompressed matrices checked against the BF16 weights, {bad} differ")
        d = GraphDecoder(model, ids, T + C)
        # eager reference of the first C steps
        d.prefill()
        prefill_logits = d.logits.clone()
        eager = []
        for _ in range(C):
            d.step()
            eager.append(d.logits.clone())
        eager_tokens = d.res[: C + 1].clone()
        d.capture()
        d.prefill()
        same = 0
        for i in range(C):                                 # replays with host work and a sync between them
            d.graph.replay()
            torch.cuda.synchronize()
            same += int(torch.equal(d.logits, eager[i]))
        tokens_ok = bool(torch.equal(d.res[: C + 1], eager_tokens))
        log(f"decode {mode}: {same}/{C} graph replays equal to eager steps, tokens equal {tokens_ok}")
        d.prefill()
        torch.cuda.synchronize()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        w0 = time.time()
        ev0.record()
        for _ in range(T):
            d.graph.replay()
        ev1.record()
        torch.cuda.synchronize()
        wall = time.time() - w0
        ms = ev0.elapsed_time(ev1) / T
        res[mode] = {"ms_per_token": round(ms, 4), "tokens_per_s": round(1e3 / ms, 1),
                     "wall_tokens_per_s": round(T / wall, 1), "graph_replays_equal_eager": f"{same}/{C}",
                     "tokens_equal_eager": tokens_ok, "first_logits": eager[0], "prefill_logits": prefill_logits}
        log(f"decode {mode}: {ms:.3f} ms/token ({1e3 / ms:.1f} tokens/s)")
        del d
        torch.cuda.empty_cache()
    def rel(key):
        a, b = res["nwc"][key], res["bf16"][key]
        return {"max_abs_diff": round(float((a - b).abs().max()), 5), "max_abs": round(float(b.abs().max()), 3),
                "same_argmax": int(a.argmax()) == int(b.argmax())}
    cmp = {"prefill (dequant + hipBLASLt GEMM)": rel("prefill_logits"), "first token step (fused matvecs)": rel("first_logits")}
    for r in res.values():
        del r["first_logits"], r["prefill_logits"]
    a = QWEN3_ARCH[name]
    return {"metric": f"batch-1 greedy decode, random-init {name}, one HIP graph per token", "value": res["nwc"]["tokens_per_s"],
            "unit": "tokens/s", "higher_is_better": True, "dtype": args.decode_elem,
            "config": {"workload": f"{name} ({a['num_hidden_layers']} layers, hidden {a['hidden_size']}), 16-token "
                                   f"seeded prompt, {T} tokens timed", "layout": 0, "nwc_elem": args.decode_elem},
            "bf16_hipblaslt": res["bf16"], "nwc": res["nwc"],
            "speedup_vs_bf16": round(res["bf16"]["ms_per_token"] / res["nwc"]["ms_per_token"], 3),
            "weights_bit_exact": {"matrices": checked, "differing": bad}, "logits_vs_bf16": cmp,
            "data": "random-init N(0,0.02^2) BF16 weights (transformers init), seeded random prompt"}


def run_gather(args):
    """configs[4] embedding: --gather seeded uniform ids from the 152064 x 3584 table, per layout; 16 id sets rotate."""
    import torch
    from nwc_amd.nwc_torch import NWCWeight
    dev = torch.device("cuda:0")
    M, K, n = 152064, 3584, args.gather
    w = make_weight(M, K, 4000)
    out = {}
    for layout in (0, 1, 2):
        c = NWCWeight(w, device=dev, layout=layout)
        ids = [torch.randint(0, M, (n,), generator=torch.Generator().manual_seed(5000 + i)).to(dev) for i in range(16)]
        got = c.gather(ids[0])
        if not torch.equal(got.cpu(), w[ids[0].cpu()]):
            raise SystemExit(f"layout {layout}: gather is not bit-exact")
        g = graph_stack([(lambda j=j: c.gather(ids[j])) for j in range(16)])
        us = timed_steps(g.replay if g is not None else (lambda: [c.gather(i) for i in ids]), 5, 2) / 16 * 1e3
        out[f"layout{layout}"] = {"us": round(us, 2), "table_MB": round(c.bytes / 1e6, 1),
                                  "out_KB": round(n * K * 2 / 1e3, 1)}
        if layout <= 1:
            # NWCWeight.gather takes nwc_gather_xindex (row index) here; the reference's entry point for comparison
            from nwc_amd._abi import lib as _lib, ptr as _ptr, stream as _stream
            rows = torch.empty(n, c.K16, dtype=torch.bfloat16, device=dev)
            ref = lambda j: _lib.nwc_gather(_stream(), *c._streams(), _ptr(ids[j]), n, _ptr(rows), c.n, c.block, K, c.code)
            ref(0)
            if not torch.equal(rows[:, :K].cpu(), w[ids[0].cpu()]):
                raise SystemExit(f"layout {layout}: nwc_gather is not bit-exact")
            g2 = graph_stack([(lambda j=j: ref(j)) for j in range(16)])
            us2 = timed_steps(g2.replay if g2 is not None else (lambda: [ref(j) for j in range(16)]), 5, 2) / 16 * 1e3
            out[f"layout{layout}"]["entry"] = "nwc_gather_xindex" if c.row_index() is not None else "nwc_gather"
            out[f"layout{layout}_nwc_gather"] = {"us": round(us2, 2),
                                                 "entry": "nwc_gather (reference signature, no row index)"}
            del g2
        del c, g
        torch.cuda.empty_cache()
    return {"metric": f"embedding gather of {n} ids from a 152064x3584 compressed table, us per call",
            "value": out["layout2"]["us"], "unit": "us", "higher_is_better": False, "dtype": "bf16",
            "config": {"workload": "Qwen2.5-7B untied embedding (BASELINE configs[4])", "ids": n},
            "per_layout": out, "data": "synthetic N(0,0.02^2) BF16 table, uniform ids from fixed seeds"}


def run_cpu(args):
    """CPU baseline on BASELINE configs[0] (9728 x 2560 BF16, layout 0), each phase at 1 thread and on all host cores:
    encode (the C oracle's single-threaded restatement of the reference encoder, nwc_ops.cu:245-320; all cores: the
    library's multithreaded host encoder, byte-identical), decode (oracle, OpenMP over row groups), fp32 matvec on the
    decoded BF16 weights (oracle), end-to-end decode + fp32 matvec (oracle, the reference's CPU path of
    tests/test_format_cpu.py:36-111), and torch's CPU matvec for context (fp32 weights, and BF16).  Each phase repeats
    for about --cpu-seconds / 10.  `value` is the end-to-end rate on all cores in compressed GB/s."""
    import numpy as np
    import torch
    from nwc_amd._abi import lib as _lib, ptr as _ptr
    from nwc_amd.nwc_torch import NPAIR, HDR_BLOCK, RAW_SLACK, _geometry
    from oracle import oracle as O
    cores = len(os.sched_getaffinity(0))
    M, K = 9728, 2560
    wt = make_weight(M, K, 7)
    w = wt.view(torch.int16).numpy().view(np.uint16)
    per = args.cpu_seconds / 10

    def rate(fn, min_reps=2):
        fn()                                                       # warm-up
        reps, t0 = 0, time.perf_counter()
        while True:
            fn()
            reps += 1
            dt = time.perf_counter() - t0
            if dt >= per and reps >= min_reps:
                return dt / reps, reps

    t0 = time.perf_counter()
    enc = O.encode(w, 0, 0)
    t_enc1 = time.perf_counter() - t0
    nbytes = enc["dl"] + enc["bases"].size * 4 + enc["hdr"].size + 4096 * 4 + enc["n_low"]
    x = torch.randn(K, generator=torch.Generator().manual_seed(8)).to(torch.bfloat16).float().numpy()
    y64 = O.bf16_to_f64(w) @ x.astype(np.float64)
    for th in (1, cores):                                     # checks against the float64 closed form
        assert np.array_equal(O.decode(enc, threads=th), w)
        y = O.linear(enc, x, threads=th)
        assert np.all(np.abs(y - y64) <= 1e-3 * np.abs(y64) + 1e-5), "oracle CPU path outside tolerance"

    # the library's host encoder on all cores (byte-identical to the oracle's output)
    src = wt.view(torch.int16).contiguous()
    nb, n_low, _, _ = _geometry(M, K, 0)
    cap = M * K + M * K // 2 + nb * 64 + 4096
    bufs = dict(freq=torch.empty(NPAIR, dtype=torch.int16), psym=torch.empty(NPAIR, dtype=torch.int16),
                bases=torch.empty(nb, dtype=torch.int32), hdr=torch.empty(nb * HDR_BLOCK, dtype=torch.uint8),
                data=torch.empty(cap, dtype=torch.uint8), low=torch.zeros(n_low + RAW_SLACK, dtype=torch.uint8))
    enc_lib = lambda: _lib.nwc_encode(_ptr(src), M * K, K, 0, _ptr(bufs["freq"]), _ptr(bufs["psym"]), _ptr(bufs["bases"]),
                                      _ptr(bufs["hdr"]), _ptr(bufs["data"]), cap, _ptr(bufs["low"]))
    assert enc_lib() == enc["dl"] and np.array_equal(bufs["data"].numpy()[:enc["dl"]], enc["data"][:enc["dl"]])
    t_enc_all, _ = rate(enc_lib)

    phases = {"encode": {"unit": "M weights/s", "threads_1": round(M * K / t_enc1 / 1e6, 1),
                         f"threads_{cores}": round(M * K / t_enc_all / 1e6, 1),
                         "note": "1 thread: the oracle's restatement of the reference encoder (one run); all cores: the "
                                 "library's host encoder (nwc_encode), byte-identical"}}
    dec = {}
    for key, fn, nb_, unit in (
            ("decode", lambda th: O.decode(enc, threads=th), nbytes, "compressed GB/s"),
            ("fp32_matvec", lambda th: O.matvec_f32(w, x, threads=th), 2 * M * K, "BF16 GB/s"),
            ("end_to_end", lambda th: O.linear(enc, x, threads=th), nbytes, "compressed GB/s")):
        d = {"unit": unit}
        for th in (1, cores):
            t, reps = rate(lambda: fn(th))
            d[f"threads_{th}"] = round(nb_ / t / 1e9, 3)
            d[f"ms_threads_{th}"] = round(t * 1e3, 2)
        phases[key] = d
    nthreads = torch.get_num_threads()
    wf32, xt = wt.float(), torch.from_numpy(x)
    for key, W_, X_ in (("torch_fp32_matvec", wf32, xt), ("torch_bf16_matvec", wt, xt.to(torch.bfloat16))):
        d = {"unit": "GB/s of the weights"}
        for th in (1, cores):
            torch.set_num_threads(th)
            t, reps = rate(lambda: W_ @ X_)
            d[f"threads_{th}"] = round(W_.numel() * W_.element_size() / t / 1e9, 3)
            d[f"ms_threads_{th}"] = round(t * 1e3, 3)
        phases[key] = d
    torch.set_num_threads(nthreads)
    e2e = phases["end_to_end"]
    return {"value": e2e[f"threads_{cores}"], "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"configs[0]: 9728x2560 BF16 layout 0 ({nbytes/1e6:.1f} MB compressed); value = the C oracle's "
                      f"decode + fp32 matvec on {cores} threads ({e2e[f'ms_threads_{cores}']} ms per matvec; "
                      f"{e2e['ms_threads_1']} ms on 1 thread); each phase timed ~{per:.1f} s",
            "us_per_matvec": round(e2e[f"ms_threads_{cores}"] * 1e3, 1), "phases": phases}


def run_encode(args):
    """Host encoder throughput on BASELINE configs[0] (9728 x 2560 BF16, layout 0): the library's multithreaded
    nwc_encode against the C oracle's single-threaded restatement of the reference encoder (nwc_ops.cu:245-320, which
    is single-threaded too), outputs byte-identical.  No GPU needed."""
    import numpy as np
    import torch
    from nwc_amd._abi import lib as _lib, ptr as _ptr
    from nwc_amd.nwc_torch import NPAIR, HDR_BLOCK, RAW_SLACK, _geometry
    from oracle import oracle as O
    M, K = 9728, 2560
    w = make_weight(M, K, 7)
    src = w.view(torch.int16).contiguous()
    n = M * K
    nb, n_low, _, _ = _geometry(M, K, 0)
    cap = n + n // 2 + nb * 64 + 4096
    bufs = dict(freq=torch.empty(NPAIR, dtype=torch.int16), psym=torch.empty(NPAIR, dtype=torch.int16),
                bases=torch.empty(nb, dtype=torch.int32), hdr=torch.empty(nb * HDR_BLOCK, dtype=torch.uint8),
                data=torch.empty(cap, dtype=torch.uint8), low=torch.zeros(n_low + RAW_SLACK, dtype=torch.uint8))

    def ours():
        return _lib.nwc_encode(_ptr(src), n, K, 0, _ptr(bufs["freq"]), _ptr(bufs["psym"]), _ptr(bufs["bases"]),
                               _ptr(bufs["hdr"]), _ptr(bufs["data"]), cap, _ptr(bufs["low"]))
    dl = ours()
    times = []
    for _ in range(5):
        t0 = time.perf_counter()
        ours()
        times.append(time.perf_counter() - t0)
    t_ours = statistics.median(times)
    wn = src.numpy().view(np.uint16)
    t0 = time.perf_counter()
    enc = O.encode(wn, 0, 0)
    t_ref = time.perf_counter() - t0
    same = (enc["dl"] == dl and np.array_equal(enc["data"][:dl], bufs["data"].numpy()[:dl])
            and np.array_equal(enc["bases"], bufs["bases"].numpy().view(np.uint32))
            and np.array_equal(enc["hdr"], bufs["hdr"].numpy()) and np.array_equal(enc["low"], bufs["low"].numpy()))
    if not same:
        raise SystemExit("encoder output differs from the oracle's")
    cores = len(os.sched_getaffinity(0))
    return {"metric": "host encode throughput, 9728x2560 BF16 layout 0 (BASELINE configs[0])",
            "value": round(n / t_ours / 1e6, 1), "unit": "M weights/s", "higher_is_better": True,
            "ms": round(t_ours * 1e3, 2), "byte_identical_to_oracle": same, "cores": cores,
            "cpu_baseline": {"value": round(n / t_ref / 1e6, 1), "unit": "M weights/s", "cores": 1, "kind": "port",
                             "ms": round(t_ref * 1e3, 1),
                             "sample": "the C oracle's single-threaded restatement of the reference encoder, one run"},
            "speedup": round(t_ref / t_ours, 2)}


def _sweep_summary(g, blas_ref=None):
    """The per-token figures of one run_gpu result, for the extra-config keys of the driver line."""
    us = g["ms_step"] * 1e3
    gbps = g["bytes_tok"] / (us * 1e-6) / 1e9
    out = {"us_per_token": round(us, 1), "GBps": round(gbps, 1), "hbm_frac": round(gbps / PEAK_HBM_GBS, 4),
           "bytes_per_token": g["bytes_tok"],
           "per_layer_us": {p["layer"]: round(p["nwc_us"], 2) for p in g["per"]},
           "per_layer_hbm_frac": {p["layer"]: round(p["hbm_frac"], 4) for p in g["per"]}}
    blas = g["blas"] or blas_ref
    if blas is not None:
        out["hipblaslt_us_per_token"] = round(blas["us_per_token_graph"], 1)
        out["speedup_vs_hipblaslt"] = round(blas["us_per_token_graph"] / us, 3)
    if g["bf16rows"] is not None:
        out["uncompressed_bf16_tuned_us_per_token"] = round(g["bf16rows"]["us_per_token_graph"], 1)
        out["speedup_vs_uncompressed_bf16_tuned"] = round(g["bf16rows"]["us_per_token_graph"] / us, 3)
    return out


def run_extras(args):
    """Every other BASELINE config's figure in the default run (sweeps graph-timed as the headline is, without the
    per-launch event timings): configs[1] Qwen3-0.6B layout 0; configs[2] Qwen3-4B layout 1; configs[3] Qwen3-4B fp8
    layouts 0 and 1 against the uncompressed fp8 matvec; configs[4] Qwen2.5-7B layout 2; the 512-token Qwen3-4B
    prefill (layout 0) and the 64-id embedding gather."""
    import copy
    import torch

    def sub(**kw):
        a = copy.copy(args)
        a.light, a.no_cpu, a.no_baseline, a.no_blas = True, True, False, False
        for k, v in kw.items():
            setattr(a, k, v)
        return a

    def cfg(name, layout):
        layers, shapes, elem, _, workload = CONFIGS[name]
        return (layers, shapes, elem, layout), workload

    out = {}
    for key, name, layout, kw in (("qwen3_0.6b_layout0", "qwen3-0.6b", 0, {}),
                                  ("qwen3_4b_layout1", "qwen3-4b", 1, {"no_blas": True}),
                                  ("qwen3_4b_fp8_layout0", "qwen3-4b-fp8", 0, {"no_blas": True}),
                                  ("qwen3_4b_fp8_layout1", "qwen3-4b-fp8", 1, {"no_baseline": True}),
                                  ("qwen2.5_7b_layout2", "qwen2.5-7b-l2", 2, {})):
        t0 = time.time()
        c, workload = cfg(name, layout)
        g = run_gpu(sub(**kw), c, None)
        r = {"workload": f"{workload}, layout {layout}", **_sweep_summary(g)}
        if g["fp8"] is not None:
            r["native_fp8_us_per_token"] = round(g["fp8"]["us_per_token_graph"], 1)
            r["native_fp8_per_layer_us"] = {p["layer"]: round(p["us"], 2) for p in g["fp8"]["per_layer"]}
            out["_native_fp8"] = g["fp8"]["us_per_token_graph"]
        if "fp8" in name and "_native_fp8" in out:
            r["speedup_vs_native_fp8"] = round(out["_native_fp8"] / (g["ms_step"] * 1e3), 3)
        out[key] = r
        log(f"extra config {key}: {r['us_per_token']} us/token ({time.time() - t0:.1f} s)")
        torch.cuda.empty_cache()
    out.pop("_native_fp8", None)
    t0 = time.time()
    pf = run_prefill(sub(prefill=512, layout=0))
    out["qwen3_4b_prefill512_layout0"] = {"us_per_stack": pf["per_stack"], "overhead_vs_resident": pf["overhead_vs_resident"],
                                          "per_layer": pf["per_layer"]}
    log(f"extra: prefill {pf['per_stack']} ({time.time() - t0:.1f} s)")
    torch.cuda.empty_cache()
    t0 = time.time()
    ga = run_gather(sub(gather=64))
    out["qwen2.5_7b_gather64"] = {"per_layout": ga["per_layout"], "unit": "us per call"}
    log(f"extra: gather ({time.time() - t0:.1f} s)")
    return out


def traffic_bytes():
    """HBM bytes per gate_up launch from the committed rocprofv3 counter summary (FETCH_SIZE + WRITE_SIZE, each scaled
    by the factor a plain copy of known size gives), or None when there is none."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)["bytes_per_launch"]
    except (OSError, ValueError, KeyError):
        return None


def run_profile(args):
    """Counter target: --profile-launches launches of one matrix of --config (--profile-shape, default gate_up), after
    three device copies of 256 MiB (the calibration kernel of known size); with --profile-gemm T, launches of the
    prefill GEMM on T tokens and that matrix's shape instead.  Run under rocprofv3 --pmc; prints one line per phase."""
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
    _, shapes, elem, layout0, _ = CONFIGS[args.config]
    layout = args.layout if args.config in ("qwen3-4b", "qwen3-4b-fp8") else layout0
    name, M, K = next(s for s in shapes if s[0] == args.profile_shape)
    if args.profile_gemm:
        # the prefill GEMM alone (nwc_gemm_xbf16) on --profile-gemm tokens and this matrix's shape
        from nwc_amd.nwc_torch import gemm_xbf16
        g = torch.Generator().manual_seed(2)
        x = torch.randn(args.profile_gemm, K, generator=g).to(torch.bfloat16).to(dev)
        ws = [(torch.randn(M, K, generator=g) * 0.02).to(torch.bfloat16).to(dev) for _ in range(4)]
        for i in range(args.profile_launches):
            gemm_xbf16(x, ws[i % len(ws)])
        torch.cuda.synchronize()
        print(f"{name}: {args.profile_launches} launches of nwc_gemm_xbf16, {args.profile_gemm} x {M} x {K}", flush=True)
        return
    c = NWCWeight(make_weight(M, K, 1000 + [s[0] for s in shapes].index(name)), device=dev, layout=layout, elem=elem)
    cs = [c] + [clone_weight(c) for _ in range(7)]
    x = torch.randn(K, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(dev)
    ys = [torch.empty(M, dtype=torch.bfloat16, device=dev) for _ in cs]
    L = [Launch(cc, x, y) for cc, y in zip(cs, ys)]
    sh = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for i in range(args.profile_launches):
        L[i % len(L)](sh)
    torch.cuda.synchronize()
    print(f"{name}: {args.profile_launches} launches, {c.token_bytes() + 2 * K + 2 * M} algorithmic bytes each", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layout", type=int, default=0, choices=[0, 1, 2])
    ap.add_argument("--runs", type=int, default=60, help="launches per shape for the per-launch medians")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-baseline", action="store_true")
    ap.add_argument("--no-lm-head", action="store_true", help="skip the vocabulary matrix's timings")
    ap.add_argument("--no-extras", action="store_true",
                    help="default run: skip the other configs' sweeps, prefill, gather and the streaming ceiling")
    ap.add_argument("--profile-launches", type=int, default=0,
                    help="only run the counter target (copies + this many gate_up launches), for rocprofv3 --pmc")
    ap.add_argument("--profile-shape", default=DOMINANT, choices=[s[0] for s in SHAPES],
                    help="the Qwen3-4B matrix --profile-launches runs")
    ap.add_argument("--profile-gemm", type=int, default=0,
                    help="with --profile-launches: launch the prefill GEMM (nwc_gemm_xbf16) on this many tokens instead")
    ap.add_argument("--config", default="qwen3-4b", choices=sorted(CONFIGS))
    ap.add_argument("--prefill", type=int, default=0, help="time the prefill path for this many tokens instead")
    ap.add_argument("--gather", type=int, default=0, help="time the embedding gather of this many ids instead")
    ap.add_argument("--batch", type=int, default=0,
                    help="time the batched token path for this many tokens (2..8) through each 4B matrix instead")
    ap.add_argument("--encode", action="store_true", help="time the host encoder on configs[0] (no GPU)")
    ap.add_argument("--decode-elem", default="bf16", choices=["bf16", "fp8"],
                    help="--decode: the NWC model's weights, lossless BF16 or weight-only fp8 (BASELINE configs[3])")
    ap.add_argument("--decode", type=int, default=0,
                    help="model-level decode of a random-init Qwen3 (--config qwen3-4b or qwen3-0.6b): this many tokens")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this path (a batch-1 decode-matvec) is not run across GPUs in this build; "
              "use --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.profile_launches:
        run_profile(args)
        return
    if args.prefill or args.gather:
        print(json.dumps(run_prefill(args) if args.prefill else run_gather(args)), flush=True)
        return
    if args.batch:
        print(json.dumps(run_batch(args)), flush=True)
        return
    if args.decode:
        print(json.dumps(run_decode(args)), flush=True)
        return
    if args.encode:
        print(json.dumps(run_encode(args)), flush=True)
        return

    layers, shapes, elem, layout0, workload = CONFIGS[args.config]
    layout = args.layout if args.config in ("qwen3-4b", "qwen3-4b-fp8") else layout0
    g = run_gpu(args, (layers, shapes, elem, layout), None if args.no_lm_head else HEADS[args.config])
    headline = args.config == "qwen3-4b" and layout == 0
    extras = None if args.no_extras or not headline else run_extras(args)
    ceiling = None if args.no_extras or not headline else run_stream_ceiling(args)
    cpu = None if args.no_cpu or args.config != "qwen3-4b" else run_cpu(args)
    us_tok = g["ms_step"] * 1e3
    value = g["bytes_tok"] / (g["ms_step"] * 1e-3) / 1e9
    blas = g["blas"]
    rnd = lambda d: {k: (round(v, 2) if isinstance(v, float) else v) for k, v in d.items()}
    line = {
        "metric": METRIC if args.config == "qwen3-4b" else f"per-token matvec µs + effective HBM GB/s, {args.config} "
                  "shapes batch 1", "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(g["ms_step"], 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp8" if elem == "fp8" else "bf16",
        "data": f"synthetic: N(0,0.02^2) {'weights quantized to fp8 e4m3 per row' if elem == 'fp8' else 'BF16 weights'} "
                f"and N(0,1) activations from fixed seeds; {len(shapes)} matrices encoded once, {layers} device copies each",
        "config": {"workload": f"{workload}, layout {layout}", "layers": layers,
                   "shapes": {n: [M, K] for n, M, K in shapes}, "layout": layout, "elem": elem, "batch": 1,
                   "step": f"one token = {layers * len(shapes)} fused decode-matvecs replayed as one HIP graph"
                           if g["graph"] else f"one token = {layers * len(shapes)} fused decode-matvecs (eager)"},
        "us_per_token": round(us_tok, 1),
        "us_per_token_sum_of_launches": round(g["sum_launch_us"], 1),
        "bytes_per_token": g["bytes_tok"], "bytes_per_token_bf16": g["bf16_tok"],
        "hbm_frac": round(value / PEAK_HBM_GBS, 4),
        # the uncompressed weights' bytes per token over the same time (the reference kernbench's "equivalent" column)
        "bf16_equivalent_GBps": round(g["bf16_tok"] / (us_tok * 1e-6) / 1e9, 1),
        "per_layer": [rnd(p) for p in g["per"]],
        "lm_head": None if g["lm_head"] is None else rnd(g["lm_head"]),
        "with_lm_head": None if g["lm_head"] is None else {
            "us_per_token": round(g["lm_head"]["us_per_token_with_lm_head"], 1),
            "bytes_per_token": g["bytes_tok"] + g["lm_head"]["bytes"],
            "GBps": round((g["bytes_tok"] + g["lm_head"]["bytes"]) / g["lm_head"]["us_per_token_with_lm_head"] / 1e3, 1),
            "hbm_frac": round((g["bytes_tok"] + g["lm_head"]["bytes"]) / g["lm_head"]["us_per_token_with_lm_head"] / 1e3
                              / PEAK_HBM_GBS, 4),
            "hipblaslt_us_per_token": None if blas is None else round(blas["us_per_token_with_lm_head"], 1),
            "native_fp8_us_per_token": None if g["fp8"] is None else round(g["fp8"]["us_per_token_with_lm_head"], 1),
            "speedup_vs_hipblaslt": None if blas is None else round(blas["us_per_token_with_lm_head"] /
                                                                     g["lm_head"]["us_per_token_with_lm_head"], 3),
            "step": f"the {layers * len(shapes)} matvecs of the sweep + the {HEADS[args.config][0]}x"
                    f"{HEADS[args.config][1]} vocabulary matvec, one HIP graph per token"},
        "hipblaslt": None if blas is None else rnd({**blas, "per_layer": [rnd(p) for p in blas["per_layer"]]}),
        "speedup_vs_hipblaslt": None if blas is None else round(blas["us_per_token_graph"] / us_tok, 3),
        "uncompressed_bf16_tuned": None if g["bf16rows"] is None else rnd({**g["bf16rows"], "per_layer": [rnd(p) for p in g["bf16rows"]["per_layer"]]}),
        "speedup_vs_uncompressed_bf16_tuned": None if g["bf16rows"] is None else round(g["bf16rows"]["us_per_token_graph"] / us_tok, 3),
        "stream_ceiling": ceiling,
        "native_fp8": None if g["fp8"] is None else rnd({**g["fp8"], "per_layer": [rnd(p) for p in g["fp8"]["per_layer"]]}),
        "speedup_vs_native_fp8": None if g["fp8"] is None else round(g["fp8"]["us_per_token_graph"] / us_tok, 3),
        "roofline": {"bound": "hbm", "achieved": round(g["achieved"], 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(g["achieved"] / PEAK_HBM_GBS, 4), "traffic": traffic_bytes() if args.config == "qwen3-4b" and layout == 0 else None,
                     "kernel": f"{'k_layout0p<BF16, 8 rows> (token path, BF16 x, one round, 13-bit table, preloaded arguments)' if layout == 0 else f'layout {layout} kernel'}"
                               f": gate_up {dict((n, (M, K)) for n, M, K in shapes)['gate_up']}",
                     "bytes_per_launch": g["dom_bytes"], "avg_launch_us": round(g["dom_us"], 2),
                     "achieved_basis": "NWCWeight.bytes (+ row-index entries read) + x + y of one gate_up launch / "
                                       f"average time of {4 * layers} launches (a HIP graph of {layers} back-to-back "
                                       "launches replayed 4 times between HIP events on the launch stream), median of "
                                       "5 such measurements",
                     "sweep_achieved": round(g["bytes_tok"] / (g["sum_launch_us"] * 1e-6) / 1e9, 1)},
        "cpu_baseline": cpu,
        "configs": extras,
        "device": g["device"],
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
