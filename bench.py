#!/usr/bin/env python3
"""Benchmark of the fused 3-bit codebook MoE decode layer on one MI355X.

Headline workload (one "step" = one MoE layer over one decode batch, inputs resident in HBM):
  D = 6144, 64 routed experts (top-8) + 1 shared expert, SwiGLU intermediate 2048, gate/up/down all CB3 3-bit
  codebook (10 codes per u32, 8 bf16 centroids per (row, 128-column group)), batch 1, router logits ~ N(0,1),
  softmax top-8 renormalized, x bf16 ~ N(0,1).  Synthetic random weights generated on the GPU.
metric: effective weight GB/s = stored bytes of every distinct expert read in the step / step time
        (as % of the 8 TB/s HBM peak), plus microseconds per MoE layer at batch 1 / 8 / 16.

Cache: the layer's weights are rotated over several independent copies (> 256 MB Infinity Cache) and the routing
changes every step, so each step streams cold weights.  Steps are captured back to back in one HIP graph of
--steps steps and replayed; each timed replay is bracketed by device synchronizations and HIP events on the launch
stream, and the headline is the median of --replays timed replays (p10 / p90 under "timing").
CPU baseline: the oracle's C++ OpenMP restatement of the decode (and its NumPy restatement alongside) on the host's
cores, on a bounded sample of the same layer.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20]
"""
import argparse
import ctypes
import json
import re
import math
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0         # dense bf16 matrix-core peak of MI355X
D, E_ROUTED, TOPK, INTER = 6144, 64, 8, 2048
SHARED = E_ROUTED                      # expert index of the shared expert (appended to every table)
LIMIT = 10.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=6, help="independent layer copies rotated between steps")
    ap.add_argument("--replays", type=int, default=9, help="timed replays of the headline graphs (median, p10/p90)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only-b1", action="store_true", help="headline only (profiling runs)")
    ap.add_argument("--only-b816", action="store_true", help="the CB3 layer at batch 8 and 16 only (profiling runs)")
    ap.add_argument("--only-batch", type=int, default=0,
                    help="the CB3 layer at this batch only, with its gate/up and down algorithmic bytes (profiling runs)")
    ap.add_argument("--only-layout", default=None,
                    help="decode at batch 1 and 8 of one table layout only, e.g. iq2s_iq4xs (profiling runs)")
    ap.add_argument("--only-prefill", action="store_true", help="the 512-token prefill chunk only (profiling runs)")
    ap.add_argument("--only-int8", action="store_true", help="the int8 projections and shared MLP only")
    ap.add_argument("--only-bf16", action="store_true", help="the shared expert's MLP over bf16 leaves only")
    ap.add_argument("--only-route", action="store_true", help="the router at 1, 8 and 512 tokens only")
    ap.add_argument("--read-ceiling", action="store_true",
                    help="only the streaming-read probe (the part's practical HBM read rate)")
    ap.add_argument("--tune", action="append", default=[], metavar="NAME=VALUE",
                    help="launch-plan override through mi_tuning_set, for measurement runs (repeatable)")
    ap.add_argument("--calib", action="store_true",
                    help="end with one plain 256 MiB device copy (calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


# ------------------------------------------------------------------------------------------------ synthetic weights
def cb3_bytes(R, K):
    return R * (4 * math.ceil(K / 10) + 16 * (K // 128))


def iq3s_bytes(R, K):
    return R * (K // 256) * 110       # 110-byte blocks of 256 weights (the planes hold exactly these bytes)


def iq4xs_bytes(R, K):
    return R * (K // 256) * 136       # 136-byte blocks of 256 weights


def iq2s_bytes(R, K):
    return R * (K // 256) * 82        # 82-byte blocks of 256 weights


def q2k_bytes(R, K):
    return R * (K // 256) * 84        # 84-byte blocks (the planes hold exactly these)


def q3k_bytes(R, K):
    return R * (K // 256) * 116       # 110-byte blocks; the planes hold the scales unpacked and d padded: 116


def softmax_topk(rng, N, E, k):
    logits = rng.standard_normal((N, E))
    p = np.exp(logits - logits.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    idx = np.argsort(-p, axis=-1)[:, :k].astype(np.int32)
    w = np.take_along_axis(p, idx, -1)
    return idx, (w / w.sum(-1, keepdims=True)).astype(np.float32)


def zipf_topk(rng, N, E, k, s=1.1):
    logp = -s * np.log(np.arange(1, E + 1, dtype=np.float64))
    perm = rng.permutation(E)
    idx = np.zeros((N, k), np.int32)
    for n in range(N):
        idx[n] = perm[np.argsort(-(logp + rng.gumbel(size=E)))[:k]]
    logits = rng.standard_normal((N, k))
    w = np.exp(logits - logits.max(-1, keepdims=True))
    return idx, (w / w.sum(-1, keepdims=True)).astype(np.float32)


# ------------------------------------------------------------------------------------------------ timing
class Timer:
    """Times per-step callables (each one step of the hot path on its own weight copy, used in turn).  The timed
    steps are captured back to back into one HIP graph, so the timed region is the GPU's own time for exactly
    `steps` consecutive steps with no host submission gaps; the warmup steps are a graph of their own."""

    def __init__(self, torch, fns):
        self.torch = torch
        self.fns = fns
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for f in fns:
                f()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()

    def _graph(self, n):
        g = self.torch.cuda.CUDAGraph()
        with self.torch.cuda.graph(g):
            for i in range(n):
                self.fns[i % len(self.fns)]()
        return g

    def run(self, steps, warmup, replays=1):
        """ms per step of the `steps`-step graph: the median over `replays` timed replays (each replay exactly
        `steps` steps, timed on its own between device synchronizations); `self.stats` holds that median and the
        p10 / p90.  The graph's first replay (its one-time upload to the device) is part of the untimed warmup."""
        torch = self.torch
        timed = self._graph(steps)
        if warmup > 0:
            self._graph(warmup).replay()
            timed.replay()
        torch.cuda.synchronize()
        ms = []
        for _ in range(max(1, replays)):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            timed.replay()
            end.record()
            torch.cuda.synchronize()
            ms.append(start.elapsed_time(end) / steps)
        self.stats = stats(ms)
        return float(np.median(ms))                       # ms per step


def stats(values):
    """median, p10 and p90 of a list of per-step times (ms), and their count."""
    v = np.asarray(values, dtype=np.float64)
    return {"n": int(v.size), "median": round(float(np.median(v)), 5), "p10": round(float(np.percentile(v, 10)), 5),
            "p90": round(float(np.percentile(v, 90)), 5)}


# ------------------------------------------------------------------------------------------------ CPU baseline
def host_cores():
    """Host cores this process may use: the affinity set, capped by OMP_NUM_THREADS when that is set."""
    n = len(os.sched_getaffinity(0))
    try:
        n = min(n, int(os.environ.get("OMP_NUM_THREADS", n)))
    except ValueError:
        pass
    return max(1, n)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _timed_reps(fn, budget_s, min_reps=5, max_reps=50):
    """Times fn() repeatedly (after one untimed warm-up call) until budget_s is spent, at least min_reps times."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_reps or (time.perf_counter() < t_end and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return times


def cpu_baseline():
    """The oracle's restatements of the reference's decode path on one batch-1 layer of the same workload (8 routed +
    1 shared CB3 experts), timed on this host's cores: (1) the C++ OpenMP leg (oracle/cpu_moe.cpp: CB3 decoded per
    row, f64 dots, threads over rows) -- `value`; (2) the NumPy leg (oracle.moe.decode_apply: gather -> exact
    dequant to f32 -> f64 matvec, resident.py:122-135 / pallas_moe.py:310-323) with BLAS on the same cores.  Each
    leg: one warm-up, then >= 5 timed layers within a few seconds; median and p10 / p90."""
    from threadpoolctl import threadpool_limits
    from oracle import cb3 as ocb3, cpu_moe, moe as omoe
    cores = host_cores()
    rng = np.random.default_rng(1)
    experts = 9
    gen = {}
    for name, (R, K) in (("gate", (INTER, D)), ("up", (INTER, D)), ("down", (D, INTER))):
        gen[name] = [ocb3.generate(rng, R, K) for _ in range(experts)]
    packed = {name: (np.stack([ocb3.pack_canonical(c) for c, _ in g]), np.stack([cb for _, cb in g]))
              for name, g in gen.items()}
    x = ocb3.bf16_normal(rng, (1, D))
    idx = np.arange(8, dtype=np.int32)[None]
    w = np.full((1, 8), 1.0 / 8, np.float32)
    nbytes = experts * (2 * cb3_bytes(INTER, D) + cb3_bytes(D, INTER))

    cpp = lambda: cpu_moe.decode_cb3(packed["gate"], packed["up"], packed["down"], x, idx, w, LIMIT, shared=8,
                                     threads=cores)
    t_cpp = _timed_reps(cpp, 8.0)
    deq = lambda name, e: ocb3.dequant(*gen[name][e])
    npy = lambda: omoe.decode_apply(deq, x, idx, w, LIMIT) + omoe.shared_apply(lambda m: deq(m, 8), x, LIMIT)
    with threadpool_limits(cores):
        t_npy = _timed_reps(npy, 8.0, min_reps=5, max_reps=5)
    # the two legs compute the same layer
    assert float(np.max(np.abs(cpp() - npy()))) < 1e-6 * float(np.max(np.abs(npy())))
    leg = lambda t: {"us_per_layer": round(float(np.median(t)) * 1e6, 1),
                     "GBps": round(nbytes / float(np.median(t)) / 1e9, 4),
                     "p10_us": round(float(np.percentile(t, 10)) * 1e6, 1),
                     "p90_us": round(float(np.percentile(t, 90)) * 1e6, 1), "layers": len(t)}
    return {"value": round(nbytes / float(np.median(t_cpp)) / 1e9, 4), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": "batch-1 MoE layers (8 routed + 1 shared CB3 experts, D=6144, I=2048, %.0f MB of weights): "
                      "the oracle's C++ OpenMP restatement of the decode path on %d threads, median of %d layers "
                      "(%.1f s); NumPy leg alongside" % (nbytes / 1e6, cores, len(t_cpp), sum(t_cpp)),
            "cpu_model": cpu_model(), "cpp_openmp": leg(t_cpp), "numpy": leg(t_npy)}


def measured_traffic():
    """HBM bytes per gate/up launch of this workload, as measured by the rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    (copy-calibrated) recorded in profiles/gateup_cb3_moe_b1_hbm_traffic.md; None when that record is absent."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "gateup_cb3_moe_b1_hbm_traffic.md")
    try:
        m = re.search(r"HBM bytes per gate/up launch: (\d+)", open(path).read())
    except OSError:
        return None
    return int(m.group(1)) if m else None


# ------------------------------------------------------------------------------------------------ main
def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py measures one GPU: the decode path runs on a single MI355X holding one layer's full expert "
              "set (multi-GPU expert parallelism is a design note, not part of this build); run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import __graft_entry__ as ge
    pkg = ge.load_package()
    pkg._lib.lib()
    for item in args.tune:
        name, _, value = item.partition("=")
        pkg._lib.check("mi_tuning_set(%s)" % name, pkg._lib.lib().mi_tuning_set(name.encode(), int(value)))
    if args.read_ceiling:
        print(json.dumps({"read_ceiling": bench_read_ceiling(torch, pkg, args)}))
        return
    if args.only_int8:
        print(json.dumps({"int8_b8": bench_int8(torch, pkg, torch.Generator(device="cuda"), args)}))
        return
    if args.only_bf16:
        print(json.dumps({"bf16_mlp": bench_bf16_mlp(torch, pkg, torch.Generator(device="cuda"), args)}))
        return
    if args.only_route:
        print(json.dumps({"route": bench_route(torch, pkg, torch.Generator(device="cuda"), args)}))
        return
    torch.manual_seed(0)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1234)
    E = E_ROUTED + 1
    L = args.copies
    per_expert = 2 * cb3_bytes(INTER, D) + cb3_bytes(D, INTER)

    shapes = (("gate", (INTER, D)), ("up", (INTER, D)), ("down", (D, INTER)))
    layers = [{name: pkg.random_cb3_table(E, R, K, gen) for name, (R, K) in shapes} for _ in range(L)]
    torch.cuda.synchronize()
    # the reference's GGUF formats, for their own lines; made on demand, one layout at a time.  A layout names the
    # gate/up format and the down format ("iq2s_iq4xs": the production mix of the reference's GGUF layers).
    makers = {"iq3s": (pkg.random_iq3s_table, iq3s_bytes), "iq4xs": (pkg.random_iq4xs_table, iq4xs_bytes),
              "iq2s": (pkg.random_iq2s_table, iq2s_bytes),
              "q2k": (lambda *a: pkg.random_kq_table("Q2_K", *a), q2k_bytes),
              "q3k": (lambda *a: pkg.random_kq_table("Q3_K", *a), q3k_bytes)}
    made = {}

    def fmts(layout):
        gu, _, dn = layout.partition("_")
        return gu, dn or gu

    def iq_layers(layout):
        if layout not in made:
            made.clear()
            torch.cuda.empty_cache()
            gu, dn = fmts(layout)
            made[layout] = [{name: makers[dn if name == "down" else gu][0](E, R, K, gen) for name, (R, K) in shapes}
                            for _ in range(L)]
            torch.cuda.synchronize()
        return made[layout]

    def iq_pe(layout):
        gu, dn = fmts(layout)
        return 2 * makers[gu][1](INTER, D) + makers[dn][1](D, INTER)

    rng = np.random.default_rng(2026)
    extra = {}

    def layer_fns(N, routing, phases=3, fused=False, tables=None, pe=per_expert, pe_gu=None):
        """Per-copy step callables for batch N (fixed routing per copy, fresh per copy): mi_moe_decode, or the
        one-launch form mi_moe_decode_fused."""
        tables = tables or layers
        pe_gu = pe_gu or 2 * cb3_bytes(INTER, D)
        fns, nbytes = [], []
        ws = torch.zeros(pkg.resident.decode_workspace_bytes(tables[0]["gate"], tables[0]["down"], N, TOPK, SHARED),
                         dtype=torch.uint8, device="cuda")
        out = torch.empty((N, D), dtype=torch.bfloat16, device="cuda")
        for c in range(L):
            idx, w = routing(rng, N, E_ROUTED, TOPK)
            x = torch.randn((N, D), device="cuda", generator=gen).to(torch.bfloat16)
            it, wt = torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda()
            t = tables[c]
            f = (lambda t=t, x=x, it=it, wt=wt: pkg.moe_decode(t["gate"], t["up"], t["down"], x, it, wt, LIMIT,
                                                              shared_expert=SHARED, want_f32=False, out_bf16=out,
                                                              workspace=ws, phases=phases, fused=fused))
            fns.append(f)
            n_exp = len(np.unique(idx)) + 1
            nbytes.append(n_exp * (pe if phases == 3 else pe_gu))
        return fns, nbytes

    timing = {}

    def measure(N, routing, phases=3, steps=args.steps, fused=False, replays=1, key=None, **kw):
        fns, nbytes = layer_fns(N, routing, phases, fused, **kw)
        t = Timer(torch, fns)
        ms = t.run(steps, args.warmup, replays)
        if key:
            timing[key] = t.stats
        avg_bytes = float(np.mean([nbytes[i % L] for i in range(steps)]))
        return ms, avg_bytes

    if args.only_prefill:
        print(json.dumps({"prefill_t512": bench_prefill(torch, pkg, gen, args, layers, rng, per_expert),
                          "prefill_t512_iq3s": bench_prefill(torch, pkg, gen, args, iq_layers("iq3s"), rng,
                                                             iq_pe("iq3s")),
                          "prefill_t512_iq4xs": bench_prefill(torch, pkg, gen, args, iq_layers("iq4xs"), rng,
                                                              iq_pe("iq4xs")),
                          "prefill_t512_iq2s_iq4xs": bench_prefill(torch, pkg, gen, args, iq_layers("iq2s_iq4xs"),
                                                                   rng, iq_pe("iq2s_iq4xs"))}))
        return
    if args.only_batch:
        N = args.only_batch
        ms, b = measure(N, zipf_topk if N > 1 else softmax_topk)
        n_exp = b / per_expert          # distinct experts + the shared one, mean over the timed steps
        print(json.dumps({"b%d" % N: {"us_per_layer": round(ms * 1e3, 2), "GBps": round(b / (ms * 1e-3) / 1e9, 1),
                                       "experts_read_mean": round(n_exp, 3),
                                       "gateup_bytes_mean": int(n_exp * 2 * cb3_bytes(INTER, D)),
                                       "down_bytes_mean": int(n_exp * cb3_bytes(D, INTER))}}))
        if args.calib:
            calib_copy(torch)
        return
    if args.only_b816:
        res = {}
        for N in (8, 16):
            ms, b = measure(N, zipf_topk)
            res["b%d" % N] = {"us_per_layer": round(ms * 1e3, 2), "GBps": round(b / (ms * 1e-3) / 1e9, 1)}
        print(json.dumps(res))
        return
    if args.only_layout:
        fmt = args.only_layout
        res = {}
        for N, routing in ((1, softmax_topk), (8, zipf_topk)):
            ms, b = measure(N, routing, tables=iq_layers(fmt), pe=iq_pe(fmt))
            res["b%d_%s" % (N, fmt)] = {"us_per_layer": round(ms * 1e3, 2), "GBps": round(b / (ms * 1e-3) / 1e9, 1)}
        print(json.dumps(res))
        if args.calib:
            calib_copy(torch)
        return
    # headline: batch 1 layer (mi_moe_decode)
    ms1, bytes1 = measure(1, softmax_topk, replays=args.replays, key="b1")
    gbs1 = bytes1 / (ms1 * 1e-3) / 1e9
    extra["b1"] = {"us_per_layer": round(ms1 * 1e3, 2), "GBps": round(gbs1, 1), "pct_hbm": round(100 * gbs1 / HBM_PEAK_GBS, 1),
                   "bytes_per_layer": int(bytes1)}
    # the gate/up launch alone (gate and up partials; the three-launch form's dominant kernel)
    msg, bytesg = measure(1, softmax_topk, phases=1, replays=args.replays, key="b1_gateup_kernel")
    gbsg = bytesg / (msg * 1e-3) / 1e9
    extra["b1_gateup_kernel"] = {"us": round(msg * 1e3, 2), "GBps": round(gbsg, 1), "bytes": int(bytesg)}
    # the same layer as one persistent launch (mi_moe_decode_fused), for comparison
    msf, bytesf = measure(1, softmax_topk, fused=True)
    extra["b1_one_launch"] = {"us_per_layer": round(msf * 1e3, 2), "GBps": round(bytesf / (msf * 1e-3) / 1e9, 1)}
    # this box's streaming-read rate for the gate/up launch's bytes (parts differ by box): what the launch reaches of it
    rc = bench_read_ceiling(torch, pkg, args, sizes=(118996992,), wgs=(1024, 16384))
    extra["read_ceiling_gateup_bytes"] = {"GBps": rc["best_GBps"], "pct_hbm": rc["pct_hbm"],
                                          "gateup_pct_of_it": round(100 * gbsg / rc["best_GBps"], 1)}
    if not args.only_b1:
        for N in (8, 16):
            ms, b = measure(N, zipf_topk)
            gbs = b / (ms * 1e-3) / 1e9
            extra["b%d" % N] = {"us_per_layer": round(ms * 1e3, 2), "GBps": round(gbs, 1),
                                "pct_hbm": round(100 * gbs / HBM_PEAK_GBS, 1), "bytes_per_layer": int(b)}
        extra["prefill_t512"] = bench_prefill(torch, pkg, gen, args, layers, rng, per_expert)
        # the reference's GGUF formats: IQ3_S and IQ4_XS tables (decode and prefill on the matrix cores)
        for fmt in ("iq3s", "iq4xs", "iq2s", "iq2s_iq4xs", "q2k_q3k"):
            for N, routing in ((1, softmax_topk), (8, zipf_topk)):
                ms, b = measure(N, routing, tables=iq_layers(fmt), pe=iq_pe(fmt))
                gbs = b / (ms * 1e-3) / 1e9
                extra["b%d_%s" % (N, fmt)] = {"us_per_layer": round(ms * 1e3, 2), "GBps": round(gbs, 1),
                                             "pct_hbm": round(100 * gbs / HBM_PEAK_GBS, 1), "bytes_per_layer": int(b)}
            extra["prefill_t512_" + fmt] = bench_prefill(torch, pkg, gen, args, iq_layers(fmt), rng, iq_pe(fmt))
        extra["int8_b8"] = bench_int8(torch, pkg, gen, args)
        extra["bf16_mlp"] = bench_bf16_mlp(torch, pkg, gen, args)
        extra["route"] = bench_route(torch, pkg, gen, args)
        extra["cfg0_matvec"] = bench_matvec(torch, pkg, gen, args)

    kind = pkg.resident.decode_plan(layers[0]["gate"], layers[0]["down"], 1, TOPK, SHARED)["sep_kind"]
    gateup_kernel = {0: "grouped_kernel<gate/up, CB3>", 1: "pstream_kernel<gate/up>",
                     2: "custream_kernel<gate/up>"}[kind]
    roof = {"kernel": gateup_kernel + " (CB3 gate + up partials, batch 1)", "achieved": gbsg,
            "bytes_per_launch": int(bytesg), "us_per_launch": round(msg * 1e3, 2)}
    cpu = None if args.no_cpu else cpu_baseline()
    res = {
        "metric": "effective weight GB/s (% of HBM peak) + µs/MoE layer at batch 1/8/16",
        "value": round(gbs1, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms1, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (random CB3 codes/centroids generated on the GPU; N(0,1) router logits and bf16 activations)",
        "config": {"workload": "moe_decode_layer_b1_cb3", "hidden": D, "routed_experts": E_ROUTED, "topk": TOPK,
                   "shared_experts": 1, "moe_intermediate": INTER, "batch": 1, "format": "CB3",
                   "layer_copies": L, "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": round(roof["achieved"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(roof["achieved"] / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "kernel": roof["kernel"], "bytes_per_launch": roof["bytes_per_launch"],
                     "us_per_launch": roof["us_per_launch"]},
        "timing": {"what": "ms per step over %d timed replays of the %d-step graph (value and ms_per_step: the "
                           "median replay)" % (args.replays, args.steps), **timing},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(res))
    if args.calib:
        calib_copy(torch)


def calib_copy(torch):
    """One plain 256 MiB device-to-device copy: a dispatch of known bytes that calibrates FETCH_SIZE / WRITE_SIZE."""
    a = torch.empty(64 * 1024 * 1024, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()


def bench_read_ceiling(torch, pkg, args, launches=40, sizes=(118996992, 2 * 118996992),
                       wgs=(1024, 2048, 4096, 8192, 16384)):
    """The part's practical streaming-read rate (mi_read_probe): four regions of one size rotated between launches
    (three other regions, > the 256 MB last-level cache, are read between two reads of one region), `launches`
    launches captured in one graph and timed with events; sizes: one gate/up launch of the headline layer
    (118,996,992 B) and twice that; 1024 .. 16384 workgroups of 256 threads.  GB/s per configuration."""
    R, P = pkg.resident, pkg._lib
    res = {}
    for size in sizes:
        regions = [torch.full((size,), i + 1, dtype=torch.uint8, device="cuda") for i in range(4)]
        sink = torch.empty(16384 * 4, dtype=torch.int32, device="cuda")
        for wg in wgs:
            fns = [lambda r=r, wg=wg: P.check("mi_read_probe", P.probe_lib().mi_read_probe(R._ptr(r), size, R._ptr(sink), wg,
                                                                                  R._stream()))
                   for r in regions]
            t = Timer(torch, fns)
            t.run(launches, 4, replays=5)
            ms = t.stats["median"]
            res["%dMB_wg%d" % (size // 1000000, wg)] = {"GBps": round(size / (ms * 1e-3) / 1e9, 1),
                                                        "us": round(ms * 1e3, 2)}
        del regions
        torch.cuda.empty_cache()
    best = max(v["GBps"] for v in res.values())
    return {"best_GBps": best, "pct_hbm": round(100 * best / HBM_PEAK_GBS, 1), "configs": res}


def bench_prefill(torch, pkg, gen, args, layers, rng, per_expert, T=512):
    """Config: a prefill chunk of 512 tokens through the same layer (top-8 of 64 routed experts from N(0,1) router
    logits, plus the shared expert on every token), grouped GEMMs on the matrix cores.  Algorithmic work: every
    (token, expert) row costs 2 * 3 * D * I flops; weight bytes are those of every distinct expert the chunk uses."""
    fns, nbytes = [], []
    tb0 = layers[0]
    ws = torch.zeros(pkg.resident.prefill_workspace_bytes(tb0["gate"], tb0["down"], T, TOPK, SHARED),
                     dtype=torch.uint8, device="cuda")
    out = torch.empty((T, D), dtype=torch.bfloat16, device="cuda")
    for t in layers:
        idx, w = softmax_topk(rng, T, E_ROUTED, TOPK)
        x = torch.randn((T, D), device="cuda", generator=gen).to(torch.bfloat16)
        it, wt = torch.from_numpy(idx).cuda(), torch.from_numpy(w).cuda()
        fns.append(lambda t=t, x=x, it=it, wt=wt: pkg.moe_prefill(t["gate"], t["up"], t["down"], x, it, wt, LIMIT,
                                                                 shared_expert=SHARED, want_f32=False,
                                                                 out_bf16=out, workspace=ws))
        nbytes.append((len(np.unique(idx)) + 1) * per_expert)
    steps = max(1, args.steps // 4)
    ms = Timer(torch, fns).run(steps, max(1, args.warmup // 4))
    rows = T * (TOPK + 1)
    flops = rows * 2.0 * 3 * D * INTER
    tflops = flops / (ms * 1e-3) / 1e12
    gbs = float(np.mean(nbytes)) / (ms * 1e-3) / 1e9
    return {"us_per_layer": round(ms * 1e3, 1), "tokens_per_s": round(T / (ms * 1e-3), 0),
            "TFLOPs": round(tflops, 1), "pct_mfma_bf16_peak": round(100 * tflops / MFMA_BF16_PEAK_TFLOPS, 1),
            "weight_GBps": round(gbs, 1), "rows": rows, "steps": steps}


def bench_route(torch, pkg, gen, args):
    """Config: the MoE block's router (moe_route) over the benchmark layer's 64 routed experts, D = 6144, top-8 with
    normalised, scaled weights, at 1, 8 and 512 tokens.  Work: the f32 router matrix (1.5 MB) read per call."""
    out = {}
    rw = torch.randn((D, E_ROUTED), device="cuda", generator=gen) / math.sqrt(D)
    bias = torch.randn(E_ROUTED, device="cuda", generator=gen) * 0.05
    for N in (1, 8, 512):
        x = torch.randn((N, D), device="cuda", generator=gen).to(torch.bfloat16)
        ws = torch.empty(pkg._lib.lib().mi_moe_route_workspace(N, D, E_ROUTED), dtype=torch.uint8, device="cuda")
        fns = [lambda x=x, ws=ws: pkg.route(x, rw, bias, TOPK, True, 2.5, workspace=ws)]
        ms = Timer(torch, fns).run(args.steps, args.warmup)
        out["n%d" % N] = {"us": round(ms * 1e3, 2), "GBps": round(rw.numel() * 4 / (ms * 1e-3) / 1e9, 1)}
    return out


def bench_int8(torch, pkg, gen, args):
    """Config: the int8 dense projections at batch 8 (Q, K, V, O 6144x6144; the shared expert's MLP 6144 -> 2048 ->
    6144), per-output-channel scales on every projection, bf16 activations, weights in the tiled layout
    (MI355MOE_I8_ROWS=1: the row-major qT, for comparison).  A
    step is the layer's three dependent stages -- Q/K/V of the attention input in one launch, O, and the shared
    expert's mlp_partial (mi_int8_mlp: gate and up in one launch that forms h, then down) -- so projections that share
    their input share a launch, as they can in the model; every launch adds its split-K partials itself.  3 weight
    copies rotated (> the last-level cache)."""
    stages = [[(6144, 6144)] * 3, [(6144, 6144)]]
    B, D, I = 8, 6144, 2048
    copies = 3
    fns = []
    total = sum(i * o + 4 * o for st in stages for i, o in st) + 3 * D * I + 4 * (2 * I + D)
    # weights in the tiled layout (mi_int8_tile, repacked once at load as the IQ planes are)
    tile = (lambda w: w) if os.environ.get("MI355MOE_I8_ROWS") == "1" else pkg.int8_tile
    mk_q = lambda n_out, n_in: tile(torch.randint(-127, 128, (n_out, n_in), dtype=torch.int8, device="cuda",
                                                  generator=gen))
    mk_s = lambda n: torch.rand((n,), device="cuda", generator=gen) * 1.5e-3 + 0.5e-3
    for c in range(copies):
        ops = []
        for st in stages:
            n_in = st[0][0]
            x = torch.randn((B, n_in), device="cuda", generator=gen).to(torch.bfloat16)
            projs, outs = [], []
            for (_, n_out) in st:
                projs.append((mk_q(n_out, n_in), mk_s(n_out)))
                outs.append((torch.empty((B, n_out), dtype=torch.bfloat16, device="cuda"), None))
            n_outs = (ctypes.c_int32 * len(st))(*[o for _, o in st])
            ws = torch.zeros(max(256, pkg._lib.lib().mi_int8_project_many_workspace(B, n_in, n_outs, len(st), 1)),
                             dtype=torch.uint8, device="cuda")
            ops.append((x, projs, outs, ws))
        x = torch.randn((B, D), device="cuda", generator=gen).to(torch.bfloat16)
        mlp = ((mk_q(I, D), mk_s(I), 1), (mk_q(I, D), mk_s(I), 1), (mk_q(D, I), mk_s(D), 1))
        y = torch.empty((B, D), dtype=torch.bfloat16, device="cuda")
        wsm = torch.zeros(pkg._lib.lib().mi_int8_mlp_workspace(B, D, I, 1, 1), dtype=torch.uint8, device="cuda")
        fns.append(lambda ops=ops, x=x, mlp=mlp, y=y, wsm=wsm: (
            [pkg.int8_project_many(xx, projs, outputs=outs, workspace=ws) for (xx, projs, outs, ws) in ops],
            pkg.int8_mlp(x, *mlp, LIMIT, y_bf16=y, workspace=wsm)))
    ms = Timer(torch, fns).run(args.steps, args.warmup)
    gbs = total / (ms * 1e-3) / 1e9
    return {"us_per_layer_int8": round(ms * 1e3, 2), "GBps": round(gbs, 1), "pct_hbm": round(100 * gbs / HBM_PEAK_GBS, 1),
            "bytes": int(total), "launches": "Q+K+V | O | shared MLP: gate+up (forms h), down; split sums in each launch"}


def bench_bf16_mlp(torch, pkg, gen, args, copies=6):
    """The shared expert's mlp_partial over bf16 leaves (the engine's default non-expert weights): D 6144 -> I 2048
    -> 6144, bf16 activations, at batch 1 and 8 (mi_bf16_mlp: gate and up in one launch that forms h, then down).
    A step is one call; `copies` weight copies (75.5 MB each) rotated, more than the last-level cache holds."""
    D, I = 6144, 2048
    total = 3 * D * I * 2
    out = {}
    for B in (1, 8):
        fns = []
        for c in range(copies):
            mk = lambda n_in, n_out: pkg.bf16_leaf(
                (torch.randn((n_in, n_out), device="cuda", generator=gen) * 0.05).to(torch.bfloat16))
            w = (mk(D, I), mk(D, I), mk(I, D))
            x = torch.randn((B, D), device="cuda", generator=gen).to(torch.bfloat16)
            y = torch.empty((B, D), dtype=torch.bfloat16, device="cuda")
            ws = torch.zeros(pkg._lib.lib().mi_bf16_mlp_workspace(B, D, I), dtype=torch.uint8, device="cuda")
            fns.append(lambda x=x, w=w, y=y, ws=ws: pkg.bf16_mlp(x, *w, LIMIT, y_bf16=y, workspace=ws))
        ms = Timer(torch, fns).run(args.steps, args.warmup)
        gbs = total / (ms * 1e-3) / 1e9
        out["b%d" % B] = {"us": round(ms * 1e3, 2), "GBps": round(gbs, 1), "pct_hbm": round(100 * gbs / HBM_PEAK_GBS, 1),
                          "bytes": int(total)}
    return out


def bench_matvec(torch, pkg, gen, args):
    """Config: one CB3 matvec, W 1024 x 2048, x bf16 [1, 2048] (launch-bound correctness config)."""
    R, K = 1024, 2048
    fns = []
    for c in range(4):
        tb = pkg.random_cb3_table(1, R, K, gen)
        x = torch.randn((1, K), device="cuda", generator=gen).to(torch.bfloat16)
        idx = torch.zeros((1,), dtype=torch.int32, device="cuda")
        out = torch.empty((1, R), dtype=torch.float32, device="cuda")
        ws = torch.zeros(pkg._lib.lib().mi_matvec_workspace(tb.c, 1), dtype=torch.uint8, device="cuda")
        fns.append(lambda tb=tb, x=x, idx=idx, out=out, ws=ws: pkg.resident.matvec_into(tb, idx, x, out, ws))
    ms = Timer(torch, fns).run(args.steps, args.warmup)
    nbytes = cb3_bytes(R, K)
    return {"us": round(ms * 1e3, 2), "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1), "bytes": nbytes}


if __name__ == "__main__":
    main()
