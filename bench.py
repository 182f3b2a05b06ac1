#!/usr/bin/env python3
"""ZipGEMM benchmark on one MI355X (the benchmark spec's headline metric, config 2).

Workload (benchmark config 2): Llama-3-8B-shaped projections
qkv 6144x4096, o 4096x4096, gate/up 14336x4096, down 4096x14336 with
W ~ N(0, 0.02) bf16 and 0.1% of entries scaled x30, X[N, K] ~ N(0, 1) bf16.
One *step* is one decoder layer's five ZipGEMMs at every N in {1, 8, 16, 32,
64, 128} (30 launches, split-K 1).  `--layers` distinct compressed layers are
resident in HBM and stepped through round-robin so that weights come from
HBM, not the 256 MB Infinity Cache.  Each layer's 30 launches are captured in
one HIP graph; the timed region replays K graphs.

value  = effective TB/s = sum(2*M*K) / time (uncompressed weight bytes per
         second, the reference's "effective bandwidth",
         kernel_benchmark/bench_zipserv_gemm_sweep.cu:1240-1241).
dense  = the same sweep with torch.matmul over the dense bf16 weights.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "ZipGEMM µs + effective TB/s vs dense BF16 GEMM at N=1–128; compression ratio"
SHAPES = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate", 14336, 4096), ("up", 14336, 4096),
          ("down", 4096, 14336)]
NS = [1, 8, 16, 32, 64, 128]
SPLITS = [1, 2, 4]
HBM_PEAK_GBS = 8000.0
CALIB_BYTES = 256 << 20
COLD_BYTES = 1 << 30      # compressed bytes rotated per (shape, N) timing
COLD_MIN_COPIES = 16


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # untimed steps before the K timed ones: a captured graph runs a few
    # percent slow over its first ~10 ms of replays (the step: 0.575-0.578 ms
    # after 3 warm-up steps, 0.568 after 30, same box; the dense comparator
    # gets the same warm-up)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--layers", type=int, default=4, help="distinct resident layers (>= 3 defeats MALL)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-dense", action="store_true")
    ap.add_argument("--splits", default="1,2,4",
                    help="split-K values tried per (shape, N); the fastest is used")
    ap.add_argument("--no-c3", action="store_true", help="skip the 80-layer Llama-3.1-70B sweep")
    ap.add_argument("--no-attention", action="store_true", help="skip the decode-attention sweep")
    ap.add_argument("--no-kv", action="store_true", help="skip the KV-cache codec sweep")
    ap.add_argument("--eager", default=None, metavar="M,K,N,SPLIT[,ITERS]",
                    help="profiling mode: only launch ZipGEMM of one shape eagerly ITERS times "
                         "(default 32) over HBM-cold copies (for rocprofv3 counter runs, which "
                         "see no graph replays), then print its mean time")
    ap.add_argument("--eager-sweep", type=int, default=0, metavar="ITERS",
                    help="counter mode: after a 256 MiB calibration copy, launch every "
                         "(shape, N, split-K) ZipGEMM of the step's sweep eagerly ITERS times "
                         "over HBM-cold copies, in a fixed order (see pmc_sweep_order)")
    ap.add_argument("--pmc-summary", nargs=2, default=None, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="print the markdown summary of two rocprofv3 --pmc runs (FETCH_SIZE, "
                         "then WRITE_SIZE) of --eager-sweep; no GPU needed")
    ap.add_argument("--pmc-iters", type=int, default=6,
                    help="ITERS of the --eager-sweep run that --pmc-summary reads")
    return ap.parse_args()


def eager_gemm(spec):
    """--eager: one (M, K, N, split-K) ZipGEMM launched eagerly over rotated
    cold copies of N(0, 0.02) bf16 weights (re-tiled layout), preceded by the
    256 MiB negation bench.py uses to calibrate the HBM counters."""
    import torch

    import zipserv_asplos26_amd as zs
    v = [int(x) for x in spec.split(",")]
    M, K, N, sk = v[:4]
    iters = v[4] if len(v) > 4 else 32
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    w = (torch.randn(M, K, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    r = zs.compress_retiled(w, window="weights")
    del w
    copies = [r] + [clone_retiled(r) for _ in range(max(COLD_MIN_COPIES, -(-COLD_BYTES // r.compressed_bytes)) - 1)]
    x = torch.randn(N, K, device=dev, generator=g).to(torch.bfloat16)
    y = torch.empty(N, M, device=dev, dtype=torch.bfloat16)
    ws = zs.codec.splitk_workspace(r, N, sk)
    ca = torch.empty(CALIB_BYTES // 2, device=dev, dtype=torch.bfloat16).fill_(1.0)
    torch.neg(ca, out=torch.empty_like(ca))
    for c in copies[:4]:
        zs.zipgemm(c, x, split_k=sk, out=y, workspace=ws)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for i in range(iters):
        zs.zipgemm(copies[i % len(copies)], x, split_k=sk, out=y, workspace=ws)
    e.record()
    torch.cuda.synchronize()
    t = s.elapsed_time(e) / 1e3 / iters
    print(json.dumps({"eager": {"M": M, "K": K, "N": N, "split_k": sk, "iters": iters,
                                "copies": len(copies), "us": round(t * 1e6, 3),
                                "comp_TBps": round(r.compressed_bytes / t / 1e12, 3)}}))


def schedules(N, splits=SPLITS):
    """Split-K values the step's search tries for batch N: the given
    split-K slices, and for N <= 16 the stream-K schedule (0)."""
    return ([0] if N <= 16 else []) + list(splits)


def pmc_sweep_order():
    """The (shape, M, K, N, split-K) launch groups of --eager-sweep, in the
    order they are dispatched: every combination the step's split-K search
    can pick, so the counters cover whatever split a bench run chooses."""
    return [(name, M, K, N, sk) for name, M, K in SHAPES for N in NS for sk in schedules(N)]


def eager_sweep(iters):
    """--eager-sweep: the 256 MiB calibration negation, then for every entry
    of pmc_sweep_order() `iters` eager ZipGEMM launches (re-tiled layout,
    in-kernel split-K sum, exactly one GEMM dispatch per call) rotating over
    HBM-cold copies of that shape's weights (config 2 distribution)."""
    import torch

    import zipserv_asplos26_amd as zs
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    ca = torch.empty(CALIB_BYTES // 2, device=dev, dtype=torch.bfloat16).fill_(1.0)
    torch.neg(ca, out=torch.empty_like(ca))
    torch.cuda.synchronize()
    del ca
    order = pmc_sweep_order()
    for name, M, K in SHAPES:
        w = torch.randn(M, K, device=dev, generator=g) * 0.02
        mask = torch.rand(M, K, device=dev, generator=g) < 0.001
        w = torch.where(mask, w * 30.0, w).to(torch.bfloat16)
        r = zs.compress_retiled(w)
        del w, mask
        nc = max(COLD_MIN_COPIES, -(-COLD_BYTES // r.compressed_bytes))
        copies = [r] + [clone_retiled(r) for _ in range(nc - 1)]
        for (n2, _, _, N, sk) in [o for o in order if o[0] == name]:
            progress(f"eager sweep {name} N={N} split_k={sk} (0: stream-K)")
            x = torch.randn(N, K, device=dev, generator=g).to(torch.bfloat16)
            y = torch.empty(N, M, device=dev, dtype=torch.bfloat16)
            ws = zs.codec.splitk_workspace(r, N, sk)
            torch.cuda.synchronize()
            for i in range(iters):
                zs.zipgemm(copies[i % nc], x, split_k=sk, out=y, workspace=ws)
            torch.cuda.synchronize()
        del copies, r
        torch.cuda.empty_cache()
    print(json.dumps({"eager_sweep": {"iters": iters, "groups": len(order)}}))


def _read_counter_csv(d):
    """rocprofv3 counter_collection CSV under directory d -> list of
    (kernel name, counter value) in dispatch order."""
    import csv
    import glob
    files = sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True))
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {d}")
    rows = []
    for fn in files:
        with open(fn, newline="") as f:
            for r in csv.DictReader(f):
                rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    rows.sort()
    return [(k, v) for _, k, v in rows]


def pmc_summary(fetch_dir, write_dir, iters):
    """Markdown summary of a FETCH_SIZE and a WRITE_SIZE run of --eager-sweep:
    the negation's reading gives each counter's KiB -> bytes factor, and each
    (shape, N, split-K) group's mean over its `iters` dispatches gives the
    HBM bytes per launch that the roofline's `traffic` averages."""
    fetch, write = _read_counter_csv(fetch_dir), _read_counter_csv(write_dir)
    out = {}
    for label, rows in (("FETCH_SIZE", fetch), ("WRITE_SIZE", write)):
        neg = [v for k, v in rows if "neg" in k.lower()]
        if not neg:
            raise SystemExit(f"{label}: no negation (calibration) dispatch found")
        gem = [(k, v) for k, v in rows if k.startswith("void zs::rgemm") or k.startswith("zs::rgemm")]
        order = pmc_sweep_order()
        if len(gem) != iters * len(order):
            raise SystemExit(f"{label}: {len(gem)} ZipGEMM dispatches, expected "
                             f"{iters} x {len(order)}")
        out[label] = (max(neg), gem)
    cal_f, gf = out["FETCH_SIZE"]
    cal_w, gw = out["WRITE_SIZE"]
    f_fac = (CALIB_BYTES / 1024) / cal_f
    w_fac = (CALIB_BYTES / 1024) / cal_w
    lines = [
        f"Calibration: the {CALIB_BYTES >> 20} MiB bf16 negation reads {cal_f:.0f} KiB "
        f"(FETCH_SIZE factor {f_fac:.4f}) and writes {cal_w:.0f} KiB (WRITE_SIZE factor "
        f"{w_fac:.4f}).",
        "",
        "| shape | M x K | N | split-K | kernel | FETCH KiB | WRITE KiB | HBM bytes per launch |",
        "|---|---|---|---|---|---|---|---|",
    ]
    tail = []
    for gi, (name, M, K, N, sk) in enumerate(pmc_sweep_order()):
        fk = [gf[gi * iters + i] for i in range(iters)]
        wk = [gw[gi * iters + i] for i in range(iters)]
        kern = fk[0][0].replace("void ", "").split("(")[0]
        if any(k.replace("void ", "").split("(")[0] != kern for k, _ in fk + wk):
            raise SystemExit(f"group {name} N={N} split_k={sk}: mixed kernels")
        f = sum(v for _, v in fk) / iters
        w = sum(v for _, v in wk) / iters
        b = int(round(f * 1024 * f_fac + w * 1024 * w_fac))
        lines.append(f"| {name} | {M}x{K} | {N} | {sk} | `{kern}` | {f:.0f} | {w:.0f} | {b} |")
        tail.append(f"traffic {name} N={N} split_k={sk} kernel=`{kern}`: {b}")
    return "\n".join(lines + [""] + tail) + "\n"


PMC_PROFILE = os.path.join("profiles", "zs_rgemm_kernel_pmc_llama3-8b_sweep.md")


def traffic_table(path=None):
    """{(shape, N, split_k): (kernel, HBM bytes per launch)} from the committed
    counter summary, {} when it is absent."""
    path = path or os.path.join(ROOT, PMC_PROFILE)
    tab = {}
    if not os.path.exists(path):
        return tab
    with open(path) as f:
        for line in f:
            if not line.startswith("traffic "):
                continue
            head, val = line.rsplit(":", 1)
            parts = head.split()
            name = parts[1]
            N = int(parts[2].split("=")[1])
            sk = int(parts[3].split("=")[1])
            kern = head.split("kernel=`", 1)[1].rstrip("`")
            tab[(name, N, sk)] = (kern, int(val.strip()))
    return tab


def roofline_traffic(per, kernel, table):
    """Mean counted HBM bytes per launch of `kernel` over the step's launches
    of it (each (shape, N) at the split-K the step uses), or None unless the
    counter table holds every one of those launches under the same kernel."""
    vals = []
    for row in per:
        if row["kernel"] != kernel:
            continue
        hit = table.get((row["shape"], row["N"], row["split_k"]))
        if hit is None or hit[0] != kernel:
            return None
        vals.append(hit[1])
    return int(sum(vals) / len(vals)) if vals else None


def progress(msg):
    """One progress line on stderr (the JSON result alone goes to stdout)."""
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def detail(name, data):
    """One stdout line of detail (`{"detail": name, "data": ...}`), printed
    before the final result line."""
    print(json.dumps({"detail": name, "data": data}), flush=True)


def final_line(res):
    """The compact result line (the last stdout line): the contract's keys,
    the roofline, the CPU baseline and one short summary per benchmark
    config; the per-launch, per-kernel, KV, attention and 70B-sweep rows go
    on the detail lines before it."""
    out = {k: res[k] for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup",
                               "ms_per_step", "higher_is_better", "scaling", "vs_baseline",
                               "dtype", "data", "config", "compression_ratio",
                               "dense_TBps_effective", "speedup_vs_dense")}
    rl = res["roofline"]
    out["roofline"] = {k: rl[k] for k in ("bound", "achieved", "peak", "unit", "frac", "traffic",
                                          "kernel", "avg_launch_us", "launches",
                                          "alg_bytes_per_launch")}
    cb = res.get("cpu_baseline")
    if cb is not None:
        out["cpu_baseline"] = {k: cb[k] for k in ("value", "unit", "cores", "kind", "sample",
                                                  "host_cpu", "compression_ratio",
                                                  "round_trip_bit_exact")}
        out["cpu_baseline"]["value_1core"] = cb["single_core"]["value"]
    per = res.get("per_launch", [])
    if per:
        sp = [r["speedup"] for r in per if "speedup" in r]
        out["per_launch_summary"] = {
            "launches": len(per),
            "speedup_min": min(sp) if sp else None, "speedup_max": max(sp) if sp else None,
            "below_dense": sum(1 for s in sp if s < 1.0)}
    c3 = res.get("c3_70b")
    if c3 is not None:
        out["c3_70b"] = {
            "ratio": c3["compression_ratio"], "gpu_compress_GBps": c3["gpu_compress_GBps"],
            "gpu_compress_kernels_GBps": c3["gpu_compress_kernels_GBps"],
            "per_N [ms/token, comp TB/s, x dense]": {
                str(r["N"]): [r["zip_ms_per_token"], r["comp_TBps"], r["speedup"]]
                for r in c3["per_N"]}}
    at = res.get("attention")
    if at is not None:
        cs = at["cases"]
        out["attention"] = {
            "cases": len(cs), "speedup_min": min(r["speedup"] for r in cs),
            "speedup_max": max(r["speedup"] for r in cs),
            "token_major_vs_head_major": [min(r["token_major_vs_head_major"] for r in cs),
                                          max(r["token_major_vs_head_major"] for r in cs)],
            "B64_T32k_us": next((r["zip_us"] for r in cs if r["B"] == 64 and r["T"] == 32768),
                                None)}
    kv = res.get("kv_cache")
    if kv is not None:
        cs = kv["cases"]
        out["kv_cache"] = {
            "cases": len(cs),
            "bit_exact": all(r.get("bit_exact", True) and r["bit_exact_retiled"] for r in cs),
            "ratio_retiled": [min(r["ratio_retiled"] for r in cs),
                              max(r["ratio_retiled"] for r in cs)]}
    return out


def capture(torch, stream, fn):
    """HIP graph of fn() on `stream` (fn runs once eagerly first to warm)."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        fn()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=stream):
            fn()
    torch.cuda.synchronize()
    return g


def timed(torch, stream, graphs, steps, warmup):
    """Seconds for `steps` replays (round-robin over `graphs`), HIP events on `stream`."""
    for i in range(warmup):
        graphs[i % len(graphs)].replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record(stream)
    with torch.cuda.stream(stream):
        for i in range(steps):
            graphs[i % len(graphs)].replay()
    e.record(stream)
    torch.cuda.synchronize()
    return s.elapsed_time(e) / 1e3


def timed_dist(torch, stream, graph, replays, warmup):
    """Seconds of each of `replays` replays of `graph`, HIP events on `stream`."""
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(replays + 1)]
    with torch.cuda.stream(stream):
        ev[0].record(stream)
        for i in range(replays):
            graph.replay()
            ev[i + 1].record(stream)
    torch.cuda.synchronize()
    return [ev[i].elapsed_time(ev[i + 1]) / 1e3 for i in range(replays)]


# Untimed replays of a freshly captured per-launch graph before its timed
# ones (each replay is one launch on every cold copy, 0.2-1.5 ms): a graph's
# first replays run a few percent slow.
LAUNCH_WARMUP = 8


def pick_schedule(torch, stream, scheds, make_run):
    """The fastest of `scheds` (split-K values) for the launches make_run(sk)
    returns: every candidate is captured first (its workspace allocated),
    then each is timed twice, once in each order, after two warm-up
    replays, and its faster time kept -- a candidate timed right after its
    workspace was allocated, or after a pause, otherwise reads 5-12% slow.
    Returns (split-K, {split-K: seconds})."""
    graphs = {sk: capture(torch, stream, make_run(sk)) for sk in scheds}
    res = {}
    for order in (list(scheds), list(scheds)[::-1]):
        for sk in order:
            t = timed(torch, stream, [graphs[sk]], 2, 2)
            res[sk] = min(t, res.get(sk, float("inf")))
    return min(scheds, key=lambda sk: res[sk]), res


def pct(v, q):
    """q-th percentile (nearest rank) of a list."""
    v = sorted(v)
    return v[min(len(v) - 1, max(0, int(round(q / 100 * (len(v) - 1)))))]


C3_SHAPES = [("qkv", 10240, 8192), ("o", 8192, 8192), ("gate", 28672, 8192), ("up", 28672, 8192),
             ("down", 8192, 28672)]
C3_NS = [1, 8, 16, 32, 64, 128, 256]
C3_LAYERS = 80


def bench_c3(torch, zs, stream, gen, dev):
    """Benchmark config 3: 80 Llama-3.1-70B layers (W ~ N(0, 0.02) bf16) compressed on
    the GPU into the re-tiled layout and resident; per-token time of the 400
    ZipGEMMs at each N, the dense comparator timed on 8 distinct resident layers
    and scaled to 80."""
    comp, enc_t, enc_bytes = [], 0.0, 0
    single_t, single_bytes = 0.0, 0
    dense = []
    group = 8  # layers per encoder call
    for l0 in range(0, C3_LAYERS, group):
        if l0 % 20 == 0:
            progress(f"config 3: compressing layer {l0} of {C3_LAYERS}")
        ws = [(torch.randn(M, K, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
              for _ in range(group) for name, M, K in C3_SHAPES]
        torch.cuda.synchronize()
        # eight layers' forty matrices in one call: the host waits for each
        # outlier total while the GPU encodes the next matrices (the call's
        # last matrices drain with the GPU idle in between: ~0.15 ms a call)
        t0 = time.perf_counter()
        out = zs.compress_retiled_many(ws)
        torch.cuda.synchronize()
        enc_t += time.perf_counter() - t0
        enc_bytes += sum(w.numel() * 2 for w in ws)
        if l0 == 0:  # one call per matrix (a host synchronisation each), for comparison
            for w in ws[:len(C3_SHAPES)]:
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                zs.compress_retiled(w)
                torch.cuda.synchronize()
                single_t += time.perf_counter() - t0
                single_bytes += w.numel() * 2
        if l0 < 8:
            dense.extend(ws)
        del ws
        n = len(C3_SHAPES)
        comp.extend(out[i:i + n] for i in range(0, len(out), n))
    comp_bytes = sum(c.compressed_bytes for L in comp for c in L)
    dense_bytes = C3_LAYERS * sum(2 * M * K for _, M, K in C3_SHAPES)
    # encoder kernels alone on layer 0 (no host size synchronisation)
    k_t = sum(compress_kernel_seconds(torch, zs, w) for w in dense[:len(C3_SHAPES)])
    k_bytes = sum(2 * M * K for _, M, K in C3_SHAPES)
    rows = []
    for N in C3_NS:
        progress(f"config 3: N={N}")
        xs = {K: torch.randn(N, K, device=dev, generator=gen).to(torch.bfloat16)
              for K in {k for _, _, k in C3_SHAPES}}
        ys = {M: torch.empty(N, M, device=dev, dtype=torch.bfloat16) for M in {m for _, m, _ in C3_SHAPES}}

        # split-K per shape (fastest of 1/2/4 over 4 resident layers)
        sk_of, ws_of = {}, {}
        for si, (name, M, K) in enumerate(C3_SHAPES):
            wsk = {sk: zs.codec.splitk_workspace(comp[0][si], N, sk) for sk in schedules(N)}

            def make_run(sk, si=si, M=M, K=K):
                def srun():
                    for li in range(4):
                        zs.zipgemm(comp[li][si], xs[K], split_k=sk, out=ys[M], workspace=wsk[sk])
                return srun
            sk_of[si], _ = pick_schedule(torch, stream, schedules(N), make_run)
            ws_of[si] = wsk[sk_of[si]]

        def zrun():
            for L in comp:
                for si, ((name, M, K), c) in enumerate(zip(C3_SHAPES, L)):
                    zs.zipgemm(c, xs[K], split_k=sk_of[si], out=ys[M], workspace=ws_of[si])

        def drun():
            for li in range(8):
                for si, (name, M, K) in enumerate(C3_SHAPES):
                    torch.matmul(xs[K], dense[li * 5 + si].t(), out=ys[M])
        tz = timed(torch, stream, [capture(torch, stream, zrun)], 3, 1) / 3
        td = timed(torch, stream, [capture(torch, stream, drun)], 3, 1) / 3 * (C3_LAYERS / 8)
        # each shape alone: its 80 resident layers in one graph (ZipGEMM), its
        # 8 dense copies (hipBLASLt), time per GEMM
        shapes = []
        for si, (name, M, K) in enumerate(C3_SHAPES):
            def zone(si=si, M=M, K=K):
                for L in comp:
                    zs.zipgemm(L[si], xs[K], split_k=sk_of[si], out=ys[M], workspace=ws_of[si])

            def done(si=si, M=M, K=K):
                for li in range(8):
                    torch.matmul(xs[K], dense[li * 5 + si].t(), out=ys[M])
            t1 = timed(torch, stream, [capture(torch, stream, zone)], 3, 1) / (3 * C3_LAYERS)
            d1 = timed(torch, stream, [capture(torch, stream, done)], 3, 1) / (3 * 8)
            cb = sum(L[si].compressed_bytes for L in comp) / C3_LAYERS
            shapes.append({"shape": name, "M": M, "K": K, "split_k": sk_of[si],
                           "zip_us": round(t1 * 1e6, 2), "dense_us": round(d1 * 1e6, 2),
                           "speedup": round(d1 / t1, 3),
                           "comp_TBps": round(cb / t1 / 1e12, 3),
                           "eff_TBps": round(2 * M * K / t1 / 1e12, 3)})
        rows.append({"N": N, "split_k": [sk_of[i] for i in range(len(C3_SHAPES))],
                     "zip_ms_per_token": round(tz * 1e3, 3),
                     "dense_ms_per_token": round(td * 1e3, 3), "speedup": round(td / tz, 3),
                     "eff_TBps": round(dense_bytes / tz / 1e12, 3),
                     "comp_TBps": round(comp_bytes / tz / 1e12, 3), "per_shape": shapes})
        del xs, ys
    del comp, dense
    torch.cuda.empty_cache()
    return {"layers": C3_LAYERS, "shapes": {n: [m, k] for n, m, k in C3_SHAPES},
            "weights": "N(0,0.02) bf16", "compression_ratio": round(dense_bytes / comp_bytes, 4),
            "compressed_GB": round(comp_bytes / 1e9, 3), "dense_GB": round(dense_bytes / 1e9, 3),
            "gpu_compress_GBps": round(enc_bytes / enc_t / 1e9, 2),
            "gpu_compress_timing": "host clock around compress_retiled_many over eight layers' "
                                   "forty matrices per call, all 80 layers",
            "gpu_compress_single_call_GBps": round(single_bytes / single_t / 1e9, 2),
            "gpu_compress_kernels_GBps": round(k_bytes / k_t / 1e9, 2),
            "dense_timing": "8 distinct resident layers, scaled x10", "per_N": rows}


ATTN_CASES = [(1, 4096), (1, 16384), (1, 32768), (8, 4096), (8, 16384), (8, 32768), (32, 4096),
              (32, 16384), (32, 32768), (64, 4096), (64, 16384), (64, 32768)]


def kv_tensor(torch, gen, dev, B, T, Hkv=8, D=128):
    """Benchmark configs 4/5: N(0,1) times per-(head, channel) lognormal(0,1) scales."""
    scale = torch.exp(torch.randn(1, 1, Hkv, D, device=dev, generator=gen))
    return (torch.randn(B, T, Hkv, D, device=dev, generator=gen) * scale).to(torch.bfloat16)


def bench_attention(torch, zs, stream, gen, dev):
    """Benchmark config 5: GQA 64/8, D 128, one query token, compressed vs dense KV.
    At B=64, T=32k one K tensor holds 2^31 elements, past the int32 stream
    offsets of the canonical format: that case runs on the re-tiled layout only
    (canonical_us null)."""
    import zipserv_asplos26_amd.attention as za
    rows = []
    for B, T in ATTN_CASES:
        progress(f"config 5: attention B={B} T={T}")
        k = kv_tensor(torch, gen, dev, B, T)
        v = kv_tensor(torch, gen, dev, B, T)
        q = torch.randn(B, 1, 64, 128, device=dev, generator=gen).to(torch.bfloat16)
        canonical = k.numel() <= 2**31 - 1
        ck, cv = (za.compress_kv(k), za.compress_kv(v)) if canonical else (None, None)
        rk, rv = za.compress_kv(k, retiled=True), za.compress_kv(v, retiled=True)
        # token-major caches (rows b * batch_stride + t * Hkv + h): fused attention,
        # and the staged comparator (bench_zipserv_decode_attention.py:752-796) --
        # the caches decompressed into dense buffers, then the dense kernel
        sk_, sv_ = (za.compress_kv(k, layout="token_major", retiled=True),
                    za.compress_kv(v, layout="token_major", retiled=True))
        kbuf = torch.empty(sk_.rows, sk_.cols, dtype=torch.bfloat16, device=dev)
        vbuf = torch.empty(sv_.rows, sv_.cols, dtype=torch.bfloat16, device=dev)
        cap = sk_.rows // B // 8
        sl = torch.full((B,), T, dtype=torch.int32, device=dev)

        def staged():
            zs.decompress_retiled(sk_, kbuf)
            zs.decompress_retiled(sv_, vbuf)
            za.flash_attn_with_kvcache_dense(q, kbuf.view(B, cap, 8, 128), vbuf.view(B, cap, 8, 128),
                                             cache_seqlens=sl)
        torch.cuda.synchronize()
        reps = 10
        tc = timed(torch, stream, [capture(torch, stream, lambda: [
            za.flash_attn_with_kvcache_zipserv(q, ck, cv, 8, T) for _ in range(reps)])], 3, 1) / (
            3 * reps) if canonical else None
        tz = timed(torch, stream, [capture(torch, stream, lambda: [
            za.flash_attn_with_kvcache_zipserv(q, rk, rv, 8, T) for _ in range(reps)])], 3, 1) / (3 * reps)
        td = timed(torch, stream, [capture(torch, stream, lambda: [
            za.flash_attn_with_kvcache_dense(q, k, v) for _ in range(reps)])], 3, 1) / (3 * reps)
        tt = timed(torch, stream, [capture(torch, stream, lambda: [
            za.flash_attn_with_kvcache_zipserv(q, sk_, sv_, 8, T) for _ in range(reps)])], 3, 1) / (
            3 * reps)
        ts = timed(torch, stream, [capture(torch, stream, lambda: [
            staged() for _ in range(reps)])], 3, 1) / (3 * reps)
        comp = rk.compressed_bytes + rv.compressed_bytes
        dense = 2 * k.numel() * 2
        rows.append({"B": B, "T": T, "zip_us": round(tz * 1e6, 2),
                     "canonical_us": round(tc * 1e6, 2) if tc else None,
                     "dense_us": round(td * 1e6, 2),
                     "token_major_us": round(tt * 1e6, 2),
                     "staged_us": round(ts * 1e6, 2),
                     "speedup": round(td / tz, 3), "speedup_vs_staged": round(ts / tz, 3),
                     "token_major_vs_head_major": round(tz / tt, 3),
                     "token_major_speedup": round(td / tt, 3),
                     "ratio": round(dense / comp, 4),
                     "comp_TBps": round((comp + 2 * 2 * B * 64 * 128) / tz / 1e12, 3),
                     "dense_TBps": round((dense + 2 * 2 * B * 64 * 128) / td / 1e12, 3)})
        del k, v, q, ck, cv, rk, rv, sk_, sv_, kbuf, vbuf
        torch.cuda.empty_cache()
    return {"heads": 64, "heads_k": 8, "head_dim": 128, "kv": "N(0,1) x lognormal(0,1) per channel",
            "note": "reps captured in one HIP graph; time per call; zip_us = fused over re-tiled "
                    "head-major KV, canonical_us = fused over canonical TCA-TBE KV, "
                    "token_major_us = fused over re-tiled token-major KV, staged_us = the "
                    "token-major caches decompressed into dense buffers then the dense kernel, "
                    "dense_us = the dense kernel over bf16 KV", "cases": rows}


# Benchmark config 4 (B 1-32, 8 KV heads, T 1k-128k, D 128); (32, 128k) is
# 2^32 elements per tensor.
KV_CASES = [(1, 1024), (1, 32768), (1, 131072), (8, 32768), (8, 131072), (32, 16384),
            (32, 131072)]


def bench_kv(torch, zs, dev, gen):
    """Benchmark config 4: KV-cache compress / decompress throughput (GB/s of
    original bytes), ratio and bit-exact recovery, by_kv_head layout, for the
    canonical streams and the re-tiled layout."""
    import zipserv_asplos26_amd.attention as za

    def clock(fn, reps=5):
        fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / (reps * 1e3)

    def host_clock(fn):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        res = fn()
        torch.cuda.synchronize()
        return time.perf_counter() - t0, res

    rows = []
    for B, T in KV_CASES:
        progress(f"config 4: KV codec B={B} T={T}")
        x = kv_tensor(torch, gen, dev, B, T)
        mat, _, _ = za.pad_batched_kv_prefix_by_kv_head(x)
        mat = mat.contiguous()
        del x
        nbytes = mat.numel() * 2
        out = torch.empty_like(mat)
        # canonical streams hold int32 offsets: caches past 2^31 elements
        # are re-tiled only
        canonical = mat.numel() <= 2**31 - 1 - 16 * (mat.numel() // 4096)
        row = {"B": B, "T": T, "elements": mat.numel()}
        if canonical:
            tc, c = host_clock(lambda: zs.compress(mat))
            td = clock(lambda: zs.decompress_zipserv_into(
                out, *c.streams(), c.rows, c.cols, c.max_high_freq_count, c.max_full_count,
                c.start_exp))
            row.update({"ratio": round(nbytes / c.compressed_bytes, 4),
                        "compress_GBps": round(nbytes / tc / 1e9, 2),
                        "decompress_GBps": round(nbytes / td / 1e9, 2),
                        "bit_exact": bool(torch.equal(out.view(torch.int16), mat.view(torch.int16)))})
            del c
        tr, r = host_clock(lambda: zs.compress_retiled(mat))
        tk = compress_kernel_seconds(torch, zs, mat)
        tdr = clock(lambda: zs.decompress_retiled(r, out))
        row.update({"ratio_retiled": round(nbytes / r.compressed_bytes, 4),
                    "compress_retiled_GBps": round(nbytes / tr / 1e9, 2),
                    "compress_retiled_kernels_GBps": round(nbytes / tk / 1e9, 2),
                    "decompress_retiled_GBps": round(nbytes / tdr / 1e9, 2),
                    "bit_exact_retiled": bool(torch.equal(out.view(torch.int16),
                                                          mat.view(torch.int16)))})
        rows.append(row)
        del mat, r, out
        torch.cuda.empty_cache()
    return {"layout": "by_kv_head",
            "compress_timing": "host clock around one call incl. its size sync; *_kernels_GBps: "
                               "HIP events around the encoder's kernels alone",
            "decompress_timing": "HIP events, 5 calls", "cases": rows}


def kernel_name(N, M, split_k, K):
    """Kernel that zs_retiled_mm launches for batch N (mirrors its dispatch):
    N <= 16 -> rgemm_kernel<F, 1, W, D, XD> (F bands per wave: 2 when N > 8
    and M/16 >= 384, else 1; one 16-column block; W = 4 waves when M/16 >= 640
    (N > 1) or M/16 >= 896 (N = 1), else 8; records D = 4 tiles ahead with one
    band per wave, 3
    with two; X staged through LDS in XD-row loads: 1 for N <= 2, 2 for
    N <= 4, 4 for N <= 8, none (0) above); N > 16 ->
    rgemm_wide_kernel<NB, 4, PH, 2> with NB = 2, 4 or 8
    column blocks, 4 row bands, 4 K phases when M/64 * split_k <= the CU
    count (2 otherwise), records 2 steps ahead; on grids of >= 160 128-row
    workgroups rgemm_wide2_kernel<NB, 8, 2> (two bands per wave) instead,
    for N > 64 at any split-K and for 16 < N <= 64 at split-K 1 or 2;
    4 <= N <= 16 on grids of M/64 * split_k >= 7/8 of the CU count ->
    rgemm_wide_kernel<1, 4, PH, 2>; NB = 8 outside the two-band case takes 3
    K phases when the split-K slice has >= 32 K tiles."""
    import torch
    nb = (N + 15) // 16
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if split_k == 0:  # stream-K schedule (narrow batches)
        xd = 1 if N <= 2 else (2 if N <= 4 else (4 if N <= 8 else 0))
        return f"zs::rgemm_sk_kernel<4, {xd}>"
    if nb <= 1 and N >= 4 and (M // 64) * split_k * 8 >= cus * 7:
        ph = 4 if (M // 64) * split_k <= cus else 2
        return f"zs::rgemm_wide_kernel<1, 4, {ph}, 2>"
    if nb <= 1:
        waves = 4 if M // 16 >= (640 if N > 1 else 896) else 8
        f = 2 if (N > 8 and M // 16 >= 384) else 1
        xd = 1 if N <= 2 else (2 if N <= 4 else (4 if N <= 8 else 0))
        return f"zs::rgemm_kernel<{f}, 1, {waves}, {4 if f == 1 else 3}, {xd}>"
    nb = 2 if nb <= 2 else (4 if nb <= 4 else 8)
    if nb == 2 and M % 128 == 0 and split_k <= 2 and (M // 128) * split_k >= 160:
        return "zs::rgemm_wide2_kernel<2, 8, 2>"
    if nb == 8 and M % 128 == 0 and (M // 128) * split_k * ((N + 127) // 128) >= 160:
        return "zs::rgemm_wide2_kernel<8, 8, 2>"
    if nb == 4 and M % 128 == 0 and split_k <= 2 and (M // 128) * split_k >= 160:
        return "zs::rgemm_wide2_kernel<4, 8, 2>"
    ph = 4 if (nb <= 4 and (M // 64) * split_k <= cus) else 2
    if nb == 8 and ((K // 64) - 1) // split_k + 1 >= 32:
        ph = 3
    return f"zs::rgemm_wide_kernel<{nb}, 4, {ph}, 2>"


def compress_kernel_seconds(torch, zs, x, window="kv", reps=3):
    """Device time of the re-tiled GPU encoder's kernels on the bf16 matrix x
    (window guess from a sample, fixed parts + counts + full histogram in one
    input pass, window check -- a second pass only when the guess was wrong --
    offset scan, exponent-byte compaction), HIP events on the current stream,
    with every buffer allocated beforehand so that no host size
    synchronisation sits between the phases (compress_retiled needs one to
    size the stream)."""
    L = zs.lib()
    rows, cols = x.shape
    nrec = rows // 16 * (cols // 64)
    dev = x.device
    i32 = dict(dtype=torch.int32, device=dev)
    top, hist = torch.empty(7, **i32), torch.empty(256, dtype=torch.int64, device=dev)
    cnt, eoff = torch.empty(nrec, **i32), torch.empty(nrec + 1, **i32)
    total = torch.empty(1, dtype=torch.int64, device=dev)
    fixed = torch.empty(nrec * 1408, dtype=torch.uint8, device=dev)
    tmp = torch.empty(nrec * zs._lib.ZS_RETILED_EXP_SLOT_BYTES, dtype=torch.uint8, device=dev)
    work = torch.empty(zs._lib.ZS_RETILED_AUTO_WORK_BYTES, dtype=torch.uint8, device=dev)
    nexp = zs.compress_retiled(x, window=window).num_outliers
    exps = torch.empty(nexp + 64, dtype=torch.uint8, device=dev)
    rule = zs._lib.ZS_WINDOW_KV if window == "kv" else zs._lib.ZS_WINDOW_WEIGHTS

    def run():
        st = torch.cuda.current_stream().cuda_stream
        assert L.zs_compress_retiled_auto_gpu(st, x.data_ptr(), rows, cols, rule, hist.data_ptr(),
                                              top.data_ptr(), work.data_ptr(), fixed.data_ptr(),
                                              cnt.data_ptr(), eoff.data_ptr(), total.data_ptr(),
                                              tmp.data_ptr()) == 0
        assert L.zs_compress_retiled_exps_gpu(st, x.data_ptr(), rows, cols, top.data_ptr(),
                                              eoff.data_ptr(), tmp.data_ptr(), exps.data_ptr()) == 0
    run()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        run()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / 1e3 / reps


def clone_retiled(r):
    """A second resident copy of a re-tiled matrix (distinct addresses)."""
    import dataclasses
    return dataclasses.replace(r, fixed=r.fixed.clone(), exps=r.exps.clone(), eoff=r.eoff.clone())


def clone_canonical(c):
    """A second resident copy of canonical device streams."""
    import dataclasses
    return dataclasses.replace(
        c, sign_mantissa=c.sign_mantissa.clone(), compressed_full=c.compressed_full.clone(),
        bitmap1=c.bitmap1.clone(), bitmap2=c.bitmap2.clone(), bitmap3=c.bitmap3.clone(),
        tile_offsets_median=c.tile_offsets_median.clone(),
        tile_offsets_global=c.tile_offsets_global.clone())


def make_layer(torch, zs, gen, dev):
    """Synthetic bf16 weights of one layer, compressed on the GPU into the
    canonical streams (c) and the re-tiled device layout built from them (r)."""
    layer = []
    for name, M, K in SHAPES:
        w = torch.randn(M, K, device=dev, generator=gen) * 0.02
        mask = torch.rand(M, K, device=dev, generator=gen) < 0.001
        w = torch.where(mask, w * 30.0, w).to(torch.bfloat16)
        c = zs.compress(w)
        layer.append((name, M, K, w, c, zs.retile(c)))
    return layer


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo) and the cores this process may use."""
    name = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return name, usable


def median_time(fn, runs=10, warmup=2):
    """Median seconds of `runs` calls after `warmup` (steady_clock-style wall
    time, as the reference's CPU benchmarks time their codec)."""
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def cpu_baseline(threads_cap=16):
    """Benchmark config 1 on the host: the seed-0 4096x4096 N(0, 0.02) bf16
    matrix through the oracle's C restatement of the reference's CPU codec --
    window (utils.h:189-272), InitBF16MatrixTripleBitmap (scalar 7-way search,
    L_API.cu:314-557) and _Reuse_SIMD (SSE, L_API.cu:773-1053), the CPU
    decoder (bench_kv_cache_zipserv_decompress_token_scaling.cu:2106-2218) --
    with a bit-exact round-trip check, then Y = X W^T with X [8, 4096] ~ N(0, 1)
    and fp32 accumulation.  Each stage: median of 10 runs after 2 warm-ups,
    on 1 core and on all usable cores (OpenMP over global tiles / rows, the
    reference benchmarks' MT mode); output allocation (malloc + memset, inside
    the reference's timed compress) reported apart from the encode.  `value`
    is the all-cores decode + GEMM rate in the metric's unit (effective TB/s,
    uncompressed weight bytes over time)."""
    import numpy as np

    import oracle as zo
    model, usable = cpu_model()
    threads = max(1, min(usable, threads_cap))
    rng = np.random.default_rng(0)
    W = zo.f32_to_bf16(rng.standard_normal((4096, 4096), dtype=np.float32) * np.float32(0.02))
    X = zo.f32_to_bf16(np.random.default_rng(1).standard_normal((8, 4096), dtype=np.float32))
    M, K = W.shape
    nbytes = 2 * M * K
    t_an = median_time(lambda: zo.analyze_cpu(W))
    top = zo.analyze_cpu(W)
    enc = {}
    for variant, nt in (("plain", 1), ("sse", 1), ("sse_mt", threads)):
        tm = []

        def run(variant=variant, nt=nt):
            t = {}
            zo.compress(W, top=top, variant=variant, threads=nt, timings=t)
            tm.append(t)
        median_time(run)
        tm = tm[2:]
        enc[variant] = {"alloc_ms": round(sorted(t["alloc_s"] for t in tm)[len(tm) // 2] * 1e3, 3),
                        "encode_ms": round(sorted(t["encode_s"] for t in tm)[len(tm) // 2] * 1e3, 3)}
    e = zo.compress(W, top=top, variant="sse")
    exact = bool(np.array_equal(zo.decompress(e), W))
    ratio = nbytes / e.compressed_bytes()
    t_dec1 = median_time(lambda: zo.decompress_mt(e, 1))
    t_decN = median_time(lambda: zo.decompress_mt(e, threads))
    t_gemm1 = median_time(lambda: zo.gemm_f32_mt(W, X, 1))
    t_gemmN = median_time(lambda: zo.gemm_f32_mt(W, X, threads))
    tN = t_decN + t_gemmN
    t1 = t_dec1 + t_gemm1
    return {
        "value": round(nbytes / tN / 1e12, 6),
        "unit": "TB/s",
        "cores": threads,
        "kind": "port",
        "sample": ("benchmark config 1: 4096x4096 N(0,0.02) bf16 (seed 0) decompressed by the "
                   "oracle's CPU decoder, then Y = X W^T with X [8, 4096] and fp32 accumulation; "
                   f"median of 10 runs on {threads} threads (effective TB/s = 2*M*K / time)"),
        "host_cpu": model,
        "host_cores_usable": usable,
        "compression_ratio": round(ratio, 4),
        "round_trip_bit_exact": exact,
        "analyze_ms": round(t_an * 1e3, 3),
        "compress_ms": {"scalar_1core": enc["plain"], "sse_1core": enc["sse"],
                        f"sse_{threads}threads": enc["sse_mt"]},
        "compress_GBps_sse_all_cores": round(nbytes / (enc["sse_mt"]["encode_ms"] * 1e-3) / 1e9, 3),
        "decompress_ms": {"1core": round(t_dec1 * 1e3, 3), f"{threads}threads": round(t_decN * 1e3, 3)},
        "gemm_n8_ms": {"1core": round(t_gemm1 * 1e3, 3), f"{threads}threads": round(t_gemmN * 1e3, 3)},
        "single_core": {"value": round(nbytes / t1 / 1e12, 6), "unit": "TB/s",
                        "seconds": round(t1, 4)},
        "seconds": round(tN, 4),
    }


def main():
    args = parse()
    if args.pmc_summary:
        print(pmc_summary(args.pmc_summary[0], args.pmc_summary[1], args.pmc_iters), end="")
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1 "
                          "(multi-GPU sharding is a design note, not a run mode)"}))
        sys.exit(2)
    import torch

    import zipserv_asplos26_amd as zs
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.eager:
        eager_gemm(args.eager)
        return
    if args.eager_sweep:
        eager_sweep(args.eager_sweep)
        return
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)

    progress("config 2: compressing layers")
    t0 = time.perf_counter()
    layers = [make_layer(torch, zs, gen, dev) for _ in range(args.layers)]
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t0
    xs = {(N, K): torch.randn(N, K, device=dev, generator=gen).to(torch.bfloat16)
          for N in NS for K in {k for _, _, k in SHAPES}}
    outs = {(N, M): torch.empty(N, M, device=dev, dtype=torch.bfloat16)
            for N in NS for M in {m for _, m, _ in SHAPES}}

    # GPU encoder throughput on one layer (config 2 weights), GB/s of original bytes.
    enc_t, enc_c_t, enc_k_t, enc_bytes = 0.0, 0.0, 0.0, 0
    for name, M, K, w, c, r in layers[0]:
        enc_k_t += compress_kernel_seconds(torch, zs, w)
        zs.compress_retiled(w)
        zs.compress_zipserv(w)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        zs.compress_retiled(w)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        zs.compress_zipserv(w)
        torch.cuda.synchronize()
        enc_t += t2 - t1
        enc_c_t += time.perf_counter() - t2
        enc_bytes += 2 * M * K

    # Calibration kernel for HBM counters: an elementwise negation of 256 MiB
    # (reads and writes exactly CALIB_BYTES each); rocprofv3 --pmc runs of this
    # script scale FETCH_SIZE / WRITE_SIZE of the GEMM kernels by its reading.
    ca = torch.empty(CALIB_BYTES // 2, device=dev, dtype=torch.bfloat16).fill_(1.0)
    cb = torch.empty_like(ca)
    torch.neg(ca, out=cb)
    torch.cuda.synchronize()
    del ca, cb

    stream = torch.cuda.Stream()

    # HBM-cold copies per shape (see the per-launch timing below): the
    # layers' own matrices plus clones, >= COLD_MIN_COPIES and >= COLD_BYTES
    # of compressed weights, so one launch's weights were last touched more
    # than 1 GiB of traffic earlier (past the 256 MB Infinity Cache).
    colds = []
    for si, (name, M, K) in enumerate(SHAPES):
        comp = layers[0][si][5].compressed_bytes
        nc = max(COLD_MIN_COPIES, -(-COLD_BYTES // comp))
        cold = [L[si] for L in layers]
        while len(cold) < nc:
            _, _, _, w0, c0, r0 = layers[len(cold) % len(layers)][si]
            cold.append((name, M, K, w0.clone(), clone_canonical(c0), clone_retiled(r0)))
        colds.append(cold)
    torch.cuda.synchronize()

    # Split-K per (shape, N): the reference sweeps Split_K in {1, 2, 4}
    # (benchmark config 2); the fastest on this GPU (cold weights) is kept.
    splits, wss = {}, {}
    for si, (name, M, K) in enumerate(SHAPES):
        for N in NS:
            cand = schedules(N, [int(v) for v in args.splits.split(",")])
            wsk = {sk: zs.codec.splitk_workspace(layers[0][si][5], N, sk) for sk in cand}

            def make_run(sk, si=si, N=N, M=M, K=K):
                def srun():
                    for cp in colds[si]:
                        zs.zipgemm(cp[5], xs[(N, K)], split_k=sk, out=outs[(N, M)],
                                   workspace=wsk[sk])
                return srun
            splits[(si, N)], _ = pick_schedule(torch, stream, cand, make_run)
            wss[(si, N)] = wsk[splits[(si, N)]]

    def zip_layer(layer):
        def run():
            for N in NS:
                for si, (name, M, K, w, c, r) in enumerate(layer):
                    zs.zipgemm(r, xs[(N, K)], split_k=splits[(si, N)], out=outs[(N, M)],
                               workspace=wss[(si, N)])
        return run

    def dense_layer(layer):
        def run():
            for N in NS:
                for name, M, K, w, c, r in layer:
                    torch.matmul(xs[(N, K)], w.t(), out=outs[(N, M)])
        return run

    zg = [capture(torch, stream, zip_layer(L)) for L in layers]
    step_bytes = sum(2 * M * K for _, M, K in SHAPES) * len(NS)
    t_zip = timed(torch, stream, zg, args.steps, args.warmup)
    value = step_bytes * args.steps / t_zip / 1e12

    result_dense = None
    if not args.no_dense:
        dg = [capture(torch, stream, dense_layer(L)) for L in layers]
        t_dense = timed(torch, stream, dg, args.steps, args.warmup)
        result_dense = step_bytes * args.steps / t_dense / 1e12

    # Per-(shape, N) kernel timing, HBM-cold: one graph launches the shape
    # once on each of `nc` distinct resident copies (the layers' own plus
    # clones, >= 16 and >= COLD_BYTES of compressed weights, so a launch's
    # weights were last touched > 1 GiB of traffic ago, past the 256 MB
    # Infinity Cache), timed with events on the replay stream around each of
    # 9 replays; zip_us is the median replay / nc, p10/p90 beside it.  The
    # dense and canonical comparators rotate their own copies the same way.
    per = []
    sum_alg_bytes, sum_kernel_s = 0.0, 0.0
    for si, (name, M, K) in enumerate(SHAPES):
        progress(f"config 2: per-launch timing {name} {M}x{K}")
        cold = colds[si]
        nc = len(cold)
        for N in NS:
            def zrun(si=si, N=N, M=M, K=K):
                for cp in cold:
                    zs.zipgemm(cp[5], xs[(N, K)], split_k=splits[(si, N)],
                               out=outs[(N, M)], workspace=wss[(si, N)])
            dz = [t / nc for t in timed_dist(torch, stream, capture(torch, stream, zrun), 9, LAUNCH_WARMUP)]
            tz = pct(dz, 50)
            comp = layers[0][si][5].compressed_bytes
            sk = splits[(si, N)]
            alg = comp + 2 * N * K + 2 * N * M + (4 * sk * M * N if sk > 1 else 0)
            sum_alg_bytes += alg
            sum_kernel_s += tz
            # the drop-in entry point on the canonical streams, at its own
            # fastest split-K of the same set
            tc, csk = None, 1
            for sk_c in [int(v) for v in args.splits.split(",")]:
                cws = zs.codec.splitk_workspace(layers[0][si][4], N, sk_c)
                def crun(si=si, N=N, M=M, K=K, sk_c=sk_c, cws=cws):
                    for cp in cold:
                        zs.zipgemm(cp[4], xs[(N, K)], split_k=sk_c, out=outs[(N, M)],
                                   workspace=cws)
                t = timed(torch, stream, [capture(torch, stream, crun)], 3, LAUNCH_WARMUP) / (3 * nc)
                if tc is None or t < tc:
                    tc, csk = t, sk_c
                del cws
            row = {"shape": name, "M": M, "K": K, "N": N, "kernel": kernel_name(N, M, sk, K),
                   "split_k": sk, "cold_copies": nc,
                   "canonical_us": round(tc * 1e6, 3), "canonical_split_k": csk,
                   "zip_us": round(tz * 1e6, 3),
                   "zip_us_p10": round(pct(dz, 10) * 1e6, 3),
                   "zip_us_p90": round(pct(dz, 90) * 1e6, 3),
                   "alg_bytes": alg,
                   "eff_TBps": round(2 * M * K / tz / 1e12, 3),
                   "comp_TBps": round(alg / tz / 1e12, 3),
                   # MFMA use: dense-equivalent flops against the 2.5 PFLOP/s bf16 peak
                   "TFLOPs": round(2 * M * N * K / tz / 1e12, 2),
                   "mfma_frac": round(2 * M * N * K / tz / 2.5e15, 4)}
            if not args.no_dense:
                def drun(si=si, N=N, M=M, K=K):
                    for cp in cold:
                        torch.matmul(xs[(N, K)], cp[3].t(), out=outs[(N, M)])
                td = pct([t / nc for t in
                          timed_dist(torch, stream, capture(torch, stream, drun), 9, LAUNCH_WARMUP)], 50)
                row["dense_us"] = round(td * 1e6, 2)
                row["speedup"] = round(td / tz, 3)
            per.append(row)
    del colds, cold
    torch.cuda.empty_cache()

    ratio = sum(2 * M * K for _, M, K in SHAPES) / sum(r.compressed_bytes for *_, r in layers[0])
    ratio_canonical = (sum(2 * M * K for _, M, K in SHAPES)
                       / sum(c.compressed_bytes for *_, c, r in layers[0]))
    # Per-kernel roll-up: launches of one instantiation, its average launch
    # time and average algorithmic bytes; the dominant one carries the roofline.
    kernels = {}
    for row in per:
        k = kernels.setdefault(row["kernel"], {"launches": 0, "time_s": 0.0, "alg_bytes": 0.0})
        k["launches"] += 1
        k["time_s"] += row["zip_us"] * 1e-6
        k["alg_bytes"] += row["alg_bytes"]
    for k in kernels.values():
        k["avg_us"] = round(k["time_s"] / k["launches"] * 1e6, 3)
        k["avg_alg_bytes"] = int(k["alg_bytes"] / k["launches"])
        k["achieved_GBps"] = round(k["alg_bytes"] / k["time_s"] / 1e9, 1)
    dominant = max(kernels, key=lambda n: kernels[n]["time_s"])
    dk = kernels[dominant]
    achieved = dk["alg_bytes"] / dk["time_s"] / 1e9
    traffic = roofline_traffic(per, dominant, traffic_table())
    out = {
        "metric": METRIC,
        "value": round(value, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_zip / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "llama3-8b-projections ZipGEMM sweep (benchmark config 2)",
            "shapes": {n: [m, k] for n, m, k in SHAPES},
            "N": NS,
            "split_k": "per (shape, N), fastest of split-K 1/2/4 and, N <= 16, stream-K (0)",
            "layout": "CDNA4 re-tiled records (zs_retiled_mm_fused)",
            "layers_resident": args.layers,
            "weights": "N(0,0.02) bf16, 0.1% x30 outliers",
            "parallelism": "single-gpu",
        },
        "compression_ratio": round(ratio, 4),
        "compression_ratio_canonical": round(ratio_canonical, 4),
        "dense_TBps_effective": None if result_dense is None else round(result_dense, 4),
        "speedup_vs_dense": None if result_dense is None else round(value / result_dense, 4),
        "gpu_compress_GBps": round(enc_bytes / enc_t / 1e9, 2),
        "gpu_compress_kernels_GBps": round(enc_bytes / enc_k_t / 1e9, 2),
        "gpu_compress_canonical_GBps": round(enc_bytes / enc_c_t / 1e9, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": dominant,
            "launches": dk["launches"],
            "avg_launch_us": dk["avg_us"],
            "alg_bytes_per_launch": dk["avg_alg_bytes"],
            "algorithmic_bytes": "comp_bytes(W) + 2*N*K + 2*N*M (+ 4*S*M*N split-K partials) per "
                                 "launch, averaged over the launches of this instantiation in one step",
            "traffic_source": PMC_PROFILE if traffic is not None else None,
        },
        "kernels": kernels,
        "per_launch": per,
        "setup_s": round(setup_s, 2),
    }
    if not args.no_cpu_baseline:
        progress("CPU baseline (config 1)")
        out["cpu_baseline"] = cpu_baseline()
    del layers, xs, outs
    torch.cuda.empty_cache()
    if not args.no_kv:
        out["kv_cache"] = bench_kv(torch, zs, dev, gen)
    if not args.no_attention:
        out["attention"] = bench_attention(torch, zs, stream, gen, dev)
    if not args.no_c3:
        out["c3_70b"] = bench_c3(torch, zs, stream, gen, dev)
    for key in ("per_launch", "kernels", "cpu_baseline", "kv_cache", "attention", "c3_70b"):
        if key in out:
            detail(key, out[key])
    detail("roofline", out["roofline"])
    print(json.dumps(final_line(out)), flush=True)


if __name__ == "__main__":
    main()
