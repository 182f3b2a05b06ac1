#!/usr/bin/env python3
"""ZipGEMM benchmark on one MI355X (BASELINE.json metric, config 2).

Workload: Llama-3-8B-shaped projections
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
HBM_PEAK_GBS = 8000.0
CALIB_BYTES = 256 << 20


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=4, help="distinct resident layers (>= 3 defeats MALL)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-dense", action="store_true")
    ap.add_argument("--reps", type=int, default=20, help="graph replays per (shape, N) in the per-kernel timing")
    return ap.parse_args()


def kernel_name(N):
    """Instantiation of zs::gemm_kernel that zs_bf16_triple_bitmap_mm picks for
    split-K 1 at batch N (ceil(N/16) column blocks of 16, rounded up to a
    compiled width; 8 waves per workgroup up to 4 blocks, else 4)."""
    nb = (N + 15) // 16
    nb = next(w for w in (1, 2, 3, 4, 6, 8, 16) if w >= nb) if nb <= 16 else 16
    return f"zs::gemm_kernel<{nb}, {8 if nb <= 4 else 4}>"


def traffic_from_profile(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by a copy kernel of
    known size); None when the summary has no line for this kernel."""
    path = os.path.join(ROOT, "profiles", "zs_gemm_kernel_pmc_llama3-8b_sweep.md")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch") and f"`{kernel}`" in line:
                return {"bytes_per_launch": int(line.rsplit(":", 1)[1].strip()),
                        "source": os.path.relpath(path, ROOT)}
    return None


def make_layer(torch, zs, gen, dev):
    """Synthetic bf16 weights of one layer, compressed on the GPU."""
    layer = []
    for name, M, K in SHAPES:
        w = torch.randn(M, K, device=dev, generator=gen) * 0.02
        mask = torch.rand(M, K, device=dev, generator=gen) < 0.001
        w = torch.where(mask, w * 30.0, w).to(torch.bfloat16)
        c = zs.compress(w)
        layer.append((name, M, K, w, c))
    return layer


def cpu_baseline(torch, layer, seed):
    """Oracle (plain-C restatement, 1 thread) decode + fp32 GEMM of one layer at
    N=16: the same work per launch as the GPU step's N=16 row, measured in the
    metric's unit (effective TB/s)."""
    import numpy as np

    import oracle as zo
    rng = np.random.default_rng(seed)
    total_bytes, t_dec, t_gemm, t_enc = 0, 0.0, 0.0, 0.0
    for name, M, K, w, c in layer:
        W = w.cpu().view(torch.int16).numpy().view(np.uint16)
        t0 = time.perf_counter()
        e = zo.compress(W, variant="sse")
        t_enc += time.perf_counter() - t0
        X = zo.f32_to_bf16(rng.standard_normal((16, K), dtype=np.float32))
        t0 = time.perf_counter()
        D = zo.decompress(e)
        t1 = time.perf_counter()
        zo.gemm_f32(D, X)
        t2 = time.perf_counter()
        t_dec += t1 - t0
        t_gemm += t2 - t1
        total_bytes += 2 * M * K
    return {
        "value": round(total_bytes / (t_dec + t_gemm) / 1e12, 6),
        "unit": "TB/s",
        "cores": 1,
        "kind": "port",
        "sample": ("oracle zso_decompress + zso_gemm_f32 (fp32 accumulate) of one Llama-3-8B layer "
                   "(qkv,o,gate,up,down) at N=16, single thread"),
        "seconds": round(t_dec + t_gemm, 3),
        "decompress_s": round(t_dec, 3),
        "gemm_s": round(t_gemm, 3),
        "compress_sse_s": round(t_enc, 3),
        "compress_GBps": round(total_bytes / t_enc / 1e9, 3),
        "host_cpu": platform.processor() or platform.machine(),
        "host_nproc": os.cpu_count(),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1 "
                          "(multi-GPU sharding is design-only, see DESIGN.md)"}))
        sys.exit(2)
    import torch

    import zipserv_asplos26_amd as zs
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)

    t0 = time.perf_counter()
    layers = [make_layer(torch, zs, gen, dev) for _ in range(args.layers)]
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t0
    xs = {(N, K): torch.randn(N, K, device=dev, generator=gen).to(torch.bfloat16)
          for N in NS for K in {k for _, _, k in SHAPES}}
    outs = {(N, M): torch.empty(N, M, device=dev, dtype=torch.bfloat16)
            for N in NS for M in {m for _, m, _ in SHAPES}}

    # GPU encoder throughput on one layer (config 2 weights), GB/s of original bytes.
    enc_t, enc_bytes = 0.0, 0
    for name, M, K, w, c in layers[0]:
        zs.compress_zipserv(w)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        zs.compress_zipserv(w)
        torch.cuda.synchronize()
        enc_t += time.perf_counter() - t1
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

    def capture(fn):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            fn()  # warm (also initialises lazy state outside capture)
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=stream):
                fn()
        torch.cuda.synchronize()
        return g

    def zip_layer(layer):
        def run():
            for N in NS:
                for name, M, K, w, c in layer:
                    zs.zipgemm(c, xs[(N, K)], out=outs[(N, M)])
        return run

    def dense_layer(layer):
        def run():
            for N in NS:
                for name, M, K, w, c in layer:
                    torch.matmul(xs[(N, K)], w.t(), out=outs[(N, M)])
        return run

    def timed(graphs, steps, warmup):
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
        return s.elapsed_time(e) / 1e3  # seconds

    zg = [capture(zip_layer(L)) for L in layers]
    step_bytes = sum(2 * M * K for _, M, K in SHAPES) * len(NS)
    t_zip = timed(zg, args.steps, args.warmup)
    value = step_bytes * args.steps / t_zip / 1e12

    result_dense = None
    if not args.no_dense:
        dg = [capture(dense_layer(L)) for L in layers]
        t_dense = timed(dg, args.steps, args.warmup)
        result_dense = step_bytes * args.steps / t_dense / 1e12

    # Per-(shape, N) kernel timing: `reps` launches in one graph, cycling
    # through the resident layers, timed with events on the replay stream.
    per = []
    sum_alg_bytes, sum_kernel_s = 0.0, 0.0
    for si, (name, M, K) in enumerate(SHAPES):
        for N in NS:
            def zrun(si=si, N=N, M=M, K=K):
                for r in range(args.reps):
                    zs.zipgemm(layers[r % len(layers)][si][4], xs[(N, K)], out=outs[(N, M)])
            tz = timed([capture(zrun)], 3, 1) / (3 * args.reps)
            comp = layers[0][si][4].compressed_bytes
            alg = comp + 2 * N * K + 2 * N * M
            sum_alg_bytes += alg
            sum_kernel_s += tz
            row = {"shape": name, "M": M, "K": K, "N": N, "kernel": kernel_name(N),
                   "zip_us": round(tz * 1e6, 3), "alg_bytes": alg,
                   "eff_TBps": round(2 * M * K / tz / 1e12, 3),
                   "comp_TBps": round(alg / tz / 1e12, 3)}
            if not args.no_dense:
                def drun(si=si, N=N, M=M, K=K):
                    for r in range(args.reps):
                        torch.matmul(xs[(N, K)], layers[r % len(layers)][si][3].t(), out=outs[(N, M)])
                td = timed([capture(drun)], 3, 1) / (3 * args.reps)
                row["dense_us"] = round(td * 1e6, 2)
                row["speedup"] = round(td / tz, 3)
            per.append(row)

    ratio = sum(2 * M * K for _, M, K in SHAPES) / sum(c.compressed_bytes for _, _, _, _, c in layers[0])
    # Per-kernel roll-up: launches of one instantiation, its average launch
    # time and average algorithmic bytes; the dominant one carries the roofline.
    kernels = {}
    for row in per:
        k = kernels.setdefault(kernel_name(row["N"]), {"launches": 0, "time_s": 0.0, "alg_bytes": 0.0})
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
    traffic = traffic_from_profile(dominant)
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
            "workload": "llama3-8b-projections ZipGEMM sweep (BASELINE config 2)",
            "shapes": {n: [m, k] for n, m, k in SHAPES},
            "N": NS,
            "split_k": 1,
            "layers_resident": args.layers,
            "weights": "N(0,0.02) bf16, 0.1% x30 outliers",
            "parallelism": "single-gpu",
        },
        "compression_ratio": round(ratio, 4),
        "dense_TBps_effective": None if result_dense is None else round(result_dense, 4),
        "speedup_vs_dense": None if result_dense is None else round(value / result_dense, 4),
        "gpu_compress_GBps": round(enc_bytes / enc_t / 1e9, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None if traffic is None else traffic["bytes_per_launch"],
            "kernel": dominant,
            "avg_launch_us": dk["avg_us"],
            "alg_bytes_per_launch": dk["avg_alg_bytes"],
            "algorithmic_bytes": "comp_bytes(W) + 2*N*K + 2*N*M per launch, averaged over the "
                                 "launches of this instantiation in one step",
            "traffic_source": None if traffic is None else traffic["source"],
        },
        "kernels": kernels,
        "per_launch": per,
        "setup_s": round(setup_s, 2),
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(torch, layers[0], args.seed)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
