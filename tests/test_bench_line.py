"""bench.py's result line and counter summary, on the CPU (no GPU, no torch).

The driver parses the LAST stdout line of bench.py as the result; a line of
tens of KB (every per-launch row inline) was cut off in its captured tail.
These tests build the final line from stub rows of the real counts (30
per-launch rows, 7 x 5 config-3 rows, 12 attention and 7 KV cases) and bound
its size, and check that the counter summary written by --pmc-summary is read
back into the roofline's traffic for exactly the step's launches.
"""
import csv
import json
import os

import pytest

import bench


def _stub_result():
    per = []
    for name, M, K in bench.SHAPES:
        for N in bench.NS:
            per.append({"shape": name, "M": M, "K": K, "N": N, "split_k": 1 + (N > 16),
                        "kernel": f"zs::rgemm_wide_kernel<{min(8, -(-N // 16))}, 4, 2, 2>",
                        "cold_copies": 16, "canonical_us": 33.333, "canonical_split_k": 2,
                        "zip_us": 22.222, "zip_us_p10": 21.111, "zip_us_p90": 23.333,
                        "alg_bytes": 88824242, "eff_TBps": 4.361, "comp_TBps": 3.298,
                        "TFLOPs": 279.08, "mfma_frac": 0.1116, "dense_us": 40.12,
                        "speedup": 1.49})
    c3 = {"compression_ratio": 1.4275, "gpu_compress_GBps": 1380.12,
          "gpu_compress_kernels_GBps": 2090.55,
          "per_N": [{"N": N, "split_k": [4, 2, 1, 1, 2], "zip_ms_per_token": 17.972,
                     "dense_ms_per_token": 29.582, "speedup": 1.646, "eff_TBps": 7.617,
                     "comp_TBps": 5.333,
                     "per_shape": [{"shape": s, "M": m, "K": k, "split_k": 1, "zip_us": 60.1,
                                    "dense_us": 90.2, "speedup": 1.5, "comp_TBps": 5.3,
                                    "eff_TBps": 7.6} for s, m, k in bench.C3_SHAPES]}
                    for N in bench.C3_NS]}
    att = {"cases": [{"B": B, "T": T, "zip_us": 16.23, "canonical_us": 24.51, "dense_us": 11.71,
                      "staged_us": 31.4, "speedup": 0.722, "speedup_vs_staged": 1.935,
                      "token_major_us": 18.5, "token_major_vs_head_major": 0.88,
                      "token_major_speedup": 0.63,
                      "ratio": 1.3509, "comp_TBps": 0.767, "dense_TBps": 1.435}
                     for B, T in bench.ATTN_CASES]}
    kv = {"cases": [{"B": B, "T": T, "ratio_retiled": 1.35, "bit_exact": True,
                     "bit_exact_retiled": True} for B, T in bench.KV_CASES]}
    cpu = {"value": 0.004503, "unit": "TB/s", "cores": 16, "kind": "port",
           "sample": "benchmark config 1: 4096x4096 N(0,0.02) bf16 (seed 0) decompressed by the "
                     "oracle's CPU decoder, then Y = X W^T with X [8, 4096] and fp32 "
                     "accumulation; median of 10 runs on 16 threads",
           "host_cpu": "AMD EPYC 9575F 64-Core Processor", "compression_ratio": 1.4189,
           "round_trip_bit_exact": True, "single_core": {"value": 0.000339}}
    return {
        "metric": bench.METRIC, "value": 4.3184, "unit": "TB/s", "n_gpus": 1, "steps": 20,
        "warmup": 3, "ms_per_step": 0.6061, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": "llama3-8b-projections ZipGEMM sweep (benchmark config 2)",
                   "shapes": {n: [m, k] for n, m, k in bench.SHAPES}, "N": bench.NS,
                   "split_k": "per (shape, N), fastest of split-K 1/2/4 and, N <= 16, stream-K (0)",
                   "layout": "CDNA4 re-tiled records (zs_retiled_mm_fused)",
                   "layers_resident": 4, "weights": "N(0,0.02) bf16, 0.1% x30 outliers",
                   "parallelism": "single-gpu"},
        "compression_ratio": 1.4275, "dense_TBps_effective": 3.266, "speedup_vs_dense": 1.32,
        "roofline": {"bound": "hbm", "achieved": 3969.7, "peak": 8000.0, "unit": "GB/s",
                     "frac": 0.4962, "traffic": 84710085,
                     "kernel": "zs::rgemm_wide_kernel<1, 4, 4, 2>", "launches": 6,
                     "avg_launch_us": 20.902, "alg_bytes_per_launch": 82975173,
                     "algorithmic_bytes": "long text " * 20, "traffic_source": bench.PMC_PROFILE},
        "kernels": {}, "per_launch": per, "cpu_baseline": cpu, "c3_70b": c3,
        "attention": att, "kv_cache": kv,
    }


def test_final_line_is_compact_and_complete():
    res = _stub_result()
    line = json.dumps(bench.final_line(res))
    assert len(line) < 3000, len(line)
    got = json.loads(line)
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
              "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
              "roofline", "cpu_baseline"):
        assert k in got, k
    for k in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert k in got["roofline"], k
    for k in ("value", "unit", "cores", "kind", "sample"):
        assert k in got["cpu_baseline"], k
    assert "per_launch" not in got and "kernels" not in got
    assert len(got["c3_70b"]["per_N [ms/token, comp TB/s, x dense]"]) == len(bench.C3_NS)
    # a detail line carries one section on its own
    assert len(json.dumps({"detail": "per_launch", "data": res["per_launch"]})) > len(line)


def test_final_line_without_optional_sections():
    res = _stub_result()
    for k in ("cpu_baseline", "c3_70b", "attention", "kv_cache"):
        del res[k]
    got = bench.final_line(res)
    assert "cpu_baseline" not in got and "c3_70b" not in got
    assert got["value"] == res["value"]


def _write_counter_csv(d, counter, rows):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        for i, (k, v) in enumerate(rows):
            w.writerow([i + 1, k, counter, v])


def test_pmc_summary_round_trip(tmp_path):
    iters = 2
    order = bench.pmc_sweep_order()

    def kern(name, N, sk):
        return f"void zs::rgemm_kernel<{N}, {sk}>(int, int)"
    fetch = [("void at::native::neg_kernel(int)", 131072.0), ("void other(int)", 5.0)]
    write = [("void at::native::neg_kernel(int)", 262144.0)]
    for gi, (name, M, K, N, sk) in enumerate(order):
        for _ in range(iters):
            fetch.append((kern(name, N, sk), 1000.0 + gi))
            write.append((kern(name, N, sk), 10.0))
    _write_counter_csv(str(tmp_path / "f"), "FETCH_SIZE", fetch)
    _write_counter_csv(str(tmp_path / "w"), "WRITE_SIZE", write)
    md = bench.pmc_summary(str(tmp_path / "f"), str(tmp_path / "w"), iters)
    p = tmp_path / "summary.md"
    p.write_text(md)
    tab = bench.traffic_table(str(p))
    assert len(tab) == len(order)
    gi = order.index(("gate", 14336, 4096, 8, 2))
    k, b = tab[("gate", 8, 2)]
    assert k == "zs::rgemm_kernel<8, 2>"
    # FETCH factor 2 (the negation reads 128 MiB of KiB for 256 MiB), WRITE factor 1
    assert b == int(round((1000.0 + gi) * 1024 * 2 + 10.0 * 1024))
    per = [{"shape": "gate", "N": 8, "split_k": 2, "kernel": k},
           {"shape": "up", "N": 8, "split_k": 2, "kernel": "zs::rgemm_kernel<8, 2>"},
           {"shape": "o", "N": 1, "split_k": 1, "kernel": "zs::rgemm_kernel<1, 1>"}]
    t = bench.roofline_traffic(per, "zs::rgemm_kernel<8, 2>", tab)
    assert t == (tab[("gate", 8, 2)][1] + tab[("up", 8, 2)][1]) // 2
    # a step launch the table lists under another kernel: no traffic figure
    per[1]["split_k"] = 4
    assert bench.roofline_traffic(per, "zs::rgemm_kernel<8, 2>", tab) is None


def test_pmc_summary_rejects_wrong_dispatch_count(tmp_path):
    _write_counter_csv(str(tmp_path / "f"), "FETCH_SIZE",
                       [("neg", 1.0), ("void zs::rgemm_kernel<1>(int)", 1.0)])
    _write_counter_csv(str(tmp_path / "w"), "WRITE_SIZE",
                       [("neg", 1.0), ("void zs::rgemm_kernel<1>(int)", 1.0)])
    with pytest.raises(SystemExit):
        bench.pmc_summary(str(tmp_path / "f"), str(tmp_path / "w"), 2)
