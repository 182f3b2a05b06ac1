"""Prints the stage profile of the re-tiled record pipeline for one matrix:
    python -m zipserv_asplos26_amd.stage_report [M K] [--warm]
(N(0, 0.02) bf16 weights with 0.1% x30 outliers, seed 0; records ~1 MiB apart,
or the same record over and over with --warm)."""
import sys

import torch

import zipserv_asplos26_amd as zs
from zipserv_asplos26_amd.profiler import STAGES, measure_record_stages


def main(argv):
    warm = "--warm" in argv
    nums = [int(a) for a in argv if not a.startswith("--")]
    M, K = (nums + [8192, 8192])[:2]
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    w = torch.randn(M, K, device="cuda", generator=g) * 0.02
    w = torch.where(torch.rand(M, K, device="cuda", generator=g) < 0.001, w * 30, w)
    r = zs.compress_retiled(w.to(torch.bfloat16))
    res = measure_record_stages(r, stride=0 if warm else None, warmup=8, iters=256)
    print(f"matrix {M}x{K}, {'one record (cache-warm)' if warm else 'records ~1 MiB apart'}; "
          f"shader clock {res['clock_mhz']:.0f} MHz, bracket {res['bracket_cycles']} cycles")
    print("| stage | cycles | us |")
    print("|---|---:|---:|")
    for s in STAGES:
        print(f"| {s} | {res['cycles'][s]} | {res['us'][s]:.3f} |")
    return 0


if __name__ == "__main__":
    raise SystemExit(main(sys.argv[1:]))
