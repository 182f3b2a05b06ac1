"""Stage profiler of the re-tiled record pipeline (counterpart of
kernel_benchmark/zipserv_tile_stage_bench_ext.cu measure_zipserv_tile_stages):
one wave consumes records step by step with a shader-clock stamp between the
steps; the result is the mean time of each step, bracket cost removed, as the
reference reports its stages.  The kernel is zs_measure_record_stages."""
from __future__ import annotations

from . import _lib
from ._lib import check, lib
from .codec import ZipservRetiled, _dptr, _stream, _torch

STAGES = ("offsets", "fixed", "exps", "stage", "decode", "mfma", "record")


def measure_record_stages(r: ZipservRetiled, record: int = 0, stride: int | None = None,
                          warmup: int = 4, iters: int = 64, x=None) -> dict:
    """Per-step cycles and microseconds of consuming records of `r`.  stride
    (records between iterations) defaults to ~1 MiB apart so the loads miss
    the caches; x is the 16 x 64 bf16 right-hand tile of the MFMA step.
    Returns {"cycles": {...}, "us": {...}, "clock_mhz", "bracket_cycles",
    "fragment" (the last record's decoded operands, lane order)}."""
    torch = _torch()
    if not isinstance(r, ZipservRetiled):
        raise TypeError("measure_record_stages takes a ZipservRetiled matrix")
    dev = r.device
    nrec = r.rows // 16 * (r.cols // 64)
    if stride is None:
        stride = max(1, min(nrec - 1, (1 << 20) // 1408 + 1))
    if x is None:
        x = torch.ones(16, 64, dtype=torch.bfloat16, device=dev)
    x = x.contiguous()
    out = torch.zeros(11, dtype=torch.int64, device=dev)
    frag = torch.empty(64 * 16, dtype=torch.bfloat16, device=dev)
    check("zs_measure_record_stages", lib().zs_measure_record_stages(
        _stream(), _dptr(r.fixed), _dptr(r.exps), _dptr(r.eoff), r.start_exp & 0xFF, r.rows,
        r.cols, int(record), int(stride), int(warmup), int(iters), _dptr(x), _dptr(out),
        _dptr(frag)))
    v = out.cpu().tolist()
    bracket = v[0]
    mhz = v[8] / max(v[9], 1) * 100.0  # shader cycles per 100 MHz real-time tick
    cyc = {s: max(0, v[i + 1] - bracket) for i, s in enumerate(STAGES)}
    return {"cycles": cyc, "us": {s: c / mhz for s, c in cyc.items()}, "clock_mhz": mhz,
            "bracket_cycles": bracket, "fragment": frag}
