"""Stage profiler (zipserv_tile_stage_bench_ext.cu counterpart): it runs the
real record decode -- the operands it decoded equal the matrix -- and reports
stage times that are positive and add up."""
import numpy as np
import pytest

import zipserv_asplos26_amd as zs
from zipserv_asplos26_amd.profiler import STAGES, measure_record_stages
from zs_testutil import from_torch_bf16, to_torch_bf16, weights_bf16

pytestmark = pytest.mark.gpu


def test_record_stage_profiler(torch_cuda):
    rng = np.random.default_rng(3)
    M, K = 1024, 2048
    W = weights_bf16(rng, (M, K), outlier_frac=0.01)
    r = zs.compress_retiled(to_torch_bf16(W))
    nrec = M // 16 * (K // 64)
    warmup, iters, stride, rec0 = 2, 16, 97, 5
    res = measure_record_stages(r, record=rec0, stride=stride, warmup=warmup, iters=iters)
    c = res["cycles"]
    assert set(c) == set(STAGES)
    assert 300 < res["clock_mhz"] < 5000
    for s in ("fixed", "decode", "mfma", "record"):
        assert c[s] > 0, s
    # each global load waits out a memory latency; the record step is no
    # slower than its parts in sequence
    assert c["fixed"] > c["stage"]
    assert c["record"] <= sum(c[s] for s in STAGES if s != "record") * 1.5
    # the decoded operands of the last record are the matrix's elements
    rec = (rec0 + (warmup + iters - 1) * stride) % nrec
    band, kt = divmod(rec, K // 64)
    f = from_torch_bf16(res["fragment"]).reshape(64, 2, 8)  # lane, half, element
    for l in range(64):
        for h in range(2):
            row, col = 16 * band + l % 16, 64 * kt + 32 * h + 8 * (l // 16)
            np.testing.assert_array_equal(f[l, h], W[row, col:col + 8])
