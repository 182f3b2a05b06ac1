"""The exact unit-vector probe check of the GPU shape tests, on the CPU.

tests/test_gpu_shapes.py probes every C2 / C3 ZipGEMM with rows of X equal
to unit vectors e_k and requires every probed output column to equal the
weight column W[:, k] bit for bit.  Here the same helpers run against the
oracle (CPU) to show (1) that the identity holds exactly through an fp32
GEMM and through the split-K model (bf16 partials summed in fp32,
Reduction_Kernel.cuh:15-37), (2) that the probe set covers every K tile and
every split-K slice boundary, and (3) that a single planted wrong weight -- an
exponent off by one, or a flipped sign -- in a probed column is caught, where
the normwise 1e-2 bound of the real-shape tests lets it through.  The
mistake is planted in the oracle's decoded matrix, on the CPU.
"""
import numpy as np
import pytest

import oracle as zo
from zs_testutil import (normal_bf16, probe_batches, probe_columns, probe_mismatches,
                         weights_bf16)


def _probe_x(cols, K):
    X = np.zeros((len(cols), K), np.float32)
    X[np.arange(len(cols)), cols] = 1.0
    return zo.f32_to_bf16(X)


@pytest.mark.parametrize("K,split_k", [(4096, 1), (4096, 2), (4096, 4), (14336, 4),
                                       (28672, 2), (8192, 4)])
def test_probe_columns_cover_tiles_and_slices(K, split_k):
    cols = probe_columns(K, split_k)
    kt = K // 64
    assert sorted(set(c // 64 for c in cols)) == list(range(kt))
    assert cols[0] == 0 and cols[-1] == K - 1
    per = (kt - 1) // split_k + 1
    for s in range(split_k):
        if s * per < kt:
            assert 64 * s * per in cols and 64 * min(kt, (s + 1) * per) - 1 in cols
    for n in (1, 8, 16, 128, 256):
        b = probe_batches(cols, n)
        assert all(len(x) == n for x in b) and set(c for x in b for c in x) == set(cols)


@pytest.mark.parametrize("split_k", [1, 2, 4])
def test_probes_reproduce_weight_columns_exactly(split_k):
    rng = np.random.default_rng(5)
    M, K = 128, 512
    W = weights_bf16(rng, (M, K), outlier_frac=0.01)
    e = zo.compress(W, variant="sse")
    Wd = zo.decompress(e)
    assert np.array_equal(Wd, W)
    cols = probe_columns(K, split_k)
    X = _probe_x(cols, K)
    if split_k == 1:
        Y = zo.f32_to_bf16(zo.gemm_f32(Wd, X))
    else:
        Y = zo.gemm_splitk_bf16(Wd, X, split_k)
    want = zo.bf16_to_f32(W[:, cols].T.copy())
    assert probe_mismatches(zo.bf16_to_f32(Y), want) == 0


@pytest.mark.parametrize("plant", ["exponent", "sign"])
def test_planted_single_weight_error_is_caught(plant):
    # A C2-sized matrix (4096 x 4096, N(0, 0.02) with 0.1% x30 outliers).
    rng = np.random.default_rng(1000 + 4096 + 4096)
    M, K = 4096, 4096
    W = weights_bf16(rng, (M, K), outlier_frac=0.001)
    bad = W.copy()
    m, k = 1234, probe_columns(K, 2)[17]
    if plant == "exponent":
        bad[m, k] = np.uint16(int(bad[m, k]) + (1 << 7))  # exponent + 1
    else:
        bad[m, k] = np.uint16(int(bad[m, k]) ^ 0x8000)
    # exact probes: the planted weight's column is probed
    cols = probe_columns(K, 2)
    X = _probe_x(cols, K)
    Y = zo.gemm_splitk_bf16(bad, X, 2)
    want = zo.bf16_to_f32(W[:, cols].T.copy())
    assert probe_mismatches(zo.bf16_to_f32(Y), want) == 1
    # the normwise bound on N(0, 1) batches does not see it (rows 1230..1239)
    Xn = normal_bf16(np.random.default_rng(3), (16, K))
    rows = np.arange(1230, 1240)
    ref = zo.gemm_f32(W[rows], Xn)
    got = zo.bf16_to_f32(zo.f32_to_bf16(zo.gemm_f32(bad[rows], Xn)))
    assert np.abs(got - ref).max() / np.abs(ref).max() <= 1e-2
