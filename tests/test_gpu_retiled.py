"""GPU parity of the CDNA4 re-tiled layout: encoders byte-identical to the
oracle, decompress bit-exact, and ZipGEMM over the re-tiled layout identical
(bit for bit, N <= 16 in 8-wave 16-row workgroups) or equal up to fp32
summation order (N > 16, the 4-wave workgroups of N > 1 on >= 640 bands and
of N = 1 on >= 896, and the 64-row workgroups of 4 <= N <= 16 on >= 224 of
them) to ZipGEMM
over the canonical streams it was built from, and within 1e-2 relative
error of the fp32-accumulated product."""
import numpy as np
import pytest

import oracle as zo
import zipserv_asplos26_amd as zs
from zs_testutil import arbitrary_bf16, from_torch_bf16, kv_bf16, pad_by_kv_head, to_torch_bf16, upload, weights_bf16

pytestmark = pytest.mark.gpu

SHAPES = [((64, 64), 0.0, 0), ((128, 192), 0.001, 1), ((256, 512), 0.05, 2), ((64, 4096), 0.01, 3),
          ((1024, 64), 0.3, 4)]


def _host(r):
    torch = __import__("torch")
    torch.cuda.synchronize()
    return (r.fixed.cpu().numpy(), r.exps[: r.num_outliers].cpu().numpy(), r.eoff.cpu().numpy())


@pytest.mark.parametrize("kind", ["random_bits", "specials"])
def test_retiled_encoder_arbitrary_bits(torch_cuda, kind):
    # every bit pattern, NaNs / Infs / subnormals / signed zeros included:
    # byte-identical to the oracle and decoded back to the same bits.  With
    # random bits nearly every element is an outlier, so records overflow the
    # encoder's per-record slot (re-emitted from the input) and the decoders'
    # LDS stage (outlier windows read from global memory).
    rng = np.random.default_rng(43)
    W = arbitrary_bf16(rng, (256, 512), kind)
    r = zs.compress_retiled(to_torch_bf16(W))
    top = zo.analyze_gpu(W)
    ref = zo.compress_retiled(W, top[0] - 1)
    assert r.start_exp == ref.start_exp and r.num_outliers == ref.exps.size
    fixed, exps, eoff = _host(r)
    np.testing.assert_array_equal(fixed, ref.fixed)
    np.testing.assert_array_equal(exps, ref.exps)
    np.testing.assert_array_equal(eoff, ref.eoff)
    np.testing.assert_array_equal(from_torch_bf16(zs.decompress_retiled(r)), W)


@pytest.mark.parametrize("shape,frac,seed", SHAPES)
def test_retiled_encoder_matches_oracle(torch_cuda, shape, frac, seed):
    rng = np.random.default_rng(200 + seed)
    W = weights_bf16(rng, shape, outlier_frac=frac)
    r = zs.compress_retiled(to_torch_bf16(W))
    top = zo.analyze_gpu(W)
    ref = zo.compress_retiled(W, top[0] - 1)
    assert r.start_exp == ref.start_exp and r.num_outliers == ref.exps.size
    fixed, exps, eoff = _host(r)
    np.testing.assert_array_equal(fixed, ref.fixed)
    np.testing.assert_array_equal(exps, ref.exps)
    np.testing.assert_array_equal(eoff, ref.eoff)
    assert r.compressed_bytes == ref.compressed_bytes()


@pytest.mark.parametrize("shape,frac,seed", SHAPES)
def test_retile_from_canonical_matches(torch_cuda, shape, frac, seed):
    rng = np.random.default_rng(300 + seed)
    W = weights_bf16(rng, shape, outlier_frac=frac)
    e = zo.compress(W)                       # CPU window (weights path)
    r = zs.retile(upload(e))
    ref = zo.retile(e)
    fixed, exps, eoff = _host(r)
    np.testing.assert_array_equal(fixed, ref.fixed)
    np.testing.assert_array_equal(exps, ref.exps)
    np.testing.assert_array_equal(eoff, ref.eoff)


@pytest.mark.parametrize("shape,frac,seed", SHAPES)
def test_retiled_decompress_bit_exact(torch_cuda, shape, frac, seed):
    rng = np.random.default_rng(400 + seed)
    W = weights_bf16(rng, shape, outlier_frac=frac)
    out = zs.decompress_retiled(zs.compress_retiled(to_torch_bf16(W)))
    np.testing.assert_array_equal(from_torch_bf16(out), W)


@pytest.mark.parametrize("kind", ["random_bits", "zeros", "uniform", "wrap", "kv"])
def test_retiled_edge_inputs(torch_cuda, kind):
    rng = np.random.default_rng(31)
    if kind == "random_bits":
        W = rng.integers(0, 65536, size=(128, 256), dtype=np.uint16)
    elif kind == "zeros":
        W = np.zeros((64, 128), np.uint16)            # every element an outlier
    elif kind == "uniform":
        W = np.full((64, 128), 0x3F80, np.uint16)     # no outliers
    elif kind == "wrap":
        W = np.tile(np.array([(e_ << 7) | 9 for e_ in range(7)] * 10, np.uint16)[:64], (64, 1))
    else:
        W, _ = pad_by_kv_head(kv_bf16(rng, 2, 100, 8, 128))
    if kind == "wrap":
        e = zo.compress(W, top=list(range(0, 7)))
        assert e.start_exp == 255
        r = zs.retile(upload(e))
    else:
        r = zs.compress_retiled(to_torch_bf16(W))
    out = zs.decompress_retiled(r)
    np.testing.assert_array_equal(from_torch_bf16(out), W)


@pytest.mark.parametrize("M,K", [(64, 64), (256, 512), (192, 1024), (128, 4480)])
@pytest.mark.parametrize("N", [1, 5, 16, 17, 32, 64, 100, 128, 200])
def test_retiled_zipgemm_equals_canonical(torch_cuda, M, K, N):
    torch = torch_cuda
    rng = np.random.default_rng(M * 7 + K + N)
    W = weights_bf16(rng, (M, K), outlier_frac=0.01)
    X = zo.f32_to_bf16(rng.standard_normal((N, K), dtype=np.float32))
    c = upload(zo.compress(W))
    r = zs.retile(c)
    x = to_torch_bf16(X)
    Yc = zs.zipgemm(c, x)
    Yr = zs.zipgemm(r, x)
    torch.cuda.synchronize()
    yr = from_torch_bf16(Yr)
    yc = from_torch_bf16(Yc)
    ref = zo.gemm_f32(W, X)
    err = np.abs(zo.bf16_to_f32(yr) - ref).max() / max(np.abs(ref).max(), 1e-30)
    assert err <= 1e-2
    if N <= 16:
        # same workgroup shape and summation order as the canonical kernel
        np.testing.assert_array_equal(yr, yc)
    else:
        # 64-row kernel: two or three K phases instead of the canonical
        # kernel's waves, so the fp32 sums differ only in rounding
        assert_same_sum_up_to_order(zo.bf16_to_f32(yr), zo.bf16_to_f32(yc), W, X)


def assert_same_sum_up_to_order(a, b, W, X):
    """a and b are bf16-rounded results of the same K-term fp32 sums of exact
    products in two orders: per element they differ by at most one bf16
    rounding of each (unit roundoff 2^-8) plus twice the fp32 summation bound
    K * 2^-24 * sum |w x|."""
    K = W.shape[1]
    s = zo.gemm_f32(W & 0x7FFF, X & 0x7FFF)  # sum of |w| |x| per element
    bound = 2.0 ** -8 * (np.abs(a) + np.abs(b)) + 2.0 * K * 2.0 ** -24 * s
    assert np.all(np.abs(a - b) <= bound), float(np.max(np.abs(a - b) - bound))


@pytest.mark.parametrize("M", [64 * 100, 64 * 193])
@pytest.mark.parametrize("N", [1, 9, 16])
def test_retiled_zipgemm_two_bands_per_wave(torch_cuda, N, M):
    # N > 8 with M / 16 >= 384 selects two bands per wave.  With 8 waves per
    # workgroup the per-band summation order is the canonical kernel's, so
    # the result is bit-identical; N > 1 on >= 640 bands (M = 12352) runs 4
    # waves per workgroup, whose fp32 sums differ from it only in rounding.
    torch = torch_cuda
    rng = np.random.default_rng(501 + N + M)
    K = 256
    W = weights_bf16(rng, (M, K), outlier_frac=0.01)
    X = zo.f32_to_bf16(rng.standard_normal((N, K), dtype=np.float32))
    c = upload(zo.compress(W))
    r = zs.retile(c)
    x = to_torch_bf16(X)
    Yc = zs.zipgemm(c, x)
    Yr = zs.zipgemm(r, x)
    torch.cuda.synchronize()
    if N == 1 or M // 16 < 640:
        np.testing.assert_array_equal(from_torch_bf16(Yr), from_torch_bf16(Yc))
    else:
        assert_same_sum_up_to_order(zo.bf16_to_f32(from_torch_bf16(Yr)),
                                    zo.bf16_to_f32(from_torch_bf16(Yc)), W, X)
    ref = zo.gemm_f32(W, X)
    y = zo.bf16_to_f32(from_torch_bf16(Yr))
    assert np.abs(y - ref).max() / np.abs(ref).max() <= 1e-2


@pytest.mark.parametrize("N,split_k,M", [(20, 1, 24576), (64, 1, 24576), (128, 1, 24576),
                                         (40, 2, 24576), (100, 1, 24576), (200, 1, 24576),
                                         (128, 2, 20480), (128, 1, 24640), (64, 1, 20480),
                                         (50, 2, 20480), (4, 1, 24576), (5, 1, 24576),
                                         (8, 1, 16384), (13, 2, 8192), (16, 1, 24640),
                                         (3, 1, 24576)])
def test_retiled_zipgemm_large_grid(torch_cuda, N, split_k, M):
    # M / 64 * split_k >= 384 selects the two-phase 64-row kernel; N > 32 with
    # M % 128 == 0 and >= 160 128-row workgroups the two-bands-per-wave one
    # (M = 24640 is not a multiple of 128: the 64-row kernel); 4 <= N <= 16
    # on >= 224 64-row workgroups the 64-row kernel over one column block
    # (four phases below 384 workgroups); N = 3 stays on the 16-row kernel
    torch = torch_cuda
    rng = np.random.default_rng(N * 3 + split_k + M)
    K = 128
    W = weights_bf16(rng, (M, K), outlier_frac=0.01)
    X = zo.f32_to_bf16(rng.standard_normal((N, K), dtype=np.float32))
    r = zs.compress_retiled(to_torch_bf16(W))
    Y = zs.zipgemm(r, to_torch_bf16(X), split_k=split_k)
    torch.cuda.synchronize()
    y = zo.bf16_to_f32(from_torch_bf16(Y))
    ref = zo.gemm_f32(W, X) if split_k == 1 else zo.bf16_to_f32(zo.gemm_splitk_bf16(W, X, split_k))
    assert np.abs(y - ref).max() / np.abs(ref).max() <= 1e-2


@pytest.mark.parametrize("M,K,N,split_k", [(14336, 320, 9, 4), (14336, 448, 16, 1),
                                           (14336, 1600, 5, 1), (14336, 1600, 12, 2)])
def test_retiled_zipgemm_64row_narrow_batches(torch_cuda, M, K, N, split_k):
    # 4 <= N <= 16 on >= 224 64-row workgroups: the 64-row kernel over one
    # column block -- K tiles not a multiple of the phases (phases with one
    # tile fewer), an empty last split, a steady loop of several steps.
    torch = torch_cuda
    rng = np.random.default_rng(M + K + N + split_k)
    W = weights_bf16(rng, (M, K), outlier_frac=0.01)
    X = zo.f32_to_bf16(rng.standard_normal((N, K), dtype=np.float32))
    r = zs.compress_retiled(to_torch_bf16(W))
    Y = zs.zipgemm(r, to_torch_bf16(X), split_k=split_k)
    torch.cuda.synchronize()
    y = zo.bf16_to_f32(from_torch_bf16(Y))
    ref = zo.gemm_f32(W, X) if split_k == 1 else zo.bf16_to_f32(zo.gemm_splitk_bf16(W, X, split_k))
    assert np.abs(y - ref).max() / np.abs(ref).max() <= 1e-2


@pytest.mark.parametrize("N,M,K", [(1, 256, 1024), (16, 256, 1024), (32, 256, 2048),
                                   (64, 256, 1024), (128, 256, 2048), (8, 14336, 512)])
def test_retiled_mixed_direct_and_staged_records(torch_cuda, N, M, K):
    # Some records carry more outlier bytes than the LDS stage (zero bands:
    # every element an outlier) next to ordinary records decoded by other waves
    # of the same workgroup; both decode paths must leave each other intact
    # (N >= 32 and the 14336-row N = 8 case: the 64-row kernels, whose steady
    # loop decodes a record one step ahead of its MFMAs).
    torch = torch_cuda
    rng = np.random.default_rng(77 + N)
    W = weights_bf16(rng, (M, K), outlier_frac=0.01)
    W[16:32, :] = 0                    # one band of all-outlier records
    W[100:116, 128:256] = 0            # two records of another band
    X = zo.f32_to_bf16(rng.standard_normal((N, K), dtype=np.float32))
    r = zs.compress_retiled(to_torch_bf16(W))
    out = zs.decompress_retiled(r)
    Y = zs.zipgemm(r, to_torch_bf16(X))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_torch_bf16(out), W)
    y = zo.bf16_to_f32(from_torch_bf16(Y))
    ref = zo.gemm_f32(W, X)
    assert np.abs(y - ref).max() / np.abs(ref).max() <= 1e-2


@pytest.mark.parametrize("split_k,N", [(2, 24), (4, 16), (3, 100), (8, 1)])
def test_retiled_zipgemm_splitk(torch_cuda, split_k, N):
    torch = torch_cuda
    rng = np.random.default_rng(split_k * 100 + N)
    M, K = 256, 1024
    W = weights_bf16(rng, (M, K), outlier_frac=0.01)
    X = zo.f32_to_bf16(rng.standard_normal((N, K), dtype=np.float32))
    r = zs.compress_retiled(to_torch_bf16(W))
    Y = zs.zipgemm(r, to_torch_bf16(X), split_k=split_k)
    torch.cuda.synchronize()
    y = zo.bf16_to_f32(from_torch_bf16(Y))
    ref = zo.bf16_to_f32(zo.gemm_splitk_bf16(W, X, split_k))
    assert np.abs(y - ref).max() / np.abs(ref).max() <= 1e-2


@pytest.mark.parametrize("N", [1, 16, 40, 128])
def test_retiled_zipgemm_empty_split(torch_cuda, N):
    """K = 320 (5 tiles) over 4 splits of 2 tiles: the last split has no
    tiles at all and contributes zeros (every kernel width)."""
    torch = torch_cuda
    rng = np.random.default_rng(N + 7)
    M, K, split_k = 256, 320, 4
    W = weights_bf16(rng, (M, K), outlier_frac=0.01)
    X = zo.f32_to_bf16(rng.standard_normal((N, K), dtype=np.float32))
    r = zs.compress_retiled(to_torch_bf16(W))
    Y = zs.zipgemm(r, to_torch_bf16(X), split_k=split_k)
    torch.cuda.synchronize()
    y = zo.bf16_to_f32(from_torch_bf16(Y))
    ref = zo.bf16_to_f32(zo.gemm_splitk_bf16(W, X, split_k))
    assert np.abs(y - ref).max() / np.abs(ref).max() <= 1e-2


def test_retiled_unit_vectors_exact(torch_cuda):
    torch = torch_cuda
    rng = np.random.default_rng(9)
    M, K = 128, 256
    W = weights_bf16(rng, (M, K), outlier_frac=0.02)
    cols = [0, 1, 63, 64, 100, 255]
    X = np.zeros((len(cols), K), np.uint16)
    for n, k in enumerate(cols):
        X[n, k] = 0x3F80
    Y = zs.zipgemm(zs.compress_retiled(to_torch_bf16(W)), to_torch_bf16(X))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_torch_bf16(Y), W[:, cols].T)


def test_retiled_rejects_bad_args(torch_cuda):
    torch = torch_cuda
    L = zs.lib()
    r = zs.compress_retiled(to_torch_bf16(weights_bf16(np.random.default_rng(0), (64, 128))))
    x = torch.zeros(4, 128, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(4, 64, dtype=torch.bfloat16, device="cuda")
    args = lambda M=64, N=4, K=128, sk=1, ws=None: (  # noqa: E731
        0, r.fixed.data_ptr(), r.exps.data_ptr(), r.eoff.data_ptr(), r.start_exp, x.data_ptr(),
        y.data_ptr(), M, N, K, ws, sk)
    assert L.zs_retiled_mm(*args()) == 0
    torch.cuda.synchronize()
    assert L.zs_retiled_mm(*args(M=65)) == zs._lib.ZS_E_INVAL
    assert L.zs_retiled_mm(*args(K=96)) == zs._lib.ZS_E_INVAL
    assert L.zs_retiled_mm(*args(N=0)) == zs._lib.ZS_E_INVAL
    assert L.zs_retiled_mm(*args(sk=2)) == zs._lib.ZS_E_INVAL    # split-K needs a workspace
    assert L.zs_retiled_mm(*args(sk=3)) == zs._lib.ZS_E_INVAL    # more slices than K tiles
    assert L.zs_retiled_mm(*args(sk=0)) == zs._lib.ZS_E_INVAL


# (M, K, N, split_k) -> the kernel zs_retiled_mm picks: narrow F = 1, 64-row
# one-column-block 2-phase, 4-phase, 2-phase (N <= 16 on >= 224 workgroups),
# an empty last split, wide 4-phase, wide 2-phase, two-band wide (4 and 8
# column blocks), wide 8 column blocks, narrow F = 2, narrow 4-wave F = 1.
FUSED_CASES = [(1024, 1024, 1, 2), (6144, 512, 16, 4), (10240, 512, 8, 2), (10240, 256, 12, 3),
               (256, 320, 8, 4), (512, 2048, 32, 3),
               (12288, 256, 32, 2), (10240, 256, 64, 2), (10240, 256, 128, 2), (512, 1024, 100, 3),
               (6144, 512, 16, 2), (10240, 512, 3, 2)]


@pytest.mark.parametrize("M,K,N,split_k", FUSED_CASES)
def test_retiled_zipgemm_fused_splitk(torch_cuda, M, K, N, split_k):
    """In-kernel split-K reduction: bit-identical to the two-kernel path on
    three calls in a row (the counters return to zero), within 1e-2 of the
    split-K rounding model."""
    torch = torch_cuda
    rng = np.random.default_rng(M + K + N + split_k)
    W = weights_bf16(rng, (M, K), outlier_frac=0.01)
    X = zo.f32_to_bf16(rng.standard_normal((N, K), dtype=np.float32))
    r = zs.compress_retiled(to_torch_bf16(W))
    x = to_torch_bf16(X)
    y2 = zs.zipgemm(r, x, split_k=split_k, fused=False)
    cnt = torch.zeros(int(zs.lib().zs_retiled_mm_counters(M, N)), dtype=torch.int32, device="cuda")
    for _ in range(3):
        y1 = zs.zipgemm(r, x, split_k=split_k, counters=cnt)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(from_torch_bf16(y1), from_torch_bf16(y2))
        assert int(cnt.abs().sum()) == 0
    y = zo.bf16_to_f32(from_torch_bf16(y1))
    ref = zo.bf16_to_f32(zo.gemm_splitk_bf16(W, X, split_k))
    assert np.abs(y - ref).max() / np.abs(ref).max() <= 1e-2


def test_retiled_zipgemm_fused_default_counters_and_graph(torch_cuda):
    """The per-stream counter buffer (default path), calls of different
    shapes sharing it, and a captured graph replayed with eager work between
    replays: every result equals the two-kernel reduction's."""
    torch = torch_cuda
    rng = np.random.default_rng(5)
    mats = [(zs.compress_retiled(to_torch_bf16(weights_bf16(rng, (M, K), outlier_frac=0.01))), K)
            for M, K in ((2048, 1024), (512, 512))]
    xs = [to_torch_bf16(zo.f32_to_bf16(rng.standard_normal((n, K), dtype=np.float32)))
          for (r, K), n in zip(mats, (24, 3))]
    refs = [zs.zipgemm(r, x, split_k=4, fused=False) for (r, _), x in zip(mats, xs)]
    for _ in range(2):
        for (r, _), x, ref in zip(mats, xs, refs):
            torch.testing.assert_close(zs.zipgemm(r, x, split_k=4), ref, rtol=0, atol=0)
    st = torch.cuda.Stream()
    outs = [torch.empty_like(ref) for ref in refs]
    with torch.cuda.stream(st):
        for (r, _), x, o in zip(mats, xs, outs):   # counters for this stream, outside capture
            zs.zipgemm(r, x, split_k=4, out=o)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            for (r, _), x, o in zip(mats, xs, outs):
                zs.zipgemm(r, x, split_k=4, out=o)
    for _ in range(3):
        for o in outs:
            o.fill_(0)
        g.replay()
        torch.cuda.synchronize()
        for o, ref in zip(outs, refs):
            torch.testing.assert_close(o, ref, rtol=0, atol=0)
        torch.ones(1 << 20, device="cuda").sum().item()   # eager work between replays


def test_retiled_mm_fused_rejects_bad_args(torch_cuda):
    torch = torch_cuda
    L = zs.lib()
    r = zs.compress_retiled(to_torch_bf16(weights_bf16(np.random.default_rng(0), (64, 128))))
    x = torch.zeros(4, 128, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(4, 64, dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(2 * 4 * 64 + 8, dtype=torch.bfloat16, device="cuda")
    cnt = torch.zeros(int(L.zs_retiled_mm_counters(64, 4)) + 1, dtype=torch.int32, device="cuda")
    args = lambda sk=2, w=ws.data_ptr(), c=cnt.data_ptr(): (  # noqa: E731
        0, r.fixed.data_ptr(), r.exps.data_ptr(), r.eoff.data_ptr(), r.start_exp, x.data_ptr(),
        y.data_ptr(), 64, 4, 128, w, sk, c)
    assert L.zs_retiled_mm_counters(64, 4) == 4 and L.zs_retiled_mm_counters(0, 4) == 0
    assert L.zs_retiled_mm_fused(*args(c=None)) == zs._lib.ZS_E_INVAL       # no counters
    assert L.zs_retiled_mm_fused(*args(c=cnt.data_ptr() + 2)) == zs._lib.ZS_E_INVAL
    assert L.zs_retiled_mm_fused(*args(w=ws.data_ptr() + 4)) == zs._lib.ZS_E_INVAL
    assert L.zs_retiled_mm_fused(*args(w=None)) == zs._lib.ZS_E_INVAL       # no workspace
    assert L.zs_retiled_mm_fused(*args(sk=1, c=None, w=None)) == 0          # no split: none needed
    assert L.zs_retiled_mm_fused(*args()) == 0
    torch.cuda.synchronize()
    assert int(cnt.abs().sum()) == 0


@pytest.mark.parametrize("kind", ["weights", "kv", "random_bits", "zeros"])
def test_two_pass_encoder_equals_three_pass(torch_cuda, kind):
    # zs_compress_retiled_fixed_gpu / _exps_gpu (input read once after the
    # histogram; outlier bytes parked in 256-byte slots, records with more
    # re-read their tile) against zs_compress_retiled_count_gpu / _emit_gpu
    torch = torch_cuda
    L = zs.lib()
    rng = np.random.default_rng(91)
    if kind == "weights":
        W = weights_bf16(rng, (512, 1024), outlier_frac=0.01)
    elif kind == "kv":
        W, _ = pad_by_kv_head(kv_bf16(rng, 2, 200, 8, 128))
    elif kind == "random_bits":
        W = rng.integers(0, 65536, size=(128, 256), dtype=np.uint16)  # > 256 outliers per record
    else:
        W = np.zeros((64, 192), np.uint16)
    x = to_torch_bf16(W)
    M, K = W.shape
    nrec = M // 16 * (K // 64)
    st = int(torch.cuda.current_stream().cuda_stream)
    i32 = dict(dtype=torch.int32, device="cuda")
    # zeros: the weights-path window (121..127) makes every element an outlier
    top = torch.tensor(zo.analyze_cpu(W) if kind == "zeros" else zo.analyze_gpu(W), **i32)
    cnt3, eoff3, cnt2, eoff2 = (torch.empty(n, **i32) for n in (nrec, nrec + 1, nrec, nrec + 1))
    tot3, tot2 = (torch.empty(1, dtype=torch.int64, device="cuda") for _ in range(2))
    fixed3 = torch.empty(nrec * 1408, dtype=torch.uint8, device="cuda")
    fixed2 = torch.empty_like(fixed3)
    tmp = torch.empty(nrec * 256, dtype=torch.uint8, device="cuda")
    assert L.zs_compress_retiled_count_gpu(st, x.data_ptr(), M, K, top.data_ptr(), cnt3.data_ptr(),
                                           eoff3.data_ptr(), tot3.data_ptr()) == 0
    assert L.zs_compress_retiled_fixed_gpu(st, x.data_ptr(), M, K, top.data_ptr(),
                                           fixed2.data_ptr(), cnt2.data_ptr(), eoff2.data_ptr(),
                                           tot2.data_ptr(), tmp.data_ptr()) == 0
    total = int(tot3.item())
    assert int(tot2.item()) == total
    exps3 = torch.zeros(total + 64, dtype=torch.uint8, device="cuda")
    exps2 = torch.zeros_like(exps3)
    assert L.zs_compress_retiled_emit_gpu(st, x.data_ptr(), M, K, top.data_ptr(), eoff3.data_ptr(),
                                          fixed3.data_ptr(), exps3.data_ptr()) == 0
    assert L.zs_compress_retiled_exps_gpu(st, x.data_ptr(), M, K, top.data_ptr(), eoff2.data_ptr(),
                                          tmp.data_ptr(), exps2.data_ptr()) == 0
    torch.cuda.synchronize()
    assert torch.equal(cnt2, cnt3) and torch.equal(eoff2, eoff3)
    assert torch.equal(fixed2, fixed3) and torch.equal(exps2, exps3)
    if kind in ("random_bits", "zeros"):
        assert int(cnt2.max()) > 256  # the re-read path ran


_DIFFERS = 2 * 16 * 256 * 8 + 32  # the flag's byte offset in the auto encoder's scratch


def _guess_miss_matrix(rng, M, K):
    """Sampled chunks (every 32nd run of 2048 elements) hold exponents near 100,
    the rest near 120, so the sample's window is not the full histogram's."""
    W = np.empty(M * K, np.uint16)
    chunks = W.reshape(-1, 2048)
    for c in range(chunks.shape[0]):
        base = 100 if c % 32 == 0 else 120
        e = rng.integers(base - 3, base + 4, 2048).astype(np.uint16)
        chunks[c] = (e << 7) | rng.integers(0, 128, 2048, dtype=np.uint16)
    return W.reshape(M, K)


@pytest.mark.parametrize("rule", ["kv", "weights"])
@pytest.mark.parametrize("kind", ["weights", "kv", "random_bits", "zeros", "guess_miss"])
def test_one_pass_encoder_equals_analyze_then_fixed(torch_cuda, kind, rule):
    # zs_compress_retiled_auto_gpu (window guessed from a sample, histogram
    # counted during the encoding pass, second pass only on a wrong guess)
    # against zs_analyze_* followed by zs_compress_retiled_fixed_gpu / _exps_gpu
    torch = torch_cuda
    L = zs.lib()
    rng = np.random.default_rng(92)
    if kind == "weights":
        W = weights_bf16(rng, (1024, 2048), outlier_frac=0.01)
    elif kind == "kv":
        W, _ = pad_by_kv_head(kv_bf16(rng, 2, 300, 8, 128))
    elif kind == "random_bits":
        W = rng.integers(0, 65536, size=(128, 256), dtype=np.uint16)
    elif kind == "zeros":
        W = np.zeros((64, 192), np.uint16)
    else:
        W = _guess_miss_matrix(rng, 512, 4096)
    x = to_torch_bf16(W)
    M, K = W.shape
    nrec = M // 16 * (K // 64)
    st = int(torch.cuda.current_stream().cuda_stream)
    i32 = dict(dtype=torch.int32, device="cuda")
    want_top = zo.analyze_gpu(W) if rule == "kv" else zo.analyze_cpu(W)
    u8 = dict(dtype=torch.uint8, device="cuda")
    outs = []
    for path in ("auto", "two_step"):
        hist, top = torch.empty(256, dtype=torch.int64, device="cuda"), torch.empty(7, **i32)
        cnt, eoff = torch.empty(nrec, **i32), torch.empty(nrec + 1, **i32)
        tot = torch.empty(1, dtype=torch.int64, device="cuda")
        fixed, tmp = torch.empty(nrec * 1408, **u8), torch.empty(nrec * 256, **u8)
        work = torch.empty(zs._lib.ZS_RETILED_AUTO_WORK_BYTES, **u8)
        if path == "auto":
            r = zs._lib.ZS_WINDOW_KV if rule == "kv" else zs._lib.ZS_WINDOW_WEIGHTS
            assert L.zs_compress_retiled_auto_gpu(st, x.data_ptr(), M, K, r, hist.data_ptr(),
                                                  top.data_ptr(), work.data_ptr(),
                                                  fixed.data_ptr(), cnt.data_ptr(),
                                                  eoff.data_ptr(), tot.data_ptr(),
                                                  tmp.data_ptr()) == 0
        else:
            fn = (L.zs_analyze_top_exponents_u64_gpu if rule == "kv"
                  else L.zs_analyze_exponents_weights_gpu)
            assert fn(st, x.data_ptr(), W.size, hist.data_ptr(), top.data_ptr()) == 0
            assert L.zs_compress_retiled_fixed_gpu(st, x.data_ptr(), M, K, top.data_ptr(),
                                                   fixed.data_ptr(), cnt.data_ptr(),
                                                   eoff.data_ptr(), tot.data_ptr(),
                                                   tmp.data_ptr()) == 0
        total = int(tot.item())
        exps = torch.zeros(total + 64, **u8)
        assert L.zs_compress_retiled_exps_gpu(st, x.data_ptr(), M, K, top.data_ptr(),
                                              eoff.data_ptr(), tmp.data_ptr(),
                                              exps.data_ptr()) == 0
        torch.cuda.synchronize()
        differs = int(work[_DIFFERS:_DIFFERS + 4].view(torch.int32).item()) if path == "auto" else None
        outs.append((hist, top, cnt, eoff, total, fixed, exps, differs))
    (h1, t1, c1, e1, n1, f1, x1, differs), (h2, t2, c2, e2, n2, f2, x2, _) = outs
    np.testing.assert_array_equal(h1.cpu().numpy(), zo.histogram(W))
    assert torch.equal(h1, h2)
    assert t1.cpu().tolist() == want_top == t2.cpu().tolist()
    assert n1 == n2 and torch.equal(c1, c2) and torch.equal(e1, e2)
    assert torch.equal(f1, f2) and torch.equal(x1, x2)
    if kind == "guess_miss":
        assert differs == 1  # the second pass ran
    elif kind in ("weights", "kv"):
        assert differs == 0
    r = zo.compress_retiled(W, (want_top[0] - 1) & 0xFF)
    np.testing.assert_array_equal(f1.cpu().numpy(), r.fixed)
    np.testing.assert_array_equal(x1[:n1].cpu().numpy(), r.exps[:n1])


@pytest.mark.parametrize("first", [0, 1, 100, 248, 249])
def test_explicit_window_encoder_bytes(torch_cuda, first):
    # the GPU encoder under an explicit window, including the windows that
    # wrap the code arithmetic (first exponent 0: start_exp 255) or end at 255,
    # byte for byte against the oracle's re-tiled encoder
    torch = torch_cuda
    rng = np.random.default_rng(700 + first)
    W = rng.integers(0, 65536, size=(128, 512), dtype=np.uint16)
    # make the window's exponents frequent so that both codes and outliers occur
    e = rng.integers(first, first + 7, size=W.shape).astype(np.uint16) & 0xFF
    keep = rng.random(W.shape) < 0.6
    W = np.where(keep, (W & 0x807F) | (e << 7), W).astype(np.uint16)
    r = zs.compress_retiled(to_torch_bf16(W), window=list(range(first, first + 7)))
    o = zo.compress_retiled(W, (first - 1) & 0xFF)
    torch.cuda.synchronize()
    assert r.start_exp == (first - 1) & 0xFF
    np.testing.assert_array_equal(r.fixed.cpu().numpy(), o.fixed)
    np.testing.assert_array_equal(r.eoff.cpu().numpy(), o.eoff)
    np.testing.assert_array_equal(r.exps[: r.num_outliers].cpu().numpy(), o.exps)
    np.testing.assert_array_equal(from_torch_bf16(zs.decompress_retiled(r)), W)


@pytest.mark.parametrize("rule", ["kv", "weights"])
def test_guess_encoder_equals_sampled_guess(torch_cuda, rule):
    # zs_compress_retiled_guess_gpu with a wrong guess (a window no element
    # falls in) and with the right one writes what zs_compress_retiled_auto_gpu
    # writes; a null guess, or one aliasing d_top, is refused
    torch = torch_cuda
    import zipserv_asplos26_amd._lib as zl
    L = zs.lib()
    rng = np.random.default_rng(97)
    W = weights_bf16(rng, (512, 1024), outlier_frac=0.02)
    x = to_torch_bf16(W)
    rows, cols = W.shape
    nrec = rows // 16 * (cols // 64)
    rl = zl.ZS_WINDOW_KV if rule == "kv" else zl.ZS_WINDOW_WEIGHTS
    st = torch.cuda.current_stream().cuda_stream

    def bufs():
        return dict(hist=torch.empty(256, dtype=torch.int64, device="cuda"),
                    top=torch.empty(7, dtype=torch.int32, device="cuda"),
                    work=torch.empty(zl.ZS_RETILED_AUTO_WORK_BYTES, dtype=torch.uint8, device="cuda"),
                    fixed=torch.empty(nrec * 1408, dtype=torch.uint8, device="cuda"),
                    cnt=torch.empty(nrec, dtype=torch.int32, device="cuda"),
                    eoff=torch.empty(nrec + 1, dtype=torch.int32, device="cuda"),
                    total=torch.empty(1, dtype=torch.int64, device="cuda"),
                    tmp=torch.empty(nrec * zl.ZS_RETILED_EXP_SLOT_BYTES, dtype=torch.uint8,
                                    device="cuda"))

    def args(b):
        return [b[k].data_ptr() for k in ("hist", "top", "work", "fixed", "cnt", "eoff", "total", "tmp")]
    ref = bufs()
    assert L.zs_compress_retiled_auto_gpu(st, x.data_ptr(), rows, cols, rl, *args(ref)) == 0
    right = ref["top"].clone()
    wrong = torch.arange(200, 207, dtype=torch.int32, device="cuda")
    for guess in (wrong, right):
        b = bufs()
        assert L.zs_compress_retiled_guess_gpu(st, x.data_ptr(), rows, cols, rl, guess.data_ptr(),
                                               *args(b)) == 0
        torch.cuda.synchronize()
        for k in ("hist", "top", "fixed", "cnt", "eoff", "total"):
            assert torch.equal(b[k], ref[k]), k
        tot = int(ref["total"].item())
        # slots hold the outlier bytes of each record (the rest is unspecified)
        exps_a = torch.empty(tot + 64, dtype=torch.uint8, device="cuda")
        exps_b = torch.empty(tot + 64, dtype=torch.uint8, device="cuda")
        for bb, e in ((ref, exps_a), (b, exps_b)):
            assert L.zs_compress_retiled_exps_gpu(st, x.data_ptr(), rows, cols, bb["top"].data_ptr(),
                                                  bb["eoff"].data_ptr(), bb["tmp"].data_ptr(),
                                                  e.data_ptr()) == 0
        torch.cuda.synchronize()
        assert torch.equal(exps_a, exps_b)
    b = bufs()
    assert L.zs_compress_retiled_guess_gpu(st, x.data_ptr(), rows, cols, rl, None, *args(b)) == zl.ZS_E_INVAL
    assert L.zs_compress_retiled_guess_gpu(st, x.data_ptr(), rows, cols, rl, b["top"].data_ptr(),
                                           *args(b)) == zl.ZS_E_INVAL


@pytest.mark.parametrize("window,lookahead", [("kv", 2), ("weights", 0), ("explicit", 9)])
def test_batched_encoder_equals_one_call_per_matrix(torch_cuda, window, lookahead):
    # compress_retiled_many (outlier totals read back asynchronously, the
    # host waiting `lookahead` matrices behind the GPU) against
    # compress_retiled per matrix and the oracle, byte for byte, over matrices
    # of different shapes and outlier densities (one with no outliers at all)
    torch = torch_cuda
    rng = np.random.default_rng(811)
    mats = [weights_bf16(rng, (1024, 2048), outlier_frac=0.01),
            weights_bf16(rng, (64, 64), outlier_frac=0.2),
            np.zeros((128, 192), np.uint16),
            rng.integers(0, 65536, size=(256, 512), dtype=np.uint16),
            weights_bf16(rng, (4096, 448), outlier_frac=0.001)]
    win = list(range(115, 122)) if window == "explicit" else window
    xs = [to_torch_bf16(W) for W in mats]
    many = zs.compress_retiled_many(iter(xs), window=win, lookahead=lookahead)
    assert zs.compress_retiled_many([], window=win) == []
    assert len(many) == len(mats)
    for W, x, r in zip(mats, xs, many):
        one = zs.compress_retiled(x, window=win)
        torch.cuda.synchronize()
        assert (r.rows, r.cols, r.start_exp, r.num_outliers, r.compressed_bytes) == \
            (one.rows, one.cols, one.start_exp, one.num_outliers, one.compressed_bytes)
        assert torch.equal(r.fixed, one.fixed)
        assert torch.equal(r.eoff, one.eoff)
        assert torch.equal(r.exps, one.exps)
        o = zo.compress_retiled(W, r.start_exp)
        np.testing.assert_array_equal(r.fixed.cpu().numpy(), o.fixed)
        np.testing.assert_array_equal(r.exps[: r.num_outliers].cpu().numpy(), o.exps)
        np.testing.assert_array_equal(from_torch_bf16(zs.decompress_retiled(r)), W)
