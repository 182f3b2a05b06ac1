"""GPU parity of the codec kernels (decompress, encoder, analyze) and ZipGEMM
against the CPU oracle, through the C-ABI.  Bit-exact for codec work; ZipGEMM
within 1e-2 relative error of the fp32-accumulated product."""
import numpy as np
import pytest

import oracle as zo
import zipserv_asplos26_amd as zs
from zs_testutil import (arbitrary_bf16, from_torch_bf16, kv_bf16, normal_bf16, pad_by_kv_head,
                         to_torch_bf16, upload, weights_bf16)

pytestmark = pytest.mark.gpu

SHAPES = [((64, 64), 0.0, 0), ((128, 192), 0.001, 1), ((256, 512), 0.05, 2), ((64, 4096), 0.01, 3),
          ((1024, 64), 0.3, 4)]


@pytest.mark.parametrize("shape,frac,seed", SHAPES)
def test_decompress_bit_exact(torch_cuda, shape, frac, seed):
    rng = np.random.default_rng(seed)
    W = weights_bf16(rng, shape, outlier_frac=frac)
    c = upload(zo.compress(W))
    out = zs.decompress(c)
    torch_cuda.cuda.synchronize()
    np.testing.assert_array_equal(from_torch_bf16(out), W)


@pytest.mark.parametrize("kind", ["random_bits", "all_outliers", "uniform", "wrap"])
def test_decompress_edge_inputs(torch_cuda, kind):
    rng = np.random.default_rng(21)
    if kind == "random_bits":
        W = rng.integers(0, 65536, size=(128, 128), dtype=np.uint16)
        e = zo.compress(W)
    elif kind == "all_outliers":
        W = weights_bf16(rng, (128, 128))
        e = zo.compress(W, top=list(range(10, 17)))
    elif kind == "uniform":
        W = np.full((64, 128), 0x3F80, np.uint16)
        e = zo.compress(W)
    else:
        W = np.tile(np.array([(e_ << 7) | 9 for e_ in range(7)] * 10, np.uint16)[:64], (64, 1))
        e = zo.compress(W, top=list(range(0, 7)))
        assert e.start_exp == 255
    out = zs.decompress(upload(e))
    torch_cuda.cuda.synchronize()
    np.testing.assert_array_equal(from_torch_bf16(out), W)


@pytest.mark.parametrize("shape,frac,seed", SHAPES)
def test_gpu_encoder_matches_oracle(torch_cuda, shape, frac, seed):
    rng = np.random.default_rng(100 + seed)
    W = weights_bf16(rng, shape, outlier_frac=frac)
    parts = zs.compress_zipserv(to_torch_bf16(W))
    sm, fu, b1, b2, b3, med, tog, meta = parts
    m = meta.tolist()
    top = zo.analyze_gpu(W)
    e = zo.compress(W, top=top)
    assert m[6] == e.start_exp
    assert m[4] == e.max_high_freq_count and m[5] == e.max_full_count
    assert m[7] == e.sign_mantissa.size and m[8] == e.compressed_full.size
    np.testing.assert_array_equal(sm.cpu().numpy()[: m[7]], e.sign_mantissa)
    np.testing.assert_array_equal(from_torch_bf16(fu)[: m[8]], e.compressed_full)
    np.testing.assert_array_equal(b1.cpu().numpy().view(np.uint64), e.bitmap1)
    np.testing.assert_array_equal(b2.cpu().numpy().view(np.uint64), e.bitmap2)
    np.testing.assert_array_equal(b3.cpu().numpy().view(np.uint64), e.bitmap3)
    np.testing.assert_array_equal(med.cpu().numpy(), e.tile_offsets_median)
    np.testing.assert_array_equal(tog.cpu().numpy(), e.tile_offsets_global)
    # and the device streams decode back to W
    c = zs.make_zipserv_compressed(parts)
    np.testing.assert_array_equal(from_torch_bf16(zs.decompress(c)), W)


@pytest.mark.parametrize("kind", ["random_bits", "specials"])
def test_gpu_encoder_arbitrary_bits(torch_cuda, kind):
    # NaN payloads, infinities, subnormals and signed zeros are outliers or
    # in-window values like any other bits: the GPU encoder's streams equal
    # the oracle's byte for byte and decode back to the same bits
    rng = np.random.default_rng(41)
    W = arbitrary_bf16(rng, (192, 512), kind)
    parts = zs.compress_zipserv(to_torch_bf16(W))
    sm, fu, b1, b2, b3, med, tog, meta = parts
    m = meta.tolist()
    e = zo.compress(W, top=zo.analyze_gpu(W))
    assert m[6] == e.start_exp and m[7] == e.sign_mantissa.size and m[8] == e.compressed_full.size
    np.testing.assert_array_equal(sm.cpu().numpy()[: m[7]], e.sign_mantissa)
    np.testing.assert_array_equal(from_torch_bf16(fu)[: m[8]], e.compressed_full)
    np.testing.assert_array_equal(b1.cpu().numpy().view(np.uint64), e.bitmap1)
    np.testing.assert_array_equal(b2.cpu().numpy().view(np.uint64), e.bitmap2)
    np.testing.assert_array_equal(b3.cpu().numpy().view(np.uint64), e.bitmap3)
    np.testing.assert_array_equal(med.cpu().numpy(), e.tile_offsets_median)
    np.testing.assert_array_equal(tog.cpu().numpy(), e.tile_offsets_global)
    c = zs.make_zipserv_compressed(parts)
    np.testing.assert_array_equal(from_torch_bf16(zs.decompress(c)), W)


def test_gpu_encoder_kv_cache(torch_cuda):
    rng = np.random.default_rng(7)
    A, _ = pad_by_kv_head(kv_bf16(rng, 2, 300, 8, 128))
    c = zs.compress(to_torch_bf16(A))
    e = zo.compress(A, top=zo.analyze_gpu(A))
    assert c.total_high_freq == e.sign_mantissa.size
    np.testing.assert_array_equal(from_torch_bf16(zs.decompress(c)), A)


def test_gpu_analyze_histogram(torch_cuda):
    torch = torch_cuda
    rng = np.random.default_rng(12)
    a = rng.integers(0, 65536, size=100003, dtype=np.uint16)
    t = to_torch_bf16(a)
    counts = torch.empty(256, dtype=torch.int32, device="cuda")
    top = torch.empty(7, dtype=torch.int32, device="cuda")
    done = torch.empty(1, dtype=torch.int32, device="cuda")
    rc = zs.lib().zs_analyze_top_exponents_gpu(int(torch.cuda.current_stream().cuda_stream), t.data_ptr(),
                                              a.size, counts.data_ptr(), top.data_ptr(), done.data_ptr())
    assert rc == 0
    np.testing.assert_array_equal(counts.cpu().numpy(), np.bincount((a >> 7) & 0xFF, minlength=256))
    assert top.cpu().tolist() == zo.select_gpu(np.bincount((a >> 7) & 0xFF, minlength=256))


def _data_with_counts(counts, rng):
    """bf16 values whose exponent histogram is exactly `counts`."""
    e = np.repeat(np.arange(256, dtype=np.uint16), counts)
    rng.shuffle(e)
    return (e << 7) | rng.integers(0, 128, e.size, dtype=np.uint16)


@pytest.mark.parametrize("rule", ["kv", "weights"])
@pytest.mark.parametrize("case", ["evict_first_min_slot", "ties_at_seventh", "few_present",
                                  "all_equal", "top_edge", "noncontiguous", "one_exponent",
                                  "zeros_only", "bottom_edge"])
def test_gpu_select_window_special_cases(torch_cuda, case, rule):
    # window selection of zipserv_decode_attention_ext.cu:65-134 (streaming
    # top-7 evicting the first minimum slot; "kv") and of
    # kernel_benchmark/utils.h:189-272 (seven largest-count passes; "weights")
    # against the oracle restatements
    torch = torch_cuda
    rng = np.random.default_rng(31)
    c = np.zeros(256, np.int64)
    if case == "evict_first_min_slot":
        c[0], c[1], c[7] = 5, 3, 4          # 7 evicts exponent 2 (first zero slot)
    elif case == "ties_at_seventh":
        c[100:112] = 9
        c[105] = 20
    elif case == "few_present":
        c[120], c[121], c[125] = 50, 40, 30
    elif case == "all_equal":
        c[:] = 3
    elif case == "top_edge":
        c[250:256] = [10, 20, 30, 40, 50, 60]
    elif case == "one_exponent":
        c[127] = 4096                        # the rules differ: 121..127 vs 1..7
    elif case == "zeros_only":
        c[0] = 4096
    elif case == "bottom_edge":
        c[0:5] = [60, 50, 40, 30, 20]
    else:
        c[[10, 11, 12, 40, 41, 90, 200]] = [7, 8, 9, 30, 31, 5, 6]
    a = _data_with_counts(c, rng)
    t = to_torch_bf16(a)
    top = torch.empty(7, dtype=torch.int32, device="cuda")
    st = int(torch.cuda.current_stream().cuda_stream)
    if rule == "kv":
        counts = torch.empty(256, dtype=torch.int32, device="cuda")
        rc = zs.lib().zs_analyze_top_exponents_gpu(st, t.data_ptr(), a.size, counts.data_ptr(),
                                                  top.data_ptr(), None)
        want = zo.select_gpu(c)
    else:
        counts = torch.empty(256, dtype=torch.int64, device="cuda")
        rc = zs.lib().zs_analyze_exponents_weights_gpu(st, t.data_ptr(), a.size,
                                                      counts.data_ptr(), top.data_ptr())
        want = zo.select_cpu(c)
    assert rc == 0
    np.testing.assert_array_equal(counts.cpu().numpy(), c)
    assert top.cpu().tolist() == want


def rel_err(y, ref):
    return np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30)


@pytest.mark.parametrize("M,K", [(64, 64), (256, 512), (192, 1024)])
@pytest.mark.parametrize("N", [1, 5, 8, 16, 17, 32, 64, 100, 128, 200])
def test_zipgemm_matches_oracle(torch_cuda, M, K, N):
    rng = np.random.default_rng(M * 7 + K + N)
    W = weights_bf16(rng, (M, K), outlier_frac=0.001)
    X = normal_bf16(rng, (N, K))
    c = upload(zo.compress(W))
    Y = zs.zipgemm(c, to_torch_bf16(X))
    torch_cuda.cuda.synchronize()
    y = zo.bf16_to_f32(from_torch_bf16(Y))
    ref = zo.gemm_f32(W, X)
    assert y.shape == (N, M)
    assert rel_err(y, ref) <= 1e-2
    np.testing.assert_allclose(y, ref, rtol=1e-2, atol=1e-2 * np.abs(ref).max())


@pytest.mark.parametrize("split_k,N", [(2, 24), (3, 24), (4, 24), (2, 1), (4, 16), (2, 64),
                                       (3, 100), (5, 128)])
def test_zipgemm_splitk(torch_cuda, split_k, N):
    rng = np.random.default_rng(split_k * 1000 + N)
    M, K = 128, 320
    W = weights_bf16(rng, (M, K), outlier_frac=0.01)
    X = normal_bf16(rng, (N, K))
    c = upload(zo.compress(W))
    Y = zs.zipgemm(c, to_torch_bf16(X), split_k=split_k)
    torch_cuda.cuda.synchronize()
    y = zo.bf16_to_f32(from_torch_bf16(Y))
    assert rel_err(y, zo.gemm_f32(W, X)) <= 1e-2
    model = zo.bf16_to_f32(zo.gemm_splitk_bf16(W, X, split_k))
    assert rel_err(y, model) <= 1e-2


@pytest.mark.parametrize("M,K,N,split_k", [(256, 2048, 16, 4), (192, 4096, 8, 8), (512, 1024, 32, 2),
                                           (128, 64 * 70, 1, 3)])
def test_zipgemm_splitk_long_slices(torch_cuda, M, K, N, split_k):
    """Slices longer than the 64-tile offset chunk and heavy outliers."""
    rng = np.random.default_rng(M + K + N + split_k)
    W = weights_bf16(rng, (M, K), outlier_frac=0.05)
    X = normal_bf16(rng, (N, K))
    c = upload(zo.compress(W))
    Y = zs.zipgemm(c, to_torch_bf16(X), split_k=split_k)
    y = zo.bf16_to_f32(from_torch_bf16(Y))
    assert rel_err(y, zo.gemm_f32(W, X)) <= 1e-2
    assert rel_err(y, zo.bf16_to_f32(zo.gemm_splitk_bf16(W, X, split_k))) <= 1e-2


def test_zipgemm_unit_vectors_exact(torch_cuda):
    rng = np.random.default_rng(31)
    M, K = 128, 256
    W = weights_bf16(rng, (M, K), outlier_frac=0.05)
    ks = [0, 7, 8, 31, 32, 63, 64, 200, 255]
    X = np.zeros((len(ks), K), np.uint16)
    for i, k in enumerate(ks):
        X[i, k] = 0x3F80
    Y = from_torch_bf16(zs.zipgemm(upload(zo.compress(W)), to_torch_bf16(X)))
    for i, k in enumerate(ks):
        np.testing.assert_array_equal(Y[i], W[:, k])


# 64-row workgroups (X tiles staged in LDS) run every split-K launch and a
# single slice at N > 16 on grids of >= 160 row blocks (>= 96 for N > 112):
# M = 10240 / 6144 select them with one slice, M = 12352 with two slices
# selects two K phases per workgroup instead of four; N = 200 spans two
# column blocks of 128.
@pytest.mark.parametrize("M,K,N,split_k", [(10240, 256, 17, 1), (10240, 256, 40, 1),
                                           (10240, 320, 100, 1), (10240, 256, 128, 1),
                                           (10240, 256, 200, 1), (6144, 512, 128, 1),
                                           (12352, 512, 1, 2), (12352, 512, 8, 2),
                                           (12352, 256, 40, 2), (12352, 384, 128, 3)])
def test_zipgemm_64row_workgroups(torch_cuda, M, K, N, split_k):
    rng = np.random.default_rng(M + K + N + split_k)
    W = weights_bf16(rng, (M, K), outlier_frac=0.01)
    X = normal_bf16(rng, (N, K))
    c = upload(zo.compress(W))
    Y = zs.zipgemm(c, to_torch_bf16(X), split_k=split_k)
    y = zo.bf16_to_f32(from_torch_bf16(Y))
    ref = zo.gemm_f32(W, X)
    assert rel_err(y, ref) <= 1e-2
    if split_k > 1:
        assert rel_err(y, zo.bf16_to_f32(zo.gemm_splitk_bf16(W, X, split_k))) <= 1e-2


@pytest.mark.parametrize("M,split_k", [(10240, 1), (128, 2), (12352, 3)])
def test_zipgemm_64row_unit_vectors_exact(torch_cuda, M, split_k):
    """One nonzero per batch row: every output is one weight, exactly, which
    pins the K phase of each tile and the B-fragment slot of each batch row."""
    rng = np.random.default_rng(M + split_k)
    K = 256
    W = weights_bf16(rng, (M, K), outlier_frac=0.05)
    ks = [0, 7, 8, 31, 32, 63, 64, 65, 100, 127, 128, 191, 192, 200, 255] * 3
    X = np.zeros((len(ks), K), np.uint16)
    for i, k in enumerate(ks):
        X[i, k] = 0x3F80
    Y = from_torch_bf16(zs.zipgemm(upload(zo.compress(W)), to_torch_bf16(X), split_k=split_k))
    for i, k in enumerate(ks):
        np.testing.assert_array_equal(Y[i], W[:, k])


@pytest.mark.parametrize("M,N,split_k,shift", [(128, 15, 1, 4), (128, 15, 2, 4), (10240, 15, 1, 4),
                                               (10240, 30, 1, 4), (12352, 15, 3, 4), (128, 15, 1, None),
                                               (10240, 30, 2, None)])
def test_zipgemm_outlier_dominated_unit_vectors_exact(torch_cuda, M, N, split_k, shift):
    """Median tiles with more than 264 outliers (33 staged FULL chunks) take
    their FULL values from global memory instead of the LDS stage.  The window
    moved `shift` exponents up from the analysed one leaves 262-361 outliers
    per median tile (both paths in one matrix at M = 10240); None: a window
    far below every exponent, all 1024 elements outliers.  16-row kernel at
    one slice and N <= 16, 64-row kernel with split-K and at N = 30."""
    rng = np.random.default_rng(M + N + split_k)
    K = 256
    W = weights_bf16(rng, (M, K), outlier_frac=0.01)
    e0 = zo.compress(W)
    E0 = e0.start_exp + 1
    lo = 10 if shift is None else E0 + shift
    e = zo.compress(W, top=list(range(lo, lo + 7)))
    ex = (W.astype(np.int64) >> 7) & 0xFF
    per_tile = ((ex < lo) | (ex > lo + 6)).reshape(M // 16, 16, K // 64, 64).sum(axis=(1, 3))
    assert per_tile.max() > 264
    ks = ([0, 7, 8, 31, 32, 63, 64, 65, 100, 127, 128, 191, 192, 200, 255] * 2)[:N]
    X = np.zeros((N, K), np.uint16)
    for i, k in enumerate(ks):
        X[i, k] = 0x3F80
    Y = from_torch_bf16(zs.zipgemm(upload(e), to_torch_bf16(X), split_k=split_k))
    for i, k in enumerate(ks):
        np.testing.assert_array_equal(Y[i], W[:, k])


def test_zipgemm_rejects_bad_args(torch_cuda):
    rng = np.random.default_rng(0)
    W = weights_bf16(rng, (64, 128))
    c = upload(zo.compress(W))
    X = to_torch_bf16(normal_bf16(rng, (4, 128)))
    with pytest.raises(zs.ZipServError):
        zs.zipgemm(c, X, split_k=3)  # split_k > K/64
