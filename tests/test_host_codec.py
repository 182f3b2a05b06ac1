"""Product CPU codec (libzipserv host encoders, C-ABI) against the oracle."""
import numpy as np
import pytest

import oracle as zo
import zipserv_asplos26_amd as zs
from zs_testutil import kv_bf16, pad_by_kv_head, weights_bf16

FIELDS = ["sign_mantissa", "compressed_full", "bitmap1", "bitmap2", "bitmap3", "tile_offsets",
          "tile_offsets_median", "tile_offsets_global"]


def assert_same(h, e):
    for f in FIELDS:
        np.testing.assert_array_equal(getattr(h, f), getattr(e, f), err_msg=f)
    assert h.max_high_freq_count == e.max_high_freq_count
    assert h.max_full_count == e.max_full_count
    assert h.start_exp == e.start_exp


@pytest.mark.parametrize("variant", ["alloc", "reuse", "reuse_simd"])
@pytest.mark.parametrize("shape,frac,seed", [((64, 64), 0.0, 0), ((192, 128), 0.001, 1),
                                             ((128, 320), 0.1, 2)])
def test_host_encoders_match_oracle(variant, shape, frac, seed):
    rng = np.random.default_rng(seed)
    W = weights_bf16(rng, shape, outlier_frac=frac)
    assert zs.analyze_exponents(W) == zo.analyze_cpu(W)
    assert_same(zs.compress_host(W, variant=variant), zo.compress(W))


def test_host_encoder_kv_cache():
    rng = np.random.default_rng(3)
    kv = kv_bf16(rng, 2, 100, 2, 128)
    A, _ = pad_by_kv_head(kv)  # padding zeros count as exponent 0 in the histogram
    assert zs.analyze_exponents(A) == zo.analyze_cpu(A)
    assert_same(zs.compress_host(A), zo.compress(A))


def test_noncontiguous_window_lut_variants():
    # the LUT encoders accept any 7 exponents; the SIMD one uses [top0, top0+6]
    rng = np.random.default_rng(4)
    W = weights_bf16(rng, (64, 128))
    top = [110, 116, 117, 118, 119, 120, 121]
    h = zs.compress_host(W, top=top, variant="reuse")
    e = zo.compress(W, top=top, variant="lut")
    assert_same(h, e)
    assert_same(zs.compress_host(W, top=top, variant="alloc"), zo.compress(W, top=top, variant="plain"))


@pytest.mark.parametrize("shape", [(64, 64), (128, 192)])
def test_host_roundtrip_random_bits(shape):
    rng = np.random.default_rng(8)
    W = rng.integers(0, 65536, size=shape, dtype=np.uint16)
    h = zs.compress_host(W)
    e = zo.compress(W)
    assert_same(h, e)
    np.testing.assert_array_equal(zo.decompress(e), W)


def test_host_rejects_bad_shapes():
    W = np.zeros((64, 96), np.uint16)
    with pytest.raises(zs.ZipServError):
        zs.compress_host(W, top=list(range(120, 127)))
    L = zs.lib()
    top = np.arange(120, 127, dtype=np.int32)
    # wrong tile sizes -> ZS_E_UNSUPPORTED
    import ctypes as C
    ptrs = [C.c_void_p() for _ in range(8)]
    a = np.zeros((64, 64), np.uint16)
    rc = L.zs_init_bf16_matrix_triple_bitmap(a.ctypes.data, 64, 64, 8, 16, 64, 8, 32, 64,
                                             top.ctypes.data, *[C.byref(p) for p in ptrs],
                                             C.byref(C.c_int32()), C.byref(C.c_int32()))
    assert rc == -2
