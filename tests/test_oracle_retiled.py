"""CPU oracle of the CDNA4 re-tiled layout (this build's device layout; it has
no counterpart in the reference).  Pinned by: the round trip back to the exact
bf16 input, equality with the canonical encoder's content (outlier count,
code planes), hand-built known answers, and the exponent wrap mod 256."""
import numpy as np
import pytest

import oracle as zo
from zs_testutil import normal_bf16, weights_bf16


def _lane_of(row, col):
    """(record, h, lane, i) of matrix element (row, col) for K = 64*KT."""
    band, r16 = divmod(row, 16)
    kt, c64 = divmod(col, 64)
    h, c32 = divmod(c64, 32)
    q, i = divmod(c32, 8)
    return band, kt, h, 16 * q + r16, i


@pytest.mark.parametrize("shape,frac,seed", [((64, 64), 0.0, 0), ((128, 192), 0.01, 1),
                                             ((256, 128), 0.05, 2), ((64, 640), 0.3, 3)])
def test_retiled_round_trip(shape, frac, seed):
    rng = np.random.default_rng(seed)
    W = weights_bf16(rng, shape, outlier_frac=frac)
    e = zo.compress(W)
    r = zo.retile(e)
    np.testing.assert_array_equal(zo.decompress_retiled(r), W)
    # same content as the canonical streams: every unpadded FULL value is one outlier byte
    ind = zo_in_window_mask(W, e.start_exp)
    assert r.exps.size == int((~ind).sum())
    assert np.all(np.diff(r.eoff) >= 0) and r.eoff[0] == 0 and r.eoff[-1] == r.exps.size
    # size: fixed records + outlier bytes + offsets
    nrec = (shape[0] // 16) * (shape[1] // 64)
    assert r.compressed_bytes() == nrec * 1408 + r.exps.size + 4 * (nrec + 1)


def zo_in_window_mask(W, start_exp):
    d = (((W.astype(np.int32) >> 7) & 0xFF) - start_exp) & 0xFF
    return (d >= 1) & (d <= 7)


def test_retiled_all_ones_known_answer():
    W = np.full((64, 64), 0x3F80, np.uint16)  # 1.0: exponent 127 -> window start 126, code 1
    r = zo.compress_retiled(W, 126)
    f = r.fixed.reshape(4, 1408)
    assert np.all(f[:, :1024] == 0)                      # mantissa 0, partner sign 0
    p32 = f[:, 1024:1280].copy().view(np.uint32)
    p16 = f[:, 1280:1408].copy().view(np.uint16)
    # eight 3-bit codes 1 per half: 0o11111111 = 0x249249
    assert np.all(p32 == 0x49249249) and np.all(p16 == 0x2492)
    assert r.exps.size == 0 and np.all(r.eoff == 0)


def _codes(f, lane, h):
    w32 = int(f[1024 + 4 * lane:1028 + 4 * lane].view(np.uint32)[0])
    w16 = int(f[1280 + 2 * lane:1282 + 2 * lane].view(np.uint16)[0])
    c = ((w32 >> 24) | (w16 << 8)) if h else (w32 & 0xFFFFFF)
    return [(c >> (3 * i)) & 7 for i in range(8)]


def test_retiled_single_outlier_placement():
    W = np.full((128, 128), 0x3F80, np.uint16)
    row, col = 37, 101
    W[row, col] = 0xC4A5  # sign 1, exponent 137 (outside 127..133), mantissa 0x25
    r = zo.compress_retiled(W, 126)
    band, kt, h, lane, i = _lane_of(row, col)
    rec = band * 2 + kt
    assert r.exps.tolist() == [137]                      # the raw exponent byte
    assert np.diff(r.eoff).tolist() == [1 if k == rec else 0 for k in range(16)]
    f = r.fixed.reshape(16, 1408)[rec]
    assert f[16 * lane + 8 * h + i] == 0x25 << 1         # mantissa << 1, partner sign 0
    assert f[16 * lane + 8 * h + (i ^ 1)] == 0x01        # partner: mantissa 0, this sign 1
    assert _codes(f, lane, h) == [0 if k == i else 1 for k in range(8)]
    assert _codes(f, lane, 1 - h) == [1] * 8
    np.testing.assert_array_equal(zo.decompress_retiled(r), W)


def test_retiled_signs_follow_partner():
    # every sign pattern of a pair, every mantissa, in-window and outlier
    a = np.arange(1 << 16, dtype=np.uint32)
    W = (a.astype(np.uint16)).reshape(1024, 64)
    for st in (0, 120, 250):
        r = zo.compress_retiled(W, st)
        np.testing.assert_array_equal(zo.decompress_retiled(r), W)


def test_retiled_exponent_wrap():
    # start_exp 255 (window 0..6): code c decodes to (255 + c) mod 256 = c - 1
    rng = np.random.default_rng(3)
    W = (rng.integers(0, 7, (64, 64)) << 7).astype(np.uint16) | rng.integers(0, 128, (64, 64)).astype(np.uint16)
    W[5, 5] = 0x4000  # exponent 128: outlier
    r = zo.compress_retiled(W, 255)
    assert r.exps.size == 1 and r.exps[0] == 128
    np.testing.assert_array_equal(zo.decompress_retiled(r), W)


def test_retiled_all_outliers_and_zeros():
    rng = np.random.default_rng(4)
    Z = np.zeros((64, 128), np.uint16)
    r = zo.compress_retiled(Z, 126)      # exponent 0 is outside 127..133: all outliers
    assert r.exps.size == Z.size and np.all(r.exps == 0)
    np.testing.assert_array_equal(zo.decompress_retiled(r), Z)
    X = normal_bf16(rng, (64, 128), std=1e-30)
    r = zo.compress_retiled(X, 10)
    np.testing.assert_array_equal(zo.decompress_retiled(r), X)
