"""The container of csrc/zs_container.cpp (no counterpart in the reference,
which keeps compressed matrices only in memory): CRC-32C against its
published check value and a bitwise restatement of the polynomial, byte
layout, round trips of the canonical streams through bytes, files and
bundles, and rejection of damaged images."""
import numpy as np
import pytest

import zipserv_asplos26_amd as zs
from zipserv_asplos26_amd import container as ct
from zs_testutil import weights_bf16


def _crc32c_bitwise(data: bytes) -> int:
    # CRC-32C: reflected Castagnoli polynomial 0x82F63B78, init and final xor ~0
    crc = 0xFFFFFFFF
    for byte in data:
        crc ^= byte
        for _ in range(8):
            crc = (crc >> 1) ^ (0x82F63B78 if crc & 1 else 0)
    return crc ^ 0xFFFFFFFF


def _crc(data: bytes, crc: int = 0) -> int:
    buf = np.frombuffer(data, np.uint8) if data else np.zeros(1, np.uint8)
    return int(zs.lib().zs_crc32c(crc, buf.ctypes.data, len(data)))


def test_crc32c_known_answers():
    assert _crc(b"123456789") == 0xE3069283  # the published CRC-32C check value
    assert _crc(b"") == 0
    rng = np.random.default_rng(0)
    for n in (1, 7, 8, 9, 63, 64, 1000):
        d = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert _crc(d) == _crc32c_bitwise(d)
        # incremental over any split, unaligned starts included
        k = n // 3
        assert _crc(d[k:], _crc(d[:k])) == _crc(d)


def _host_matrix(seed=1, shape=(128, 192), frac=0.01):
    rng = np.random.default_rng(seed)
    return zs.compress_host(weights_bf16(rng, shape, outlier_frac=frac))


def _same(a, b):
    for f in ("rows", "cols", "start_exp", "max_high_freq_count", "max_full_count"):
        assert getattr(a, f) == getattr(b, f), f
    for f in ("sign_mantissa", "compressed_full", "bitmap1", "bitmap2", "bitmap3",
              "tile_offsets", "tile_offsets_median", "tile_offsets_global"):
        np.testing.assert_array_equal(getattr(a, f), getattr(b, f), err_msg=f)


def test_container_layout_and_round_trip():
    h = _host_matrix()
    b = ct.to_bytes(h, name="layer0.qkv")
    assert bytes(b[:8]) == b"ZSRVCNTR"
    assert int(b[8:12].view(np.uint32)[0]) == 1 and int(b[12:16].view(np.uint32)[0]) == 256
    sizes = [h.sign_mantissa.size, 2 * h.compressed_full.size] + [8 * h.bitmap1.size] * 3 + \
        [4 * h.tile_offsets_median.size, 4 * h.tile_offsets_global.size]
    table = b[128:256].view(np.uint64).reshape(8, 2)
    assert [int(table[i, 0]) for i in range(7)] == sizes
    assert b.size == 256 + sum((n + 63) // 64 * 64 for n in sizes)
    assert int(b[56:64].view(np.uint64)[0]) == b.size
    assert bytes(b[64:74]) == b"layer0.qkv"
    # stream 0 starts right after the header, byte for byte
    np.testing.assert_array_equal(b[256:256 + sizes[0]], h.sign_mantissa)
    _same(ct.from_bytes(b), h)


def test_container_files_and_bundles(tmp_path):
    h0, h1 = _host_matrix(2, (64, 64), 0.0), _host_matrix(3, (192, 128), 0.2)
    p = tmp_path / "one.zsc"
    assert ct.save(str(p), h1, "w") == p.stat().st_size
    _same(ct.load(str(p)), h1)
    q = tmp_path / "bundle.zsc"
    ct.save_bundle(str(q), {"a": h0, "b": h1, "c": h0})
    got = ct.load_bundle(str(q))
    assert list(got) == ["a", "b", "c"]
    _same(got["a"], h0)
    _same(got["b"], h1)
    _same(got["c"], h0)


@pytest.mark.parametrize("where", ["magic", "header", "sm", "full", "bitmap", "global", "pad"])
def test_container_rejects_damage(where):
    h = _host_matrix(4)
    b = ct.to_bytes(h)
    sm = h.sign_mantissa.size
    at = {"magic": 0, "header": 30, "sm": 256 + sm // 2,
          "full": 256 + (sm + 63) // 64 * 64 + 1, "bitmap": b.size - 4096,
          "global": b.size - 40, "pad": None}[where]
    bad = b.copy()
    if at is None:  # a stream table size that no longer matches the shape
        bad[128 + 16 * 2] ^= 8
    else:
        bad[at] ^= 0x40
    with pytest.raises(zs.ZipServError):
        ct.from_bytes(bad)


def test_container_rejects_truncation_and_version():
    b = ct.to_bytes(_host_matrix(5))
    with pytest.raises(zs.ZipServError):
        ct.from_bytes(b[:-64])
    v = b.copy()
    v[8] = 2  # another version: unsupported, whatever its CRC says
    with pytest.raises(zs.ZipServError) as e:
        ct.from_bytes(v)
    assert e.value.status == zs._lib.ZS_E_UNSUPPORTED


def test_container_golden_image():
    # the committed v1 image of a fixed 64x64 matrix still parses to it, and
    # encoding that matrix again reproduces the image byte for byte
    import os
    here = os.path.join(os.path.dirname(__file__), "golden")
    matrix = np.load(os.path.join(here, "container_v1_matrix.npy"))
    image = np.fromfile(os.path.join(here, "container_v1.zsc"), np.uint8)
    _same(ct.from_bytes(image), zs.compress_host(matrix))
    np.testing.assert_array_equal(ct.to_bytes(zs.compress_host(matrix), "golden"), image)


def _reseal(b):
    """Recompute every stream CRC and the header CRC of a container image, so
    a planted change passes the CRC checks and only the offset checks remain."""
    b = b.copy()
    n = int(b[20:24].view(np.uint32)[0])
    off = 256
    for i in range(n):
        size = int(b[128 + 16 * i: 136 + 16 * i].view(np.uint64)[0])
        crc = _crc(b[off: off + size].tobytes()) if size else 0
        b[136 + 16 * i: 140 + 16 * i] = np.array([crc], np.uint32).view(np.uint8)
        off += (size + 63) // 64 * 64
    b[52:56] = 0
    b[52:56] = np.array([_crc(b[:256].tobytes())], np.uint32).view(np.uint8)
    return b


def _stream_at(b, i):
    off = 256
    for j in range(i):
        off += (int(b[128 + 16 * j: 136 + 16 * j].view(np.uint64)[0]) + 63) // 64 * 64
    return off


def _retiled_host(seed=6, shape=(128, 192), frac=0.05):
    import oracle as zo
    rng = np.random.default_rng(seed)
    W = weights_bf16(rng, shape, outlier_frac=frac)
    r = zo.compress_retiled(W, zo.analyze_gpu(W)[0] - 1)
    return zs.ZipservRetiled(r.fixed, r.exps, r.eoff, r.rows, r.cols, r.rows, r.cols,
                             r.start_exp, r.exps.size, r.compressed_bytes())


def test_container_reseal_keeps_good_images():
    # the CRC rewrite alone changes nothing: a resealed good image still loads
    h = _host_matrix(7)
    _same(ct.from_bytes(_reseal(ct.to_bytes(h))), h)
    b = ct.to_bytes(_retiled_host())
    np.testing.assert_array_equal(_reseal(b), b)
    d, _, streams, _ = ct._parse(b)
    assert d.layout == zs._lib.ZS_CONTAINER_RETILED and len(streams) == 3


@pytest.mark.parametrize("plant", ["eoff0", "swap", "over1024", "code"])
def test_container_rejects_crc_valid_bad_retiled_offsets(plant):
    # a CRC-valid image whose outlier offsets disagree with the record codes
    # would steer the decoders past the exponent stream: rejected on load
    r = _retiled_host()
    b = ct.to_bytes(r)
    fx, eo = _stream_at(b, 0), _stream_at(b, 2)
    eoff = b[eo: eo + 4 * r.eoff.size].view(np.int32)
    bad = b.copy()
    beoff = bad[eo: eo + 4 * r.eoff.size].view(np.int32)
    if plant == "eoff0":
        beoff[:] = eoff + 1                      # not starting at 0 (last offset moved too)
    elif plant == "swap":
        i = int(np.argmax(np.diff(eoff) > 0))    # a record with outliers
        beoff[i + 1] = eoff[i]                   # its bytes handed to the next record
    elif plant == "over1024":
        beoff[1:] = eoff[1:] + 2000              # a record with 2000 "outliers"
    else:
        # one in-window code turned into an outlier code, offsets untouched
        p32 = bad[fx + 1024: fx + 1028].view(np.uint32)
        codes = int(p32[0])
        k = next(i for i in range(8) if (codes >> (3 * i)) & 7)
        p32[0] = codes & ~(7 << (3 * k))
    with pytest.raises(zs.ZipServError):
        ct.from_bytes(_reseal(bad), device="cpu")


@pytest.mark.parametrize("plant", ["global", "median", "pad"])
def test_container_rejects_crc_valid_bad_canonical_offsets(plant):
    h = _host_matrix(8, (128, 192), 0.05)
    b = ct.to_bytes(h)
    bad = b.copy()
    if plant == "global":
        tog = bad[_stream_at(b, 6): _stream_at(b, 6) + 4 * h.tile_offsets_global.size].view(np.int32)
        tog[2] += 16                              # GT 1 starts 16 SM bytes late
    elif plant == "median":
        tom = bad[_stream_at(b, 5): _stream_at(b, 5) + 4 * h.tile_offsets_median.size].view(np.int32)
        tom[2] += 1                               # median 1 of GT 0 off by one
    else:
        tog = bad[_stream_at(b, 6): _stream_at(b, 6) + 4 * h.tile_offsets_global.size].view(np.int32)
        tog[2:] += 1                              # padding no longer a multiple of 16
    with pytest.raises(zs.ZipServError):
        ct.from_bytes(_reseal(bad))
