"""The C-ABI library loads and exports every symbol include/zipserv.h declares.

No device entry point is called here (this suite runs without a GPU)."""
import ctypes as C
import os
import re

import zipserv_asplos26_amd as zs
from zipserv_asplos26_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    src = open(os.path.join(ROOT, "include", "zipserv.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(zs_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for must in ["zs_bf16_triple_bitmap_mm", "zs_bf16_triple_bitmap_decompress",
                 "zs_init_bf16_matrix_triple_bitmap", "zs_init_bf16_matrix_triple_bitmap_reuse",
                 "zs_init_bf16_matrix_triple_bitmap_reuse_simd",
                 "zs_init_bf16_matrix_triple_bitmap_gpu", "zs_analyze_exponents_host",
                 "zs_analyze_top_exponents_gpu", "zs_decode_attention"]:
        assert must in names


def test_library_exports_every_declared_symbol():
    raw = C.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(raw, n)]
    assert not missing, missing
    # and the Python binding knows the signature of each
    assert set(declared_functions()) <= set(_lib.SIGNATURES)


def test_size_queries():
    L = zs.lib()
    assert L.zs_num_global_tiles(4096, 4096) == 4096
    assert L.zs_sign_mantissa_capacity(64, 64) >= 4096 + 16 + 64
    assert L.zs_splitk_workspace_bytes(128, 8, 1) == 0
    assert L.zs_splitk_workspace_bytes(128, 8, 4) == 4 * 128 * 8 * 2
    mk = 4096 * 4096
    assert L.zs_compressed_bytes(4096, 4096, 100, 10) == 100 + 20 + 24 * mk // 64 + 8 * mk // 1024 + 8 * (mk // 4096 + 1)
    assert L.zs_version().startswith(b"zipserv")
    assert L.zs_status_string(-1) == b"invalid argument"


def test_retiled_mm_refuses_k_past_row_blocks():
    # X of N*K*2 > 2^31 bytes runs as row blocks of X; with K > 2^26 not even
    # a 16-row block fits 2^31 bytes, which must be refused up front
    # (ZS_E_OVERFLOW) rather than split again.  Fake, aligned pointers: the
    # call returns during argument checks, before touching memory or a GPU.
    L = zs.lib()
    fake = 1 << 20
    K = (1 << 26) + 64
    assert L.zs_retiled_mm(None, fake, fake, fake, 120, fake, fake, 64, 16, K, None, 1) == \
        _lib.ZS_E_OVERFLOW


def test_batched_encoder_argument_checks():
    # compress_retiled_many refuses a negative lookahead before any device
    # work, and an empty batch is an empty list
    import pytest
    import zipserv_asplos26_amd as zs
    with pytest.raises(ValueError):
        zs.compress_retiled_many([], lookahead=-1)
    assert zs.compress_retiled_many([]) == []
