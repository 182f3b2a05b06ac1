"""ctypes binding of libzipserv.so (the C-ABI declared in include/zipserv.h).

The library is built in-tree (zipserv_asplos26_amd/_build/libzipserv.so) by
`make -C zipserv_asplos26_amd` or `build()`.  Loading fails loudly when it is
missing: there is no Python or CPU fallback for any device entry point.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "_build", "libzipserv.so")

ZS_OK = 0
ZS_E_INVAL = -1
ZS_E_UNSUPPORTED = -2
ZS_E_OVERFLOW = -3
ZS_E_NOMEM = -4
ZS_STREAM_SLACK_BYTES = 64
ZS_RETILED_EXP_SLOT_BYTES = 256
ZS_WINDOW_KV = 0
ZS_WINDOW_WEIGHTS = 1
ZS_RETILED_AUTO_WORK_BYTES = 65600
ZS_LAYOUT_HEAD_MAJOR = 0
ZS_LAYOUT_TOKEN_MAJOR = 1

_lib = None

_p = C.c_void_p
_i32 = C.c_int32
_i64 = C.c_int64

# name -> (restype, argtypes); mirrors include/zipserv.h exactly.
SIGNATURES = {
    "zs_version": (C.c_char_p, []),
    "zs_status_string": (C.c_char_p, [C.c_int]),
    "zs_num_global_tiles": (_i64, [C.c_int, C.c_int]),
    "zs_sign_mantissa_capacity": (_i64, [C.c_int, C.c_int]),
    "zs_full_capacity": (_i64, [C.c_int, C.c_int]),
    "zs_compressed_bytes": (_i64, [C.c_int, C.c_int, _i64, _i64]),
    "zs_splitk_workspace_bytes": (_i64, [C.c_int, C.c_int, C.c_int]),
    "zs_analyze_exponents_host": (C.c_int, [_p, _i64, _p]),
    "zs_init_bf16_matrix_triple_bitmap": (
        C.c_int, [_p, C.c_int, C.c_int] + [C.c_int] * 6 + [_p] + [_p] * 8 + [_p, _p]),
    "zs_host_free": (None, [_p]),
    "zs_init_bf16_matrix_triple_bitmap_reuse": (
        C.c_int, [_p, C.c_int, C.c_int] + [C.c_int] * 6 + [_p] + [_p] * 8 + [_p] * 6 + [_p] * 4),
    "zs_init_bf16_matrix_triple_bitmap_reuse_simd": (
        C.c_int, [_p, C.c_int, C.c_int] + [C.c_int] * 6 + [_p] + [_p] * 8 + [_p] * 6 + [_p] * 4),
    "zs_bf16_triple_bitmap_decompress": (
        C.c_int, [_p] + [_p] * 7 + [C.c_int, C.c_int, C.c_uint8, _p, C.c_int, C.c_int]),
    "zs_bf16_triple_bitmap_mm": (
        C.c_int, [_p] + [_p] * 7 + [C.c_int, C.c_int, C.c_uint8, _p, _p, C.c_int, C.c_int,
                                    C.c_int, _p, C.c_int]),
    "zs_analyze_top_exponents_gpu": (C.c_int, [_p, _p, _i64, _p, _p, _p]),
    "zs_analyze_top_exponents_u64_gpu": (C.c_int, [_p, _p, _i64, _p, _p]),
    "zs_analyze_exponents_weights_gpu": (C.c_int, [_p, _p, _i64, _p, _p]),
    "zs_init_bf16_matrix_triple_bitmap_gpu": (
        C.c_int, [_p, _p, C.c_int, C.c_int, _p] + [_p] * 8 + [_p] * 2 + [_p] * 4 + [_p] * 4),
    "zs_retiled_num_records": (C.c_int64, [C.c_int, C.c_int]),
    "zs_retiled_fixed_bytes": (C.c_int64, [C.c_int, C.c_int]),
    "zs_compress_retiled_count_gpu": (C.c_int, [_p, _p, C.c_int, C.c_int, _p, _p, _p, _p]),
    "zs_compress_retiled_emit_gpu": (C.c_int, [_p, _p, C.c_int, C.c_int, _p, _p, _p, _p]),
    "zs_compress_retiled_fixed_gpu": (C.c_int, [_p, _p, C.c_int, C.c_int, _p, _p, _p, _p, _p,
                                                _p]),
    "zs_compress_retiled_auto_gpu": (C.c_int, [_p, _p, C.c_int, C.c_int, C.c_int, _p, _p, _p, _p, _p,
                                               _p, _p, _p]),
    "zs_compress_retiled_guess_gpu": (C.c_int, [_p, _p, C.c_int, C.c_int, C.c_int, _p, _p, _p, _p,
                                                _p, _p, _p, _p, _p]),
    "zs_compress_retiled_exps_gpu": (C.c_int, [_p, _p, C.c_int, C.c_int, _p, _p, _p, _p]),
    "zs_retile_triple_bitmap_count_gpu": (
        C.c_int, [_p, _p, _p, _p, _p, _p, _p, _p, C.c_int, C.c_int, _p, _p, _p]),
    "zs_retile_triple_bitmap_emit_gpu": (
        C.c_int, [_p, _p, _p, _p, _p, _p, _p, _p, C.c_uint8, C.c_int, C.c_int, _p, _p, _p]),
    "zs_retiled_decompress": (C.c_int, [_p, _p, _p, _p, C.c_uint8, _p, C.c_int, C.c_int]),
    "zs_retiled_mm": (C.c_int, [_p, _p, _p, _p, C.c_uint8, _p, _p, C.c_int, C.c_int, C.c_int,
                                _p, C.c_int]),
    "zs_retiled_mm_counters": (C.c_int64, [C.c_int, C.c_int]),
    "zs_retiled_mm_streamk_workspace_bytes": (C.c_int64, [C.c_int, C.c_int, C.c_int]),
    "zs_retiled_mm_streamk": (C.c_int, [_p, _p, _p, _p, C.c_uint8, _p, _p, C.c_int, C.c_int,
                                        C.c_int, _p, C.c_size_t, _p]),
    "zs_retiled_mm_fused": (C.c_int, [_p, _p, _p, _p, C.c_uint8, _p, _p, C.c_int, C.c_int,
                                      C.c_int, _p, C.c_int, _p]),
    "zs_retiled_mm_fused_noalloc": (C.c_int, [_p, _p, _p, _p, C.c_uint8, _p, _p, C.c_int,
                                              C.c_int, C.c_int, C.c_int]),
    "zs_decode_attention": (
        C.c_int, [_p, _p, _p, _p, _p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                  _p, _p, _p, C.c_size_t, C.c_int]),
    "zs_kv_staging_bytes": (C.c_int64, [C.c_int, C.c_int, C.c_int]),
    "zs_kv_retiled_staging_bytes": (C.c_int64, [C.c_int, C.c_int, C.c_int, C.c_int]),
    "zs_decode_attention_workspace_bytes": (
        C.c_size_t, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "zs_decode_attention_retiled": (
        C.c_int, [_p, _p, _p, _p, _p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                  _p, _p, _p, C.c_size_t, C.c_int]),
    "zs_decode_attention_dense": (
        C.c_int, [_p, _p, _p, _p, _p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                  C.c_float, _p, _p, _p, C.c_size_t, C.c_int]),
    "zs_decode_attention_dense_paged": (
        C.c_int, [_p, _p, _p, _p, _p, C.c_int, C.c_int, C.c_int, _p, C.c_int, C.c_int, C.c_int,
                  C.c_int, C.c_int, C.c_float, _p, _p, _p, C.c_size_t, C.c_int]),
    "zs_measure_record_stages": (
        C.c_int, [_p, _p, _p, _p, C.c_uint8, C.c_int, C.c_int, _i64, _i64, C.c_int, C.c_int,
                  _p, _p, _p]),
    "zs_crc32c": (C.c_uint32, [C.c_uint32, _p, _i64]),
    "zs_container_bytes": (_i64, [_p]),
    "zs_container_write": (C.c_int, [_p, C.c_char_p, _p, _p, _i64]),
    "zs_container_parse": (C.c_int, [_p, _i64, _p, _p, _p]),
}

ZS_CONTAINER_CANONICAL = 0
ZS_CONTAINER_RETILED = 1


class ContainerDesc(C.Structure):
    """zs_container_desc_t of include/zipserv.h."""
    _fields_ = [
        ("layout", _i32),
        ("rows", _i32),
        ("cols", _i32),
        ("logical_rows", _i32),
        ("logical_cols", _i32),
        ("start_exp", _i32),
        ("max_high_freq_count", _i32),
        ("max_full_count", _i32),
        ("num_streams", _i32),
        ("stream_bytes", _i64 * 8),
    ]


class ZipServError(RuntimeError):
    def __init__(self, fn: str, status: int):
        self.status = status
        msg = lib().zs_status_string(status).decode() if _lib is not None else str(status)
        super().__init__(f"{fn} failed with status {status} ({msg})")


def build(force: bool = False) -> str:
    """Compile libzipserv.so for gfx950 with hipcc (zipserv_asplos26_amd/Makefile)."""
    cmd = ["make", "-s", "-j8", "-C", PKG_DIR]
    if force:
        subprocess.run(["make", "-s", "-C", PKG_DIR, "clean"], check=True)
    subprocess.run(cmd, check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    """Load libzipserv.so; raise if it has not been built.

    torch is imported first when it is installed: torch's wheel ships its own
    HIP runtime under another file name, and the library must bind to that
    same runtime (one per process) rather than pull in /opt/rocm's copy
    before torch loads its own."""
    global _lib
    if _lib is None:
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libzipserv.so not found at {LIB_PATH}; build it with "
                "`make -C zipserv_asplos26_amd` (the HIP path has no fallback)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(fn: str, status: int) -> None:
    if status != ZS_OK:
        raise ZipServError(fn, status)


class KVRetiled(C.Structure):
    """zs_kv_retiled_t of include/zipserv.h."""
    _fields_ = [
        ("fixed", _p),
        ("exps", _p),
        ("eoff", _p),
        ("rows", _i32),
        ("cols", _i32),
        ("batch_stride_rows", _i32),
        ("head_stride_rows", _i32),
        ("start_exp", _i32),
        ("layout", _i32),
    ]


class KVCompressed(C.Structure):
    """zs_kv_compressed_t of include/zipserv.h (flash.h:51-68 ZipservCompressedKVParams)."""
    _fields_ = [
        ("sign_mantissa", _p),
        ("compressed_full", _p),
        ("bitmap1", _p),
        ("bitmap2", _p),
        ("bitmap3", _p),
        ("tile_offsets_median", _p),
        ("tile_offsets_global", _p),
        ("rows", _i32),
        ("cols", _i32),
        ("batch_stride_rows", _i32),
        ("head_stride_rows", _i32),
        ("max_high_freq_count", _i32),
        ("max_full_count", _i32),
        ("start_exp", _i32),
        ("layout", _i32),
    ]
