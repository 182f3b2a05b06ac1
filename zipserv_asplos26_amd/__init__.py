"""ZipServ hot path for AMD MI355X (gfx950): TCA-TBE codec, ZipGEMM, KV-cache
compression and decode attention over compressed K/V.

The compute lives in libzipserv.so (HIP kernels + C++ host codec) behind the
C-ABI of include/zipserv.h; this package is the Python host-side mirror of the
reference's operator interfaces (see codec.py and attention.py).
"""
from ._lib import LIB_PATH, ZipServError, build, lib  # noqa: F401
from . import container  # noqa: F401
from .codec import (  # noqa: F401
    HostCompressed,
    ZipservCompressed,
    ZipservRetiled,
    analyze_exponents,
    compress,
    compress_host,
    compress_retiled,
    compress_retiled_many,
    compress_zipserv,
    decompress,
    decompress_retiled,
    decompress_zipserv,
    decompress_zipserv_into,
    make_zipserv_compressed,
    retile,
    to_device,
    zipgemm,
)

__all__ = [
    "LIB_PATH", "ZipServError", "build", "lib", "HostCompressed", "ZipservCompressed",
    "ZipservRetiled", "compress_retiled", "compress_retiled_many", "decompress_retiled", "retile",
    "analyze_exponents", "compress", "compress_host", "compress_zipserv", "decompress",
    "decompress_zipserv", "decompress_zipserv_into", "make_zipserv_compressed", "to_device",
    "zipgemm", "container",
]
