"""Persistent form of a compressed matrix: the container of
csrc/zs_container.cpp (versioned header, per-stream CRC-32C, 64-byte aligned
streams) for the canonical TCA-TBE streams and the re-tiled layout.

The reference holds compressed matrices only in memory (seven tensors and
the meta tensor of kernel_benchmark/zipserv_decode_attention_ext.cu:250-262);
a container lets a checkpoint be compressed once.  A bundle is containers
back to back (each one's header gives its length), one per named matrix.
Encoding, validation and CRCs run in libzipserv.so; this module moves bytes
between files, numpy and device tensors.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import check, lib
from .codec import (HostCompressed, ZipservCompressed, ZipservRetiled, _torch, to_device)

_HEADER = 256


def _host(t) -> np.ndarray:
    """A tensor or array as a contiguous uint8 numpy view (device -> host copy)."""
    if isinstance(t, np.ndarray):
        return np.ascontiguousarray(t).view(np.uint8).reshape(-1)
    torch = _torch()
    return t.detach().contiguous().view(torch.uint8).cpu().numpy().reshape(-1)


def _parts(c):
    """(descriptor fields, stream byte arrays) of a compressed matrix."""
    if isinstance(c, HostCompressed):
        streams = [c.sign_mantissa, c.compressed_full, c.bitmap1, c.bitmap2, c.bitmap3,
                   c.tile_offsets_median, c.tile_offsets_global]
        f = dict(layout=_lib.ZS_CONTAINER_CANONICAL, rows=c.rows, cols=c.cols,
                 logical_rows=c.rows, logical_cols=c.cols, start_exp=c.start_exp,
                 max_high_freq_count=c.max_high_freq_count, max_full_count=c.max_full_count)
        return f, [_host(s) for s in streams]
    if isinstance(c, ZipservCompressed):
        streams = [_host(c.sign_mantissa)[: c.total_high_freq],
                   _host(c.compressed_full)[: 2 * c.total_full]]
        streams += [_host(t) for t in (c.bitmap1, c.bitmap2, c.bitmap3, c.tile_offsets_median,
                                       c.tile_offsets_global)]
        f = dict(layout=_lib.ZS_CONTAINER_CANONICAL, rows=c.rows, cols=c.cols,
                 logical_rows=c.logical_rows, logical_cols=c.logical_cols,
                 start_exp=c.start_exp, max_high_freq_count=c.max_high_freq_count,
                 max_full_count=c.max_full_count)
        return f, streams
    if isinstance(c, ZipservRetiled):
        streams = [_host(c.fixed), _host(c.exps)[: c.num_outliers], _host(c.eoff)]
        f = dict(layout=_lib.ZS_CONTAINER_RETILED, rows=c.rows, cols=c.cols,
                 logical_rows=c.logical_rows, logical_cols=c.logical_cols,
                 start_exp=c.start_exp, max_high_freq_count=0, max_full_count=0)
        return f, streams
    raise TypeError(f"cannot store {type(c).__name__}")


def to_bytes(c, name: str = "") -> np.ndarray:
    """HostCompressed / ZipservCompressed / ZipservRetiled -> container bytes."""
    f, streams = _parts(c)
    d = _lib.ContainerDesc(**f)
    d.num_streams = len(streams)
    for i, s in enumerate(streams):
        d.stream_bytes[i] = s.size
    L = lib()
    n = int(L.zs_container_bytes(C.byref(d)))
    if n < 0:
        check("zs_container_bytes", n)
    out = np.empty(n, np.uint8)
    ptrs = (C.c_void_p * len(streams))(*[s.ctypes.data for s in streams])
    check("zs_container_write", L.zs_container_write(C.byref(d), name.encode()[:63], ptrs,
                                                     out.ctypes.data, n))
    return out


def _parse(buf: np.ndarray, at: int = 0):
    d = _lib.ContainerDesc()
    name = C.create_string_buffer(64)
    offs = (C.c_int64 * 8)()
    view = buf[at:]
    check("zs_container_parse", lib().zs_container_parse(view.ctypes.data, view.size, C.byref(d),
                                                         name, offs))
    streams = [view[offs[i]: offs[i] + d.stream_bytes[i]] for i in range(d.num_streams)]
    total = int(np.frombuffer(view[56:64].tobytes(), np.uint64)[0])
    return d, name.value.decode(errors="replace"), streams, total


def from_bytes(buf, device=None, layout: str = "by_kv_head"):
    """Container bytes -> the matrix: HostCompressed (canonical, device None),
    ZipservCompressed (canonical) or ZipservRetiled on `device`."""
    buf = np.frombuffer(bytes(buf), np.uint8) if not isinstance(buf, np.ndarray) else buf
    d, _, streams, _ = _parse(buf)
    return _build(d, streams, device, layout)


def _build(d, s, device, layout):
    if d.layout == _lib.ZS_CONTAINER_CANONICAL:
        mk = d.rows * d.cols
        b = [s[i].copy().view(np.uint64) for i in (2, 3, 4)]
        hf = np.bitwise_count(b[0] | b[1] | b[2]).astype(np.int32)
        tiles = np.stack([hf, 64 - hf], axis=1).reshape(-1)
        h = HostCompressed(
            sign_mantissa=s[0].copy(), compressed_full=s[1].copy().view(np.uint16),
            bitmap1=b[0], bitmap2=b[1], bitmap3=b[2], tile_offsets=tiles,
            tile_offsets_median=s[5].copy().view(np.int32),
            tile_offsets_global=s[6].copy().view(np.int32), rows=d.rows, cols=d.cols,
            max_high_freq_count=d.max_high_freq_count, max_full_count=d.max_full_count,
            start_exp=d.start_exp)
        assert tiles.size == 2 * (mk // 64)
        if device is None:
            return h
        c = to_device(h, device, d.logical_rows, d.logical_cols)
        c.layout = layout
        return c
    if device is None:
        raise ValueError("a re-tiled container loads onto a device")
    torch = _torch()
    total = int(d.stream_bytes[1])
    exps = np.zeros(total + _lib.ZS_STREAM_SLACK_BYTES, np.uint8)
    exps[:total] = s[1]
    nrec = d.rows // 16 * (d.cols // 64)

    def dev(x):
        return torch.from_numpy(np.ascontiguousarray(x)).to(device)
    return ZipservRetiled(dev(s[0]), dev(exps), dev(s[2].copy().view(np.int32)), d.rows, d.cols,
                          d.logical_rows, d.logical_cols, d.start_exp, total,
                          nrec * 1408 + total + 4 * (nrec + 1), layout)


def save(path: str, c, name: str = "") -> int:
    """Write one matrix as a container file; returns its size in bytes."""
    b = to_bytes(c, name)
    b.tofile(path)
    return b.size


def load(path: str, device=None, layout: str = "by_kv_head"):
    """Read a container file (see from_bytes)."""
    return from_bytes(np.fromfile(path, np.uint8), device, layout)


def save_bundle(path: str, items: dict) -> int:
    """Write named matrices as containers back to back; returns the bytes written."""
    n = 0
    with open(path, "wb") as f:
        for name, c in items.items():
            b = to_bytes(c, name)
            f.write(b.tobytes())
            n += b.size
    return n


def load_bundle(path: str, device=None, layout: str = "by_kv_head") -> dict:
    """Read every container of a bundle into {name: matrix}."""
    buf = np.fromfile(path, np.uint8)
    out, at = {}, 0
    while at < buf.size:
        d, name, streams, total = _parse(buf, at)
        out[name] = _build(d, streams, device, layout)
        at += total
    return out
