"""Host-side mirror of the reference's codec interfaces, over the C-ABI.

* numpy (CPU) entry points mirror build/L_API.cuh's host encoders and
  kernel_benchmark/utils.h's analyzeExponentDistribution_BF16;
* torch (GPU) entry points mirror the PyTorch extension
  kernel_benchmark/zipserv_decode_attention_ext.cpp:81-181
  (compress_zipserv / decompress_zipserv / decompress_zipserv_into) and the
  ZipservCompressed record of bench_zipserv_decode_attention.py:49-68, plus
  zipgemm() over BF16TripleBitmap_MM_API.

Every device call goes through libzipserv.so; nothing here computes on the
CPU on behalf of a GPU call.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from ._lib import check, lib

TILE_ARGS = (8, 16, 64, 8, 64, 64)


def _np_ptr(a: np.ndarray) -> int:
    return a.ctypes.data


# --------------------------------------------------------------------------
# Host codec (numpy)
# --------------------------------------------------------------------------
@dataclass
class HostCompressed:
    """Canonical TCA-TBE streams held in numpy arrays (csrc/L_API.cu:314-557)."""
    sign_mantissa: np.ndarray        # uint8  [total_high_freq]
    compressed_full: np.ndarray      # uint16 [total_full]
    bitmap1: np.ndarray              # uint64 [M*K/64]
    bitmap2: np.ndarray
    bitmap3: np.ndarray
    tile_offsets: np.ndarray         # int32 [2*M*K/64]
    tile_offsets_median: np.ndarray  # int32 [2*M*K/1024]
    tile_offsets_global: np.ndarray  # int32 [2*(M*K/4096+1)]
    rows: int
    cols: int
    max_high_freq_count: int
    max_full_count: int
    start_exp: int
    top_exponents: list = field(default_factory=list)

    @property
    def total_high_freq(self) -> int:
        return int(self.sign_mantissa.size)

    @property
    def total_full(self) -> int:
        return int(self.compressed_full.size)

    @property
    def num_global_tiles(self) -> int:
        return (self.rows // 64) * (self.cols // 64)

    def compressed_bytes(self) -> int:
        return int(lib().zs_compressed_bytes(self.rows, self.cols, self.total_high_freq,
                                             self.total_full))

    def ratio(self) -> float:
        return 2.0 * self.rows * self.cols / self.compressed_bytes()


def analyze_exponents(a: np.ndarray) -> list[int]:
    """kernel_benchmark/utils.h:189-272 -> 7 contiguous exponents."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    top = np.zeros(7, np.int32)
    check("zs_analyze_exponents_host", lib().zs_analyze_exponents_host(_np_ptr(a), a.size, _np_ptr(top)))
    return top.tolist()


def compress_host(a: np.ndarray, top=None, variant: str = "reuse_simd") -> HostCompressed:
    """Encode a bf16 [M, K] bit-pattern matrix on the CPU.

    variant: "alloc" (InitBF16MatrixTripleBitmap, L_API.cuh:53),
             "reuse" (_Reuse, L_API.cuh:76), "reuse_simd" (_Reuse_SIMD, L_API.cuh:109).
    """
    a = np.ascontiguousarray(a, dtype=np.uint16)
    if a.ndim != 2:
        raise ValueError("compress_host expects a 2D bf16 matrix")
    M, K = a.shape
    if top is None:
        top = analyze_exponents(a)
    topa = np.ascontiguousarray(top, dtype=np.int32)
    L = lib()
    mk = M * K
    ngt = mk // 4096
    if variant == "alloc":
        ptrs = [C.c_void_p() for _ in range(8)]
        mh, mf = C.c_int32(), C.c_int32()
        rc = L.zs_init_bf16_matrix_triple_bitmap(
            _np_ptr(a), M, K, *TILE_ARGS, _np_ptr(topa), *[C.byref(p) for p in ptrs],
            C.byref(mh), C.byref(mf))
        if rc < 0:
            check("zs_init_bf16_matrix_triple_bitmap", rc)
        tog = np.ctypeslib.as_array(C.cast(ptrs[7], C.POINTER(C.c_int32)), (2 * (ngt + 1),)).copy()
        th, tf = int(tog[-2]), int(tog[-1])

        def grab(p, ctype, n, dt):
            return np.ctypeslib.as_array(C.cast(p, C.POINTER(ctype)), (n,)).astype(dt, copy=True)
        out = HostCompressed(
            sign_mantissa=grab(ptrs[0], C.c_uint8, max(th, 1), np.uint8)[:th],
            compressed_full=grab(ptrs[1], C.c_uint16, max(tf, 1), np.uint16)[:tf],
            bitmap1=grab(ptrs[2], C.c_uint64, mk // 64, np.uint64),
            bitmap2=grab(ptrs[3], C.c_uint64, mk // 64, np.uint64),
            bitmap3=grab(ptrs[4], C.c_uint64, mk // 64, np.uint64),
            tile_offsets=grab(ptrs[5], C.c_int32, 2 * (mk // 64), np.int32),
            tile_offsets_median=grab(ptrs[6], C.c_int32, 2 * (mk // 1024), np.int32),
            tile_offsets_global=tog, rows=M, cols=K, max_high_freq_count=mh.value,
            max_full_count=mf.value, start_exp=(int(topa[0]) - 1) & 0xFF, top_exponents=topa.tolist())
        for p in ptrs:
            L.zs_host_free(p)
        return out
    fn = {"reuse": L.zs_init_bf16_matrix_triple_bitmap_reuse,
          "reuse_simd": L.zs_init_bf16_matrix_triple_bitmap_reuse_simd}[variant]
    sm = np.zeros(mk + 16 * ngt + 16, np.uint8)
    fu = np.zeros(mk + 8 * ngt + 8, np.uint16)
    b1, b2, b3 = (np.zeros(mk // 64, np.uint64) for _ in range(3))
    tiles = np.zeros(2 * (mk // 64), np.int32)
    med = np.zeros(2 * (mk // 1024), np.int32)
    tog = np.zeros(2 * (ngt + 1), np.int32)
    tsm = np.zeros(ngt * (4096 + 15) + 16, np.uint8)
    tfu = np.zeros(ngt * (4096 + 7), np.uint16)
    ghf, gfu = np.zeros(ngt, np.int32), np.zeros(ngt, np.int32)
    hoff, foff = np.zeros(ngt + 1, np.int32), np.zeros(ngt + 1, np.int32)
    mh, mf, th, tf = C.c_int32(), C.c_int32(), C.c_int32(), C.c_int32()
    rc = fn(_np_ptr(a), M, K, *TILE_ARGS, _np_ptr(topa), _np_ptr(sm), _np_ptr(fu), _np_ptr(b1),
            _np_ptr(b2), _np_ptr(b3), _np_ptr(tiles), _np_ptr(med), _np_ptr(tog), _np_ptr(tsm),
            _np_ptr(tfu), _np_ptr(ghf), _np_ptr(gfu), _np_ptr(hoff), _np_ptr(foff),
            C.byref(mh), C.byref(mf), C.byref(th), C.byref(tf))
    if rc < 0:
        check(variant, rc)
    return HostCompressed(
        sign_mantissa=sm[: th.value].copy(), compressed_full=fu[: tf.value].copy(),
        bitmap1=b1, bitmap2=b2, bitmap3=b3, tile_offsets=tiles, tile_offsets_median=med,
        tile_offsets_global=tog, rows=M, cols=K, max_high_freq_count=mh.value,
        max_full_count=mf.value, start_exp=(int(topa[0]) - 1) & 0xFF, top_exponents=topa.tolist())


# --------------------------------------------------------------------------
# Device codec (torch tensors on the GPU)
# --------------------------------------------------------------------------
def _torch():
    import torch
    return torch


def _dptr(t) -> int:
    return 0 if t is None else int(t.data_ptr())


def _stream() -> int:
    torch = _torch()
    return int(torch.cuda.current_stream().cuda_stream)


@dataclass
class ZipservCompressed:
    """Device-resident compressed matrix (bench_zipserv_decode_attention.py:49-68).

    sign_mantissa / compressed_full keep ZS_STREAM_SLACK_BYTES of readable slack
    past total_high_freq / total_full.
    """
    sign_mantissa: object
    compressed_full: object
    bitmap1: object
    bitmap2: object
    bitmap3: object
    tile_offsets_median: object
    tile_offsets_global: object
    rows: int
    cols: int
    logical_rows: int
    logical_cols: int
    max_high_freq_count: int
    max_full_count: int
    start_exp: int
    total_high_freq: int
    total_full: int
    num_global_tiles: int
    compressed_bytes: int
    tile_offsets: object = None
    layout: str = "by_kv_head"

    @property
    def device(self):
        return self.sign_mantissa.device

    def ratio(self) -> float:
        return 2.0 * self.rows * self.cols / self.compressed_bytes

    def streams(self):
        """The 7 buffers in L_API argument order."""
        return (self.sign_mantissa, self.compressed_full, self.bitmap1, self.bitmap2,
                self.bitmap3, self.tile_offsets_median, self.tile_offsets_global)


def to_device(h: HostCompressed, device="cuda", logical_rows=None, logical_cols=None) -> ZipservCompressed:
    """Upload host-compressed streams (with stream slack) to the GPU."""
    torch = _torch()
    slack = _lib.ZS_STREAM_SLACK_BYTES
    sm = np.zeros(h.total_high_freq + slack, np.uint8)
    sm[: h.total_high_freq] = h.sign_mantissa
    fu = np.zeros(h.total_full + slack // 2, np.uint16)
    fu[: h.total_full] = h.compressed_full

    def dev(x):
        return torch.from_numpy(np.ascontiguousarray(x)).to(device)
    return ZipservCompressed(
        sign_mantissa=dev(sm), compressed_full=dev(fu.view(np.int16)).view(torch.bfloat16),
        bitmap1=dev(h.bitmap1.view(np.int64)), bitmap2=dev(h.bitmap2.view(np.int64)),
        bitmap3=dev(h.bitmap3.view(np.int64)), tile_offsets_median=dev(h.tile_offsets_median),
        tile_offsets_global=dev(h.tile_offsets_global), rows=h.rows, cols=h.cols,
        logical_rows=h.rows if logical_rows is None else logical_rows,
        logical_cols=h.cols if logical_cols is None else logical_cols,
        max_high_freq_count=h.max_high_freq_count, max_full_count=h.max_full_count,
        start_exp=h.start_exp, total_high_freq=h.total_high_freq, total_full=h.total_full,
        num_global_tiles=h.num_global_tiles, compressed_bytes=h.compressed_bytes(),
        tile_offsets=dev(h.tile_offsets))


def _check_cuda(t, name, dtype=None):
    torch = _torch()
    if not (isinstance(t, torch.Tensor) and t.is_cuda):
        raise ValueError(f"{name} must be a CUDA tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}")


WINDOW_RULES = ("kv", "weights")


def _device_window(input, window, top, counts_u64=None):
    """Writes the 7 window exponents of `input` into the int32 device tensor
    `top` on the current stream.

    window: "kv"      -- AnalyzeTopExponentsGPU's rule
                         (zipserv_decode_attention_ext.cu:65-134), the
                         reference's KV-cache compressor;
            "weights" -- analyzeExponentDistribution_BF16's rule
                         (kernel_benchmark/utils.h:189-272), the reference's
                         weight path (same window as analyze_exponents());
            7 ints    -- an explicit window (top[0] .. top[0] + 6).
    """
    torch = _torch()
    L = lib()
    if isinstance(window, str):
        if window not in WINDOW_RULES:
            raise ValueError(f"window must be one of {WINDOW_RULES} or 7 exponents")
        counts = counts_u64 if counts_u64 is not None else torch.empty(
            256, dtype=torch.int64, device=input.device)
        fn = "zs_analyze_top_exponents_u64_gpu" if window == "kv" else \
            "zs_analyze_exponents_weights_gpu"
        check(fn, getattr(L, fn)(_stream(), _dptr(input), input.numel(), _dptr(counts),
                                 _dptr(top)))
        return
    w = [int(v) for v in window]
    if len(w) != 7 or any(w[i] != w[0] + i for i in range(7)):
        raise ValueError("an explicit window is 7 consecutive exponents")
    top.copy_(torch.tensor(w, dtype=torch.int32))


def compress_zipserv(input, logical_rows: int | None = None, logical_cols: int | None = None,
                     window="kv", _with_tiles: bool = False):
    """zipserv_decode_attention_ext.cpp:81-88 / .cu:157-265 on the GPU.

    `window` picks the exponent-window rule (see _device_window): "kv" is the
    reference compressor's own; "weights" reproduces the host encoder's
    window (InitBF16MatrixTripleBitmap after analyzeExponentDistribution_BF16)
    so the streams equal zs_init_bf16_matrix_triple_bitmap's bytes.

    Returns [sign_mantissa, compressed_full, bitmap1, bitmap2, bitmap3,
    tile_offsets_median, tile_offsets_global, meta] where meta is the int64
    [rows, cols, logical_rows, logical_cols, max_hf, max_full, start_exp,
    total_hf, total_full, num_global_tiles, comp_bytes] tensor of ext.cu:250-262
    (comp_bytes uses the inclusive formula of ext.cu:23-33).
    """
    torch = _torch()
    _check_cuda(input, "input", torch.bfloat16)
    if input.dim() != 2:
        raise ValueError("input must be 2D")
    rows, cols = input.shape
    if rows % 64 or cols % 64:
        raise ValueError("rows and cols must be padded to multiples of 64")
    L = lib()
    dev = input.device
    mk = rows * cols
    ngt = mk // 4096
    if mk + 16 * ngt > 2**31 - 1:  # int32 stream offsets of the format (ext.cu:184)
        check("zs_init_bf16_matrix_triple_bitmap_gpu", _lib.ZS_E_OVERFLOW)
    i32 = dict(dtype=torch.int32, device=dev)
    sm = torch.empty(int(L.zs_sign_mantissa_capacity(rows, cols)), dtype=torch.uint8, device=dev)
    fu = torch.empty(int(L.zs_full_capacity(rows, cols)), dtype=torch.bfloat16, device=dev)
    b1, b2, b3 = (torch.empty(mk // 64, dtype=torch.int64, device=dev) for _ in range(3))
    tiles = torch.empty(2 * (mk // 64), **i32)
    med = torch.empty(2 * (mk // 1024), **i32)
    tog = torch.empty(2 * (ngt + 1), **i32)
    ghf, gfu = torch.empty(ngt, **i32), torch.empty(ngt, **i32)
    hoff, foff = torch.empty(ngt + 1, **i32), torch.empty(ngt + 1, **i32)
    small = torch.empty(12, **i32)  # top[0:7] | scalars[8:12]: one D2H copy below
    top, scal = small[0:7], small[8:12]
    counts = torch.empty(256, **i32)
    done = torch.empty(4, **i32)
    st = _stream()
    if isinstance(window, str) and window == "kv":
        check("zs_analyze_top_exponents_gpu",
              L.zs_analyze_top_exponents_gpu(st, _dptr(input), mk, _dptr(counts), _dptr(top),
                                             _dptr(done)))
    else:
        _device_window(input, window, top)
    check("zs_init_bf16_matrix_triple_bitmap_gpu",
          L.zs_init_bf16_matrix_triple_bitmap_gpu(
              st, _dptr(input), rows, cols, _dptr(top), _dptr(sm), _dptr(fu), _dptr(b1),
              _dptr(b2), _dptr(b3), _dptr(tiles), _dptr(med), _dptr(tog), None, None,
              _dptr(ghf), _dptr(gfu), _dptr(hoff), _dptr(foff), _dptr(scal[0:]),
              _dptr(scal[1:]), _dptr(scal[2:]), _dptr(scal[3:])))
    host = small.cpu().tolist()  # synchronises, as ext.cu:234-245
    top0 = host[0]
    max_hf, max_full, total_hf, total_full = host[8:12]
    # The slack a decoder may read past the streams is zeroed so it is defined.
    slack = _lib.ZS_STREAM_SLACK_BYTES
    sm[total_hf:total_hf + slack].zero_()
    fu[total_full:total_full + slack // 2].zero_()
    start_exp = top0 - 1
    inclusive = (total_hf + 2 * total_full + (mk // 64) * 3 * 8 + (mk // 64) * 2 * 4
                 + (mk // 1024) * 2 * 4 + (ngt + 1) * 2 * 4 + 7 * 4)
    meta = torch.tensor([rows, cols, rows if logical_rows is None else logical_rows,
                         cols if logical_cols is None else logical_cols, max_hf, max_full,
                         start_exp, total_hf, total_full, ngt, inclusive], dtype=torch.int64)
    parts = [sm, fu, b1, b2, b3, med, tog, meta]
    return (parts, tiles) if _with_tiles else parts


def make_zipserv_compressed(parts, layout: str = "by_kv_head") -> ZipservCompressed:
    """bench_zipserv_decode_attention.py:375-405 make_zipserv_compressed_from_parts."""
    sm, fu, b1, b2, b3, med, tog, meta = parts
    m = meta.tolist()
    rows, cols = int(m[0]), int(m[1])
    return ZipservCompressed(
        sign_mantissa=sm, compressed_full=fu, bitmap1=b1, bitmap2=b2, bitmap3=b3,
        tile_offsets_median=med, tile_offsets_global=tog, rows=rows, cols=cols,
        logical_rows=int(m[2]), logical_cols=int(m[3]), max_high_freq_count=int(m[4]),
        max_full_count=int(m[5]), start_exp=int(m[6]), total_high_freq=int(m[7]),
        total_full=int(m[8]), num_global_tiles=int(m[9]),
        compressed_bytes=int(lib().zs_compressed_bytes(rows, cols, int(m[7]), int(m[8]))),
        layout=layout)


def compress(input, logical_rows=None, logical_cols=None, layout="by_kv_head",
             window="kv") -> ZipservCompressed:
    parts, tiles = compress_zipserv(input, logical_rows, logical_cols, window, _with_tiles=True)
    c = make_zipserv_compressed(parts, layout)
    c.tile_offsets = tiles  # per-small-tile (hf, full) counts; no kernel reads them
    return c


def decompress_zipserv_into(output, sign_mantissa, compressed_full, bitmap1, bitmap2, bitmap3,
                            tile_offsets_median, tile_offsets_global, rows, cols,
                            max_high_freq_count, max_full_count, start_exp):
    """zipserv_decode_attention_ext.cpp:144-175 -> BF16TripleBitmap_Decompress_API."""
    torch = _torch()
    _check_cuda(output, "output", torch.bfloat16)
    if tuple(output.shape) != (rows, cols):
        raise ValueError("output shape must be (rows, cols)")
    for name, t in (("sign_mantissa", sign_mantissa), ("compressed_full", compressed_full),
                    ("bitmap1", bitmap1), ("bitmap2", bitmap2), ("bitmap3", bitmap3),
                    ("tile_offsets_median", tile_offsets_median),
                    ("tile_offsets_global", tile_offsets_global)):
        _check_cuda(t, name)
    check("zs_bf16_triple_bitmap_decompress",
          lib().zs_bf16_triple_bitmap_decompress(
              _stream(), _dptr(sign_mantissa), _dptr(compressed_full), _dptr(bitmap1),
              _dptr(bitmap2), _dptr(bitmap3), _dptr(tile_offsets_median),
              _dptr(tile_offsets_global), int(max_high_freq_count), int(max_full_count),
              int(start_exp) & 0xFF, _dptr(output), int(rows), int(cols)))
    return output


def decompress_zipserv(sign_mantissa, compressed_full, bitmap1, bitmap2, bitmap3,
                       tile_offsets_median, tile_offsets_global, rows, cols,
                       max_high_freq_count, max_full_count, start_exp):
    """zipserv_decode_attention_ext.cpp:90-142."""
    torch = _torch()
    out = torch.empty((rows, cols), dtype=torch.bfloat16, device=sign_mantissa.device)
    return decompress_zipserv_into(out, sign_mantissa, compressed_full, bitmap1, bitmap2, bitmap3,
                                   tile_offsets_median, tile_offsets_global, rows, cols,
                                   max_high_freq_count, max_full_count, start_exp)


def decompress(c: ZipservCompressed, out=None):
    torch = _torch()
    if out is None:
        out = torch.empty((c.rows, c.cols), dtype=torch.bfloat16, device=c.sign_mantissa.device)
    return decompress_zipserv_into(out, *c.streams(), c.rows, c.cols, c.max_high_freq_count,
                                   c.max_full_count, c.start_exp)


def splitk_workspace(c, n: int, split_k: int):
    """Workspace of zipgemm(c, x[n], split_k): the bf16 partial slabs of
    split-K, or with split_k == 0 (stream-K, re-tiled layout) the fp32
    partials of the bands shared between workgroups; None when none is
    needed."""
    torch = _torch()
    if split_k == 0:
        nbytes = int(lib().zs_retiled_mm_streamk_workspace_bytes(c.rows, n, c.cols))
        if nbytes <= 0:
            return None
        return torch.empty(nbytes, dtype=torch.uint8, device=c.device)
    nbytes = int(lib().zs_splitk_workspace_bytes(c.rows, n, split_k))
    if nbytes == 0:
        return None
    return torch.empty(nbytes // 2, dtype=torch.bfloat16, device=c.device)


# Arrival counters of the in-kernel split-K reduction, one zero-filled int32
# buffer per (device, stream): calls on one stream run one after another, so
# they can share it, and every completed call leaves it zero.  A buffer that
# a larger shape outgrows is retired, never freed: a HIP graph captured
# earlier may still hold its address and replay into it.
_SPLITK_COUNTERS = {}
_RETIRED_COUNTERS = []
_MIN_COUNTERS = 1 << 16


def splitk_counters(rows: int, n: int, device=None):
    """The current stream's counter buffer for zs_retiled_mm_fused (at least
    zs_retiled_mm_counters(rows, n) entries), or None while a graph is being
    captured and no large enough buffer exists yet (a new one would be
    allocated inside the graph's memory pool)."""
    torch = _torch()
    need = int(lib().zs_retiled_mm_counters(rows, n))
    dev = torch.device(device) if device is not None else torch.device("cuda",
                                                                       torch.cuda.current_device())
    key = (dev.index, torch.cuda.current_stream(dev).cuda_stream)
    buf = _SPLITK_COUNTERS.get(key)
    if buf is None or buf.numel() < need:
        if torch.cuda.is_current_stream_capturing():
            return None
        if buf is not None:
            _RETIRED_COUNTERS.append(buf)
        buf = torch.zeros(max(need, _MIN_COUNTERS), dtype=torch.int32, device=dev)
        _SPLITK_COUNTERS[key] = buf
    return buf


# ---------------------------------------------------------------------------
# CDNA4 re-tiled layout (the library's device layout; see include/zipserv.h)
# ---------------------------------------------------------------------------
@dataclass
class ZipservRetiled:
    """Device-resident re-tiled matrix: fixed 1408-byte records per 16x64 tile
    (sign|mantissa bytes and code bit-planes in MFMA lane order) + outlier
    exponent bytes with per-record offsets.  Same content and size as the
    canonical streams, laid out for contiguous per-band streaming."""
    fixed: object          # uint8 [num_records * 1408]
    exps: object           # uint8 [num_outliers + slack]
    eoff: object           # int32 [num_records + 1]
    rows: int
    cols: int
    logical_rows: int
    logical_cols: int
    start_exp: int
    num_outliers: int
    compressed_bytes: int
    layout: str = "by_kv_head"

    @property
    def device(self):
        return self.fixed.device

    def ratio(self) -> float:
        return 2.0 * self.rows * self.cols / self.compressed_bytes


def _retiled_alloc(rows, cols, total, dev):
    torch = _torch()
    nrec = rows // 16 * (cols // 64)
    fixed = torch.empty(nrec * 1408, dtype=torch.uint8, device=dev)
    exps = torch.zeros(int(total) + _lib.ZS_STREAM_SLACK_BYTES, dtype=torch.uint8, device=dev)
    return fixed, exps, nrec


def _retiled_encode(input, window, guess=None):
    """First phase of the re-tiled GPU encoder on the current stream: the
    window, the fixed parts, the per-record outlier counts and offsets, and
    the outlier bytes in per-record slots; the outlier total and the window
    land in one int64 [5] tensor (`meta`) that the host reads to size the
    exponent stream.  Under a window rule, `guess` (int32 [7] on the device,
    e.g. the previous matrix's window) replaces the sampled guess; the bytes
    are the same either way.  Returns the state _retiled_finish takes."""
    torch = _torch()
    _check_cuda(input, "input", torch.bfloat16)
    if input.dim() != 2:
        raise ValueError("input must be 2D")
    rows, cols = input.shape
    if rows % 64 or cols % 64:
        raise ValueError("rows and cols must be padded to multiples of 64")
    L = lib()
    dev = input.device
    i32 = dict(dtype=torch.int32, device=dev)
    nrec = rows // 16 * (cols // 64)
    # the outlier total and the window share one buffer, so that a single
    # synchronising copy brings both to the host
    meta = torch.empty(5, dtype=torch.int64, device=dev)
    total, top = meta[:1], meta[1:].view(torch.int32)[:7]
    counts = torch.empty(256, dtype=torch.int64, device=dev)
    cnt, eoff = torch.empty(nrec, **i32), torch.empty(nrec + 1, **i32)
    fixed = torch.empty(nrec * 1408, dtype=torch.uint8, device=dev)
    tmp = torch.empty(nrec * _lib.ZS_RETILED_EXP_SLOT_BYTES, dtype=torch.uint8, device=dev)
    st = _stream()
    if isinstance(window, str):
        if window not in WINDOW_RULES:
            raise ValueError(f"window must be one of {WINDOW_RULES} or 7 exponents")
        rule = _lib.ZS_WINDOW_KV if window == "kv" else _lib.ZS_WINDOW_WEIGHTS
        work = torch.empty(_lib.ZS_RETILED_AUTO_WORK_BYTES, dtype=torch.uint8, device=dev)
        # 64-bit bins: the re-tiled layout takes matrices past 2^31 elements.
        if guess is not None:
            _check_cuda(guess, "guess", torch.int32)
            check("zs_compress_retiled_guess_gpu",
                  L.zs_compress_retiled_guess_gpu(st, _dptr(input), rows, cols, rule, _dptr(guess),
                                                  _dptr(counts), _dptr(top), _dptr(work),
                                                  _dptr(fixed), _dptr(cnt), _dptr(eoff),
                                                  _dptr(total), _dptr(tmp)))
        else:
            check("zs_compress_retiled_auto_gpu",
                  L.zs_compress_retiled_auto_gpu(st, _dptr(input), rows, cols, rule, _dptr(counts),
                                                 _dptr(top), _dptr(work), _dptr(fixed), _dptr(cnt),
                                                 _dptr(eoff), _dptr(total), _dptr(tmp)))
    else:
        _device_window(input, window, top, counts)
        check("zs_compress_retiled_fixed_gpu",
              L.zs_compress_retiled_fixed_gpu(st, _dptr(input), rows, cols, _dptr(top),
                                              _dptr(fixed), _dptr(cnt), _dptr(eoff),
                                              _dptr(total), _dptr(tmp)))
    return dict(input=input, rows=rows, cols=cols, nrec=nrec, meta=meta, top=top, eoff=eoff,
                fixed=fixed, tmp=tmp)


def _retiled_finish(s, host_meta, logical_rows, logical_cols, layout) -> ZipservRetiled:
    """Second phase: the exponent stream sized from the host copy of `meta`
    and the outlier bytes moved into it."""
    torch = _torch()
    tot, top0 = int(host_meta[0]), int(host_meta[1:].view(torch.int32)[0])
    if tot > 2**31 - 1:
        raise OverflowError("outlier count exceeds the int32 offsets")
    rows, cols, nrec = s["rows"], s["cols"], s["nrec"]
    # every byte is written by the compaction, the slack bytes as zeros
    exps = torch.empty(tot + _lib.ZS_STREAM_SLACK_BYTES, dtype=torch.uint8,
                       device=s["input"].device)
    check("zs_compress_retiled_exps_gpu",
          lib().zs_compress_retiled_exps_gpu(_stream(), _dptr(s["input"]), rows, cols,
                                             _dptr(s["top"]), _dptr(s["eoff"]), _dptr(s["tmp"]),
                                             _dptr(exps)))
    s.pop("tmp")  # stream-ordered: the allocator reuses it only after the compaction
    return ZipservRetiled(s["fixed"], exps, s["eoff"], rows, cols,
                          rows if logical_rows is None else logical_rows,
                          cols if logical_cols is None else logical_cols,
                          (top0 - 1) & 0xFF, tot, nrec * 1408 + tot + 4 * (nrec + 1), layout)


def compress_retiled(input, logical_rows=None, logical_cols=None, layout="by_kv_head",
                     window="kv") -> ZipservRetiled:
    """bf16 [rows, cols] on the GPU -> re-tiled layout.  The window is chosen on
    the GPU, by default with the rule of zipserv_decode_attention_ext.cu:35-135
    ("kv"); "weights" applies kernel_benchmark/utils.h:189-272 instead (see
    _device_window).  Under a rule the encoder reads the input once when the
    window guessed from a sample of it is the rule's (zs_compress_retiled_auto_gpu),
    twice otherwise; an explicit window is one more input pass.  The host
    synchronises once, to size the exponent stream (compress_retiled_many
    overlaps that wait with the next matrices' encoding)."""
    s = _retiled_encode(input, window)
    host = s["meta"].cpu()  # synchronises (sizes the stream)
    return _retiled_finish(s, host, logical_rows, logical_cols, layout)


def compress_retiled_many(inputs, window="kv", layout="by_kv_head", lookahead=4) -> list:
    """compress_retiled over several bf16 matrices without the GPU idling
    between them: each matrix's outlier total (the one figure the host needs,
    to size its exponent stream) comes back by an asynchronous copy into pinned
    memory, and the host waits for it only once the first phases of the next
    `lookahead` matrices are queued behind it.  Same bytes as one call per
    matrix (a model's weights are compressed this way, layer by layer).  At
    most lookahead + 1 matrices hold their outlier slots (256 bytes per 1024
    elements, an eighth of the bf16 bytes) at once.  Under a window rule each
    matrix after the first takes the previous one's window as its guess
    (zs_compress_retiled_guess_gpu: no sample of its input; a model's
    matrices share one window, and a wrong guess only costs a second
    encoding pass).  The default lookahead of 4 keeps the GPU busy while the
    host allocates each exponent stream: 1-2% faster than 2 over forty
    Llama-70B-sized matrices per call."""
    torch = _torch()
    if lookahead < 0:
        raise ValueError("lookahead must be >= 0")
    out, pending = [], []
    prev_top = None  # kept referenced until the next matrix's encoder is queued

    def finish_oldest():
        s, host, done = pending.pop(0)
        done.synchronize()
        out.append(_retiled_finish(s, host, None, None, layout))

    for x in inputs:
        rule = isinstance(window, str)
        same_dev = prev_top is not None and prev_top.device == x.device
        s = _retiled_encode(x, window, guess=prev_top if rule and same_dev else None)
        prev_top = s["top"]
        host = torch.empty(5, dtype=torch.int64, pin_memory=True)
        host.copy_(s["meta"], non_blocking=True)
        done = torch.cuda.Event()
        done.record(torch.cuda.current_stream(x.device))
        pending.append((s, host, done))
        if len(pending) > lookahead:
            finish_oldest()
    while pending:
        finish_oldest()
    return out


def retile(c: ZipservCompressed) -> ZipservRetiled:
    """Canonical device streams -> re-tiled layout (same window, same bytes as
    compress_retiled under that window)."""
    torch = _torch()
    L = lib()
    dev = c.sign_mantissa.device
    i32 = dict(dtype=torch.int32, device=dev)
    nrec = c.rows // 16 * (c.cols // 64)
    cnt, eoff = torch.empty(nrec, **i32), torch.empty(nrec + 1, **i32)
    total = torch.empty(1, dtype=torch.int64, device=dev)
    st = _stream()
    ptrs = [_dptr(t) for t in c.streams()]
    check("zs_retile_triple_bitmap_count_gpu",
          L.zs_retile_triple_bitmap_count_gpu(st, *ptrs, c.rows, c.cols, _dptr(cnt), _dptr(eoff),
                                              _dptr(total)))
    tot = int(total.item())
    fixed, exps, _ = _retiled_alloc(c.rows, c.cols, tot, dev)
    check("zs_retile_triple_bitmap_emit_gpu",
          L.zs_retile_triple_bitmap_emit_gpu(st, *ptrs, c.start_exp & 0xFF, c.rows, c.cols,
                                             _dptr(eoff), _dptr(fixed), _dptr(exps)))
    return ZipservRetiled(fixed, exps, eoff, c.rows, c.cols, c.logical_rows, c.logical_cols,
                          c.start_exp & 0xFF, tot, nrec * 1408 + tot + 4 * (nrec + 1), c.layout)


def decompress_retiled(r: ZipservRetiled, out=None):
    torch = _torch()
    if out is None:
        out = torch.empty((r.rows, r.cols), dtype=torch.bfloat16, device=r.device)
    _check_cuda(out, "out", torch.bfloat16)
    check("zs_retiled_decompress",
          lib().zs_retiled_decompress(_stream(), _dptr(r.fixed), _dptr(r.exps), _dptr(r.eoff),
                                      r.start_exp & 0xFF, _dptr(out), r.rows, r.cols))
    return out


def zipgemm(c, x, split_k: int = 1, out=None, workspace=None, fused: bool = True,
            counters=None):
    """Y[N, M] = X[N, K] . W[M, K]^T (build/L_API.cuh:19-37 BF16TripleBitmap_MM_API).
    `c` is a ZipservCompressed (canonical streams) or a ZipservRetiled.

    Split-K over the re-tiled layout adds the partial sums inside the GEMM
    kernel (zs_retiled_mm_fused) when `fused`, with `counters` or the current
    stream's buffer from splitk_counters(); same results as the two-kernel
    reduction, which `fused=False` selects (as do the canonical streams).

    split_k == 0 (re-tiled layout, N <= 16) selects the stream-K schedule
    (zs_retiled_mm_streamk: one round of workgroups over equal record
    ranges, fp32 partials); shapes it does not take run split-K 1."""
    torch = _torch()
    _check_cuda(x, "x", torch.bfloat16)
    if x.dim() != 2 or x.shape[1] != c.cols:
        raise ValueError(f"x must be [N, {c.cols}]")
    n = x.shape[0]
    if out is None:
        out = torch.empty((n, c.rows), dtype=torch.bfloat16, device=x.device)
    retiled = isinstance(c, ZipservRetiled)
    if split_k == 0:
        if not retiled:
            raise ValueError("split_k == 0 (stream-K) takes the re-tiled layout")
        L = lib()
        if n <= 16 and int(L.zs_retiled_mm_streamk_workspace_bytes(c.rows, n, c.cols)) > 0:
            if workspace is None:
                workspace = splitk_workspace(c, n, 0)
            if counters is None:
                counters = splitk_counters(c.rows, n, x.device)
            if counters is not None and counters.numel() >= c.rows // 16:
                check("zs_retiled_mm_streamk",
                      L.zs_retiled_mm_streamk(_stream(), _dptr(c.fixed), _dptr(c.exps),
                                              _dptr(c.eoff), c.start_exp & 0xFF, _dptr(x),
                                              _dptr(out), c.rows, n, c.cols, _dptr(workspace),
                                              workspace.numel() * workspace.element_size(),
                                              _dptr(counters)))
                return out
        split_k = 1
    if split_k > 1 and workspace is None:
        workspace = splitk_workspace(c, n, split_k)
    if retiled:
        if split_k > 1 and fused and counters is None:
            counters = splitk_counters(c.rows, n, x.device)
        if split_k > 1 and fused and counters is not None:
            if counters.dtype != torch.int32 or counters.device != x.device or \
                    counters.numel() < lib().zs_retiled_mm_counters(c.rows, n):
                raise ValueError("counters must be int32 on x's device with "
                                 "zs_retiled_mm_counters(M, N) entries")
            check("zs_retiled_mm_fused",
                  lib().zs_retiled_mm_fused(_stream(), _dptr(c.fixed), _dptr(c.exps),
                                            _dptr(c.eoff), c.start_exp & 0xFF, _dptr(x),
                                            _dptr(out), c.rows, n, c.cols, _dptr(workspace),
                                            split_k, _dptr(counters)))
            return out
        check("zs_retiled_mm",
              lib().zs_retiled_mm(_stream(), _dptr(c.fixed), _dptr(c.exps), _dptr(c.eoff),
                                  c.start_exp & 0xFF, _dptr(x), _dptr(out), c.rows, n, c.cols,
                                  _dptr(workspace), split_k))
        return out
    check("zs_bf16_triple_bitmap_mm",
          lib().zs_bf16_triple_bitmap_mm(
              _stream(), *[_dptr(t) for t in c.streams()], c.max_high_freq_count,
              c.max_full_count, c.start_exp & 0xFF, _dptr(x), _dptr(out), c.rows, n, c.cols,
              _dptr(workspace), split_k))
    return out
