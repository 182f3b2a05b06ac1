"""CPU oracle for the ZipServ hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker.  The product package never imports it.

numpy wrappers over oracle/_build/libzsoracle.so (built from zs_oracle.c by
oracle/Makefile).  Each function names the reference file:line it restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libzsoracle.so")
_lib = None


def build() -> str:
    """Compile the oracle with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        p = C.c_void_p
        L.zso_bf16_to_f32.restype = C.c_float
        L.zso_bf16_to_f32.argtypes = [C.c_uint16]
        L.zso_f32_to_bf16.restype = C.c_uint16
        L.zso_f32_to_bf16.argtypes = [C.c_float]
        L.zso_small_tile_pos.argtypes = [C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int)]
        for name in ("zso_analyze_cpu", "zso_analyze_gpu"):
            getattr(L, name).argtypes = [p, C.c_int64, p]
        for name in ("zso_select_cpu", "zso_select_gpu"):
            getattr(L, name).argtypes = [p, p]
        L.zso_histogram.argtypes = [p, C.c_int64, p]
        for name in ("zso_compress_plain", "zso_compress_lut", "zso_compress_sse"):
            fn = getattr(L, name)
            fn.restype = C.c_int
            fn.argtypes = [p, C.c_int, C.c_int, p, p]
        L.zso_compress_sse_mt.restype = C.c_int
        L.zso_compress_sse_mt.argtypes = [p, C.c_int, C.c_int, p, p, C.c_int]
        L.zso_decompress.restype = C.c_int
        L.zso_decompress.argtypes = [p, C.c_int64, p, C.c_int64, p, p, p, p, C.c_int, C.c_int, C.c_int, p]
        L.zso_gemm_f32.argtypes = [p, p, C.c_int, C.c_int, C.c_int, p]
        L.zso_decompress_mt.restype = C.c_int
        L.zso_decompress_mt.argtypes = [p, C.c_int64, p, C.c_int64, p, p, p, p, C.c_int, C.c_int,
                                        C.c_int, p, C.c_int]
        L.zso_gemm_f32_mt.argtypes = [p, p, C.c_int, C.c_int, C.c_int, p, C.c_int]
        L.zso_gemm_splitk_bf16.argtypes = [p, p, C.c_int, C.c_int, C.c_int, C.c_int, p]
        L.zso_decode_attention_f64.argtypes = [p, p, p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                               p, C.c_double, p, p]
        L.zso_decode_attention_absv_f64.argtypes = [p, p, p, C.c_int, C.c_int, C.c_int, C.c_int,
                                                    C.c_int, p, C.c_double, p, p, p]
        L.zso_compress_retiled.restype = C.c_int64
        L.zso_compress_retiled.argtypes = [p, C.c_int, C.c_int, C.c_int, p, p, p]
        L.zso_decompress_retiled.argtypes = [p, p, p, C.c_int, C.c_int, C.c_int, p]
        _lib = L
    return _lib


class _Encoded(C.Structure):
    _fields_ = [
        ("sign_mantissa", C.c_void_p),
        ("compressed_full", C.c_void_p),
        ("bitmap1", C.c_void_p),
        ("bitmap2", C.c_void_p),
        ("bitmap3", C.c_void_p),
        ("tile_offsets", C.c_void_p),
        ("tile_offsets_median", C.c_void_p),
        ("tile_offsets_global", C.c_void_p),
        ("max_high_freq_count", C.c_int32),
        ("max_full_count", C.c_int32),
        ("total_high_freq", C.c_int64),
        ("total_full", C.c_int64),
    ]


@dataclass
class Encoded:
    """Canonical TCA-TBE streams of one matrix (csrc/L_API.cu:314-557)."""
    sign_mantissa: np.ndarray      # uint8  [total_high_freq]
    compressed_full: np.ndarray    # uint16 [total_full]
    bitmap1: np.ndarray            # uint64 [M*K/64]
    bitmap2: np.ndarray
    bitmap3: np.ndarray
    tile_offsets: np.ndarray       # int32 [2*M*K/64]
    tile_offsets_median: np.ndarray  # int32 [2*M*K/1024]
    tile_offsets_global: np.ndarray  # int32 [2*(M*K/4096+1)]
    max_high_freq_count: int
    max_full_count: int
    start_exp: int
    rows: int
    cols: int

    @property
    def num_global_tiles(self) -> int:
        return (self.rows // 64) * (self.cols // 64)

    def compressed_bytes(self) -> int:
        """GEMM-path size formula (kernel_benchmark/bench_zipserv_gemm_sweep.cu:424-429)."""
        mk = self.rows * self.cols
        return (self.sign_mantissa.size + 2 * self.compressed_full.size + 24 * (mk // 64)
                + 8 * (mk // 1024) + 8 * (mk // 4096 + 1))


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    return (a.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns (NaN kept quiet)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    out = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    out[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return out


def small_tile_pos(st: int) -> tuple[int, int]:
    r, c = C.c_int(), C.c_int()
    lib().zso_small_tile_pos(st, C.byref(r), C.byref(c))
    return r.value, c.value


def histogram(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.zeros(256, dtype=np.int64)
    lib().zso_histogram(_ptr(a), a.size, _ptr(out))
    return out


def analyze_cpu(a: np.ndarray) -> list[int]:
    """kernel_benchmark/utils.h:189-272 analyzeExponentDistribution_BF16."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    top = np.zeros(7, dtype=np.int32)
    lib().zso_analyze_cpu(_ptr(a), a.size, _ptr(top))
    return top.tolist()


def analyze_gpu(a: np.ndarray) -> list[int]:
    """kernel_benchmark/zipserv_decode_attention_ext.cu:35-135 selection."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    top = np.zeros(7, dtype=np.int32)
    lib().zso_analyze_gpu(_ptr(a), a.size, _ptr(top))
    return top.tolist()


def select_cpu(counts) -> list[int]:
    c = np.ascontiguousarray(counts, dtype=np.int64)
    top = np.zeros(7, dtype=np.int32)
    lib().zso_select_cpu(_ptr(c), _ptr(top))
    return top.tolist()


def select_gpu(counts) -> list[int]:
    c = np.ascontiguousarray(counts, dtype=np.int64)
    top = np.zeros(7, dtype=np.int32)
    lib().zso_select_gpu(_ptr(c), _ptr(top))
    return top.tolist()


def _zeroed(n, dt):
    """malloc + memset of the output buffers (the reference's encoder does both
    inside its timed region, L_API.cu:350-357)."""
    b = np.empty(n, dt)
    b.fill(0)
    return b


def compress(a: np.ndarray, top=None, variant: str = "plain", threads: int = 0,
             timings: dict | None = None) -> Encoded:
    """Encode a bf16 [M, K] matrix; variant in {plain, lut, sse, sse_mt}
    (sse_mt: the sse encoder over `threads` OpenMP threads, 0 = all).  With
    `timings`, the output allocation (malloc + memset) and the encode are
    timed separately into timings["alloc_s"] / timings["encode_s"]."""
    import time
    a = np.ascontiguousarray(a, dtype=np.uint16)
    M, K = a.shape
    if top is None:
        top = analyze_cpu(a)
    topa = np.ascontiguousarray(top, dtype=np.int32)
    mk = M * K
    t0 = time.perf_counter()
    bufs = dict(
        sign_mantissa=_zeroed(mk + 16, np.uint8),
        compressed_full=_zeroed(mk + 8, np.uint16),
        bitmap1=_zeroed(mk // 64, np.uint64),
        bitmap2=_zeroed(mk // 64, np.uint64),
        bitmap3=_zeroed(mk // 64, np.uint64),
        tile_offsets=_zeroed(2 * (mk // 64), np.int32),
        tile_offsets_median=_zeroed(2 * (mk // 1024), np.int32),
        tile_offsets_global=_zeroed(2 * (mk // 4096 + 1), np.int32),
    )
    enc = _Encoded(**{k: _ptr(v) for k, v in bufs.items()})
    t1 = time.perf_counter()
    if variant == "sse_mt":
        rc = lib().zso_compress_sse_mt(_ptr(a), M, K, _ptr(topa), C.byref(enc), int(threads))
    else:
        fn = {"plain": lib().zso_compress_plain, "lut": lib().zso_compress_lut,
              "sse": lib().zso_compress_sse}[variant]
        rc = fn(_ptr(a), M, K, _ptr(topa), C.byref(enc))
    if timings is not None:
        timings["alloc_s"] = t1 - t0
        timings["encode_s"] = time.perf_counter() - t1
    if rc < 0:
        raise ValueError(f"oracle compress failed for shape {a.shape}")
    return Encoded(
        sign_mantissa=bufs["sign_mantissa"][: enc.total_high_freq].copy(),
        compressed_full=bufs["compressed_full"][: enc.total_full].copy(),
        bitmap1=bufs["bitmap1"], bitmap2=bufs["bitmap2"], bitmap3=bufs["bitmap3"],
        tile_offsets=bufs["tile_offsets"], tile_offsets_median=bufs["tile_offsets_median"],
        tile_offsets_global=bufs["tile_offsets_global"],
        max_high_freq_count=enc.max_high_freq_count, max_full_count=enc.max_full_count,
        start_exp=(int(topa[0]) - 1) & 0xFF, rows=M, cols=K)


def decompress(e: Encoded, start_exp: int | None = None) -> np.ndarray:
    """bench_kv_cache_zipserv_decompress_token_scaling.cu:2106-2218."""
    out = np.zeros((e.rows, e.cols), np.uint16)
    se = e.start_exp if start_exp is None else start_exp
    sm = np.ascontiguousarray(e.sign_mantissa)
    fu = np.ascontiguousarray(e.compressed_full)
    rc = lib().zso_decompress(_ptr(sm), sm.size, _ptr(fu), fu.size,
                              _ptr(e.bitmap1), _ptr(e.bitmap2), _ptr(e.bitmap3),
                              _ptr(e.tile_offsets_global), e.rows, e.cols, se, _ptr(out))
    if rc != 0:
        raise ValueError("oracle decompress: stream index out of range")
    return out


def decompress_mt(e: Encoded, threads: int = 0) -> np.ndarray:
    """decompress() parallel over global tiles (CPU baseline; same output)."""
    out = np.zeros((e.rows, e.cols), np.uint16)
    sm = np.ascontiguousarray(e.sign_mantissa)
    fu = np.ascontiguousarray(e.compressed_full)
    rc = lib().zso_decompress_mt(_ptr(sm), sm.size, _ptr(fu), fu.size,
                                 _ptr(e.bitmap1), _ptr(e.bitmap2), _ptr(e.bitmap3),
                                 _ptr(e.tile_offsets_global), e.rows, e.cols, e.start_exp,
                                 _ptr(out), int(threads))
    if rc != 0:
        raise ValueError("oracle decompress: stream index out of range")
    return out


def gemm_f32_mt(W: np.ndarray, X: np.ndarray, threads: int = 0) -> np.ndarray:
    """gemm_f32() with each W row widened once, parallel over rows (same result)."""
    W = np.ascontiguousarray(W, dtype=np.uint16)
    X = np.ascontiguousarray(X, dtype=np.uint16)
    M, K = W.shape
    N = X.shape[0]
    Y = np.zeros((N, M), np.float32)
    lib().zso_gemm_f32_mt(_ptr(W), _ptr(X), M, N, K, _ptr(Y), int(threads))
    return Y


def gemm_f32(W: np.ndarray, X: np.ndarray) -> np.ndarray:
    """Y[N, M] = X[N, K] . W[M, K]^T with fp32 accumulation (csrc/L_Kernel.cuh:294-571 semantics)."""
    W = np.ascontiguousarray(W, dtype=np.uint16)
    X = np.ascontiguousarray(X, dtype=np.uint16)
    M, K = W.shape
    N = X.shape[0]
    Y = np.zeros((N, M), np.float32)
    lib().zso_gemm_f32(_ptr(W), _ptr(X), M, N, K, _ptr(Y))
    return Y


def gemm_splitk_bf16(W: np.ndarray, X: np.ndarray, split_k: int) -> np.ndarray:
    """Split-K rounding model (csrc/L_Kernel.cuh:316-326, csrc/Reduction_Kernel.cuh:15-37)."""
    W = np.ascontiguousarray(W, dtype=np.uint16)
    X = np.ascontiguousarray(X, dtype=np.uint16)
    M, K = W.shape
    N = X.shape[0]
    Y = np.zeros((N, M), np.uint16)
    lib().zso_gemm_splitk_bf16(_ptr(W), _ptr(X), M, N, K, split_k, _ptr(Y))
    return Y


def decode_attention_f64(q, k, v, seqlens=None, scale=None, return_absv=False):
    """q [B,H,D], k/v [B,T,Hkv,D] (bf16 bits) -> (out [B,H,D] f64, lse [B,H] f64),
    plus absv [B,H,D] = sum_t p_t |v_t| (the softmax-weighted magnitude of V,
    which bounds the effect of rounding the weights to bf16) when
    `return_absv`."""
    q = np.ascontiguousarray(q, dtype=np.uint16)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    B, H, D = q.shape
    T, Hkv = k.shape[1], k.shape[2]
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    sl = None if seqlens is None else np.ascontiguousarray(seqlens, dtype=np.int32)
    out = np.zeros((B, H, D), np.float64)
    lse = np.zeros((B, H), np.float64)
    absv = np.zeros((B, H, D), np.float64) if return_absv else None
    lib().zso_decode_attention_absv_f64(_ptr(q), _ptr(k), _ptr(v), B, H, Hkv, T, D,
                                        None if sl is None else _ptr(sl), float(scale), _ptr(out),
                                        _ptr(lse), None if absv is None else _ptr(absv))
    return (out, lse, absv) if return_absv else (out, lse)


REC_BYTES = 1408


@dataclass
class Retiled:
    """This build's CDNA4 re-tiled layout (no reference counterpart): fixed
    1408-byte records per 16x64 tile + outlier exponent stream."""
    fixed: np.ndarray   # uint8 [num_records * 1408]
    exps: np.ndarray    # uint8 [num_outliers]
    eoff: np.ndarray    # int32 [num_records + 1]
    start_exp: int
    rows: int
    cols: int

    def compressed_bytes(self) -> int:
        return self.fixed.size + self.exps.size + 4 * self.eoff.size


def compress_retiled(a: np.ndarray, start_exp: int) -> Retiled:
    """bf16 [M, K] -> re-tiled layout under window start `start_exp`."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    M, K = a.shape
    nrec = (M // 16) * (K // 64)
    fixed = np.zeros(nrec * REC_BYTES, np.uint8)
    exps = np.zeros(M * K, np.uint8)
    eoff = np.zeros(nrec + 1, np.int32)
    n = lib().zso_compress_retiled(_ptr(a), M, K, int(start_exp), _ptr(fixed), _ptr(exps), _ptr(eoff))
    return Retiled(fixed, exps[:n].copy(), eoff, int(start_exp) & 0xFF, M, K)


def retile(e: Encoded) -> Retiled:
    """Canonical streams -> re-tiled layout (decode, then re-pack under the same window)."""
    return compress_retiled(decompress(e), e.start_exp)


def decompress_retiled(r: Retiled) -> np.ndarray:
    out = np.zeros((r.rows, r.cols), np.uint16)
    ex = np.ascontiguousarray(r.exps) if r.exps.size else np.zeros(1, np.uint8)
    lib().zso_decompress_retiled(_ptr(r.fixed), _ptr(ex), _ptr(r.eoff), r.start_exp, r.rows,
                                 r.cols, _ptr(out))
    return out
