"""Decode attention over a ZipServ-compressed KV cache (host-side mirror).

Mirrors the compressed-KV entry of the reference's FlashAttention fork:
`flash_attn_with_kvcache(q, k_cache, v_cache, ..., zipserv_k=, zipserv_v=,
zipserv_num_heads_k=)` (kernel_benchmark/third_party/flash_attn_v283/flash_attn/
flash_attn_interface.py:1572-1756) with its descriptor normalisation
(`_normalize_zipserv_kv`, :75-128), and the KV packing helpers of
kernel_benchmark/bench_zipserv_decode_attention.py:337-354.  The compute is
`zs_decode_attention` / `zs_decode_attention_dense` in libzipserv.so.
"""
from __future__ import annotations

import math
from typing import Optional

from . import _lib
from ._lib import check, lib
from .codec import ZipservRetiled, _check_cuda, _dptr, _stream, _torch, compress, compress_retiled

# flash_attn_interface.py:38-43 (_ZIPSERV_LAYOUT_IDS)
LAYOUT_IDS = {"by_kv_head": _lib.ZS_LAYOUT_HEAD_MAJOR, "dense": _lib.ZS_LAYOUT_TOKEN_MAJOR,
              "paged": _lib.ZS_LAYOUT_TOKEN_MAJOR, "token_major": _lib.ZS_LAYOUT_TOKEN_MAJOR}

_FIELDS = ("sign_mantissa", "compressed_full", "bitmap1", "bitmap2", "bitmap3",
           "tile_offsets_median", "tile_offsets_global", "rows", "cols",
           "max_high_freq_count", "max_full_count", "start_exp")


def pad_batched_kv_prefix_by_kv_head(x):
    """bench_zipserv_decode_attention.py:346-354: (B, T, Hkv, D) -> 2D
    [B*Hkv*pad64(T)][pad64(D)] with row ((b*Hkv + h)*rows_per_head + t).
    Returns (matrix, logical_rows, rows_per_head)."""
    torch = _torch()
    B, T, H, D = x.shape
    rph = (T + 63) // 64 * 64
    cols = (D + 63) // 64 * 64
    out = torch.zeros((B, H, rph, cols), dtype=x.dtype, device=x.device)
    out[:, :, :T, :D] = x.permute(0, 2, 1, 3)
    return out.view(B * H * rph, cols), B * H * rph, rph


def pad_batched_kv_prefix(x):
    """bench_zipserv_decode_attention.py:337-344: (B, T, Hkv, D) -> 2D
    [B*pad64(T*Hkv)][pad64(D)] with row (b*rows_per_batch + t*Hkv + h).
    Returns (matrix, logical_rows, rows_per_batch)."""
    torch = _torch()
    B, T, H, D = x.shape
    lr = T * H
    rpb = (lr + 63) // 64 * 64
    cols = (D + 63) // 64 * 64
    out = torch.zeros((B, rpb, cols), dtype=x.dtype, device=x.device)
    out[:, :lr, :D] = x.reshape(B, lr, D)
    return out.view(B * rpb, cols), lr * B, rpb


def compress_kv(x, layout: str = "by_kv_head", retiled: bool = False):
    """Pack a (B, T, Hkv, D) bf16 cache and compress it on the GPU into the
    canonical streams (ZipservCompressed) or the re-tiled layout
    (ZipservRetiled)."""
    if layout == "by_kv_head":
        mat, logical_rows, _ = pad_batched_kv_prefix_by_kv_head(x)
    elif layout in ("token_major", "dense"):
        mat, logical_rows, _ = pad_batched_kv_prefix(x)
    else:
        raise ValueError(f"unknown layout {layout!r}")
    fn = compress_retiled if retiled else compress
    return fn(mat.contiguous(), logical_rows, x.shape[-1], layout=layout)


def _retiled_desc(c, *, name, device, batch_size, num_heads_k):
    """zs_kv_retiled_t for a ZipservRetiled cache (strides as in
    _normalize_zipserv_kv)."""
    if c.device != device:
        raise ValueError(f"{name} must be on {device}")
    if c.rows % batch_size:
        raise ValueError(f"{name}.rows must be divisible by batch_size={batch_size}")
    bsr = c.rows // batch_size
    if bsr % num_heads_k:
        raise ValueError(f"{name}.rows must encode an integer rows-per-head for num_heads_k={num_heads_k}")
    d = _lib.KVRetiled()
    d.fixed, d.exps, d.eoff = _dptr(c.fixed), _dptr(c.exps), _dptr(c.eoff)
    d.rows, d.cols = c.rows, c.cols
    d.batch_stride_rows, d.head_stride_rows = bsr, bsr // num_heads_k
    d.start_exp, d.layout = c.start_exp, LAYOUT_IDS[str(c.layout)]
    return d


def _normalize_zipserv_kv(desc, *, name: str, device, batch_size: int, num_heads_k: int):
    """flash_attn_interface.py:75-128: descriptor (object / dict / sequence) ->
    zs_kv_compressed_t plus the tensors it points at (kept alive by the caller)."""
    torch = _torch()
    layout = "by_kv_head"
    if isinstance(desc, dict):
        values = tuple(desc[f] for f in _FIELDS)
        layout = desc.get("layout", layout)
    elif isinstance(desc, (list, tuple)):
        if len(desc) not in (len(_FIELDS), len(_FIELDS) + 1):
            raise ValueError(f"{name} must have {len(_FIELDS)} or {len(_FIELDS) + 1} elements")
        values = tuple(desc[: len(_FIELDS)])
        if len(desc) == len(_FIELDS) + 1:
            layout = desc[-1]
    else:
        values = tuple(getattr(desc, f) for f in _FIELDS)
        layout = getattr(desc, "layout", layout)
    tensors = []
    for f, t in zip(_FIELDS[:7], values[:7]):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name}.{f} must be a torch.Tensor")
        if t.device != device:
            raise ValueError(f"{name}.{f} must be on {device}")
        tensors.append(t.contiguous())
    rows, cols, max_hf, max_full, start_exp = (int(v) for v in values[7:])
    if batch_size <= 0 or num_heads_k <= 0:
        raise ValueError("batch_size and num_heads_k must be positive")
    if rows % batch_size:
        raise ValueError(f"{name}.rows must be divisible by batch_size={batch_size}")
    bsr = rows // batch_size
    if bsr % num_heads_k:
        raise ValueError(f"{name}.rows must encode an integer rows-per-head for num_heads_k={num_heads_k}")
    hsr = bsr // num_heads_k
    if str(layout) not in LAYOUT_IDS:
        raise ValueError(f"{name}.layout must be one of {sorted(LAYOUT_IDS)}")
    d = _lib.KVCompressed()
    for f, t in zip(_FIELDS[:7], tensors):
        setattr(d, f, _dptr(t))
    d.rows, d.cols = rows, cols
    d.batch_stride_rows, d.head_stride_rows = bsr, hsr
    d.max_high_freq_count, d.max_full_count = max_hf, max_full
    d.start_exp, d.layout = start_exp, LAYOUT_IDS[str(layout)]
    return d, tensors


def _seqlens(cache_seqlens, batch, device):
    torch = _torch()
    if cache_seqlens is None:
        return None
    if isinstance(cache_seqlens, int):
        return torch.full((batch,), cache_seqlens, dtype=torch.int32, device=device)
    t = cache_seqlens.to(device=device, dtype=torch.int32).contiguous()
    if t.numel() != batch:
        raise ValueError("cache_seqlens must have one entry per batch")
    return t


def _q3(q):
    """(B, 1, H, D) or (B, H, D) -> contiguous (B, H, D)."""
    if q.dim() == 4:
        if q.shape[1] != 1:
            raise ValueError("decode attention takes one query token (seqlen_q == 1)")
        q = q[:, 0]
    if q.dim() != 3:
        raise ValueError("q must be (batch, 1, heads, head_dim) or (batch, heads, head_dim)")
    return q.contiguous()


def flash_attn_with_kvcache_zipserv(q, zipserv_k, zipserv_v, zipserv_num_heads_k: int,
                                    seqlen_k: int, cache_seqlens=None,
                                    softmax_scale: Optional[float] = None, num_splits: int = 0,
                                    return_softmax_lse: bool = False):
    """Decode attention reading compressed K / V (flash_attn_interface.py:1572
    with zipserv_k / zipserv_v).  q: (B, 1, H, D) or (B, H, D) bf16 on the GPU;
    seqlen_k: tokens per sequence held by the caches; cache_seqlens: optional
    int / int32 tensor [B] of valid lengths.  Returns out shaped like q (and
    the natural-log softmax_lse [B, H] when asked)."""
    torch = _torch()
    shape = q.shape
    q3 = _q3(q)
    _check_cuda(q3, "q", torch.bfloat16)
    B, H, D = q3.shape
    retiled = isinstance(zipserv_k, ZipservRetiled)
    if retiled != isinstance(zipserv_v, ZipservRetiled):
        raise ValueError("zipserv_k and zipserv_v must use the same layout")
    if retiled:
        dk = _retiled_desc(zipserv_k, name="zipserv_k", device=q.device, batch_size=B,
                           num_heads_k=zipserv_num_heads_k)
        dv = _retiled_desc(zipserv_v, name="zipserv_v", device=q.device, batch_size=B,
                           num_heads_k=zipserv_num_heads_k)
        keep_k, keep_v = zipserv_k, zipserv_v
    else:
        dk, keep_k = _normalize_zipserv_kv(zipserv_k, name="zipserv_k", device=q.device,
                                           batch_size=B, num_heads_k=zipserv_num_heads_k)
        dv, keep_v = _normalize_zipserv_kv(zipserv_v, name="zipserv_v", device=q.device,
                                           batch_size=B, num_heads_k=zipserv_num_heads_k)
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    out = torch.empty_like(q3)
    lse = torch.empty((B, H), dtype=torch.float32, device=q.device) if return_softmax_lse else None
    sl = _seqlens(cache_seqlens, B, q.device)
    L = lib()
    wsb = int(L.zs_decode_attention_workspace_bytes(B, H, D, seqlen_k, num_splits))
    for d in (dk, dv):  # token-major caches are decompressed into the workspace first
        wsb += int(L.zs_kv_staging_bytes(d.layout, d.rows, d.cols))
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=q.device)
    import ctypes
    fn_name = "zs_decode_attention_retiled" if retiled else "zs_decode_attention"
    check(fn_name, getattr(L, fn_name)(
        _stream(), _dptr(q3), ctypes.byref(dk), ctypes.byref(dv), _dptr(sl), int(seqlen_k), B, H,
        int(zipserv_num_heads_k), D, scale, _dptr(out), _dptr(lse), _dptr(ws), ws.numel(),
        int(num_splits)))
    del keep_k, keep_v
    out = out.view(shape)
    return (out, lse) if return_softmax_lse else out


def flash_attn_with_kvcache_dense(q, k_cache, v_cache, cache_seqlens=None,
                                  softmax_scale: Optional[float] = None, num_splits: int = 0,
                                  return_softmax_lse: bool = False):
    """The uncompressed comparator (bench_zipserv_decode_attention.py:629-631):
    k_cache / v_cache (B, capacity, Hkv, D) bf16."""
    torch = _torch()
    shape = q.shape
    q3 = _q3(q)
    _check_cuda(q3, "q", torch.bfloat16)
    _check_cuda(k_cache, "k_cache", torch.bfloat16)
    _check_cuda(v_cache, "v_cache", torch.bfloat16)
    B, H, D = q3.shape
    if k_cache.shape != v_cache.shape or k_cache.dim() != 4 or k_cache.shape[0] != B:
        raise ValueError("k_cache / v_cache must both be (batch, capacity, heads_k, head_dim)")
    cap, Hkv = int(k_cache.shape[1]), int(k_cache.shape[2])
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    out = torch.empty_like(q3)
    lse = torch.empty((B, H), dtype=torch.float32, device=q.device) if return_softmax_lse else None
    sl = _seqlens(cache_seqlens, B, q.device)
    L = lib()
    wsb = int(L.zs_decode_attention_workspace_bytes(B, H, D, cap, num_splits))
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=q.device)
    check("zs_decode_attention_dense", L.zs_decode_attention_dense(
        _stream(), _dptr(q3), _dptr(k_cache), _dptr(v_cache), _dptr(sl), cap, cap, B, H, Hkv, D,
        scale, _dptr(out), _dptr(lse), _dptr(ws), ws.numel(), int(num_splits)))
    out = out.view(shape)
    return (out, lse) if return_softmax_lse else out
