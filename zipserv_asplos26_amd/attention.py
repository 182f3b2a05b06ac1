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


def pad_batched_kv_prefix_paged(x, page_block_size: int):
    """bench_zipserv_decode_attention.py:357-364: (B, T, Hkv, D) -> 2D
    [B*pad_page(T)*Hkv][pad64(D)] with row (b*rows_per_batch + t*Hkv + h), tokens
    padded to a whole number of pages.  Returns (matrix, logical_rows,
    rows_per_batch)."""
    torch = _torch()
    B, T, H, D = x.shape
    padded = (T + page_block_size - 1) // page_block_size * page_block_size
    rpb = padded * H
    cols = (D + 63) // 64 * 64
    out = torch.zeros((B, rpb, cols), dtype=x.dtype, device=x.device)
    out[:, : T * H, :D] = x.reshape(B, T * H, D)
    return out.view(B * rpb, cols), B * T * H, rpb


def make_batched_paged_kv_cache(x, page_block_size: int):
    """bench_zipserv_decode_attention.py:367-373: (B, T, Hkv, D) -> pages
    (B * pages_per_seq, page_block_size, Hkv, D), sequence b in pages
    b*pages_per_seq .. +pages_per_seq-1.  Returns (pages, pages_per_seq)."""
    torch = _torch()
    B, T, H, D = x.shape
    padded = (T + page_block_size - 1) // page_block_size * page_block_size
    out = torch.zeros((B, padded, H, D), dtype=x.dtype, device=x.device)
    out[:, :T] = x
    return out.view(B * (padded // page_block_size), page_block_size, H, D).contiguous(), \
        padded // page_block_size


def decompress_to_batched_paged_kv(comp, batch_size_cache: int, kv_heads: int, head_dim: int,
                                   page_block_size: int, workspace=None):
    """bench_zipserv_decode_attention.py:492-521 (the staged paged path):
    a token-major compressed cache -> dense pages (B * pages_per_seq,
    page_block_size, Hkv, head_dim), decompressed on the GPU into
    `workspace` ((rows, cols) bf16) when given."""
    from .codec import decompress, decompress_retiled
    if comp.rows % batch_size_cache:
        raise ValueError(f"Compressed rows {comp.rows} must be divisible by batch_size_cache "
                         f"{batch_size_cache}")
    rpb = comp.rows // batch_size_cache
    if rpb % kv_heads:
        raise ValueError(f"Rows per batch must be divisible by kv_heads, got rows_per_batch={rpb}, "
                         f"kv_heads={kv_heads}")
    padded = rpb // kv_heads
    if padded % page_block_size:
        raise ValueError(f"Padded tokens must be divisible by page_block_size, got tokens={padded}, "
                         f"page_block_size={page_block_size}")
    dense = (decompress_retiled if isinstance(comp, ZipservRetiled) else decompress)(comp, workspace)
    dense = dense.view(batch_size_cache, rpb, comp.cols)
    return dense[:, : padded * kv_heads, :head_dim].contiguous().view(
        batch_size_cache * (padded // page_block_size), page_block_size, kv_heads, head_dim)


def compress_kv(x, layout: str = "by_kv_head", retiled: bool = False,
                page_block_size: int = 16):
    """Pack a (B, T, Hkv, D) bf16 cache and compress it on the GPU into the
    canonical streams (ZipservCompressed) or the re-tiled layout
    (ZipservRetiled).  layout "paged" pads each sequence to whole pages of
    page_block_size tokens (token-major rows)."""
    if layout == "by_kv_head":
        mat, logical_rows, _ = pad_batched_kv_prefix_by_kv_head(x)
    elif layout in ("token_major", "dense"):
        mat, logical_rows, _ = pad_batched_kv_prefix(x)
    elif layout == "paged":
        mat, logical_rows, _ = pad_batched_kv_prefix_paged(x, page_block_size)
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
    for d in (dk, dv):  # staged token-major caches are decompressed into the workspace first
        wsb += int(L.zs_kv_retiled_staging_bytes(d.layout, d.rows, d.cols, zipserv_num_heads_k)
                   if retiled else L.zs_kv_staging_bytes(d.layout, d.rows, d.cols))
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
                                  return_softmax_lse: bool = False, block_table=None):
    """The uncompressed comparator (bench_zipserv_decode_attention.py:629-631):
    k_cache / v_cache (B, capacity, Hkv, D) bf16, or with block_table
    ((B, max_blocks_per_seq) int32, flash_attn_interface.py:1583-1658) pages
    (num_blocks, page_block_size, Hkv, D), page_block_size a multiple of 16."""
    torch = _torch()
    shape = q.shape
    q3 = _q3(q)
    _check_cuda(q3, "q", torch.bfloat16)
    _check_cuda(k_cache, "k_cache", torch.bfloat16)
    _check_cuda(v_cache, "v_cache", torch.bfloat16)
    B, H, D = q3.shape
    if block_table is not None:
        return _dense_paged(q3, shape, k_cache, v_cache, block_table, cache_seqlens,
                            softmax_scale, num_splits, return_softmax_lse)
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


def _dense_paged(q3, shape, k_cache, v_cache, block_table, cache_seqlens, softmax_scale,
                 num_splits, return_softmax_lse):
    torch = _torch()
    B, H, D = q3.shape
    if k_cache.shape != v_cache.shape or k_cache.dim() != 4:
        raise ValueError("paged k_cache / v_cache must both be (num_blocks, page_block_size, "
                         "heads_k, head_dim)")
    nblocks, page, Hkv = (int(v) for v in k_cache.shape[:3])
    _check_cuda(block_table, "block_table", torch.int32)
    if block_table.dim() != 2 or block_table.shape[0] != B:
        raise ValueError("block_table must be (batch, max_blocks_per_seq) int32")
    bt = block_table.contiguous()
    kc, vc = k_cache.contiguous(), v_cache.contiguous()  # held until the launch is queued
    maxb = int(bt.shape[1])
    cap = maxb * page
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    out = torch.empty_like(q3)
    lse = torch.empty((B, H), dtype=torch.float32, device=q3.device) if return_softmax_lse else None
    sl = _seqlens(cache_seqlens, B, q3.device)
    L = lib()
    wsb = int(L.zs_decode_attention_workspace_bytes(B, H, D, cap, num_splits))
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=q3.device)
    check("zs_decode_attention_dense_paged", L.zs_decode_attention_dense_paged(
        _stream(), _dptr(q3), _dptr(kc), _dptr(vc), _dptr(bt),
        maxb, nblocks, page, _dptr(sl), cap, B, H, Hkv, D, scale, _dptr(out), _dptr(lse),
        _dptr(ws), ws.numel(), int(num_splits)))
    out = out.view(shape)
    return (out, lse) if return_softmax_lse else out


def fwd_kvcache_zipserv(q, k_sign_mantissa, k_compressed_full, k_bitmap1, k_bitmap2, k_bitmap3,
                        k_tile_offsets_median, k_tile_offsets_global, k_rows: int, k_cols: int,
                        k_max_high_freq_count: int, k_max_full_count: int, k_start_exp: int,
                        v_sign_mantissa, v_compressed_full, v_bitmap1, v_bitmap2, v_bitmap3,
                        v_tile_offsets_median, v_tile_offsets_global, v_rows: int, v_cols: int,
                        v_max_high_freq_count: int, v_max_full_count: int, v_start_exp: int,
                        logical_kv_len: int, num_kv_heads: int, softmax_scale: float):
    """The standalone decode entry `fwd_kvcache_zipserv`
    (csrc/flash_attn_ck/zipserv_flash_api.cpp:7 -> mha_fwd_kvcache_zipserv,
    zipserv_fwd_kvcache.cu:380-533): one sequence (q (1, 1, H, D) bf16), one
    query token, head-major compressed K / V with rows_per_head =
    rows / num_kv_heads, the first logical_kv_len tokens attended.  Same
    argument checks (ValueError here for the reference's TORCH_CHECKs); the
    computation is zs_decode_attention.  Returns [out (1, 1, H, D),
    softmax_lse (1, H, 1)]."""
    torch = _torch()
    _check_cuda(q, "q", torch.bfloat16)
    if q.dim() != 4:
        raise ValueError("q must have shape (batch, seqlen_q, nheads, headdim)")
    if q.shape[0] != 1:
        raise ValueError("zipserv flash decode currently requires batch_size == 1")
    if q.shape[1] != 1:
        raise ValueError("zipserv flash decode currently requires q_len == 1")
    if k_rows != v_rows or k_cols != v_cols:
        raise ValueError("K/V rows and cols must match")
    if k_rows % 64 or k_cols % 64:
        raise ValueError("compressed K/V rows and cols must be padded to multiples of 64")
    if logical_kv_len <= 0:
        raise ValueError("logical_kv_len must be > 0")
    if num_kv_heads != 8:
        raise ValueError("zipserv flash decode currently requires num_kv_heads == 8")
    H, D = int(q.shape[2]), int(q.shape[3])
    if D <= 0 or D > 256:
        raise ValueError("zipserv flash decode currently requires head_dim <= 256")
    if H % num_kv_heads:
        raise ValueError("num_q_heads must be divisible by num_kv_heads")
    if k_rows % (num_kv_heads * 64):
        raise ValueError("compressed K rows must be head-major padded by 64 rows per kv head")
    if logical_kv_len * num_kv_heads > k_rows:
        raise ValueError("logical_kv_len exceeds compressed row capacity")
    if k_cols < D:
        raise ValueError("compressed K/V cols must be >= head_dim")
    k = dict(sign_mantissa=k_sign_mantissa, compressed_full=k_compressed_full, bitmap1=k_bitmap1,
             bitmap2=k_bitmap2, bitmap3=k_bitmap3, tile_offsets_median=k_tile_offsets_median,
             tile_offsets_global=k_tile_offsets_global, rows=k_rows, cols=k_cols,
             max_high_freq_count=k_max_high_freq_count, max_full_count=k_max_full_count,
             start_exp=k_start_exp, layout="by_kv_head")
    v = dict(sign_mantissa=v_sign_mantissa, compressed_full=v_compressed_full, bitmap1=v_bitmap1,
             bitmap2=v_bitmap2, bitmap3=v_bitmap3, tile_offsets_median=v_tile_offsets_median,
             tile_offsets_global=v_tile_offsets_global, rows=v_rows, cols=v_cols,
             max_high_freq_count=v_max_high_freq_count, max_full_count=v_max_full_count,
             start_exp=v_start_exp, layout="by_kv_head")
    out, lse = flash_attn_with_kvcache_zipserv(
        q, k, v, num_kv_heads, int(logical_kv_len), softmax_scale=float(softmax_scale),
        return_softmax_lse=True)
    return [out.view(1, 1, H, D), lse.view(1, H, 1)]
