"""Shared test data generators (numpy; bf16 carried as uint16 bit patterns)."""
import numpy as np

import oracle as zo


def normal_bf16(rng, shape, std=1.0):
    return zo.f32_to_bf16(rng.standard_normal(shape, dtype=np.float32) * np.float32(std))


def weights_bf16(rng, shape, std=0.02, outlier_frac=0.0, outlier_scale=30.0):
    """W ~ N(0, std) with a Bernoulli(outlier_frac) mask scaled by outlier_scale."""
    w = rng.standard_normal(shape, dtype=np.float32) * np.float32(std)
    if outlier_frac > 0:
        mask = rng.random(shape) < outlier_frac
        w[mask] *= np.float32(outlier_scale)
    return zo.f32_to_bf16(w)


def kv_bf16(rng, batch, tokens, heads, dim):
    """KV ~ N(0,1) * per-(head, channel) lognormal(0,1) scales (benchmark config 4)."""
    scales = np.exp(rng.standard_normal((1, 1, heads, dim))).astype(np.float32)
    x = rng.standard_normal((batch, tokens, heads, dim), dtype=np.float32) * scales
    return zo.f32_to_bf16(x)


def pad_by_kv_head(kv):
    """bench_zipserv_decode_attention.py:347-354 pad_batched_kv_prefix_by_kv_head on numpy:
    [B, T, Hkv, D] -> 2D [B*Hkv*pad64(T), pad64(D)] plus rows_per_head."""
    B, T, H, D = kv.shape
    rph = (T + 63) // 64 * 64
    cols = (D + 63) // 64 * 64
    out = np.zeros((B, H, rph, cols), np.uint16)
    out[:, :, :T, :D] = kv.transpose(0, 2, 1, 3)
    return out.reshape(B * H * rph, cols), rph


def upload(e, device="cuda"):
    """Oracle-encoded streams -> device ZipservCompressed (with stream slack)."""
    import zipserv_asplos26_amd as zs
    h = zs.HostCompressed(
        sign_mantissa=e.sign_mantissa, compressed_full=e.compressed_full, bitmap1=e.bitmap1,
        bitmap2=e.bitmap2, bitmap3=e.bitmap3, tile_offsets=e.tile_offsets,
        tile_offsets_median=e.tile_offsets_median, tile_offsets_global=e.tile_offsets_global,
        rows=e.rows, cols=e.cols, max_high_freq_count=e.max_high_freq_count,
        max_full_count=e.max_full_count, start_exp=e.start_exp)
    return zs.to_device(h, device)


def to_torch_bf16(a, device="cuda"):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(device).view(torch.bfloat16)


def from_torch_bf16(t):
    import torch
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def attention_tolerance(ref, absv):
    """Per-element bound for bf16 decode attention against the fp64 oracle:
    2e-3 absolute, plus bf16's unit roundoff 2^-8 of
    the output (its final rounding) and of absv = sum_t p_t |v_t| (the
    softmax weights rounded to bf16 before the P.V product, as FlashAttention
    does, flash_fwd_kernel.h:892-1074: each weight moves by at most 2^-8 of
    itself).  Arithmetic in fp32 adds far less than 2e-3 at these sizes."""
    return 2e-3 + 2.0 ** -8 * np.abs(ref) + 2.0 ** -8 * absv
