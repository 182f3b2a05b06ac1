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


# bf16 bit patterns a codec must carry unchanged: +-0, +-Inf, quiet and
# signalling NaNs with payloads, the smallest and largest subnormals, the
# largest finite value
SPECIAL_BF16 = np.array([0x0000, 0x8000, 0x7F80, 0xFF80, 0x7FC0, 0xFFC1, 0x7F81, 0x0001, 0x8001,
                         0x007F, 0x807F, 0x7F7F, 0xFF7F], np.uint16)


def arbitrary_bf16(rng, shape, kind):
    """"random_bits": every 16-bit pattern equally likely (mostly outliers,
    NaNs and Infs included); "specials": N(0, 0.02) weights with 5% of the
    elements replaced by SPECIAL_BF16 values."""
    if kind == "random_bits":
        return rng.integers(0, 65536, size=shape, dtype=np.uint16)
    W = weights_bf16(rng, shape)
    n = W.size // 20
    W.flat[rng.integers(0, W.size, n)] = rng.choice(SPECIAL_BF16, n)
    return W


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


def probe_columns(K, split_k):
    """Columns k of W probed with unit-vector rows of X (X[n] = e_k, so that
    Y[n] = W[:, k] exactly: one exact product per output, every other term
    zero, split-K partials W or 0).  One column in every 64-wide K tile (its
    position inside the tile moving with the tile), the first and last
    column of every split-K slice (the reference's partition, ceil(KT / S)
    tiles per slice, L_Kernel.cuh:316-326), and k = 0, K - 1.  Every K tile
    is one record per band, so every wave's K range, its first tile and any
    tile past a wave's 64th are among them."""
    kt = K // 64
    cols = {0, K - 1}
    for t in range(kt):
        cols.add(64 * t + (37 * t + 11) % 64)
    per = (kt - 1) // split_k + 1
    for s in range(split_k):
        t0, t1 = s * per, min(kt, (s + 1) * per)
        if t0 < kt:
            cols.update((64 * t0, 64 * t1 - 1))
    return sorted(cols)


def probe_batches(cols, n):
    """`cols` in batches of exactly n (the kernel choice depends on N): the
    last batch is filled up by repeating columns from the start."""
    out = []
    for i in range(0, len(cols), n):
        b = cols[i:i + n]
        while len(b) < n:
            b = b + cols[:n - len(b)]
        out.append(b)
    return out


def probe_mismatches(y, w_cols):
    """Entries of Y that differ from the probed W columns (Y[n][m] against
    W[m][k_n]), compared as values so that +0 and -0 are equal; works on
    numpy float arrays and on torch tensors (returns the count)."""
    diff = y != w_cols
    return int(diff.sum())
