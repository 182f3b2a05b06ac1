"""Decode attention over compressed K/V on the GPU vs the fp64 oracle and vs the
same kernel over the dense cache.

Reference: flash_attn_with_kvcache(..., zipserv_k=, zipserv_v=)
(kernel_benchmark/third_party/flash_attn_v283/flash_attn/flash_attn_interface.py:1572-1756,
flash_api.cpp:1346-1520).  Tolerance: 2e-3 absolute plus
one bf16 ulp of the reference value for the bf16 output, plus 2^-9 of the
largest |V| for the bf16 rounding of the softmax weights before the P.V
product (the same rounding FlashAttention applies).  The compressed and dense
paths decode to the same bf16 K/V and run the same arithmetic, so their
outputs must be bit-identical.
"""
import numpy as np
import pytest

import oracle as zo
from zs_testutil import from_torch_bf16, kv_bf16, normal_bf16, to_torch_bf16

pytestmark = pytest.mark.gpu


def _bf16_f32(a):
    return zo.bf16_to_f32(a).astype(np.float64)


def _run(torch_cuda, B, T, Hkv, H, seqlens=None, splits=0, seed=0, q_zero=False, retiled=False,
         layout="by_kv_head"):
    import zipserv_asplos26_amd.attention as za
    torch = torch_cuda
    rng = np.random.default_rng(seed)
    D = 128
    k = kv_bf16(rng, B, T, Hkv, D)
    v = kv_bf16(rng, B, T, Hkv, D)
    q = normal_bf16(rng, (B, H, D))
    if q_zero:
        q[:] = 0
    kd, vd, qd = to_torch_bf16(k), to_torch_bf16(v), to_torch_bf16(q)
    ck = za.compress_kv(kd, layout=layout, retiled=retiled)
    cv = za.compress_kv(vd, layout=layout, retiled=retiled)
    sl = None if seqlens is None else torch.tensor(seqlens, dtype=torch.int32, device="cuda")
    out, lse = za.flash_attn_with_kvcache_zipserv(
        qd.view(B, 1, H, D), ck, cv, Hkv, T, cache_seqlens=sl, num_splits=splits,
        return_softmax_lse=True)
    outd, lsed = za.flash_attn_with_kvcache_dense(
        qd.view(B, 1, H, D), kd, vd, cache_seqlens=sl, num_splits=splits,
        return_softmax_lse=True)
    torch.cuda.synchronize()
    ref, ref_lse = zo.decode_attention_f64(q, k, v, seqlens=seqlens)
    return (q, k, v, from_torch_bf16(out.view(B, H, D)), lse.cpu().numpy(),
            from_torch_bf16(outd.view(B, H, D)), lsed.cpu().numpy(), ref, ref_lse)


def _check(res, seqlens=None):
    q, k, v, out, lse, outd, lsed, ref, ref_lse = res
    np.testing.assert_array_equal(out, outd)  # compressed == dense, bit for bit
    np.testing.assert_array_equal(lse, lsed)
    o = _bf16_f32(out)
    vmax = np.abs(_bf16_f32(v)).max()
    tol = 2e-3 + np.abs(ref) * 2.0 ** -7 + vmax * 2.0 ** -9
    err = np.abs(o - ref)
    assert np.all(err <= tol), f"max err {err.max()} (tol at worst {tol[err > tol].min()})"
    finite = np.isfinite(ref_lse)
    np.testing.assert_allclose(lse[finite], ref_lse[finite], rtol=1e-4, atol=1e-3)
    assert np.all(np.isneginf(lse[~finite]))


@pytest.mark.parametrize("B,T,Hkv,H,splits", [
    (1, 64, 8, 64, 1),
    (1, 64, 8, 64, 0),
    (2, 100, 8, 64, 0),      # T not a multiple of 64 (masked tail)
    (2, 1000, 8, 64, 3),
    (1, 4096, 8, 64, 0),     # config-5 shape, automatic splits
    (2, 700, 2, 32, 5),      # GQA group 16
    (2, 300, 4, 4, 2),       # MHA (group 1)
    (3, 257, 1, 8, 64),      # more splits than needed for short sequences
])
def test_attention_matches_oracle(torch_cuda, B, T, Hkv, H, splits):
    _check(_run(torch_cuda, B, T, Hkv, H, splits=splits))


@pytest.mark.parametrize("B,T,Hkv,H,splits", [
    (1, 64, 8, 64, 1), (2, 100, 8, 64, 0), (2, 1000, 8, 64, 3), (1, 4096, 8, 64, 0),
    (2, 700, 2, 32, 5), (2, 300, 4, 4, 2), (3, 257, 1, 8, 64)])
def test_attention_retiled_matches_oracle(torch_cuda, B, T, Hkv, H, splits):
    # same decoded K/V and arithmetic as the canonical path: identical to dense
    _check(_run(torch_cuda, B, T, Hkv, H, splits=splits, retiled=True))


@pytest.mark.parametrize("splits", [1, 0])
def test_attention_retiled_ragged(torch_cuda, splits):
    seqlens = [300, 17, 0, 64]
    _check(_run(torch_cuda, 4, 300, 8, 64, seqlens=seqlens, splits=splits, seed=3, retiled=True))


@pytest.mark.parametrize("splits", [1, 0, 4])
def test_attention_ragged_seqlens(torch_cuda, splits):
    seqlens = [300, 17, 0, 64]
    _check(_run(torch_cuda, 4, 300, 8, 64, seqlens=seqlens, splits=splits, seed=3), seqlens)


@pytest.mark.parametrize("retiled", [False, True])
@pytest.mark.parametrize("B,T,Hkv,H,splits,seqlens", [
    (1, 64, 8, 64, 1, None),
    (2, 100, 8, 64, 0, None),     # T * Hkv not a multiple of 64: padded batch rows
    (2, 1000, 8, 64, 3, None),
    (2, 700, 2, 32, 5, None),     # GQA group 16
    (2, 300, 4, 4, 2, None),      # MHA
    (4, 300, 8, 64, 0, [300, 17, 0, 64]),
])
def test_attention_token_major(torch_cuda, retiled, B, T, Hkv, H, splits, seqlens):
    # token-major caches (row b*batch_stride + t*Hkv + h) run staged: the
    # result equals the dense kernel's bit for bit, and the oracle's
    _check(_run(torch_cuda, B, T, Hkv, H, seqlens=seqlens, splits=splits, seed=11,
                retiled=retiled, layout="token_major"), seqlens)


def test_attention_single_token_returns_v(torch_cuda):
    # T = 1: softmax weight 1, out = V[0] exactly (bf16 in, bf16 out).
    q, k, v, out, *_ = _run(torch_cuda, 2, 1, 8, 64, splits=1, seed=5)
    G = 8
    for b in range(2):
        for h in range(64):
            np.testing.assert_array_equal(out[b, h], v[b, 0, h // G])


def test_attention_equal_scores_mean_of_v(torch_cuda):
    # q = 0: all scores equal, out = mean of V over the sequence.
    res = _run(torch_cuda, 1, 200, 8, 64, splits=2, seed=7, q_zero=True)
    q, k, v, out, *_ = res
    mean = _bf16_f32(v).mean(axis=1)  # [B, Hkv, D]
    o = _bf16_f32(out).reshape(1, 8, 8, 128)
    ref = np.repeat(mean[:, :, None, :], 8, axis=2)
    assert np.all(np.abs(o - ref) <= 2e-3 + np.abs(ref) * 2.0 ** -7 + np.abs(_bf16_f32(v)).max() * 2.0 ** -9)
    _check(res)


def test_attention_rejects_unsupported(torch_cuda):
    import ctypes

    import zipserv_asplos26_amd as zs
    import zipserv_asplos26_amd.attention as za
    torch = torch_cuda
    rng = np.random.default_rng(0)
    k = to_torch_bf16(kv_bf16(rng, 1, 128, 8, 128))
    c = za.compress_kv(k)
    d, keep = za._normalize_zipserv_kv(c, name="k", device=k.device, batch_size=1, num_heads_k=8)
    q = torch.zeros(1, 64, 128, dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(q)
    L = zs.lib()

    def call(dk, dv, D=128, H=64, Hkv=8, T=128, splits=1, qoff=0, ooff=0):
        return L.zs_decode_attention(0, q.data_ptr() + qoff, ctypes.byref(dk), ctypes.byref(dv),
                                     None, T, 1, H, Hkv, D, 0.1, out.data_ptr() + ooff, None, None,
                                     0, splits)
    assert call(d, d) == 0
    torch.cuda.synchronize()
    assert call(d, d, qoff=2) == zs._lib.ZS_E_INVAL  # q rows are read 16 bytes at a time
    assert call(d, d, ooff=8) == zs._lib.ZS_E_INVAL
    assert call(d, d, D=64) == zs._lib.ZS_E_UNSUPPORTED
    assert call(d, d, H=63) == zs._lib.ZS_E_INVAL
    assert call(d, d, T=129) == zs._lib.ZS_E_INVAL  # rows per head (128) < seqlen_k
    assert call(d, d, splits=2) == zs._lib.ZS_E_INVAL  # two splits need a workspace
    tm = za._lib.KVCompressed.from_buffer_copy(d)
    tm.layout = zs._lib.ZS_LAYOUT_TOKEN_MAJOR
    assert call(tm, d) == zs._lib.ZS_E_UNSUPPORTED   # K and V layouts differ
    assert call(tm, tm) == zs._lib.ZS_E_INVAL        # token-major needs staging workspace
    assert L.zs_kv_staging_bytes(zs._lib.ZS_LAYOUT_TOKEN_MAJOR, 1024, 128) == 1024 * 128 * 2
    assert L.zs_kv_staging_bytes(zs._lib.ZS_LAYOUT_HEAD_MAJOR, 1024, 128) == 0
    assert L.zs_kv_staging_bytes(7, 1024, 128) == -1
    bad = za._lib.KVCompressed.from_buffer_copy(d)
    bad.head_stride_rows = 32
    assert call(bad, d) == zs._lib.ZS_E_INVAL
    del keep
