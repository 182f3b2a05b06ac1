"""Decode attention over compressed K/V on the GPU vs the fp64 oracle and vs the
same kernel over the dense cache.

Reference: flash_attn_with_kvcache(..., zipserv_k=, zipserv_v=)
(kernel_benchmark/third_party/flash_attn_v283/flash_attn/flash_attn_interface.py:1572-1756,
flash_api.cpp:1346-1520).  Tolerance per element (zs_testutil.attention_tolerance):
2e-3 absolute plus 2^-8 (bf16's unit roundoff) of the
reference value for the bf16 output and of sum_t p_t |v_t,d| for the bf16
rounding of the softmax weights before the P.V product (the rounding
FlashAttention applies).  tests/test_oracle_math.py shows that this bound
fails an oracle run that drops one token or scales the scores by one bf16 ulp
at the config-5 shape.  The compressed and dense paths decode to the same
bf16 K/V and run the same arithmetic, so their outputs must be bit-identical.
"""
import numpy as np
import pytest

import oracle as zo
from zs_testutil import attention_tolerance, from_torch_bf16, kv_bf16, normal_bf16, to_torch_bf16

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
    ref, ref_lse, absv = zo.decode_attention_f64(q, k, v, seqlens=seqlens, return_absv=True)
    return (q, k, v, from_torch_bf16(out.view(B, H, D)), lse.cpu().numpy(),
            from_torch_bf16(outd.view(B, H, D)), lsed.cpu().numpy(), ref, ref_lse, absv)


def _check(res, seqlens=None, exact=True):
    q, k, v, out, lse, outd, lsed, ref, ref_lse, absv = res
    if exact:
        np.testing.assert_array_equal(out, outd)  # compressed == dense, bit for bit
        np.testing.assert_array_equal(lse, lsed)
    o = _bf16_f32(out)
    tol = attention_tolerance(ref, absv)
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
    (2, 700, 2, 32, 5), (2, 300, 4, 4, 2), (3, 257, 1, 8, 64),
    # 2065 items: one wave per item, the last workgroup holds one item and
    # three idle waves; 128-token splits past T leave the last waves empty
    (7, 3840, 5, 10, 59)])
def test_attention_retiled_matches_oracle(torch_cuda, B, T, Hkv, H, splits):
    # same decoded K/V and arithmetic as the canonical path: identical to dense
    _check(_run(torch_cuda, B, T, Hkv, H, splits=splits, retiled=True))


@pytest.mark.parametrize("retiled,layout", [(False, "by_kv_head"), (True, "by_kv_head"),
                                            (True, "token_major")])
def test_attention_split_merge_past_one_chunk(torch_cuda, retiled, layout):
    # 600 splits of 32 tokens (the last 88 empty): the merge runs 16 waves
    # per (batch, head) and walks two chunks of at most 512 splits, its first
    # loads issued before the split maximum
    fused_tm = retiled and layout == "token_major"
    _check(_run(torch_cuda, 1, 16384, 8, 64, splits=600, seed=5, retiled=retiled, layout=layout),
           exact=not fused_tm)


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
    # token-major caches (row b*batch_stride + t*Hkv + h): canonical ones and
    # re-tiled ones with Hkv != 8 run staged (the result equals the dense
    # kernel's bit for bit); re-tiled ones with Hkv == 8 run fused, whose
    # splits follow their own rule -- the oracle bound holds either way
    fused = retiled and Hkv == 8
    _check(_run(torch_cuda, B, T, Hkv, H, seqlens=seqlens, splits=splits, seed=11,
                retiled=retiled, layout="token_major"), seqlens, exact=not fused)


@pytest.mark.parametrize("B,T,splits,seqlens", [
    (1, 64, 1, None),
    (2, 1000, 16, None),            # 64-token chunks, masked tail
    (3, 100, 2, None),              # T * 8 not a multiple of 64: padded batch rows
    (4, 300, 5, [300, 17, 0, 64]),  # ragged lengths, an empty sequence
    (8, 4096, 32, None),            # 2048 (batch, head, split) items, 128-token chunks
])
def test_attention_token_major_fused_exact(torch_cuda, B, T, splits, seqlens):
    # Fused token-major attention (8 KV heads, 64 query heads): with splits
    # whose chunks the dense kernel also walks with one wave per (batch,
    # head, split) -- 64-token chunks, or >= 2048 items -- both run the same
    # operands through the same arithmetic: bit-identical, and within the
    # oracle bound
    _check(_run(torch_cuda, B, T, 8, 64, seqlens=seqlens, splits=splits, seed=29, retiled=True,
                layout="token_major"), seqlens)


@pytest.mark.parametrize("B,T,H,splits,seqlens", [
    (1, 4096, 64, 0, None),          # automatic splits (config-5 shape)
    (2, 1000, 64, 3, None),          # 336-token chunks
    (2, 700, 8, 0, None),            # MHA-sized group 1
    (2, 333, 128, 0, None),          # GQA group 16
    (4, 300, 64, 0, [300, 17, 0, 64]),
    (2, 100, 64, 6, None),           # 32-token chunks: the last two splits are empty
    (5, 17, 64, 0, [17, 1, 16, 9, 0]),
])
def test_attention_token_major_fused_oracle(torch_cuda, B, T, H, splits, seqlens):
    _check(_run(torch_cuda, B, T, 8, H, seqlens=seqlens, splits=splits, seed=31, retiled=True,
                layout="token_major"), seqlens, exact=False)


def test_attention_token_major_fused_needs_no_staging(torch_cuda):
    import zipserv_asplos26_amd as zs
    L = zs.lib()
    tm, hm = zs._lib.ZS_LAYOUT_TOKEN_MAJOR, zs._lib.ZS_LAYOUT_HEAD_MAJOR
    assert L.zs_kv_retiled_staging_bytes(tm, 1024, 128, 8) == 0
    assert L.zs_kv_retiled_staging_bytes(tm, 1024, 128, 4) == 1024 * 128 * 2
    assert L.zs_kv_retiled_staging_bytes(hm, 1024, 128, 8) == 0
    assert L.zs_kv_retiled_staging_bytes(7, 1024, 128, 8) == -1


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
    # equal weights: absv is the mean of |V| over the sequence
    absv = np.repeat(np.abs(_bf16_f32(v)).mean(axis=1)[:, :, None, :], 8, axis=2)
    assert np.all(np.abs(o - ref) <= attention_tolerance(ref, absv))
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


def test_fwd_kvcache_zipserv_standalone(torch_cuda):
    # csrc/flash_attn_ck/zipserv_fwd_kvcache.cu:380-533 (fwd_kvcache_zipserv):
    # B = 1, head-major streams passed one by one, logical_kv_len tokens.
    import zipserv_asplos26_amd as zs
    import zipserv_asplos26_amd.attention as za
    torch = torch_cuda
    rng = np.random.default_rng(17)
    T, Hkv, H, D, L = 200, 8, 64, 128, 150
    k = kv_bf16(rng, 1, T, Hkv, D)
    v = kv_bf16(rng, 1, T, Hkv, D)
    q = normal_bf16(rng, (1, H, D))
    kd, vd, qd = to_torch_bf16(k), to_torch_bf16(v), to_torch_bf16(q)
    pk = zs.compress_zipserv(za.pad_batched_kv_prefix_by_kv_head(kd)[0].contiguous())
    pv = zs.compress_zipserv(za.pad_batched_kv_prefix_by_kv_head(vd)[0].contiguous())

    def args(parts):
        m = parts[7].tolist()
        return list(parts[:7]) + [m[0], m[1], m[4], m[5], m[6]]
    scale = 1.0 / np.sqrt(D)
    out, lse = za.fwd_kvcache_zipserv(qd.view(1, 1, H, D), *args(pk), *args(pv), L, Hkv, scale)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (1, 1, H, D) and tuple(lse.shape) == (1, H, 1)
    ref, ref_lse, absv = zo.decode_attention_f64(q, k[:, :L], v[:, :L], return_absv=True)
    o = _bf16_f32(from_torch_bf16(out.view(1, H, D)))
    assert np.all(np.abs(o - ref) <= attention_tolerance(ref, absv))
    np.testing.assert_allclose(lse.view(1, H).cpu().numpy(), ref_lse, rtol=1e-4, atol=1e-3)
    # the reference's argument checks
    with pytest.raises(ValueError):  # batch 2
        za.fwd_kvcache_zipserv(qd.view(1, 1, H, D).expand(2, 1, H, D).contiguous(), *args(pk),
                               *args(pv), L, Hkv, scale)
    with pytest.raises(ValueError):  # num_kv_heads != 8
        za.fwd_kvcache_zipserv(qd.view(1, 1, H, D), *args(pk), *args(pv), L, 4, scale)
    with pytest.raises(ValueError):  # more tokens than the rows hold
        za.fwd_kvcache_zipserv(qd.view(1, 1, H, D), *args(pk), *args(pv), 257, Hkv, scale)


def _paged(torch, x, page, rng):
    """(B, T, Hkv, D) torch cache -> pages in a random order + block table."""
    import zipserv_asplos26_amd.attention as za
    pages, per_seq = za.make_batched_paged_kv_cache(x, page)
    perm = rng.permutation(pages.shape[0])          # physical slot of logical page i
    shuffled = torch.empty_like(pages)
    shuffled[torch.as_tensor(perm, device=pages.device)] = pages
    bt = torch.as_tensor(perm.reshape(x.shape[0], per_seq), dtype=torch.int32, device=x.device)
    return shuffled, bt


@pytest.mark.parametrize("page,B,T,seqlens,splits", [
    (16, 2, 300, None, 0), (16, 4, 300, [300, 17, 0, 64], 0), (32, 3, 1000, None, 3),
    (256, 2, 700, [700, 513], 1), (16, 1, 4096, None, 0)])
def test_attention_dense_paged(torch_cuda, page, B, T, seqlens, splits):
    # block_table path of flash_attn_with_kvcache (flash_fwd_kernel.h:1229-1239):
    # pages in a shuffled order give the contiguous cache's result bit for bit
    import zipserv_asplos26_amd.attention as za
    torch = torch_cuda
    rng = np.random.default_rng(page + B)
    Hkv, H, D = 8, 64, 128
    k = kv_bf16(rng, B, T, Hkv, D)
    v = kv_bf16(rng, B, T, Hkv, D)
    q = normal_bf16(rng, (B, H, D))
    kd, vd, qd = to_torch_bf16(k), to_torch_bf16(v), to_torch_bf16(q)
    kp, bt = _paged(torch, kd, page, rng)
    vp = torch.empty_like(kp)
    vp[bt.view(-1).long()] = za.make_batched_paged_kv_cache(vd, page)[0]
    sl = None if seqlens is None else torch.tensor(seqlens, dtype=torch.int32, device="cuda")
    cap = bt.shape[1] * page
    kc = torch.zeros(B, cap, Hkv, D, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    kc[:, :T], vc[:, :T] = kd, vd
    out, lse = za.flash_attn_with_kvcache_dense(qd.view(B, 1, H, D), kp, vp, cache_seqlens=sl,
                                                num_splits=splits, return_softmax_lse=True,
                                                block_table=bt)
    outc, lsec = za.flash_attn_with_kvcache_dense(qd.view(B, 1, H, D), kc, vc, cache_seqlens=sl,
                                                  num_splits=splits, return_softmax_lse=True)
    torch.cuda.synchronize()
    if seqlens is None:  # the contiguous cache runs to its capacity: compare on T tokens
        sl_np = [T] * B
        out, lse = za.flash_attn_with_kvcache_dense(
            qd.view(B, 1, H, D), kp, vp, cache_seqlens=T, num_splits=splits,
            return_softmax_lse=True, block_table=bt)
        outc, lsec = za.flash_attn_with_kvcache_dense(
            qd.view(B, 1, H, D), kc, vc, cache_seqlens=T, num_splits=splits,
            return_softmax_lse=True)
    else:
        sl_np = seqlens
    assert torch.equal(out.view(torch.int16), outc.view(torch.int16))
    o = from_torch_bf16(out.view(B, H, D))
    ref, ref_lse, absv = zo.decode_attention_f64(q, k, v, seqlens=sl_np, return_absv=True)
    _check((q, k, v, o, lse.cpu().numpy(), o, lse.cpu().numpy(), ref, ref_lse, absv), sl_np)


def test_attention_dense_paged_rejects(torch_cuda):
    import zipserv_asplos26_amd as zs
    torch = torch_cuda
    q = torch.zeros(1, 64, 128, dtype=torch.bfloat16, device="cuda")
    out = torch.empty_like(q)
    kp = torch.zeros(4, 16, 8, 128, dtype=torch.bfloat16, device="cuda")
    bt = torch.zeros(1, 4, dtype=torch.int32, device="cuda")
    L = zs.lib()

    def call(page=16, maxb=4, nblocks=4, T=64, table=bt):
        return L.zs_decode_attention_dense_paged(
            0, q.data_ptr(), kp.data_ptr(), kp.data_ptr(), 0 if table is None else table.data_ptr(),
            maxb, nblocks, page, None, T, 1, 64, 8, 128, 0.1, out.data_ptr(), None, None, 0, 1)
    assert call() == 0
    torch.cuda.synchronize()
    assert call(page=8) == zs._lib.ZS_E_UNSUPPORTED       # pages of whole medians only
    assert call(T=65) == zs._lib.ZS_E_INVAL               # table too short for seqlen_k
    assert call(table=None) == zs._lib.ZS_E_INVAL
    assert call(nblocks=0) == zs._lib.ZS_E_INVAL


@pytest.mark.parametrize("retiled", [False, True])
def test_compress_kv_paged_staged(torch_cuda, retiled):
    # layout "paged" (bench_zipserv_decode_attention.py:357-364,492-521): the
    # compressed token-major cache decompresses to the reference's dense pages
    # bit for bit, and attention over it (fused) equals the dense paged kernel
    import zipserv_asplos26_amd.attention as za
    torch = torch_cuda
    rng = np.random.default_rng(23)
    B, T, Hkv, H, D, page = 2, 300, 8, 64, 128, 16
    kd = to_torch_bf16(kv_bf16(rng, B, T, Hkv, D))
    vd = to_torch_bf16(kv_bf16(rng, B, T, Hkv, D))
    qd = to_torch_bf16(normal_bf16(rng, (B, H, D)))
    ck = za.compress_kv(kd, layout="paged", retiled=retiled, page_block_size=page)
    cv = za.compress_kv(vd, layout="paged", retiled=retiled, page_block_size=page)
    kp = za.decompress_to_batched_paged_kv(ck, B, Hkv, D, page)
    vp = za.decompress_to_batched_paged_kv(cv, B, Hkv, D, page)
    ref_pages, per_seq = za.make_batched_paged_kv_cache(kd, page)
    assert torch.equal(kp.view(torch.int16), ref_pages.view(torch.int16))
    bt = torch.arange(B * per_seq, dtype=torch.int32, device="cuda").view(B, per_seq)
    # five splits each: the same 64-token chunks although seqlen_k differs
    # (300 / 304), one wave per (batch, head, split) in every kernel (the
    # re-tiled cache runs fused, the canonical one staged)
    out = za.flash_attn_with_kvcache_zipserv(qd.view(B, 1, H, D), ck, cv, Hkv, T, num_splits=5)
    outp = za.flash_attn_with_kvcache_dense(qd.view(B, 1, H, D), kp, vp, cache_seqlens=T,
                                            block_table=bt, num_splits=5)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), outp.view(torch.int16))
