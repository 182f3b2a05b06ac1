"""Tensors past 2^31 elements on the GPU.

The reference's GPU analyze counts exponents in int32 bins
(kernel_benchmark/zipserv_decode_attention_ext.cu:35-63) and its canonical
format holds int32 stream offsets (L_API.cu:357, ext.cu:184), so a
64 x 8 x 32k x 128 KV tensor (2^31 elements) is out of its reach.  The
64-bit-bin analyze and the re-tiled layout take it: checked here with a
histogram whose largest bin itself exceeds INT32_MAX, a bit-exact
compress -> decompress round trip of a 2.16 G-element KV cache, and decode
attention over that cache, bit-identical to the same kernel over the dense
cache and within 2e-3 (plus the bf16 rounding terms of test_gpu_attention)
of an fp32 reference on sampled batch entries, lse included.  The same at
benchmark config 4's largest cache (B = 32, T = 128k: 2^32 elements per
tensor, a fixed part past 4 GiB), and config-5 points (B = 8, T = 16k;
B = 32, T = 32k) against the fp64 oracle on sampled batch entries.  The
token-major layout's fused attention runs on the 2.16 G-element caches and
the config-5 points too: bit-identical to the dense kernel where both walk
the same chunks with one wave per (batch, head, split), and within the
oracle bound with its own automatic splits.
"""
import math

import numpy as np
import pytest

import oracle as zo
import zipserv_asplos26_amd as zs

pytestmark = pytest.mark.gpu

ZS_E_OVERFLOW = -3


def _exponent_counts(torch, x):
    """Exact int64 exponent histogram of a bf16 tensor, in chunks."""
    counts = torch.zeros(256, dtype=torch.int64, device=x.device)
    for part in x.reshape(-1).split(1 << 28):
        e = (part.view(torch.int16).to(torch.int32) >> 7) & 0xFF
        counts += torch.bincount(e, minlength=256)
    return counts


def test_analyze_u64_bins_past_int32(torch_cuda):
    torch = torch_cuda
    n = (1 << 31) + (1 << 23)
    x = torch.full((n,), 1.0, dtype=torch.bfloat16, device="cuda")  # exponent 127
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    x[: 1 << 22] = (torch.randn(1 << 22, device="cuda", generator=g) * 8).to(torch.bfloat16)
    expect = _exponent_counts(torch, x)
    assert int(expect[127]) > 2**31 - 1  # this bin overflows int32 counters
    st = int(torch.cuda.current_stream().cuda_stream)
    counts = torch.empty(256, dtype=torch.int64, device="cuda")
    top = torch.empty(7, dtype=torch.int32, device="cuda")
    rc = zs.lib().zs_analyze_top_exponents_u64_gpu(st, x.data_ptr(), n, counts.data_ptr(),
                                                  top.data_ptr())
    assert rc == 0
    c = counts.cpu().numpy()
    np.testing.assert_array_equal(c, expect.cpu().numpy())
    assert top.cpu().tolist() == zo.select_gpu(c)
    # the reference-shaped int32 entry point refuses this size up front
    c32 = torch.empty(256, dtype=torch.int32, device="cuda")
    assert zs.lib().zs_analyze_top_exponents_gpu(st, x.data_ptr(), n, c32.data_ptr(),
                                                 top.data_ptr(), None) == ZS_E_OVERFLOW


def _kv(torch, g, B, T, Hkv=8, D=128):
    scale = torch.exp(torch.randn(1, 1, Hkv, D, device="cuda", generator=g))
    return (torch.randn(B, T, Hkv, D, device="cuda", generator=g) * scale).to(torch.bfloat16)


def _fp32_reference(torch, q, k, v, b):
    """fp32 decode attention of batch entry b (matmuls on contiguous fp32
    operands): output [H, D], the natural-log lse [H] and absv [H, D] =
    sum_t p_t |v_t| (the scale of the bf16 rounding of the weights)."""
    Hkv, D = k.shape[2], k.shape[3]
    H = q.shape[2]
    G = H // Hkv
    kb = k[b].float().permute(1, 2, 0).contiguous()          # [Hkv, D, T]
    vb = v[b].float().permute(1, 0, 2).contiguous()          # [Hkv, T, D]
    qb = q[b, 0].float().view(Hkv, G, D)
    s = torch.matmul(qb, kb) / math.sqrt(D)                  # [Hkv, G, T]
    lse = torch.logsumexp(s, dim=-1).view(H)
    p = torch.softmax(s, dim=-1)
    ref = torch.matmul(p, vb).view(H, D)
    absv = torch.matmul(p, vb.abs()).view(H, D)
    return ref, lse, absv


def _check_sampled(torch, q, k, v, out, lse, batches):
    for b in batches:
        ref, ref_lse, absv = _fp32_reference(torch, q, k, v, b)
        o = out[b, 0].float()
        tol = 2e-3 + 2.0 ** -8 * ref.abs() + 2.0 ** -8 * absv  # zs_testutil.attention_tolerance
        assert bool(((o - ref).abs() <= tol).all()), (b, float((o - ref).abs().max()))
        assert bool(((lse[b] - ref_lse).abs() <= 1e-3 + 1e-4 * ref_lse.abs()).all()), b


def _large_kv_case(torch, B, T, seed, check_canonical_refused):
    import zipserv_asplos26_amd.attention as za
    Hkv, H, D = 8, 64, 128
    print(f"large KV case B={B} T={T}", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    k = _kv(torch, g, B, T)
    mat, _, _ = za.pad_batched_kv_prefix_by_kv_head(k)
    assert mat.numel() > 2**31 - 1
    rk = za.compress_kv(k, retiled=True)
    back = zs.decompress_retiled(rk)
    assert torch.equal(back.view(torch.int16), mat.view(torch.int16))  # bit-exact round trip
    del back, mat
    if check_canonical_refused:
        with pytest.raises(zs.ZipServError):  # canonical streams: int32 offsets
            za.compress_kv(k)
    v = _kv(torch, g, B, T)
    rv = za.compress_kv(v, retiled=True)
    q = torch.randn(B, 1, H, D, device="cuda", generator=g).to(torch.bfloat16)
    out, lse = za.flash_attn_with_kvcache_zipserv(q, rk, rv, Hkv, T, return_softmax_lse=True)
    outd, lsed = za.flash_attn_with_kvcache_dense(q, k, v, return_softmax_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), outd.view(torch.int16))
    assert torch.equal(lse, lsed)
    return q, k, v, rk, out, lse


def test_retiled_kv_and_attention_past_int32(torch_cuda):
    torch = torch_cuda
    B = 64
    q, k, v, _, out, lse = _large_kv_case(torch, B, 33000, 11, True)
    _check_sampled(torch, q, k, v, out, lse, (0, 37, B - 1))
    # the same caches token-major (fused attention): 4 splits give both the
    # fused and the dense kernel 8256-token chunks and 2048 (batch, head,
    # split) items of one wave each, so the outputs are the same bit for bit
    import zipserv_asplos26_amd.attention as za
    del out, lse
    tk = za.compress_kv(k, layout="token_major", retiled=True)
    tv = za.compress_kv(v, layout="token_major", retiled=True)
    outt, lset = za.flash_attn_with_kvcache_zipserv(q, tk, tv, 8, 33000, num_splits=4,
                                                    return_softmax_lse=True)
    outd, lsed = za.flash_attn_with_kvcache_dense(q, k, v, num_splits=4, return_softmax_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(outt.view(torch.int16), outd.view(torch.int16))
    assert torch.equal(lset, lsed)
    _check_sampled(torch, q, k, v, outt, lset, (0, B - 1))


def test_retiled_kv_past_4g_elements(torch_cuda):
    # Benchmark config 4's largest cache: B = 32, T = 128k, 8 KV heads,
    # head_dim 128 = 2^32 elements per K / V tensor (8 GiB bf16); its fixed
    # part (5.6 GiB) is past the 32-bit range of a buffer resource, so the
    # attention kernel's per-wave resources must saturate, not wrap.
    torch = torch_cuda
    B, T = 32, 131072
    q, k, v, rk, out, lse = _large_kv_case(torch, B, T, 17, False)
    assert rk.rows * rk.cols == 1 << 32
    assert rk.fixed.numel() > (1 << 32)
    _check_sampled(torch, q, k, v, out, lse, (0, 13, B - 1))


@pytest.mark.parametrize("B,T", [(8, 16384), (32, 32768)])
def test_attention_config5_points_against_oracle(torch_cuda, B, T):
    # benchmark config 5 points on the re-tiled layout, sampled batch entries
    # against the fp64 oracle with the per-element bound of test_gpu_attention
    import zipserv_asplos26_amd.attention as za
    from zs_testutil import attention_tolerance, from_torch_bf16
    torch = torch_cuda
    Hkv, H, D = 8, 64, 128
    print(f"config-5 point B={B} T={T}", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(B * 7 + T)
    k, v = _kv(torch, g, B, T), _kv(torch, g, B, T)
    q = torch.randn(B, 1, H, D, device="cuda", generator=g).to(torch.bfloat16)
    rk, rv = za.compress_kv(k, retiled=True), za.compress_kv(v, retiled=True)
    out, lse = za.flash_attn_with_kvcache_zipserv(q, rk, rv, Hkv, T, return_softmax_lse=True)
    outd = za.flash_attn_with_kvcache_dense(q, k, v)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), outd.view(torch.int16))
    # token-major caches, fused: automatic splits against the oracle, and with
    # T / 512 splits (>= 2048 one-wave items, equal chunks) against dense
    tk = za.compress_kv(k, layout="token_major", retiled=True)
    tv = za.compress_kv(v, layout="token_major", retiled=True)
    outt, lset = za.flash_attn_with_kvcache_zipserv(q, tk, tv, Hkv, T, return_softmax_lse=True)
    oute = za.flash_attn_with_kvcache_zipserv(q, tk, tv, Hkv, T, num_splits=T // 512)
    outde = za.flash_attn_with_kvcache_dense(q, k, v, num_splits=T // 512)
    torch.cuda.synchronize()
    assert torch.equal(oute.view(torch.int16), outde.view(torch.int16))
    for b in (0, B - 1):
        qb = from_torch_bf16(q[b:b + 1, 0])
        kb, vb = from_torch_bf16(k[b:b + 1]), from_torch_bf16(v[b:b + 1])
        ref, ref_lse, absv = zo.decode_attention_f64(qb, kb, vb, return_absv=True)
        for o_, l_ in ((out, lse), (outt, lset)):
            o = zo.bf16_to_f32(from_torch_bf16(o_[b:b + 1, 0])).astype(np.float64)
            err = np.abs(o - ref)
            assert np.all(err <= attention_tolerance(ref, absv)), (b, err.max())
            np.testing.assert_allclose(l_[b:b + 1].cpu().numpy(), ref_lse, rtol=1e-4, atol=1e-3)


def test_retiled_zipgemm_x_past_2gib(torch_cuda):
    # X of more than 2^31 bytes: zs_retiled_mm runs it as row blocks (its
    # kernels address X with 32-bit offsets); every row block must match
    import zipserv_asplos26_amd as zs_
    torch = torch_cuda
    M, K, N = 64, 4096, (1 << 18) + 48
    assert N * K * 2 > 2**31 - 1
    g = torch.Generator(device="cuda")
    g.manual_seed(13)
    w = (torch.randn(M, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(N, K, device="cuda", generator=g).to(torch.bfloat16)
    r = zs_.compress_retiled(w)
    y = zs_.zipgemm(r, x)
    ref = torch.empty(N, M, dtype=torch.float32, device="cuda")
    wf = w.float().t().contiguous()
    for n0 in range(0, N, 1 << 16):
        ref[n0:n0 + (1 << 16)] = x[n0:n0 + (1 << 16)].float() @ wf
    torch.cuda.synchronize()
    err = float((y.float() - ref).abs().max() / ref.abs().max())
    assert err < 1e-2, err


@pytest.mark.parametrize("split_k", [1, 2])
def test_canonical_zipgemm_x_past_2gib(torch_cuda, split_k):
    # The drop-in entry point addresses X with 64-bit pointers: one launch
    # over X of more than 2^31 bytes, in the 16-row kernel (one slice) and
    # the 64-row kernel (split-K), both against an fp32 product
    import zipserv_asplos26_amd as zs_
    torch = torch_cuda
    M, K, N = 64, 4096, (1 << 18) + 48
    assert N * K * 2 > 2**31 - 1
    g = torch.Generator(device="cuda")
    g.manual_seed(17 + split_k)
    w = (torch.randn(M, K, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(N, K, device="cuda", generator=g).to(torch.bfloat16)
    c = zs_.compress(w, window="weights")
    y = zs_.zipgemm(c, x, split_k=split_k)
    ref = torch.empty(N, M, dtype=torch.float32, device="cuda")
    wf = w.float().t().contiguous()
    for n0 in range(0, N, 1 << 16):
        ref[n0:n0 + (1 << 16)] = x[n0:n0 + (1 << 16)].float() @ wf
    torch.cuda.synchronize()
    err = float((y.float() - ref).abs().max() / ref.abs().max())
    assert err < 1e-2, err
