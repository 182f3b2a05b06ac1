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
of an fp32 reference on sampled batch entries.
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


def test_retiled_kv_and_attention_past_int32(torch_cuda):
    import zipserv_asplos26_amd.attention as za
    torch = torch_cuda
    B, T, Hkv, H, D = 64, 33000, 8, 64, 128
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    k = _kv(torch, g, B, T)
    mat, _, _ = za.pad_batched_kv_prefix_by_kv_head(k)
    assert mat.numel() > 2**31 - 1
    rk = za.compress_kv(k, retiled=True)
    back = zs.decompress_retiled(rk)
    assert torch.equal(back.view(torch.int16), mat.view(torch.int16))  # bit-exact round trip
    del back, mat
    with pytest.raises(zs.ZipServError):  # canonical streams: int32 offsets
        za.compress_kv(k)
    v = _kv(torch, g, B, T)
    rv = za.compress_kv(v, retiled=True)
    q = torch.randn(B, 1, H, D, device="cuda", generator=g).to(torch.bfloat16)
    out = za.flash_attn_with_kvcache_zipserv(q, rk, rv, Hkv, T)
    outd = za.flash_attn_with_kvcache_dense(q, k, v)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), outd.view(torch.int16))
    # fp32 reference for sampled sequences (matmul on contiguous fp32 operands)
    G = H // Hkv
    for b in (0, 37, B - 1):
        kb = k[b].float().permute(1, 2, 0).contiguous()          # [Hkv, D, T]
        vb = v[b].float().permute(1, 0, 2).contiguous()          # [Hkv, T, D]
        qb = q[b, 0].float().view(Hkv, G, D)
        p = torch.softmax(torch.matmul(qb, kb) / math.sqrt(D), dim=-1)
        ref = torch.matmul(p, vb).view(H, D)
        o = out[b, 0].float()
        tol = 2e-3 + ref.abs() * 2.0 ** -7 + vb.abs().max() * 2.0 ** -9
        assert bool(((o - ref).abs() <= tol).all()), float((o - ref).abs().max())


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
