"""Stream-K schedule of the re-tiled ZipGEMM (zs_retiled_mm_streamk, N <= 16).

One round of workgroups over equal record ranges; bands that a range
boundary cuts are added from fp32 partials across workgroups, segments within
a workgroup from its waves' LDS slots.  Checked against the split-K 1 kernel
of the same re-tiled matrix up to fp32 summation order (per element: one bf16
rounding of each result plus twice the fp32 summation bound of the exact
products, the bound of test_gpu_retiled.assert_same_sum_up_to_order), against
the fp32 oracle product, with unit-vector rows of X exactly (every K tile of
every band probed), deterministic over repeated calls and HIP graph replays
(the band counters return to zero), and shapes it does not take refused
(C-ABI) or run as split-K 1 (Python).

Shapes cover one record per workgroup (R <= the grid), bands shared by up
to 16 workgroups, K tiles fewer than the 8 waves, ranges meeting 2-4
bands, and every X path (N = 1..2, 3..4, 5..8 staged, 9..16 direct).
"""
import numpy as np
import pytest

import oracle as zo
import zipserv_asplos26_amd as zs
from zs_testutil import (from_torch_bf16, probe_batches, probe_columns, probe_mismatches,
                         to_torch_bf16, weights_bf16)

pytestmark = pytest.mark.gpu


def _same_sum_up_to_order(a, b, W, X):
    K = W.shape[1]
    s = zo.gemm_f32(W & 0x7FFF, X & 0x7FFF)
    bound = 2.0 ** -8 * (np.abs(a) + np.abs(b)) + 2.0 * K * 2.0 ** -24 * s
    assert np.all(np.abs(a - b) <= bound), float(np.max(np.abs(a - b) - bound))


CASES = [(64, 64, 1), (256, 512, 5), (1024, 1024, 16), (4096, 4096, 1), (1024, 4096, 3),
         (640, 8192, 8), (4096, 448, 12), (2048, 2048, 2)]


@pytest.mark.parametrize("M,K,N", CASES)
def test_streamk_matches_split1_and_oracle(torch_cuda, M, K, N):
    torch = torch_cuda
    print(f"stream-K M={M} K={K} N={N}", flush=True)
    rng = np.random.default_rng(M + 3 * K + N)
    W = weights_bf16(rng, (M, K), outlier_frac=0.01)
    X = zo.f32_to_bf16(rng.standard_normal((N, K), dtype=np.float32))
    r = zs.compress_retiled(to_torch_bf16(W), window="weights")
    x = to_torch_bf16(X)
    assert int(zs.lib().zs_retiled_mm_streamk_workspace_bytes(M, N, K)) > 0
    ys = [zs.zipgemm(r, x, split_k=0) for _ in range(3)]
    y1 = zs.zipgemm(r, x, split_k=1)
    torch.cuda.synchronize()
    for y in ys[1:]:  # deterministic, counters back at zero between calls
        assert torch.equal(y.view(torch.int16), ys[0].view(torch.int16))
    cnt = zs.codec.splitk_counters(M, N, x.device)
    assert int(cnt.abs().sum()) == 0
    a = zo.bf16_to_f32(from_torch_bf16(ys[0]))
    b = zo.bf16_to_f32(from_torch_bf16(y1))
    _same_sum_up_to_order(a, b, W, X)
    ref = zo.gemm_f32(W, X)
    assert np.abs(a - ref).max() / np.abs(ref).max() <= 1e-2


@pytest.mark.parametrize("M,K", [(256, 512), (4096, 4096), (1024, 448)])
@pytest.mark.parametrize("N", [1, 4, 8, 16])
def test_streamk_unit_vectors_exact(torch_cuda, M, K, N):
    torch = torch_cuda
    rng = np.random.default_rng(7 * M + K + N)
    W = weights_bf16(rng, (M, K), outlier_frac=0.02)
    w = to_torch_bf16(W)
    r = zs.compress_retiled(w, window="weights")
    cols = probe_columns(K, 1)
    flat = [k for bb in probe_batches(cols, N) for k in bb]
    X = np.zeros((len(flat), K), np.uint16)
    X[np.arange(len(flat)), flat] = 0x3F80
    x = to_torch_bf16(X)
    Y = torch.full((len(flat), M), float("nan"), dtype=torch.bfloat16, device="cuda")
    for j in range(0, len(flat), N):
        zs.zipgemm(r, x[j:j + N], split_k=0, out=Y[j:j + N])
    torch.cuda.synchronize()
    want = zo.bf16_to_f32(W[:, flat].T.copy())
    assert probe_mismatches(zo.bf16_to_f32(from_torch_bf16(Y)), want) == 0


def test_streamk_graph_replays(torch_cuda):
    torch = torch_cuda
    rng = np.random.default_rng(61)
    M, K, N = 1024, 2048, 6
    W = weights_bf16(rng, (M, K), outlier_frac=0.01)
    r = zs.compress_retiled(to_torch_bf16(W), window="weights")
    x = to_torch_bf16(zo.f32_to_bf16(rng.standard_normal((N, K), dtype=np.float32)))
    want = zs.zipgemm(r, x, split_k=0)
    out = torch.empty_like(want)
    ws = zs.codec.splitk_workspace(r, N, 0)
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        zs.zipgemm(r, x, split_k=0, out=out, workspace=ws)  # counters of this stream
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            zs.zipgemm(r, x, split_k=0, out=out, workspace=ws)
    torch.cuda.synchronize()
    for rep in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), want.view(torch.int16)), rep
        zs.zipgemm(r, x, split_k=0)  # eager work between the replays
        torch.cuda.synchronize()


def test_streamk_refuses_what_it_does_not_take(torch_cuda):
    torch = torch_cuda
    L = zs.lib()
    rng = np.random.default_rng(3)
    # 8192 bands of one K tile: a range of ~11 records meets ~11 bands (> 8 slots)
    M, K = 16 * 8192, 64
    W = weights_bf16(rng, (M, K))
    r = zs.compress_retiled(to_torch_bf16(W), window="weights")
    assert int(L.zs_retiled_mm_streamk_workspace_bytes(M, 1, K)) == 0
    x = to_torch_bf16(zo.f32_to_bf16(rng.standard_normal((2, K), dtype=np.float32)))
    y = torch.empty(2, M, dtype=torch.bfloat16, device="cuda")
    cnt = torch.zeros(M // 16, dtype=torch.int32, device="cuda")
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda")
    st = int(torch.cuda.current_stream().cuda_stream)

    def call(n=2, ws_bytes=ws.numel(), counters=cnt.data_ptr(), mm=M, kk=K):
        return L.zs_retiled_mm_streamk(st, r.fixed.data_ptr(), r.exps.data_ptr(),
                                       r.eoff.data_ptr(), r.start_exp, x.data_ptr(),
                                       y.data_ptr(), mm, n, kk, ws.data_ptr(), ws_bytes, counters)
    assert call() == zs._lib.ZS_E_UNSUPPORTED
    assert call(n=17) == zs._lib.ZS_E_UNSUPPORTED
    assert call(kk=96) == zs._lib.ZS_E_INVAL
    # Python runs such shapes as split-K 1
    yp = zs.zipgemm(r, x, split_k=0)
    y1 = zs.zipgemm(r, x, split_k=1)
    torch.cuda.synchronize()
    assert torch.equal(yp.view(torch.int16), y1.view(torch.int16))
    # a shape it takes, with too small a workspace or no counters
    M2, K2 = 1024, 1024
    r2 = zs.compress_retiled(to_torch_bf16(weights_bf16(rng, (M2, K2))), window="weights")
    need = int(L.zs_retiled_mm_streamk_workspace_bytes(M2, 2, K2))
    assert need > 0
    x2 = torch.zeros(2, K2, dtype=torch.bfloat16, device="cuda")
    y2 = torch.empty(2, M2, dtype=torch.bfloat16, device="cuda")

    def call2(ws_bytes, counters):
        return L.zs_retiled_mm_streamk(st, r2.fixed.data_ptr(), r2.exps.data_ptr(),
                                       r2.eoff.data_ptr(), r2.start_exp, x2.data_ptr(),
                                       y2.data_ptr(), M2, 2, K2, ws.data_ptr(), ws_bytes, counters)
    assert call2(need - 1, cnt.data_ptr()) == zs._lib.ZS_E_INVAL
    assert call2(need, None) == zs._lib.ZS_E_INVAL
    assert call2(need, cnt.data_ptr()) == zs._lib.ZS_OK
    torch.cuda.synchronize()
