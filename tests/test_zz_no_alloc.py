"""zs_retiled_mm_fused_noalloc (the ZipGEMM entry point that allocates
nothing: split-K partials and arrival counters in the library's static device
scratch) against zs_retiled_mm_fused with caller buffers, through the C-ABI:
bit-identical outputs on two calls in a row, the second with a smaller input,
for split-K 1, 2 and 4, replays of a captured HIP graph bit-identical to the
eager result, and oversized or invalid requests refused before any launch.
Named to be collected last: it must pass alone in a
fresh process and after every other GPU test (scratch already in use)."""
import numpy as np
import pytest

import oracle as zo
import zipserv_asplos26_amd as zs
from zipserv_asplos26_amd import _lib
from zs_testutil import to_torch_bf16, weights_bf16

pytestmark = pytest.mark.gpu


def _noalloc():
    return zs.lib().zs_retiled_mm_fused_noalloc


def _call_noalloc(torch, r, x, split_k):
    out = torch.full((x.shape[0], r.rows), float("nan"), dtype=torch.bfloat16, device=x.device)
    st = int(torch.cuda.current_stream().cuda_stream)
    rc = _noalloc()(st, r.fixed.data_ptr(), r.exps.data_ptr(), r.eoff.data_ptr(),
                    r.start_exp & 0xFF, x.data_ptr(), out.data_ptr(), r.rows, x.shape[0],
                    r.cols, split_k)
    assert rc == _lib.ZS_OK, rc
    return out


def _call_fused(torch, r, x, split_k):
    n = x.shape[0]
    out = torch.empty((n, r.rows), dtype=torch.bfloat16, device=x.device)
    ws = torch.empty(max(split_k * n * r.rows, 1), dtype=torch.bfloat16, device=x.device)
    cnt = torch.zeros(int(zs.lib().zs_retiled_mm_counters(r.rows, n)), dtype=torch.int32,
                      device=x.device)
    st = int(torch.cuda.current_stream().cuda_stream)
    rc = zs.lib().zs_retiled_mm_fused(st, r.fixed.data_ptr(), r.exps.data_ptr(),
                                      r.eoff.data_ptr(), r.start_exp & 0xFF, x.data_ptr(),
                                      out.data_ptr(), r.rows, n, r.cols, ws.data_ptr(), split_k,
                                      cnt.data_ptr())
    assert rc == _lib.ZS_OK, rc
    return out


@pytest.mark.parametrize("split_k", [1, 2, 4])
def test_noalloc_equals_fused_on_two_calls(torch_cuda, split_k):
    torch = torch_cuda
    rng = np.random.default_rng(70 + split_k)
    cases = [((2048, 4096), 40), ((512, 1024), 7)]  # second call: smaller input
    for (M, K), N in cases:
        print(f"noalloc split_k={split_k} M={M} K={K} N={N}", flush=True)
        W = weights_bf16(rng, (M, K), outlier_frac=0.01)
        X = zo.f32_to_bf16(rng.standard_normal((N, K), dtype=np.float32))
        r = zs.compress_retiled(to_torch_bf16(W), window="weights")
        x = to_torch_bf16(X)
        got = _call_noalloc(torch, r, x, split_k)
        want = _call_fused(torch, r, x, split_k)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        ref = zo.gemm_f32(W, X)
        y = got.float().cpu().numpy()
        assert np.abs(y - ref).max() / np.abs(ref).max() <= 1e-2


def test_noalloc_refuses_oversized_requests(torch_cuda):
    torch = torch_cuda
    cap = 16 << 20  # bf16 partials the 32 MiB scratch holds
    M, K = 4096, 128
    N = cap // (2 * M) + 16  # 2 * M * N partials exceed the scratch at split-K 2
    r = zs.compress_retiled(to_torch_bf16(np.zeros((M, K), np.uint16)), window="weights")
    x = torch.zeros((N, K), dtype=torch.bfloat16, device="cuda")
    out = torch.empty((N, M), dtype=torch.bfloat16, device="cuda")
    st = int(torch.cuda.current_stream().cuda_stream)
    rc = _noalloc()(st, r.fixed.data_ptr(), r.exps.data_ptr(), r.eoff.data_ptr(), r.start_exp,
                    x.data_ptr(), out.data_ptr(), M, N, K, 2)
    assert rc == _lib.ZS_E_OVERFLOW


def test_noalloc_under_graph_capture(torch_cuda):
    # Callers that cannot allocate include code under HIP graph capture: one
    # eager call, then split-K 2 and 4 calls captured in one graph, replayed
    # several times with eager work and synchronisation between the replays,
    # every replay bit-identical to zs_retiled_mm_fused with caller buffers.
    torch = torch_cuda
    rng = np.random.default_rng(91)
    M, K, N = 1024, 2048, 24
    W = weights_bf16(rng, (M, K), outlier_frac=0.01)
    r = zs.compress_retiled(to_torch_bf16(W), window="weights")
    x = to_torch_bf16(zo.f32_to_bf16(rng.standard_normal((N, K), dtype=np.float32)))
    _call_noalloc(torch, r, x, 2)
    want = {sk: _call_fused(torch, r, x, sk) for sk in (2, 4)}
    torch.cuda.synchronize()
    outs = {sk: torch.empty((N, M), dtype=torch.bfloat16, device="cuda") for sk in (2, 4)}
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for sk in (2, 4):
                rc = _noalloc()(int(s.cuda_stream), r.fixed.data_ptr(), r.exps.data_ptr(),
                                r.eoff.data_ptr(), r.start_exp & 0xFF, x.data_ptr(),
                                outs[sk].data_ptr(), M, N, K, sk)
                assert rc == _lib.ZS_OK, rc
    torch.cuda.synchronize()
    for rep in range(3):
        print(f"noalloc graph replay {rep}", flush=True)
        for o in outs.values():
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for sk in (2, 4):
            assert torch.equal(outs[sk].view(torch.int16), want[sk].view(torch.int16)), (rep, sk)
        _call_noalloc(torch, r, x[:8], 2)  # eager work on the same scratch between replays
        torch.cuda.synchronize()


def test_noalloc_rejects_bad_arguments(torch_cuda):
    torch = torch_cuda
    r = zs.compress_retiled(to_torch_bf16(np.zeros((64, 128), np.uint16)), window="weights")
    x = torch.zeros((4, 128), dtype=torch.bfloat16, device="cuda")
    out = torch.empty((4, 64), dtype=torch.bfloat16, device="cuda")
    st = int(torch.cuda.current_stream().cuda_stream)
    args = [st, r.fixed.data_ptr(), r.exps.data_ptr(), r.eoff.data_ptr(), r.start_exp,
            x.data_ptr(), out.data_ptr(), 64, 4, 128, 2]
    bad_out = list(args)
    bad_out[6] = 0
    assert _noalloc()(*bad_out) == _lib.ZS_E_INVAL
    bad_k = list(args)
    bad_k[9] = 100  # K not a multiple of 64
    assert _noalloc()(*bad_k) == _lib.ZS_E_INVAL
    bad_split = list(args)
    bad_split[10] = 3  # more slices than K tiles (2)
    assert _noalloc()(*bad_split) == _lib.ZS_E_INVAL
    assert _noalloc()(*args) == _lib.ZS_OK
    torch.cuda.synchronize()
