"""zs_retiled_mm_fused_noalloc (the ZipGEMM entry point that allocates
nothing: split-K partials and arrival counters in the library's static device
scratch) against zs_retiled_mm_fused with caller buffers, through the C-ABI:
bit-identical outputs on two calls in a row, the second with a smaller input,
for split-K 1, 2 and 4, and oversized requests refused with ZS_E_OVERFLOW
before any launch.  Named to be collected last: it must pass alone in a
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
