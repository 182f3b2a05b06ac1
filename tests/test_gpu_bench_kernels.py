"""bench.py labels every timed launch with the kernel the library dispatches
for its (M, N, K, split-K) (`bench.kernel_name`, a mirror of the dispatch in
zs_retiled_mm).  Here the kernel that actually ran, as the HIP profiler
records it, must carry that name, over one case of every dispatch branch."""
import pytest

import zipserv_asplos26_amd as zs

pytestmark = pytest.mark.gpu

# (M, K, N, split_k): N = 1 on 640 / 896 bands (8 / 4 waves), N = 8 and 16 on
# the 16-row kernels and the 64-row one-column-block kernel, N = 24 / 32 /
# 64 / 128 with 4 and 2 K phases, three-phase NB = 8, the two-band kernels
# at NB = 2 / 4 / 8, and the stream-K schedule
CASES = [(10240, 1024, 1, 1), (14336, 1024, 1, 1), (4096, 1024, 8, 1), (14336, 1024, 8, 1),
         (6144, 1024, 16, 1), (4096, 1024, 16, 1), (4096, 1024, 32, 1), (14336, 1024, 32, 2),
         (28672, 1024, 32, 1), (28672, 1024, 24, 4), (10240, 1024, 32, 2),
         (4096, 1024, 64, 4), (28672, 1024, 64, 1), (8192, 1024, 48, 4), (14336, 1024, 64, 2), (6144, 4096, 128, 1), (6144, 1024, 128, 1), (6144, 4096, 128, 2),
         (4096, 4096, 128, 4),
         (28672, 1024, 128, 1), (4096, 1024, 8, 0)]


@pytest.mark.parametrize("M,K,N,split_k", CASES)
def test_bench_kernel_name_is_the_dispatched_kernel(torch_cuda, M, K, N, split_k):
    import torch
    from torch.profiler import ProfilerActivity, profile

    import bench

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(M + N)
    w = (torch.randn(M, K, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    r = zs.compress_retiled(w, window="weights")
    x = torch.randn(N, K, device=dev, generator=g).to(torch.bfloat16)
    ws = zs.codec.splitk_workspace(r, N, split_k)
    zs.zipgemm(r, x, split_k=split_k, workspace=ws)
    torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        zs.zipgemm(r, x, split_k=split_k, workspace=ws)
        torch.cuda.synchronize()
    ran = sorted({e.name for e in prof.events() if "rgemm" in e.name})
    want = bench.kernel_name(N, M, split_k, K)
    print(f"M={M} K={K} N={N} split_k={split_k}: want {want}, ran {ran}", flush=True)
    assert any(n.split("(")[0].replace("void ", "") == want for n in ran), (want, ran)
