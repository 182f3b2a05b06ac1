"""GPU parity at the benchmark's real GEMM shapes (benchmark configs 1-3).

Reference checks this mirrors: test_mm.cu:861-936 (every element of the
benchmark shapes against a reference GEMM) and test_decompress.cu:174-242
(full-size bit compare of decompress).

* C1: the seed-0 4096x4096 N(0, 0.02) matrix compressed on the GPU under the
  weights-path window (kernel_benchmark/utils.h:189-272) reproduces the
  committed SHA-256 digests of every stream (canonical and re-tiled, written
  by the CPU oracle, tests/golden/make_golden.py); both layouts decompress
  bit-exactly; ZipGEMM at N = 8 is within 1e-2 of the fp32 oracle GEMM on
  every element, split-K 1/2/4.
* C2: the five Llama-3-8B projections (0.1% x30 outliers) at N in
  {1, 8, 16, 32, 64, 128} x split-K {1, 2, 4}, in-kernel and two-kernel
  split-K reduction (bit-identical to each other).
* C3: one Llama-3.1-70B layer at N in {1, 8, 16, 32, 64, 128, 256} x
  split-K {1, 2, 4}.
* Waves that own more than 64 K tiles (the narrow kernel's outlier-offset
  chunk reload): 10240 x 20480 at N = 8 (4-wave workgroups) and 1024 x 36864
  at N = 1 (8-wave workgroups).

Every shape: decompress bit-exact against the original bf16 matrix.  ZipGEMM
error = max |Y - ref| / max |ref| <= 1e-2 on 512
sampled rows of W (first and last band included) against the CPU oracle
zso_gemm_f32_mt, and on every element against an fp32 GEMM of the same bf16
operands on the GPU.  Batches of one shape are the first N rows of one X, so
one oracle GEMM per shape serves every N.

That normwise bound cannot see one wrong weight (an exponent off by one moves
Y by less than the tolerance at these sizes), so every C2 and C3 shape is
also probed exactly (test_*_exact_probes): rows of X are unit vectors e_k
(tests/zs_testutil.py probe_columns: one k in every K tile, the first and
last column of every split-K slice), and every probed output column must
equal the bf16 weight column W[:, k] bit for bit (as values: +0 == -0), for
the re-tiled and the canonical (drop-in) kernels at every N and split-K
{1, 2, 4} -- the mirror of test_mm.cu:861-936's full compare, made exact.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as zo
import zipserv_asplos26_amd as zs
from zs_testutil import (from_torch_bf16, probe_batches, probe_columns, probe_mismatches,
                         to_torch_bf16)

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
TOL = 1e-2
C2_SHAPES = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate", 14336, 4096),
             ("up", 14336, 4096), ("down", 4096, 14336)]
C2_NS = [1, 8, 16, 32, 64, 128]
C3_SHAPES = [("qkv", 10240, 8192), ("o", 8192, 8192), ("gate", 28672, 8192),
             ("up", 28672, 8192), ("down", 8192, 28672)]
C3_NS = [1, 8, 16, 32, 64, 128, 256]
SPLITS = [1, 2, 4]
SAMPLE_ROWS = 512


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _weights(torch, M, K, seed, outliers):
    """W ~ N(0, 0.02) bf16 on the GPU, 0.1% of entries x30 when `outliers`."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    w = torch.randn(M, K, device="cuda", generator=g) * 0.02
    if outliers:
        mask = torch.rand(M, K, device="cuda", generator=g) < 0.001
        w = torch.where(mask, w * 30.0, w)
    return w.to(torch.bfloat16)


class Case:
    """One weight matrix on the GPU (dense and re-tiled), the sampled rows of W
    on the host, a batch X of the largest N and the oracle over those rows."""

    def __init__(self, torch, M, K, nmax, seed, outliers):
        print(f"case M={M} K={K} nmax={nmax} seed={seed}", flush=True)
        self.M, self.K = M, K
        self.w = _weights(torch, M, K, seed, outliers)
        self.r = zs.compress_retiled(self.w, window="weights")
        rng = np.random.default_rng(seed)
        X = zo.f32_to_bf16(rng.standard_normal((nmax, K), dtype=np.float32))
        self.x = to_torch_bf16(X)
        rows = np.concatenate([np.arange(16), np.arange(M - 16, M),
                               rng.choice(np.arange(16, M - 16), SAMPLE_ROWS - 32, replace=False)])
        self.rows = np.sort(rows)
        Ws = from_torch_bf16(self.w[torch.from_numpy(self.rows).cuda()])
        self.ref = zo.gemm_f32_mt(Ws, X)                      # [nmax, 512] fp32
        self.dense = self.w.float().t().contiguous()          # [K, M] fp32 for the GPU check
        torch.cuda.synchronize()

    def check(self, torch, y, n, what):
        """Sampled rows against the oracle, every element against fp32 on the GPU."""
        ys = zo.bf16_to_f32(from_torch_bf16(y[:, torch.from_numpy(self.rows).cuda()]))
        ref = self.ref[:n]
        err = np.abs(ys - ref).max() / max(np.abs(ref).max(), 1e-30)
        assert err <= TOL, f"{what}: oracle rows error {err}"
        full = self.x[:n].float() @ self.dense
        errf = float((y.float() - full).abs().max() / full.abs().max())
        assert errf <= TOL, f"{what}: full-matrix error {errf}"


_CACHE = {}


def _case(torch, key, M, K, nmax, seed, outliers):
    if key not in _CACHE:
        _CACHE.clear()  # one resident case at a time keeps memory bounded
        _CACHE[key] = Case(torch, M, K, nmax, seed, outliers)
    return _CACHE[key]


def _run_all_splits(torch, c, n, what):
    x = c.x[:n]
    if n <= 16:  # stream-K schedule (fp32 partials)
        c.check(torch, zs.zipgemm(c.r, x, split_k=0), n, f"{what} stream-K")
    for sk in SPLITS:
        yf = zs.zipgemm(c.r, x, split_k=sk)                   # in-kernel split-K sum
        c.check(torch, yf, n, f"{what} split_k={sk}")
        if sk > 1:
            y2 = zs.zipgemm(c.r, x, split_k=sk, fused=False)  # two-kernel reduction
            torch.cuda.synchronize()
            assert torch.equal(yf.view(torch.int16), y2.view(torch.int16)), \
                f"{what} split_k={sk}: in-kernel and two-kernel split-K sums differ"


def test_c1_gpu_streams_match_golden_digests(torch_cuda):
    torch = torch_cuda
    with open(os.path.join(HERE, "golden", "c1_digests.json")) as f:
        gold = json.load(f)
    rng = np.random.default_rng(0)
    W = zo.f32_to_bf16(rng.standard_normal((4096, 4096), dtype=np.float32) * np.float32(0.02))
    assert _sha(W) == gold["input"]
    w = to_torch_bf16(W)
    c = zs.compress(w, window="weights")
    torch.cuda.synchronize()
    assert c.start_exp == gold["start_exp"]
    got = {
        "sign_mantissa": c.sign_mantissa[: c.total_high_freq].cpu().numpy(),
        "compressed_full": c.compressed_full[: c.total_full].cpu().view(torch.int16).numpy(),
        "bitmap1": c.bitmap1.cpu().numpy(), "bitmap2": c.bitmap2.cpu().numpy(),
        "bitmap3": c.bitmap3.cpu().numpy(), "tile_offsets": c.tile_offsets.cpu().numpy(),
        "tile_offsets_median": c.tile_offsets_median.cpu().numpy(),
        "tile_offsets_global": c.tile_offsets_global.cpu().numpy(),
        "max_hf": np.array([c.max_high_freq_count], np.int32),
        "max_full": np.array([c.max_full_count], np.int32),
    }
    for k, v in got.items():
        assert _sha(v) == gold[k], k
    r = zs.compress_retiled(w, window="weights")
    torch.cuda.synchronize()
    assert _sha(r.fixed.cpu().numpy()) == gold["rt_fixed"]
    assert _sha(r.exps[: r.num_outliers].cpu().numpy()) == gold["rt_exps"]
    assert _sha(r.eoff.cpu().numpy()) == gold["rt_eoff"]
    # decompress bit-exact, both layouts
    assert torch.equal(zs.decompress(c).view(torch.int16), w.view(torch.int16))
    assert torch.equal(zs.decompress_retiled(r).view(torch.int16), w.view(torch.int16))
    # ZipGEMM N = 8 on every element against the fp32 oracle (X[8, 4096] ~ N(0, 1))
    X = zo.f32_to_bf16(np.random.default_rng(1).standard_normal((8, 4096), dtype=np.float32))
    ref = zo.gemm_f32_mt(W, X)
    x = to_torch_bf16(X)
    for sk in SPLITS:
        for layout, m in (("retiled", r), ("canonical", c)):
            y = zo.bf16_to_f32(from_torch_bf16(zs.zipgemm(m, x, split_k=sk)))
            err = np.abs(y - ref).max() / np.abs(ref).max()
            assert err <= TOL, f"C1 {layout} split_k={sk}: {err}"


@pytest.mark.parametrize("name,M,K", C2_SHAPES)
def test_c2_decompress_bit_exact(torch_cuda, name, M, K):
    torch = torch_cuda
    c = _case(torch, ("c2", name), M, K, max(C2_NS), 1000 + M + K, True)
    assert torch.equal(zs.decompress_retiled(c.r).view(torch.int16), c.w.view(torch.int16))
    canon = zs.compress(c.w, window="weights")
    assert torch.equal(zs.decompress(canon).view(torch.int16), c.w.view(torch.int16))
    # the re-tiled layout built from the canonical streams is the same bytes
    rt = zs.retile(canon)
    torch.cuda.synchronize()
    assert rt.num_outliers == c.r.num_outliers
    assert torch.equal(rt.fixed, c.r.fixed) and torch.equal(rt.eoff, c.r.eoff)


@pytest.mark.parametrize("N", C2_NS)
@pytest.mark.parametrize("name,M,K", C2_SHAPES)
def test_c2_zipgemm(torch_cuda, name, M, K, N):
    torch = torch_cuda
    c = _case(torch, ("c2", name), M, K, max(C2_NS), 1000 + M + K, True)
    _run_all_splits(torch, c, N, f"C2 {name} {M}x{K} N={N}")


def _exact_probes(torch, c, m, N, sk, what):
    """Unit-vector rows of X through ZipGEMM over `m` (re-tiled or canonical
    streams of c.w) in batches of N at split-K sk: every probed output column
    must equal the weight column it selects."""
    cols = probe_columns(c.K, max(sk, 1))
    flat = [k for b in probe_batches(cols, N) for k in b]
    P = len(flat)
    idx = torch.tensor(flat, device="cuda")
    X = torch.zeros(P, c.K, dtype=torch.bfloat16, device="cuda")
    X[torch.arange(P, device="cuda"), idx] = 1.0
    Y = torch.full((P, c.M), float("nan"), dtype=torch.bfloat16, device="cuda")
    ws = zs.codec.splitk_workspace(m, N, sk) if sk != 1 else None
    for j in range(0, P, N):
        zs.zipgemm(m, X[j:j + N], split_k=sk, out=Y[j:j + N], workspace=ws)
    want = c.w[:, idx].t()
    bad = probe_mismatches(Y.float(), want.float())
    assert bad == 0, f"{what}: {bad} of {P * c.M} probed weights differ ({len(cols)} columns)"


def _probe_all(torch, c, ns, what):
    canon = zs.compress(c.w, window="weights")
    for N in ns:
        if N <= 16:
            print(f"{what} N={N} stream-K", flush=True)
            _exact_probes(torch, c, c.r, N, 0, f"{what} re-tiled N={N} stream-K")
        for sk in SPLITS:
            print(f"{what} N={N} split_k={sk}", flush=True)
            _exact_probes(torch, c, c.r, N, sk, f"{what} re-tiled N={N} split_k={sk}")
            _exact_probes(torch, c, canon, N, sk, f"{what} canonical N={N} split_k={sk}")
    torch.cuda.synchronize()


@pytest.mark.parametrize("name,M,K", C2_SHAPES)
def test_c2_exact_probes(torch_cuda, name, M, K):
    torch = torch_cuda
    c = _case(torch, ("c2", name), M, K, max(C2_NS), 1000 + M + K, True)
    _probe_all(torch, c, C2_NS, f"C2 {name} {M}x{K}")


@pytest.mark.parametrize("name,M,K", C2_SHAPES)
def test_c2_canonical_zipgemm(torch_cuda, name, M, K):
    # the drop-in entry point over the canonical streams at the real shapes
    # (N = 17..32 at split-K 2 on the 14336-row shapes reaches the two-phase
    # 64-row canonical kernel, cgemm_wide_kernel<2, 2, 2>)
    torch = torch_cuda
    c = _case(torch, ("c2", name), M, K, max(C2_NS), 1000 + M + K, True)
    canon = zs.compress(c.w, window="weights")
    for N in C2_NS:
        for sk in SPLITS:
            y = zs.zipgemm(canon, c.x[:N], split_k=sk)
            c.check(torch, y, N, f"C2 canonical {name} N={N} split_k={sk}")


@pytest.mark.parametrize("name,M,K", C3_SHAPES)
def test_c3_decompress_bit_exact(torch_cuda, name, M, K):
    torch = torch_cuda
    c = _case(torch, ("c3", name), M, K, max(C3_NS), 2000 + M + K, False)
    assert torch.equal(zs.decompress_retiled(c.r).view(torch.int16), c.w.view(torch.int16))


@pytest.mark.parametrize("N", C3_NS)
@pytest.mark.parametrize("name,M,K", C3_SHAPES)
def test_c3_zipgemm(torch_cuda, name, M, K, N):
    torch = torch_cuda
    c = _case(torch, ("c3", name), M, K, max(C3_NS), 2000 + M + K, False)
    _run_all_splits(torch, c, N, f"C3 {name} {M}x{K} N={N}")


@pytest.mark.parametrize("name,M,K", C3_SHAPES)
def test_c3_exact_probes(torch_cuda, name, M, K):
    torch = torch_cuda
    c = _case(torch, ("c3", name), M, K, max(C3_NS), 2000 + M + K, False)
    _probe_all(torch, c, C3_NS, f"C3 {name} {M}x{K}")


@pytest.mark.parametrize("name,M,K", C3_SHAPES)
def test_c3_canonical_zipgemm(torch_cuda, name, M, K):
    # the drop-in entry point over the canonical streams at the 70B shapes
    torch = torch_cuda
    c = _case(torch, ("c3", name), M, K, max(C3_NS), 2000 + M + K, False)
    canon = zs.compress(c.w, window="weights")
    for N in C3_NS:
        for sk in SPLITS:
            y = zs.zipgemm(canon, c.x[:N], split_k=sk)
            c.check(torch, y, N, f"C3 canonical {name} N={N} split_k={sk}")


@pytest.mark.parametrize("M,K,N", [(10240, 20480, 8), (1024, 36864, 1)])
def test_more_than_64_tiles_per_wave(torch_cuda, M, K, N):
    # 10240 rows at N > 1: 4-wave workgroups, 320 K tiles -> 80 per wave;
    # N = 1: 8-wave workgroups, 576 K tiles -> 72 per wave.  Both reload the
    # per-wave outlier offsets after the first 64 tiles.
    torch = torch_cuda
    c = _case(torch, ("tiles", M, K), M, K, N, 3000 + M + K, True)
    assert torch.equal(zs.decompress_retiled(c.r).view(torch.int16), c.w.view(torch.int16))
    y = zs.zipgemm(c.r, c.x[:N])
    c.check(torch, y, N, f"{M}x{K} N={N}")
