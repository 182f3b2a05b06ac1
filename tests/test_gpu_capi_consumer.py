"""The C-ABI from a plain C caller: tests/capi_consumer.c (built by
tests/Makefile against include/zipserv.h and libzipserv.so, no Python in the
loop) compresses W with the host encoder, decompresses it (canonical and
re-tiled) and runs ZipGEMM at N = 1 / 8 / 40, split-K 1 / 2, checking in C
against a host GEMM of the same bf16 operands (1e-2), W bit for bit after
decompress, and unit-vector columns exactly -- the flow of the reference's
kernel_benchmark/test_mm.cu.  It runs as a child process."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def test_c_consumer_of_the_c_abi():
    exe = os.path.join(HERE, "_build", "capi_consumer")
    assert os.path.exists(exe), "tests/_build/capi_consumer is built by build() (tests/Makefile)"
    print("C consumer of the C-ABI", flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("capi_consumer: ok"), r.stdout
