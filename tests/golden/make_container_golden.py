"""Writes tests/golden/container_v1_matrix.npy, a fixed 64x64 bf16 matrix
(exponents spread over and outside a 7-exponent window), and
tests/golden/container_v1.zsc, its version-1 container image from
zipserv_asplos26_amd.container.  Run from the repository root:
    python tests/golden/make_container_golden.py"""
import os
import sys

import numpy as np

sys.path.insert(0, os.path.abspath(os.path.join(os.path.dirname(__file__), "..", "..")))
import zipserv_asplos26_amd as zs  # noqa: E402
from zipserv_asplos26_amd import container as ct  # noqa: E402

i = np.arange(64 * 64, dtype=np.uint32).reshape(64, 64)
exp = (118 + (i * 7 + i // 64) % 11).astype(np.uint32)      # 118..128: some outliers
matrix = (((i * 2654435761) >> 9) & 0x807F | (exp << 7)).astype(np.uint16)
image = ct.to_bytes(zs.compress_host(matrix), "golden")
here = os.path.dirname(__file__)
np.save(os.path.join(here, "container_v1_matrix.npy"), matrix)
image.tofile(os.path.join(here, "container_v1.zsc"))
print("container_v1.zsc:", image.size, "bytes")
