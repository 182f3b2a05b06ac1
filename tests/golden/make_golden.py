"""Writes the golden fixtures of tests/test_golden.py (run from the repository
root: python tests/golden/make_golden.py).

The reference ships no golden vectors, so these are produced by this build's
CPU oracle (oracle/zs_oracle.c, the restatement of csrc/L_API.cu:314-1053) and
frozen: they pin the oracle and the encoders against regressions.  Inputs are
generated with numpy's PCG64 generator (np.random.default_rng(seed)),
float32 normals rounded to bf16 (round to nearest even).

Files:
  <name>.npz         input matrix + canonical streams (CPU window) + re-tiled
                     layout built from them (arrays only; load with
                     allow_pickle=False)
  c1_digests.json    SHA-256 of every stream of benchmark config 1 (4096x4096,
                     N(0, 0.02), seed 0), canonical and re-tiled
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle as zo  # noqa: E402


def bf16(x):
    return zo.f32_to_bf16(np.ascontiguousarray(x, dtype=np.float32))


def cases():
    r = np.random.default_rng(1)
    w = r.standard_normal((64, 64), dtype=np.float32) * np.float32(0.02)
    w[r.random((64, 64)) < 0.01] *= 30
    yield "w64x64_outliers", bf16(w)
    r = np.random.default_rng(2)
    w = r.standard_normal((128, 192), dtype=np.float32) * np.float32(0.02)
    w[r.random((128, 192)) < 0.05] *= 30
    yield "w128x192_outliers5pct", bf16(w)
    r = np.random.default_rng(3)
    scale = np.exp(r.standard_normal((1, 128))).astype(np.float32)
    yield "kv256x128_lognormal", bf16(r.standard_normal((256, 128), dtype=np.float32) * scale)
    r = np.random.default_rng(4)
    w = r.standard_normal((64, 128), dtype=np.float32) * np.float32(0.02)
    w[16:32] = 0.0                        # an all-outlier band (exponent 0)
    w[40, :8] = [1e30, -1e-30, 3e38, -2.0, 65504.0, 1e-38, -0.0, 7.0]
    yield "edge64x128", bf16(w)


def arrays(W):
    e = zo.compress(W)
    r = zo.retile(e)
    return dict(
        input=W, start_exp=np.array([e.start_exp], np.int32),
        max_hf=np.array([e.max_high_freq_count], np.int32),
        max_full=np.array([e.max_full_count], np.int32),
        sign_mantissa=e.sign_mantissa, compressed_full=e.compressed_full,
        bitmap1=e.bitmap1, bitmap2=e.bitmap2, bitmap3=e.bitmap3,
        tile_offsets=e.tile_offsets, tile_offsets_median=e.tile_offsets_median,
        tile_offsets_global=e.tile_offsets_global,
        rt_fixed=r.fixed, rt_exps=r.exps, rt_eoff=r.eoff)


def c1_matrix():
    r = np.random.default_rng(0)
    return bf16(r.standard_normal((4096, 4096), dtype=np.float32) * np.float32(0.02))


def digests(W):
    a = arrays(W)
    out = {k: hashlib.sha256(np.ascontiguousarray(v).tobytes()).hexdigest()
           for k, v in a.items() if k != "input"}
    out["input"] = hashlib.sha256(W.tobytes()).hexdigest()
    out["start_exp"] = int(a["start_exp"][0])
    return out


def main():
    for name, W in cases():
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays(W))
    with open(os.path.join(HERE, "c1_digests.json"), "w") as f:
        json.dump(digests(c1_matrix()), f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
