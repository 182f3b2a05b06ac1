"""Containers of device-resident matrices: canonical streams from the GPU
encoder and the re-tiled layout round-trip through bytes back to the GPU,
where they decode bit-exactly and multiply like the originals."""
import numpy as np
import pytest

import zipserv_asplos26_amd as zs
from zipserv_asplos26_amd import container as ct
from zs_testutil import from_torch_bf16, to_torch_bf16, weights_bf16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("retiled", [False, True])
def test_device_container_round_trip(torch_cuda, tmp_path, retiled):
    torch = torch_cuda
    rng = np.random.default_rng(9)
    W = weights_bf16(rng, (256, 512), outlier_frac=0.01)
    w = to_torch_bf16(W)
    c = zs.compress_retiled(w) if retiled else zs.compress(w)
    p = tmp_path / "m.zsc"
    ct.save(str(p), c, "m")
    back = ct.load(str(p), device="cuda")
    assert type(back) is type(c)
    dec = zs.decompress_retiled(back) if retiled else zs.decompress(back)
    np.testing.assert_array_equal(from_torch_bf16(dec), W)
    x = to_torch_bf16(weights_bf16(rng, (8, 512), std=1.0))
    y0, y1 = zs.zipgemm(c, x), zs.zipgemm(back, x)
    torch.cuda.synchronize()
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))
    assert back.compressed_bytes == c.compressed_bytes


def test_manifest_to_bundle_on_gpu(torch_cuda, tmp_path):
    # weights from a local manifest, compressed on the GPU into a bundle,
    # loaded back and multiplied: within 1e-2 of the fp32 product
    import json

    from zipserv_asplos26_amd import weights as zw
    torch = torch_cuda
    rng = np.random.default_rng(12)
    recs, mats = [], {}
    for i, shape in enumerate(((256, 128), (128, 320))):
        a = weights_bf16(rng, shape, outlier_frac=0.001)
        p = tmp_path / f"w{i}.bin"
        a.tofile(p)
        recs.append(dict(layer=i, name=f"w{i}", shape=list(shape), dtype="bf16", path=str(p),
                         nbytes=a.nbytes))
        mats[f"w{i}"] = a
    m = tmp_path / "m.jsonl"
    m.write_text("\n".join(json.dumps(r) for r in recs))
    out = tmp_path / "w.zsc"
    assert zw.main(["--manifest", str(m), "--out", str(out)]) == 0
    got = ct.load_bundle(str(out), device="cuda")
    for name, W in mats.items():
        assert isinstance(got[name], zs.ZipservRetiled)
        x = to_torch_bf16(weights_bf16(rng, (4, W.shape[1]), std=1.0))
        y = zs.zipgemm(got[name], x).float()
        ref = x.float() @ to_torch_bf16(W).float().t()
        assert float((y - ref).abs().max() / ref.abs().max()) < 1e-2
