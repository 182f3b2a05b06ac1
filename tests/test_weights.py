"""Weight ingestion from a local path: the reference's JSONL manifest
(bench_manifest_utils.h:322-395), raw bf16 .bin tensors
(bench_llama31_70b_compress.cu:206-231,925-980), layer specs and filters,
the safetensors exporter (scripts/export_llama31_70b_weights.py:126-200),
and manifest -> container bundle on the host encoder."""
import json

import numpy as np
import pytest

import zipserv_asplos26_amd as zs
from zipserv_asplos26_amd import container as ct
from zipserv_asplos26_amd import weights as zw
from zs_testutil import weights_bf16


def _write_checkpoint(tmp_path, shapes, seed=0):
    rng = np.random.default_rng(seed)
    recs, mats = [], {}
    for i, (layer, name, shape) in enumerate(shapes):
        a = weights_bf16(rng, shape)
        p = tmp_path / f"{name}.bin"
        a.tofile(p)
        recs.append(dict(layer=layer, name=name, shape=list(shape), dtype="bf16", path=str(p),
                         nbytes=a.nbytes))
        mats[name] = a
    m = tmp_path / "manifest.jsonl"
    m.write_text("\n".join(json.dumps(r) for r in recs) + "\n\n")
    return m, mats


def test_manifest_parse_and_select(tmp_path):
    m, mats = _write_checkpoint(tmp_path, [
        (0, "model.layers.0.self_attn.q_proj.weight", (128, 64)),
        (0, "model.layers.0.mlp.down_proj.weight", (64, 192)),
        (3, "model.layers.3.self_attn.q_proj.weight", (64, 64)),
        (5, "model.layers.5.mlp.up_proj.weight", (96, 64))])   # not a 64-multiple
    ts = zw.load_manifest(str(m))
    assert [t.layer for t in ts] == [0, 0, 3, 5]
    assert ts[1].shape == [64, 192] and ts[1].nbytes == 64 * 192 * 2 and ts[1].dtype == "bf16"
    assert zw.parse_layer_spec("0-2, 5,7-7") == {0, 1, 2, 5, 7}
    assert zw.parse_layer_spec("") == set()
    assert [t.layer for t in zw.select(ts, "3-5")] == [3, 5]
    assert [t.name for t in zw.select(ts, None, ["q_proj"])] == [
        "model.layers.0.self_attn.q_proj.weight", "model.layers.3.self_attn.q_proj.weight"]
    np.testing.assert_array_equal(zw.read_bf16(ts[0]), mats[ts[0].name])
    for bad in ("3-1", "-1", "x", "1-y"):
        with pytest.raises(ValueError):
            zw.parse_layer_spec(bad)


@pytest.mark.parametrize("line,msg", [
    ('{"name": "a", "shape": [64, 64], "dtype": "bf16", "path": "p", "nbytes": 1}', "layer"),
    ('{"layer": -1, "name": "a", "shape": [64], "dtype": "bf16", "path": "p", "nbytes": 1}',
     "layer out of range"),
    ('{"layer": 0, "name": "a", "shape": [64, "x"], "dtype": "bf16", "path": "p", "nbytes": 1}',
     "shape"),
    ('{"layer": 0, "name": "a", "shape": [64], "dtype": "bf16", "path": "p", "nbytes": -2}',
     "nbytes < 0"),
    ('{"layer": 0, "name": "a", "shape": [64], "dtype": "bf16", "path": "p"}', "nbytes"),
    ("not json", "invalid JSON")])
def test_manifest_rejects(tmp_path, line, msg):
    m = tmp_path / "m.jsonl"
    good = '{"layer": 0, "name": "ok", "shape": [64, 64], "dtype": "bf16", "path": "p", "nbytes": 8192}'
    m.write_text(good + "\n" + line + "\n")
    with pytest.raises(ValueError, match=f"line 2: .*{msg}"):
        zw.load_manifest(str(m))


def test_read_bf16_checks(tmp_path):
    m, _ = _write_checkpoint(tmp_path, [(0, "w", (64, 64))])
    t = zw.load_manifest(str(m))[0]
    for field, value, err in (("dtype", "fp16", "dtype"), ("shape", [64, 64, 1], "2D"),
                              ("shape", [64, 32], "mismatch"), ("path", str(tmp_path / "no"),
                                                                "missing")):
        u = zw.ManifestTensor(**{**t.__dict__, field: value})
        with pytest.raises(ValueError, match=err):
            zw.read_bf16(u)


def test_manifest_to_bundle_on_host(tmp_path):
    m, mats = _write_checkpoint(tmp_path, [
        (0, "a", (128, 64)), (1, "b", (64, 128)), (2, "c", (96, 64))], seed=4)
    out = tmp_path / "w.zsc"
    assert zw.main(["--manifest", str(m), "--out", str(out), "--device", "cpu",
                    "--layers", "0-2"]) == 0
    got = ct.load_bundle(str(out))
    assert list(got) == ["a", "b"]          # "c" (96 rows) is skipped, as the reference does
    for name in got:
        ref = zs.compress_host(mats[name])
        np.testing.assert_array_equal(got[name].sign_mantissa, ref.sign_mantissa)
        np.testing.assert_array_equal(got[name].bitmap2, ref.bitmap2)


def test_export_safetensors_snapshot(tmp_path):
    torch = pytest.importorskip("torch")
    st = pytest.importorskip("safetensors.torch")
    snap = tmp_path / "snap"
    snap.mkdir()
    g = torch.Generator().manual_seed(0)
    tensors = {f"model.layers.{l}.{s}": torch.randn(64, 128, generator=g).to(torch.bfloat16)
               for l in range(2) for s in zw.PROJECTION_SUFFIXES}
    tensors["model.embed_tokens.weight"] = torch.zeros(64, 64, dtype=torch.bfloat16)
    names = sorted(tensors)
    shard = {n: ("a.safetensors" if i % 2 else "b.safetensors") for i, n in enumerate(names)}
    for f in ("a.safetensors", "b.safetensors"):
        st.save_file({n: tensors[n] for n in names if shard[n] == f}, str(snap / f))
    (snap / "config.json").write_text(json.dumps({"num_hidden_layers": 2}))
    (snap / "model.safetensors.index.json").write_text(json.dumps({"weight_map": shard}))
    man = tmp_path / "manifest" / "weights_manifest.jsonl"
    recs = zw.export_safetensors(str(snap), str(tmp_path / "bins"), str(man), layers="1",
                                 filters=["proj"])
    assert [r.name for r in recs] == [f"model.layers.1.{s}" for s in zw.PROJECTION_SUFFIXES]
    back = zw.load_manifest(str(man))
    assert [b.name for b in back] == [r.name for r in recs]
    for r in back:
        np.testing.assert_array_equal(zw.read_bf16(r), tensors[r.name].view(torch.int16).numpy()
                                      .view(np.uint16))
