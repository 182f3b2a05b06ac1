"""Real-weight ingestion from a local path: the JSONL manifest + raw .bin
format of the reference's weight benches, and its exporter from a
safetensors snapshot.

* Manifest (kernel_benchmark/bench_manifest_utils.h:322-395 ParseManifestLine /
  LoadManifestJsonl): one JSON object per non-empty line with "layer" (int,
  0..INT_MAX), "name", "shape" (int list), "dtype", "path", "nbytes" (>= 0).
* Raw tensors (bench_llama31_70b_compress.cu:206-231, 925-980): 2-D bf16, file
  size rows*cols*2, rows and cols multiples of 64 to be compressed.
* Layer specs "0-3,5" and substring name filters (bench_manifest_utils.h:98-150).
* Export (scripts/export_llama31_70b_weights.py:126-200): the seven
  projection weights of each selected layer from model.safetensors.index.json
  shards, as bf16 .bin files plus manifest records.

Nothing is downloaded: every path is local.  `compress_manifest` turns the
selected tensors into compressed matrices (GPU encoder, or the host encoder
when device is None) and `python -m zipserv_asplos26_amd.weights` writes them
as a container bundle.
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field

import numpy as np

INT_MAX = 2**31 - 1

# export_llama31_70b_weights.py:19-27 (CANONICAL_SUFFIXES)
PROJECTION_SUFFIXES = (
    "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
    "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
    "mlp.down_proj.weight",
)


@dataclass
class ManifestTensor:
    layer: int
    name: str
    shape: list = field(default_factory=list)
    dtype: str = ""
    path: str = ""
    nbytes: int = 0


def _parse_line(line: str) -> ManifestTensor:
    try:
        obj = json.loads(line)
    except json.JSONDecodeError as e:
        raise ValueError(f"invalid JSON ({e.msg})") from None
    if not isinstance(obj, dict):
        raise ValueError("not a JSON object")

    def get(key, kind):
        v = obj.get(key)
        if kind is int:
            if isinstance(v, bool) or not isinstance(v, int):
                raise ValueError(f"missing/invalid {key}")
        elif not isinstance(v, kind):
            raise ValueError(f"missing/invalid {key}")
        return v
    layer = get("layer", int)
    if layer < 0 or layer > INT_MAX:
        raise ValueError("layer out of range")
    name = get("name", str)
    shape = get("shape", list)
    if any(isinstance(s, bool) or not isinstance(s, int) for s in shape):
        raise ValueError("missing/invalid shape")
    dtype = get("dtype", str)
    path = get("path", str)
    nbytes = get("nbytes", int)
    if nbytes < 0:
        raise ValueError("nbytes < 0")
    return ManifestTensor(layer, name, list(shape), dtype, path, nbytes)


def load_manifest(path: str) -> list:
    """JSONL manifest -> [ManifestTensor]; ValueError names the failing line."""
    out = []
    with open(path, "r", encoding="utf-8") as f:
        for no, line in enumerate(f, 1):
            line = line.strip()
            if not line:
                continue
            try:
                out.append(_parse_line(line))
            except ValueError as e:
                raise ValueError(f"Manifest parse failed at line {no}: {e}") from None
    return out


def parse_layer_spec(spec: str) -> set:
    """"0-3,5" -> {0, 1, 2, 3, 5}; an empty spec selects every layer (empty set)."""
    layers = set()
    for token in (t.strip() for t in spec.split(",")):
        if not token:
            continue
        if "-" in token:
            a, b = (s.strip() for s in token.split("-", 1))
            try:
                start, end = int(a), int(b)
            except ValueError:
                raise ValueError(f"Invalid layer range token: {token}") from None
            if start < 0 or end < 0 or start > end:
                raise ValueError(f"Invalid layer range: {token}")
            layers.update(range(start, end + 1))
        else:
            try:
                layer = int(token)
            except ValueError:
                raise ValueError(f"Invalid layer token: {token}") from None
            if layer < 0:
                raise ValueError(f"Layer index must be non-negative: {token}")
            layers.add(layer)
    return layers


def name_matches(name: str, filters) -> bool:
    return not filters or any(f in name for f in filters)


def select(tensors, layers=None, filters=None) -> list:
    """Manifest entries in the given layers (a set or a spec string) whose names
    contain one of the filters."""
    if isinstance(layers, str):
        layers = parse_layer_spec(layers)
    return [t for t in tensors if (not layers or t.layer in layers) and name_matches(t.name, filters)]


def read_bf16(t: ManifestTensor, mmap: bool = True) -> np.ndarray:
    """The tensor's raw bf16 bits as uint16 [rows, cols] (memory-mapped by default)."""
    if t.dtype != "bf16":
        raise ValueError(f"unsupported dtype: {t.dtype} (expected bf16)")
    if len(t.shape) != 2:
        raise ValueError("tensor is not 2D")
    rows, cols = t.shape
    if rows <= 0 or cols <= 0:
        raise ValueError("shape has non-positive dimension")
    size = os.path.getsize(t.path) if os.path.exists(t.path) else 0
    if size == 0:
        raise ValueError("file_missing_or_empty")
    if size != rows * cols * 2:
        raise ValueError(f"file bytes mismatch: expected {rows * cols * 2}, got {size}")
    if mmap:
        return np.memmap(t.path, dtype=np.uint16, mode="r", shape=(rows, cols))
    return np.fromfile(t.path, np.uint16).reshape(rows, cols)


def compress_manifest(tensors, device="cuda", retiled: bool = True) -> dict:
    """{name: compressed matrix} for 2-D bf16 entries with 64-multiple shapes:
    ZipservRetiled / ZipservCompressed on `device`, or HostCompressed (host
    encoder, device None).  Entries the reference's bench skips (other shapes)
    are skipped here too."""
    from . import codec
    out = {}
    for t in tensors:
        if len(t.shape) != 2 or t.shape[0] % 64 or t.shape[1] % 64:
            continue
        a = read_bf16(t)
        if device is None:
            out[t.name] = codec.compress_host(np.ascontiguousarray(a))
            continue
        import torch
        w = torch.from_numpy(np.array(a).view(np.int16)).to(device).view(torch.bfloat16)
        out[t.name] = codec.compress_retiled(w) if retiled else codec.compress(w)
    return out


def export_safetensors(snapshot_dir: str, out_dir: str, manifest_path: str, layers="",
                       filters=None) -> list:
    """export_llama31_70b_weights.py on a local snapshot (config.json,
    model.safetensors.index.json, shards): the projection weights of the
    selected layers as bf16 .bin files in out_dir plus the JSONL manifest,
    records sorted by (layer, projection, name)."""
    import torch
    from safetensors import safe_open
    with open(os.path.join(snapshot_dir, "config.json"), encoding="utf-8") as f:
        config = json.load(f)
    with open(os.path.join(snapshot_dir, "model.safetensors.index.json"), encoding="utf-8") as f:
        weight_map = json.load(f)["weight_map"]
    max_layer = int(config["num_hidden_layers"]) - 1
    sel = parse_layer_spec(layers) if layers else set(range(max_layer + 1))
    if any(l > max_layer for l in sel):
        raise ValueError(f"layer out of range [0, {max_layer}]")
    os.makedirs(out_dir, exist_ok=True)
    records = []
    for layer in sorted(sel):
        for si, suffix in enumerate(PROJECTION_SUFFIXES):
            name = f"model.layers.{layer}.{suffix}"
            if not name_matches(name, filters) or name not in weight_map:
                continue
            with safe_open(os.path.join(snapshot_dir, weight_map[name]), framework="pt") as sf:
                src = sf.get_tensor(name)
            t = src.to(torch.bfloat16).contiguous()
            path = os.path.abspath(os.path.join(out_dir, f"{name}.bin"))
            t.view(torch.int16).numpy().tofile(path)
            nbytes = os.path.getsize(path)
            if nbytes != t.numel() * 2:
                raise RuntimeError(f"nbytes mismatch for {name}")
            records.append(((layer, si, name), dict(layer=layer, name=name, shape=list(t.shape),
                                                    dtype="bf16", path=path, nbytes=nbytes)))
    records.sort(key=lambda r: r[0])
    os.makedirs(os.path.dirname(os.path.abspath(manifest_path)), exist_ok=True)
    with open(manifest_path, "w", encoding="utf-8") as f:
        for _, rec in records:
            f.write(json.dumps(rec) + "\n")
    return [ManifestTensor(**rec) for _, rec in records]


def main(argv=None) -> int:
    import argparse
    from . import container
    ap = argparse.ArgumentParser(description="Compress the bf16 tensors of a weight manifest "
                                             "into a container bundle.")
    ap.add_argument("--manifest", required=True)
    ap.add_argument("--out", required=True, help="bundle path")
    ap.add_argument("--layers", default="", help='e.g. "0-3,5" (default: all)')
    ap.add_argument("--filter", action="append", default=[], help="substring of tensor names")
    ap.add_argument("--device", default="cuda", help='"cpu" runs the host encoder')
    ap.add_argument("--canonical", action="store_true", help="canonical streams, not re-tiled")
    a = ap.parse_args(argv)
    tensors = select(load_manifest(a.manifest), a.layers, a.filter)
    dev = None if a.device == "cpu" else a.device
    mats = compress_manifest(tensors, dev, retiled=not a.canonical and dev is not None)
    n = container.save_bundle(a.out, mats)
    print(f"{len(mats)} tensors -> {a.out} ({n} bytes)")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
