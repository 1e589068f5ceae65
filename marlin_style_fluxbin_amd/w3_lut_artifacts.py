"""On-disk W3 planar artifacts: converter, manifest and hash-bound loader.

Reference: ``src/fluxbin_style/w3_lut_artifacts.py`` (``load_w3_lut_layer``
:14-44, ``replace_w3_model_linears`` :47-118) and the offline converter
``scripts/prepare_qwen3_8b_w3_lut_artifacts.py:145-294`` in
maxiu188-afk/Marlin_Style_Fluxbin.  Contract kept: one safetensors file of
planar payloads per decoder layer (``payloads/layer-NNN.safetensors``, keys
``"<module>.<field>"``), a ``manifest.json`` that records every file's byte
size and sha256 and the canonical-semantics gate, a loader that refuses a
manifest whose sha256 differs from the caller's, a layer file whose size or
hash drifted, or an inventory that is not exactly seven complete payloads, and
a model installer that validates every layer before touching the model.

Differences, all deliberate:

* Layer count and shapes come from the model config (the reference fixes 36
  layers / 252 Linears of Qwen3-8B); a manifest records them.
* The payload may carry the ``zeros`` field and fp16 scales (``allow_zeros`` /
  ``scale_dtype``, the benchmark configs' extension); the manifest's format
  string then names the extended format, and the gate records the decoded
  zero-point set instead of requiring ``[4]``.
* Writing is staged: payloads go to ``<out>.incomplete`` and the directory is
  renamed only after the manifest is complete, so a failed conversion never
  leaves a publishable artifact.

The converter runs on the CPU (``python -m marlin_style_fluxbin_amd.w3_lut_artifacts
prepare --gptq-root DIR --output-dir DIR``): it reads raw GPTQ int3 tensors
(``qweight``, ``qzeros``, ``scales``, ``g_idx``) of every
``model.layers.N.<module>`` from the safetensors files under ``--gptq-root``.
"""
from __future__ import annotations

import argparse
import datetime as dt
import hashlib
import json
import os
from pathlib import Path
from typing import Iterable, Mapping

import torch

from .gptq_deployment import (FIELDS, FORMAT, OPTIONAL_FIELDS, REFERENCE_FORMAT, convert_gptq_w3_to_planar,
                              decode_planar_w3_codes, inspect_gptq_checkpoint, layout_storage, restore_planar_w3,
                              unpack_gptq_w3_qweight, validate_planar_w3)
from .qwen3 import QWEN3_LINEAR_MODULES

STATUS = "completed_pending_gpu_validation"
GATE_STATUS = "confirmed_before_payload_writes"
RAW_FIELDS = ("qweight", "qzeros", "scales", "g_idx")
MANIFEST = "manifest.json"


def sha256_file(path: Path, chunk: int = 1 << 22) -> str:
    digest = hashlib.sha256()
    with open(path, "rb") as handle:
        while True:
            block = handle.read(chunk)
            if not block:
                return digest.hexdigest()
            digest.update(block)


def _write_json_atomically(path: Path, value: dict) -> None:
    tmp = path.with_name(path.name + ".tmp")
    tmp.write_text(json.dumps(value, indent=1, sort_keys=True) + "\n", encoding="utf-8")
    os.replace(tmp, path)


def _layer_file(layer: int) -> str:
    return f"payloads/layer-{layer:03d}.safetensors"


# ------------------------------------------------------------------ converter
def write_w3_lut_artifacts(output_dir: Path, layers: Iterable[tuple[int, Mapping[str, Mapping[str, torch.Tensor]]]],
                           *, num_layers: int, qzero_format: int = 1, scale_dtype: torch.dtype = torch.bfloat16,
                           allow_zeros: bool = False, decoded_bf16: Mapping[str, torch.Tensor] | None = None,
                           source: dict | None = None) -> dict:
    """Convert raw GPTQ W3 Linears into a hash-bound planar artifact directory.

    ``layers`` yields ``(layer_index, {module: raw tensors})`` for every layer
    ``0 .. num_layers - 1``; it is consumed twice, so pass a re-iterable (a list,
    or an object whose ``__iter__`` re-reads the source).  The first pass is the
    canonical-semantics gate: every Linear is inspected (``inspect_gptq_checkpoint``)
    and the decoded zero-points must be ``[4]`` unless ``allow_zeros``; nothing is
    written before it passes.  The second pass converts each Linear, checks that
    the planar codes decode back to the raw codes exactly and, where
    ``decoded_bf16["model.layers.N.<module>"]`` is given, that the restored bf16
    weight equals it bit for bit, then writes one safetensors file per layer.
    Returns the manifest.
    """
    from safetensors.torch import save_file

    output_dir = Path(output_dir)
    staging = output_dir.with_name(output_dir.name + ".incomplete")
    if output_dir.exists() or staging.exists():
        raise FileExistsError(output_dir if output_dir.exists() else staging)

    def modules_of(layer_modules):
        if set(layer_modules) != set(QWEN3_LINEAR_MODULES):
            raise ValueError("each layer must hold exactly the seven Qwen3 Linears")
        for module in QWEN3_LINEAR_MODULES:
            raw = layer_modules[module]
            if set(raw) != set(RAW_FIELDS):
                raise ValueError(f"raw GPTQ fields of {module} must be exactly {RAW_FIELDS}")
            yield module, raw

    zero_sets, seen, nonidentity = set(), [], 0
    for layer, layer_modules in layers:
        for module, raw in modules_of(layer_modules):
            facts = inspect_gptq_checkpoint(raw, qzero_format=qzero_format)
            zero_sets.update(facts["decoded_zero_unique"])
            nonidentity += int(not facts["permutation_identity"])
            seen.append(f"model.layers.{layer}.{module}")
    if sorted(seen) != sorted(f"model.layers.{n}.{m}" for n in range(num_layers) for m in QWEN3_LINEAR_MODULES):
        raise ValueError("the source does not cover every Linear of every layer exactly once")
    if zero_sets != {4} and not allow_zeros:
        raise ValueError(f"constant-zero layout requires decoded zero=4, got {sorted(zero_sets)}")
    extended = allow_zeros or scale_dtype != torch.bfloat16
    gate = {"status": GATE_STATUS, "inspected_linears": len(seen), "nonidentity_permutations": nonidentity,
            "all_groups_have_128_columns": True, "decoded_zero_unique": sorted(zero_sets)}

    (staging / "payloads").mkdir(parents=True)
    files, modules, payload_bytes = [], [], 0
    try:
        for layer, layer_modules in layers:
            tensors = {}
            for module, raw in modules_of(layer_modules):
                name = f"model.layers.{layer}.{module}"
                layout = convert_gptq_w3_to_planar(raw, qzero_format=qzero_format, scale_dtype=scale_dtype,
                                                   allow_zeros=allow_zeros)
                if not torch.equal(decode_planar_w3_codes(layout), unpack_gptq_w3_qweight(raw["qweight"])):
                    raise RuntimeError(f"integer code round trip failed: {name}")
                record = {"name": name, "storage": layout_storage(layout), "integer_codes_exact": True}
                if decoded_bf16 is not None and name in decoded_bf16:
                    if not torch.equal(restore_planar_w3(layout, dtype=torch.bfloat16), decoded_bf16[name]):
                        raise RuntimeError(f"bf16 bitwise round trip failed: {name}")
                    record["decoded_bf16_bitwise_exact"] = True
                payload_bytes += record["storage"]["total_bytes"]
                modules.append(record)
                tensors.update({f"{module}.{field}": value.contiguous() for field, value in layout.items()})
            path = staging / _layer_file(layer)
            save_file(tensors, str(path))
            files.append({"layer": layer, "path": _layer_file(layer), "bytes": path.stat().st_size,
                          "sha256": sha256_file(path)})
        manifest = {
            "schema_version": 1, "status": STATUS, "format": FORMAT if extended else REFERENCE_FORMAT,
            "created_at_utc": dt.datetime.now(dt.timezone.utc).isoformat(), "layers": num_layers,
            "qzero_format": qzero_format, "scale_dtype": str(scale_dtype).replace("torch.", ""),
            "canonicalization": "per-Linear stable argsort(g_idx); the same permutation for weight K and runtime x",
            "canonical_semantics_gate": gate, "deployment_tensor_bytes": payload_bytes,
            "files": sorted(files, key=lambda f: f["layer"]), "modules": modules, "source": source or {},
        }
        _write_json_atomically(staging / MANIFEST, manifest)
        os.replace(staging, output_dir)
    except BaseException:
        if staging.exists():
            _write_json_atomically(staging / "failure.json", {"status": "failed"})
        raise
    return manifest


# ------------------------------------------------------------------ loader
def _read_manifest(root: Path, expected_manifest_sha256: str) -> dict:
    path = Path(root) / MANIFEST
    if sha256_file(path) != expected_manifest_sha256:
        raise ValueError("W3 LUT manifest drift")
    manifest = json.loads(path.read_text(encoding="utf-8"))
    if manifest.get("status") != STATUS or manifest.get("format") not in (REFERENCE_FORMAT, FORMAT):
        raise ValueError("W3 LUT manifest status/format drift")
    layers = manifest.get("layers", 36)
    gate = manifest.get("canonical_semantics_gate", {})
    zero_ok = gate.get("decoded_zero_unique") == [4] or (
        manifest["format"] == FORMAT and set(gate.get("decoded_zero_unique", [-1])) <= set(range(8)))
    if (gate.get("status") != GATE_STATUS or gate.get("inspected_linears") != 7 * layers
            or gate.get("all_groups_have_128_columns") is not True or not zero_ok):
        raise ValueError("W3 LUT canonical-semantics gate missing or drifted")
    return manifest


def load_w3_lut_layer(root: Path, layer: int, *, expected_manifest_sha256: str) -> tuple[dict, dict]:
    """``(tensors, file entry)`` of one layer, after the manifest hash, the file's
    size and sha256 and its payload inventory have been checked."""
    from safetensors.torch import load_file

    root = Path(root)
    manifest = _read_manifest(root, expected_manifest_sha256)
    if not 0 <= layer < manifest.get("layers", 36):
        raise ValueError(f"layer outside 0..{manifest.get('layers', 36) - 1}")
    relative = _layer_file(layer)
    entry = next((item for item in manifest["files"] if item["path"] == relative), None)
    if entry is None:
        raise ValueError(f"W3 LUT manifest has no entry for {relative}")
    path = root / relative
    if path.stat().st_size != entry["bytes"] or sha256_file(path) != entry["sha256"]:
        raise ValueError("W3 LUT layer hash/size drift")
    tensors = load_file(str(path))
    with_zeros = {m for m in QWEN3_LINEAR_MODULES if f"{m}.zeros" in tensors}
    expected = {f"{m}.{f}" for m in QWEN3_LINEAR_MODULES for f in FIELDS} | {f"{m}.zeros" for m in with_zeros}
    if set(tensors) != expected:
        raise ValueError("W3 LUT layer inventory drift")
    for module in QWEN3_LINEAR_MODULES:
        names = FIELDS + (OPTIONAL_FIELDS if module in with_zeros else ())
        validate_planar_w3({field: tensors[f"{module}.{field}"] for field in names})
    return tensors, entry


def replace_w3_model_linears(model, artifact_root: Path, *, expected_manifest_sha256: str,
                             allow_prefill_fallback: bool = False, route: str = "structural") -> dict:
    """Install every hash-bound W3 Linear of the artifact into ``model`` (all layers
    validated against the model's shapes first, then replaced layer by layer)."""
    from torch import nn

    from .qwen3 import expected_qwen3_linear_shape
    from .w3_lut_deployment import QWEN3_ROW_TILE_BY_SHAPE, QWEN3_W3_ROUTE_POLICIES, replace_w3_block_linears

    if route not in QWEN3_W3_ROUTE_POLICIES:
        raise ValueError(f"unknown Qwen3-8B W3 route: {route}")
    blocks = model.model.layers
    manifest = _read_manifest(Path(artifact_root), expected_manifest_sha256)
    if manifest.get("layers", 36) != len(blocks):
        raise ValueError(f"artifact has {manifest.get('layers', 36)} layers, the model {len(blocks)}")
    config = model.config.to_dict()
    entries = []
    for index, block in enumerate(blocks):
        tensors, entry = load_w3_lut_layer(artifact_root, index, expected_manifest_sha256=expected_manifest_sha256)
        for name in QWEN3_LINEAR_MODULES:
            shape = validate_planar_w3({f: tensors[f"{name}.{f}"] for f in FIELDS}, check_values=False)
            if list(shape) != expected_qwen3_linear_shape(config, name):
                raise ValueError(f"W3 shape drift: layer {index} {name}")
            target = block.get_submodule(name)
            if not isinstance(target, nn.Linear) or (target.out_features, target.in_features) != shape:
                raise ValueError(f"Linear shape/type mismatch: layer {index} {name}")
        entries.append(entry)
        del tensors
    shapes = {tuple(expected_qwen3_linear_shape(config, n)) for n in QWEN3_LINEAR_MODULES}
    tiles = None if shapes <= set(QWEN3_ROW_TILE_BY_SHAPE) else {s: 256 for s in shapes}
    coverage = []
    for index, block in enumerate(blocks):
        tensors, _ = load_w3_lut_layer(artifact_root, index, expected_manifest_sha256=expected_manifest_sha256)
        done = replace_w3_block_linears(block, tensors, fallback="dense" if allow_prefill_fallback else "error",
                                        row_tile_by_shape=tiles, route=route if tiles is None else "structural")
        coverage.extend(f"model.layers.{index}.{name}" for name in done)
    return {"format": manifest["format"], "manifest_sha256": expected_manifest_sha256, "layers": entries,
            "coverage": coverage, "linear_count": len(coverage), "prefill_fallback_enabled": allow_prefill_fallback,
            "route": route, "status": "installed_not_validated"}


# ------------------------------------------------------------------ command line
class _RawGPTQSource:
    """Re-iterable ``(layer, {module: raw tensors})`` over the safetensors files of a
    raw GPTQ checkpoint directory (keys ``model.layers.N.<module>.<field>``)."""

    def __init__(self, root: Path):
        from safetensors import safe_open

        self.index: dict[str, Path] = {}
        for path in sorted(Path(root).glob("*.safetensors")):
            with safe_open(str(path), framework="pt", device="cpu") as handle:
                for key in handle.keys():
                    if key in self.index:
                        raise ValueError(f"duplicate safetensors key: {key}")
                    self.index[key] = path
        layers = {int(k.split(".")[2]) for k in self.index if k.startswith("model.layers.") and k.endswith(".qweight")}
        if not layers or layers != set(range(max(layers) + 1)):
            raise ValueError("raw GPTQ layers must be 0..N-1 without gaps")
        self.num_layers = max(layers) + 1

    def _tensor(self, key: str) -> torch.Tensor:
        from safetensors import safe_open

        with safe_open(str(self.index[key]), framework="pt", device="cpu") as handle:
            return handle.get_tensor(key).contiguous()

    def __iter__(self):
        for layer in range(self.num_layers):
            yield layer, {m: {f: self._tensor(f"model.layers.{layer}.{m}.{f}") for f in RAW_FIELDS}
                          for m in QWEN3_LINEAR_MODULES}


def main(argv=None) -> None:
    parser = argparse.ArgumentParser(description="W3 planar artifacts from a raw GPTQ int3 checkpoint")
    sub = parser.add_subparsers(dest="command", required=True)
    prep = sub.add_parser("prepare", help="convert and write payloads + manifest")
    prep.add_argument("--gptq-root", type=Path, required=True)
    prep.add_argument("--output-dir", type=Path, required=True)
    prep.add_argument("--qzero-format", type=int, default=1)
    prep.add_argument("--allow-zeros", action="store_true")
    prep.add_argument("--fp16-scales", action="store_true")
    args = parser.parse_args(argv)
    source = _RawGPTQSource(args.gptq_root)
    manifest = write_w3_lut_artifacts(args.output_dir, source, num_layers=source.num_layers,
                                      qzero_format=args.qzero_format, allow_zeros=args.allow_zeros,
                                      scale_dtype=torch.float16 if args.fp16_scales else torch.bfloat16,
                                      source={"gptq_root": str(args.gptq_root)})
    print(f"wrote {len(manifest['files'])} layers, manifest sha256 "
          f"{sha256_file(args.output_dir / MANIFEST)}", flush=True)


if __name__ == "__main__":
    main()
