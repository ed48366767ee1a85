"""Checkpoint manifest from safetensors headers: which modules are EXL3 linears, at which K and codebook.

Same API as core/src/trellis_core/format/manifest.py:1-170 (`Manifest`, `build_manifest`, `load_manifest`,
`NgramTable`, `NGRAM_FORMAT`).  The tensor headers are the truth; `quantization_config` from config.json is only
cross-checked (mismatches become warnings).  A module key is an EXL3 linear iff a `<key>.trellis` tensor exists;
tensors nested below such a key are rejected (derivative formats), everything else is an unquantized tensor.
"""
from __future__ import annotations

import glob
import json
import os
from collections import Counter
from dataclasses import dataclass, field

from .safetensors_header import ShardHeader, read_header
from .spec import INPUT_SCALE, OUTPUT_SCALE, REQUIRED_TRELLIS, FormatError, MatrixSpec, TensorInfo, build_matrix_spec

NGRAM_FORMAT = "exl3_ngram_trellis"   # n-gram embedding tables: their own container, kept apart (manifest.py:18)
INDEX_FILE = "model.safetensors.index.json"


@dataclass(frozen=True)
class NgramTable:
    file: str
    metadata: dict[str, str]
    tensors: dict[str, TensorInfo]

    @property
    def nbytes(self) -> int:
        return sum(t.nbytes for t in self.tensors.values())


@dataclass
class Manifest:
    matrices: dict[str, MatrixSpec] = field(default_factory=dict)
    unquantized: dict[str, TensorInfo] = field(default_factory=dict)
    ngram_tables: list[NgramTable] = field(default_factory=list)
    quant_config: dict = field(default_factory=dict)
    warnings: list[str] = field(default_factory=list)

    def is_quantized(self, key: str) -> bool:
        return key in self.matrices

    def children(self, prefix: str) -> dict[str, MatrixSpec]:
        """The EXL3 linears strictly below a module prefix (e.g. every expert of one MoE block)."""
        head = prefix.rstrip(".") + "."
        return {k: m for k, m in self.matrices.items() if k.startswith(head)}

    def summary(self) -> dict:
        classes = Counter((str(m.bits), m.codebook.value) for m in self.matrices.values())
        declared_keys = ("version", "bits", "head_bits", "mtp_bits", "vision_bits", "codebook", "out_scales")
        return {
            "quantized_linears": len(self.matrices),
            "quantized_bytes": sum(m.nbytes for m in self.matrices.values()),
            "unquantized_tensors": len(self.unquantized),
            "unquantized_bytes": sum(t.nbytes for t in self.unquantized.values()),
            "ngram_tables": len(self.ngram_tables),
            "ngram_bytes": sum(t.nbytes for t in self.ngram_tables),
            "by_bits_codebook": {f"K={b} {cb}": c for (b, cb), c in sorted(classes.items())},
            "legacy_sign_linears": sum(1 for m in self.matrices.values() if m.legacy_signs),
            "biased_linears": sum(1 for m in self.matrices.values() if m.has_bias),
            "declared": {k: self.quant_config[k] for k in declared_keys if k in self.quant_config},
            "warnings": list(self.warnings),
        }


def _parents(key: str):
    """Proper ancestors of a dotted module key, nearest first."""
    parts = key.split(".")
    for i in range(len(parts) - 1, 0, -1):
        yield ".".join(parts[:i])


def _live_tensors(man: Manifest, headers: list[ShardHeader], weight_map: dict[str, str]) -> dict[str, TensorInfo]:
    live: dict[str, TensorInfo] = {}
    doubled: list[str] = []
    for h in headers:
        if h.metadata.get("format") == NGRAM_FORMAT:
            man.ngram_tables.append(NgramTable(h.file, dict(h.metadata), dict(h.tensors)))
            continue
        for name, info in h.tensors.items():
            prev = live.get(name)
            if prev is None:
                live[name] = info
                continue
            owner = weight_map.get(name)
            if owner not in (prev.file, h.file):
                raise FormatError(f"tensor {name} appears in both {prev.file} and {h.file} and the index does not say "
                                  f"which one is live")
            doubled.append(name)
            if owner == h.file:
                live[name] = info
    if doubled:
        man.warnings.append(f"{len(doubled)} tensors are stored in more than one shard (the index decides), "
                            f"e.g. {doubled[0]}")
    return live


def build_manifest(headers: list[ShardHeader], quant_config: dict | None = None,
                   weight_map: dict[str, str] | None = None) -> Manifest:
    """Manifest of the tensors in `headers`; `weight_map` (the index) decides tensors stored in several shards."""
    man = Manifest(quant_config=dict(quant_config or {}))
    live = _live_tensors(man, headers, dict(weight_map or {}))
    tail = "." + REQUIRED_TRELLIS
    keys = {name[: -len(tail)] for name in live if name.endswith(tail)}
    for key in keys:
        outer = next((p for p in _parents(key) if p in keys), None)
        if outer is not None:
            raise FormatError(f"{key}.trellis: unexpected tensor nested under EXL3 linear {outer}")
    per_key: dict[str, dict[str, TensorInfo]] = {}
    for name, info in live.items():
        parent, _, suffix = name.rpartition(".")
        if parent in keys:
            per_key.setdefault(parent, {})[suffix] = info
            continue
        outer = next((p for p in _parents(name) if p in keys), None)
        if outer is not None:
            raise FormatError(f"{name}: unexpected tensor nested under EXL3 linear {outer}")
        man.unquantized[name] = info
    for key in sorted(per_key):
        man.matrices[key] = build_matrix_spec(key, per_key[key])

    declared = man.quant_config.get("codebook")
    if declared and man.matrices:
        used = sorted({m.codebook.value for m in man.matrices.values()})
        if used != [declared]:
            man.warnings.append(f"quantization_config.codebook={declared!r} but the tensors use {used}")
    scale_names = set(INPUT_SCALE + OUTPUT_SCALE)
    stray = [n for n in man.unquantized if n.rpartition(".")[2] in scale_names]
    if stray:
        man.warnings.append(f"{len(stray)} scale tensors without a trellis, e.g. {stray[0]}")
    return man


def _quant_config(model_dir: str) -> dict:
    path = os.path.join(model_dir, "config.json")
    if not os.path.exists(path):
        return {}
    with open(path) as f:
        cfg = json.load(f)
    qc = cfg.get("quantization_config") or (cfg.get("text_config") or {}).get("quantization_config") or {}
    if qc and qc.get("quant_method") != "exl3":
        raise FormatError(f"{model_dir}: quant_method is {qc.get('quant_method')!r}, not 'exl3'")
    return qc


def load_manifest(model_dir: str | os.PathLike) -> Manifest:
    """Manifest of a local checkpoint directory: every *.safetensors header, the index, config.json."""
    model_dir = os.fspath(model_dir)
    files = sorted(glob.glob(os.path.join(model_dir, "*.safetensors")))
    if not files:
        raise FormatError(f"{model_dir}: no .safetensors files")
    headers = [read_header(f) for f in files]
    weight_map: dict[str, str] = {}
    index = os.path.join(model_dir, INDEX_FILE)
    if os.path.exists(index):
        with open(index) as f:
            weight_map = json.load(f).get("weight_map", {})
    man = build_manifest(headers, _quant_config(model_dir), weight_map)
    if weight_map:
        present = {n for h in headers if h.metadata.get("format") != NGRAM_FORMAT for n in h.tensors}
        absent = sorted(set(weight_map) - present)
        if absent:
            raise FormatError(f"{len(absent)} tensors listed in the index are in no shard, e.g. {absent[0]}")
        extra = sorted(present - set(weight_map))
        if extra:
            man.warnings.append(f"{len(extra)} tensors are not in {INDEX_FILE}, e.g. {extra[0]}")
    return man
