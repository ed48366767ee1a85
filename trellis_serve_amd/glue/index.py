"""Which linears of a checkpoint are EXL3, at which shape, bitrate and codebook: the lookups the SGLang and vLLM
configs answer `get_quant_method` from.  Built from the safetensors headers (the manifest), never from JSON hints
(the contract of cuda/src/sglang_exl3/sglang_glue/config.py:17-20, 78-93).

A checkpoint, SGLang and vLLM spell one module three ways (`model.language_model.layers.3.self_attn.q_proj`,
`model.layers.3.self_attn.q_proj` or `model.layers.3.q_proj`, `language_model.model.layers.3.self_attn.q_proj`).
`module_key` reduces every spelling to one key -- the language-model prefix dropped, `.self_attn.` dropped -- and the
index is keyed by it, so a lookup is one dictionary probe under any spelling.  A draft model built over the
checkpoint's `mtp.layers.N` asks for `model.layers.N`; that spelling falls back to the `mtp.` key when the plain one
is absent (config.py:105-109).
"""
from __future__ import annotations

import logging
from typing import Iterable, Mapping

from .stash import MatrixInfo

logger = logging.getLogger(__name__)

# language-model prefixes, longest first: what precedes `layers.N`, `mtp.` or `lm_head` in the three spellings
_LM_PREFIXES = ("model.language_model.", "language_model.model.", "language_model.", "model.")

# the engines' fused linears and the checkpoint matrices they hold, in output order (the engines' packed-modules
# maps for the model families the reference serves, config.py:122-126)
FUSED_SOURCES = {
    "qkv_proj": ("q_proj", "k_proj", "v_proj"),
    "gate_up_proj": ("gate_proj", "up_proj"),
    "in_proj_qkvz": ("in_proj_qkv", "in_proj_z"),
    "in_proj_ba": ("in_proj_b", "in_proj_a"),
}
EXPERT_ROLES = ("gate", "up", "down")


def module_key(name: str) -> str:
    """The spelling-free key of a module name: 'model.language_model.layers.3.self_attn.q_proj' ->
    'layers.3.q_proj', 'language_model.model.layers.3.mlp.gate_proj' -> 'layers.3.mlp.gate_proj',
    'model.mtp.layers.0.mlp.up_proj' -> 'mtp.layers.0.mlp.up_proj', 'lm_head' -> 'lm_head'."""
    for p in _LM_PREFIXES:
        if name.startswith(p):
            name = name[len(p):]
            break
    return name.replace(".self_attn.", ".")


class CheckpointIndex:
    """The EXL3 matrices of one checkpoint by module key."""

    def __init__(self, matrices: Mapping[str, MatrixInfo | tuple], warnings: Iterable[str] = ()):
        self.names: dict[str, str] = {}          # module key -> checkpoint spelling
        self.infos: dict[str, MatrixInfo] = {}   # module key -> what the headers declare
        for name, info in matrices.items():
            key = module_key(name)
            if key in self.infos:
                raise ValueError(f"EXL3 checkpoint: {name} and {self.names[key]} name the same module")
            self.names[key], self.infos[key] = name, MatrixInfo(*info)
        self.warnings = list(warnings)

    @classmethod
    def scan(cls, model_dir: str) -> "CheckpointIndex":
        """Reads the safetensors headers of a local checkpoint directory (no tensor data)."""
        from ..format import load_manifest
        man = load_manifest(model_dir)
        index = cls({name: MatrixInfo(m.k, m.n, m.bits.twice, m.codebook.value, m.has_bias, m.legacy_signs)
                     for name, m in man.matrices.items()}, man.warnings)
        for w in man.warnings:
            logger.warning("EXL3 checkpoint: %s", w)
        s = man.summary()
        logger.info("EXL3 checkpoint %s: %d quantized linears %s, %d other tensors", model_dir,
                    s["quantized_linears"], s["by_bits_codebook"], s["unquantized_tensors"])
        return index

    def __len__(self) -> int:
        return len(self.infos)

    def __contains__(self, name: str) -> bool:
        return self.find(name) is not None

    def forget(self, name: str) -> None:
        """Drops one matrix (a checkpoint whose module is to run unquantized)."""
        key = self._key(name)
        if key is not None:
            del self.infos[key], self.names[key]

    def _key(self, name: str) -> str | None:
        key = module_key(name)
        if key in self.infos:
            return key
        if key.startswith("layers.") and "mtp." + key in self.infos:
            return "mtp." + key
        return None

    def find(self, name: str) -> MatrixInfo | None:
        """The header entry of a module under any spelling, or None (not EXL3)."""
        key = self._key(name)
        return None if key is None else self.infos[key]

    def sources(self, prefix: str, packed: Mapping[str, Iterable[str]] | None = None) -> list[str]:
        """The checkpoint modules one engine module holds: the members of a fused linear (the engine's
        packed-modules map when it has one, else FUSED_SOURCES), else the module itself."""
        parent, _, leaf = prefix.rpartition(".")
        members = (packed or FUSED_SOURCES).get(leaf)
        if not members:
            return [prefix]
        return [f"{parent}.{m}" if parent else m for m in members]

    def linear(self, prefix: str, packed: Mapping[str, Iterable[str]] | None = None) -> list[MatrixInfo] | None:
        """Header entries of an engine linear's source matrices in output order; None when none of them is EXL3.
        A fused module with EXL3 and plain members raises ValueError (one method serves the whole module)."""
        names = self.sources(prefix, packed)
        found = [self.find(n) for n in names]
        if not any(found):
            return None
        if not all(found):
            plain = [n for n, f in zip(names, found) if f is None]
            raise ValueError(f"{prefix}: fused module mixes EXL3 and unquantized sources (plain: {plain})")
        return found

    def experts(self, prefix: str) -> dict[tuple[str, int], MatrixInfo]:
        """Routed experts under an MoE module: (role, expert id) -> entry, role in gate / up / down, for keys
        '<prefix>.<id>.<role>_proj'."""
        head = module_key(prefix) + "."
        out: dict[tuple[str, int], MatrixInfo] = {}
        for key, info in self.infos.items():
            if not key.startswith(head):
                continue
            expert, _, proj = key[len(head):].partition(".")
            role = proj[:-5] if proj.endswith("_proj") else ""
            if not expert.isdigit() or role not in EXPERT_ROLES:
                raise ValueError(f"{prefix}: unexpected EXL3 matrix under the experts: {self.names[key]}")
            out[(role, int(expert))] = info
        return out
