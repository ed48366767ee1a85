"""`Exl3Config`: SGLang's quantization config for EXL3 checkpoints on this library.

Contract of cuda/src/sglang_exl3/sglang_glue/config.py:17-183: what is quantized comes from the checkpoint's
safetensors headers (the manifest), never from JSON hints; `modules` maps a checkpoint module key to
(k, n, 2K, codebook, has_bias, legacy_signs); `get_quant_method(layer, prefix)` returns an `Exl3LinearMethod` for a
linear (fused modules resolved through the packed-modules map) or an lm_head, an `Exl3MoEMethod` for a FusedMoE
holding EXL3 experts, the engine's unquantized method for linears without EXL3 tensors, and raises for a fused module
that mixes both.  SGLang's prefix spellings (`model.` for `model.language_model.`, `.self_attn.` kept or dropped,
`mtp.` draft layers) are matched against the checkpoint keys.
"""
from __future__ import annotations

import logging
import os
from typing import Any

import torch

from ..format import load_manifest
from .engine import SGLANG

logger = logging.getLogger(__name__)
MODEL_PATH_ENV = "SGLANG_EXL3_MODEL_PATH"   # the reference's variable, so existing launch scripts keep working

DEFAULT_PACKED = {
    "qkv_proj": ["q_proj", "k_proj", "v_proj"],
    "gate_up_proj": ["gate_proj", "up_proj"],
    "in_proj_qkvz": ["in_proj_qkv", "in_proj_z"],
    "in_proj_ba": ["in_proj_b", "in_proj_a"],
}
_SPELLINGS = (("model.language_model.", "model."), (".self_attn.", "."))


def _canonical(key: str) -> str:
    """One spelling per module: `model.` for `model.language_model.`, `.self_attn.` dropped."""
    for long, short in _SPELLINGS:
        key = key.replace(long, short)
    return key


class Exl3Config(SGLANG.QuantizationConfig):
    def __init__(self, declared: dict[str, Any] | None = None, model_path: str | None = None):
        super().__init__()
        self.declared = {k: v for k, v in (declared or {}).items() if k not in ("hf_config", "packed_modules_mapping")}
        self.model_path = model_path
        self.modules: dict[str, tuple] = {}
        self.warnings: list[str] = []
        self._canon: dict[str, str] | None = None
        if not getattr(self, "packed_modules_mapping", None):
            self.packed_modules_mapping = {}
        if model_path:
            self._scan(model_path)

    # ---- QuantizationConfig contract
    def get_name(self) -> str:
        return "exl3"

    def get_supported_act_dtypes(self) -> list[torch.dtype]:
        return [torch.float16, torch.bfloat16]

    @classmethod
    def get_min_capability(cls) -> int:
        return 0   # the gfx950 check is the library's (exl3_init_device)

    @staticmethod
    def get_config_filenames() -> list[str]:
        return []

    @classmethod
    def from_config(cls, config: dict[str, Any]) -> "Exl3Config":
        hf_config = config.get("hf_config")
        name = getattr(hf_config, "_name_or_path", None)
        path = name if name and os.path.isdir(name) else (os.environ.get(MODEL_PATH_ENV) or name)
        if path and not os.path.isdir(path):
            try:   # a hub id: the local snapshot only, never a download
                from huggingface_hub import snapshot_download
                path = snapshot_download(path, local_files_only=True)
            except Exception as e:
                raise ValueError(f"EXL3: no local checkpoint directory for {path!r} ({e}); set {MODEL_PATH_ENV}") \
                    from e
        if not path:
            raise ValueError(f"EXL3: model path unknown (set {MODEL_PATH_ENV})")
        cfg = cls(config, path)
        if config.get("packed_modules_mapping"):
            cfg.packed_modules_mapping = dict(config["packed_modules_mapping"])
        return cfg

    @classmethod
    def override_quantization_method(cls, hf_quant_cfg, user_quant) -> str | None:
        if isinstance(hf_quant_cfg, dict) and hf_quant_cfg.get("quant_method") == "exl3" and user_quant in (None,
                                                                                                           "exl3"):
            return "exl3"
        return None

    def get_scaled_act_names(self) -> list[str]:
        return []

    def can_fuse_shared_expert(self) -> bool:
        return False

    # ---- checkpoint scan
    def _scan(self, model_path: str) -> None:
        man = load_manifest(model_path)
        self.modules = {k: (m.k, m.n, m.bits.twice, m.codebook.value, m.has_bias, m.legacy_signs)
                        for k, m in man.matrices.items()}
        self.warnings = list(man.warnings)
        for w in man.warnings:
            logger.warning("EXL3 checkpoint: %s", w)
        s = man.summary()
        logger.info("EXL3 checkpoint %s: %d quantized linears %s, %d other tensors", model_path,
                    s["quantized_linears"], s["by_bits_codebook"], s["unquantized_tensors"])

    def __getstate__(self):
        return self.__dict__.copy()

    def lookup(self, key: str):
        """The header-scan entry of a module key under any of SGLang's spellings (`model.` / `model.language_model.`,
        with or without `.self_attn.`; `model.layers.N` of a draft model = `mtp.layers.N`), or None."""
        if key in self.modules:
            return self.modules[key]
        if getattr(self, "_canon", None) is None or len(self._canon) != len(self.modules):
            self._canon = {_canonical(k): k for k in self.modules}
        c = _canonical(key)
        for cand in (c, "mtp." + c[len("model."):] if c.startswith("model.layers.") else None):
            if cand is not None and cand in self._canon:
                return self.modules[self._canon[cand]]
        return None

    def _sources(self, prefix: str) -> list[str]:
        parent, _, leaf = prefix.rpartition(".")
        members = (self.packed_modules_mapping or DEFAULT_PACKED).get(leaf)
        if not members:
            return [prefix]
        return [f"{parent}.{m}" if parent else m for m in members]

    def experts_of(self, prefix: str) -> dict[str, tuple]:
        head = _canonical(prefix) + "."
        return {k: v for k, v in self.modules.items() if _canonical(k).startswith(head) and ".experts." in k}

    def get_quant_method(self, layer: torch.nn.Module, prefix: str):
        from .sglang_linear import Exl3LinearMethod
        if isinstance(layer, SGLANG.FusedMoE):
            from .sglang_moe import Exl3MoEMethod
            experts = self.experts_of(prefix)
            return Exl3MoEMethod(self, prefix, experts) if experts else None
        if isinstance(layer, SGLANG.ParallelLMHead):
            info = self.lookup(prefix)
            return Exl3LinearMethod(prefix, [info]) if info else None
        if not isinstance(layer, SGLANG.LinearBase):
            return None
        sources = self._sources(prefix)
        infos = [self.lookup(p) for p in sources]
        if not any(infos):
            return SGLANG.UnquantizedLinearMethod()
        if not all(infos):
            raise ValueError(f"{prefix}: fused module mixes EXL3 and unquantized sources {sources}")
        return Exl3LinearMethod(prefix, infos)
