"""`Exl3Config`: SGLang's quantization config for EXL3 checkpoints on this library.

The SGLang `QuantizationConfig` contract of cuda/src/sglang_exl3/sglang_glue/config.py:17-183, answered from a
`CheckpointIndex` of the checkpoint's headers: `get_quant_method(layer, prefix)` gives an `Exl3LinearMethod` for a
linear or lm_head whose source matrices are EXL3, an `Exl3MoEMethod` for a FusedMoE whose routed experts are, the
engine's unquantized method for a plain linear, and raises for a fused linear that mixes both.
"""
from __future__ import annotations

import os
from typing import Any

import torch

from .engine import SGLANG
from .index import CheckpointIndex

MODEL_PATH_ENV = "SGLANG_EXL3_MODEL_PATH"   # the reference's variable, so existing launch scripts keep working


def checkpoint_dir(config: dict[str, Any]) -> str:
    """The local checkpoint directory of a model config: the HF config's local path (a draft checkpoint carries its
    own headers), else $SGLANG_EXL3_MODEL_PATH, else the hub id resolved to its local snapshot -- never a download
    (config.py:44-62)."""
    name = getattr(config.get("hf_config"), "_name_or_path", None)
    if name and os.path.isdir(name):
        return name
    path = os.environ.get(MODEL_PATH_ENV) or name
    if not path:
        raise ValueError(f"EXL3: model path unknown (set {MODEL_PATH_ENV})")
    if os.path.isdir(path):
        return path
    try:
        from huggingface_hub import snapshot_download
        return snapshot_download(path, local_files_only=True)
    except Exception as e:
        raise ValueError(f"EXL3: no local checkpoint directory for {path!r} ({e}); set {MODEL_PATH_ENV}") from e


class Exl3Config(SGLANG.QuantizationConfig):
    def __init__(self, declared: dict[str, Any] | None = None, model_path: str | None = None,
                 index: CheckpointIndex | None = None):
        super().__init__()
        self.declared = {k: v for k, v in (declared or {}).items() if k not in ("hf_config", "packed_modules_mapping")}
        self.model_path = model_path
        self.index = index if index is not None else (CheckpointIndex.scan(model_path) if model_path else
                                                      CheckpointIndex({}))
        if not getattr(self, "packed_modules_mapping", None):
            self.packed_modules_mapping = {}

    @property
    def warnings(self) -> list[str]:
        return self.index.warnings

    # ---- the engine's QuantizationConfig interface
    def get_name(self) -> str:
        return "exl3"

    def get_supported_act_dtypes(self) -> list[torch.dtype]:
        return [torch.float16, torch.bfloat16]

    @classmethod
    def get_min_capability(cls) -> int:
        return 0   # the device check is the library's (exl3_init_device accepts gfx950 only)

    @staticmethod
    def get_config_filenames() -> list[str]:
        return []

    @classmethod
    def from_config(cls, config: dict[str, Any]) -> "Exl3Config":
        cfg = cls(config, checkpoint_dir(config))
        if config.get("packed_modules_mapping"):
            cfg.packed_modules_mapping = dict(config["packed_modules_mapping"])
        return cfg

    @classmethod
    def override_quantization_method(cls, hf_quant_cfg, user_quant) -> str | None:
        declared = isinstance(hf_quant_cfg, dict) and hf_quant_cfg.get("quant_method") == "exl3"
        return "exl3" if declared and user_quant in (None, "exl3") else None

    def get_scaled_act_names(self) -> list[str]:
        return []

    def can_fuse_shared_expert(self) -> bool:
        return False   # shared experts stay ordinary EXL3 linears

    def get_quant_method(self, layer: torch.nn.Module, prefix: str):
        if isinstance(layer, SGLANG.FusedMoE):
            experts = self.index.experts(prefix)
            if not experts:
                return None
            from .sglang_moe import Exl3MoEMethod
            return Exl3MoEMethod(self, prefix, experts)
        from .sglang_linear import Exl3LinearMethod
        if isinstance(layer, SGLANG.ParallelLMHead):
            info = self.index.find(prefix)
            return Exl3LinearMethod(prefix, [info]) if info is not None else None
        if isinstance(layer, SGLANG.LinearBase):
            infos = self.index.linear(prefix, self.packed_modules_mapping)
            return Exl3LinearMethod(prefix, infos) if infos else SGLANG.UnquantizedLinearMethod()
        return None

    def __getstate__(self):   # pickled to scheduler workers: plain data only
        return self.__dict__.copy()
