"""vLLM out-of-tree quantization method "exl3" on this library.

The vLLM contract of xpu/exl3xpu/vllm_plugin.py:50-261: `Exl3Config` registered under "exl3", built from the model's
declared `bits` / `head_bits` / `mtp_bits` / `codebook`; `maybe_update_config` learns the real per-module format
from the checkpoint when its directory is local (here: a CheckpointIndex of the safetensors headers, so shapes,
bitrates and codebooks are all checked at load); `get_quant_method` gives the EXL3 linear method for linears and
lm_heads whose matrices are EXL3.

Loading differs from the reference's vLLM method, which registers real-shaped parameters and copies each shard into
its column span: the method here is the one SGLang runs (`Exl3LinearCore`), with 0-byte placeholders whose loaders
stash each shard whole, so both engines keep one resident trellis per source matrix in its stored layout.
"""
from __future__ import annotations

import logging
import os
from typing import Any

import torch

from .engine import VLLM
from .index import CheckpointIndex, module_key
from .linear_method import Exl3LinearCore

logger = logging.getLogger(__name__)

_UNQUANTIZED_TOWERS = ("visual", "vision_tower")
_PLAIN_WITHOUT_HEADERS = ("in_proj_ba",)   # GDN's small b / a projections stay plain in EXL3 checkpoints


def _register(name: str):
    try:
        from vllm.model_executor.layers.quantization import register_quantization_config
        return register_quantization_config(name)
    except Exception:
        def deco(cls):
            VLLM.QUANTIZATION_METHODS[name] = cls
            return cls
        return deco


class Exl3LinearMethod(Exl3LinearCore, VLLM.LinearMethodBase):
    set_weight_attrs = staticmethod(VLLM.set_weight_attrs)

    def embedding(self, layer, input_):
        raise NotImplementedError("exl3: quantized input embeddings are not supported")


@_register("exl3")
class Exl3Config(VLLM.QuantizationConfig):
    def __init__(self, bits: float = 4, head_bits: int = 6, codebook: str = "mul1", mtp_bits: int | None = None):
        super().__init__()
        self.bits = bits
        self.head_bits = head_bits
        self.mtp_bits = int(mtp_bits or bits)
        self.codebook = codebook
        self.index: CheckpointIndex | None = None   # set by maybe_update_config for a local checkpoint

    def __repr__(self) -> str:
        return f"Exl3Config(bits={self.bits}, head_bits={self.head_bits}, codebook={self.codebook})"

    def get_name(self) -> str:
        return "exl3"

    def get_supported_act_dtypes(self) -> list[torch.dtype]:
        return [torch.float16, torch.bfloat16]

    @classmethod
    def get_min_capability(cls) -> int:
        return 0

    @staticmethod
    def get_config_filenames() -> list[str]:
        return []

    @classmethod
    def from_config(cls, config: dict[str, Any]) -> "Exl3Config":
        return cls(bits=config.get("bits", 4), head_bits=config.get("head_bits", 6),
                   codebook=config.get("codebook", "mul1"), mtp_bits=config.get("mtp_bits"))

    def maybe_update_config(self, model_name: str, hf_config=None, revision=None) -> None:
        if not model_name or not os.path.isdir(model_name):
            logger.info("exl3: %r is not a local directory; the declared bits / codebook apply", model_name)
            return
        index = CheckpointIndex.scan(model_name)
        half = [index.names[k] for k, i in index.infos.items() if i.twice_bits % 2]
        if half:
            raise NotImplementedError(f"exl3: half-integer bitrates are not supported by the kernels ({half[0]})")
        self.index = index

    def declared_bits(self, prefix: str) -> int | None:
        """The bitrate the model config declares for a module, or None for one it leaves plain."""
        key = module_key(prefix)
        if key.endswith(_PLAIN_WITHOUT_HEADERS):
            return None
        if key == "lm_head":
            return int(self.head_bits)
        return self.mtp_bits if key.startswith("mtp.") else int(self.bits)

    def get_quant_method(self, layer: torch.nn.Module, prefix: str):
        is_linear = isinstance(layer, VLLM.LinearBase)
        if not (is_linear or isinstance(layer, VLLM.ParallelLMHead)):
            return None
        plain = VLLM.UnquantizedLinearMethod() if is_linear else None
        if any(t in prefix.split(".") for t in _UNQUANTIZED_TOWERS):
            return plain
        if self.index is not None:
            infos = self.index.linear(prefix) if is_linear else (
                [self.index.find(prefix)] if self.index.find(prefix) is not None else None)
            return Exl3LinearMethod(prefix, infos) if infos else plain
        bits = self.declared_bits(prefix)
        return Exl3LinearMethod(prefix, declared_bits=bits) if bits is not None else plain


def register() -> None:
    """The `vllm.general_plugins` entry point: importing this module registers "exl3"."""
    return None
