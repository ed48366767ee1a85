"""Engine glue: the SGLang quantization method (`Exl3Config`, `Exl3LinearMethod`, `Exl3MoEMethod`) and the vLLM
quantization method, running EXL3 checkpoints on this library.  `activate()` is the SGLang plugin entry point
(the reference's `sglang.srt.plugins: exl3 = sglang_exl3.plugin:activate`, cuda/pyproject.toml:8-9 and
cuda/src/sglang_exl3/plugin.py:16-25); `register()` is vLLM's (`vllm.general_plugins`,
xpu/exl3xpu/vllm_plugin.py:325-336).  Without an installed engine both register into local stand-in registries
(`engine.SGLANG.QUANTIZATION_METHODS`, `engine.VLLM.QUANTIZATION_METHODS`)."""
from __future__ import annotations

_activated = False


def activate() -> None:
    """Registers `QUANTIZATION_METHODS["exl3"] = Exl3Config` in SGLang (idempotent)."""
    global _activated
    if _activated:
        return
    from .engine import SGLANG
    from .sglang_config import Exl3Config
    SGLANG.QUANTIZATION_METHODS["exl3"] = Exl3Config
    if SGLANG.name == "sglang":
        try:
            from sglang.srt.arg_groups.choices import QUANTIZATION_CHOICES, add_quantization_method_choices
            if "exl3" not in QUANTIZATION_CHOICES:
                add_quantization_method_choices(["exl3"])
        except Exception:
            pass
    _activated = True


def register() -> None:
    """vLLM plugin entry point: importing the plugin module registers the "exl3" quantization config."""
    from . import vllm_plugin
    vllm_plugin.register()
