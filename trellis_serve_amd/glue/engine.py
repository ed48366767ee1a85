"""Engine classes the plugin glue builds on: SGLang's or vLLM's when they are installed, otherwise minimal local
stand-ins with the same contract (layer marker classes for isinstance checks, method base classes,
`set_weight_attrs`, `StandardCombineInput`, a quantization-method registry).  The stand-ins let the glue run -- and
be tested -- without an engine: they are the interfaces the reference's glue uses
(cuda/src/sglang_exl3/sglang_glue/linear.py:14-16, moe.py:32-34, config.py:9, xpu/exl3xpu/vllm_plugin.py:14-19).
"""
from __future__ import annotations

import types
from dataclasses import dataclass

import torch


class _QuantizeMethodBase:
    def create_weights(self, layer, *args, **kwargs):
        raise NotImplementedError

    def apply(self, layer, *args, **kwargs):
        raise NotImplementedError

    def process_weights_after_loading(self, layer) -> None:
        return None


class _QuantizationConfig:
    def __init__(self):
        self.packed_modules_mapping: dict[str, list[str]] = {}


class _LinearMethodBase(_QuantizeMethodBase):
    pass


class _FusedMoEMethodBase(_QuantizeMethodBase):
    pass


class _UnquantizedLinearMethod(_LinearMethodBase):
    """Plain fp16/bf16 weight [n, k] and F.linear, as the engines' unquantized method."""

    def create_weights(self, layer, input_size_per_partition, output_partition_sizes, input_size, output_size,
                       params_dtype, **extra):
        w = torch.nn.Parameter(torch.empty(sum(output_partition_sizes), input_size_per_partition, dtype=params_dtype),
                               requires_grad=False)
        layer.register_parameter("weight", w)

    def apply(self, layer, x, bias=None):
        return torch.nn.functional.linear(x, layer.weight, bias)


class _LinearBase(torch.nn.Module):
    pass


class _ParallelLMHead(torch.nn.Module):
    pass


class _FusedMoE(torch.nn.Module):
    pass


@dataclass
class _StandardCombineInput:
    hidden_states: torch.Tensor


def _set_weight_attrs(param, attrs: dict | None) -> None:
    for k, v in (attrs or {}).items():
        if hasattr(param, k) and k != "weight_loader":
            raise KeyError(f"overwriting existing tensor attribute {k}")
        setattr(param, k, v)


def stubs() -> types.SimpleNamespace:
    """A fresh set of stand-ins (each engine gets its own registry)."""
    return types.SimpleNamespace(
        name="stub", QuantizationConfig=_QuantizationConfig, LinearMethodBase=_LinearMethodBase,
        FusedMoEMethodBase=_FusedMoEMethodBase, UnquantizedLinearMethod=_UnquantizedLinearMethod,
        LinearBase=_LinearBase, ParallelLMHead=_ParallelLMHead, FusedMoE=_FusedMoE,
        StandardCombineInput=_StandardCombineInput, set_weight_attrs=_set_weight_attrs,
        QUANTIZATION_METHODS={})


def _sglang() -> types.SimpleNamespace | None:
    try:
        from sglang.srt.layers.linear import LinearBase
        from sglang.srt.layers.moe.fused_moe_triton.layer import FusedMoE
        from sglang.srt.layers.moe.token_dispatcher.standard import StandardCombineInput
        from sglang.srt.layers.quantization import QUANTIZATION_METHODS
        from sglang.srt.layers.quantization.base_config import (FusedMoEMethodBase, LinearMethodBase,
                                                                QuantizationConfig)
        from sglang.srt.layers.quantization.unquant import UnquantizedLinearMethod
        from sglang.srt.layers.vocab_parallel_embedding import ParallelLMHead
        from sglang.srt.utils.common import set_weight_attrs
    except Exception:
        return None
    return types.SimpleNamespace(
        name="sglang", QuantizationConfig=QuantizationConfig, LinearMethodBase=LinearMethodBase,
        FusedMoEMethodBase=FusedMoEMethodBase, UnquantizedLinearMethod=UnquantizedLinearMethod,
        LinearBase=LinearBase, ParallelLMHead=ParallelLMHead, FusedMoE=FusedMoE,
        StandardCombineInput=StandardCombineInput, set_weight_attrs=set_weight_attrs,
        QUANTIZATION_METHODS=QUANTIZATION_METHODS)


def _vllm() -> types.SimpleNamespace | None:
    try:
        from vllm.model_executor.layers.linear import LinearBase, LinearMethodBase, UnquantizedLinearMethod
        from vllm.model_executor.layers.quantization.base_config import QuantizationConfig
        from vllm.model_executor.layers.vocab_parallel_embedding import ParallelLMHead
        from vllm.model_executor.utils import set_weight_attrs
    except Exception:
        return None
    base = stubs()
    base.__dict__.update(name="vllm", QuantizationConfig=QuantizationConfig, LinearMethodBase=LinearMethodBase,
                         UnquantizedLinearMethod=UnquantizedLinearMethod, LinearBase=LinearBase,
                         ParallelLMHead=ParallelLMHead, set_weight_attrs=set_weight_attrs)
    return base


SGLANG = _sglang() or stubs()
VLLM = _vllm() or stubs()


def target_device() -> torch.device:
    """Where loaded weights go: the current GPU, or the CPU when none is visible (loading-logic tests)."""
    if torch.cuda.is_available():
        return torch.device("cuda", torch.cuda.current_device())
    return torch.device("cpu")
