"""vLLM out-of-tree quantization method "exl3" on this library.

Contract of xpu/exl3xpu/vllm_plugin.py:50-261: `Exl3Config` registered under "exl3"; `create_weights` registers
real-shaped parameters -- trellis int16 [k/16, n/16, 16K] over all output partitions, suh fp16 [S, k] (one row per
partition), svh fp16 [n], and the codebook marker -- whose loaders copy each checkpoint shard into its column span
(157-221); `process_weights_after_loading` groups the loaded shards (223-248); `apply` runs the fused linear (250-261).
Which modules are EXL3, and at which K and codebook, comes from the checkpoint's manifest when the model directory is
local (`maybe_update_config`), else from the declared `bits` / `head_bits` / `codebook`.  After loading, each shard
group keeps a contiguous trellis and svh of its own (the C-ABI takes one pointer per shard).
"""
from __future__ import annotations

import logging
import os
import re
from typing import Any

import torch

from ..format import load_manifest
from .common import CODEBOOK_ID, QKV_INDEX, fused_forward, launch_runs
from .engine import VLLM, target_device

logger = logging.getLogger(__name__)

FUSED = {
    "gate_up_proj": ["gate_proj", "up_proj"],
    "qkv_proj": ["q_proj", "k_proj", "v_proj"],
    "in_proj_qkvz": ["in_proj_qkv", "in_proj_z"],
    "in_proj_ba": ["in_proj_b", "in_proj_a"],
}


def module_key(name: str) -> str:
    """Spelling-independent module key: '...layers.3.mlp.gate_proj' -> 'layers.3.mlp.gate_proj' (any model /
    language_model prefix dropped), '...mtp.layers.0.x' -> 'mtp.layers.0.x', '...lm_head' -> 'lm_head'."""
    parts = name.split(".")
    if "mtp" in parts:
        return ".".join(["mtp"] + parts[parts.index("mtp") + 1:])
    m = re.search(r"(?:^|\.)(layers\.\d+\..*)$", name)
    return m.group(1) if m else parts[-1]


def _register(name: str):
    try:
        from vllm.model_executor.layers.quantization import register_quantization_config
        return register_quantization_config(name)
    except Exception:
        def deco(cls):
            VLLM.QUANTIZATION_METHODS[name] = cls
            return cls
        return deco


@_register("exl3")
class Exl3Config(VLLM.QuantizationConfig):
    def __init__(self, bits: float = 4, head_bits: int = 6, codebook: str = "mul1", storage: dict | None = None,
                 mtp_bits: int | None = None):
        super().__init__()
        self.bits = bits
        self.head_bits = head_bits
        self.mtp_bits = int(mtp_bits or bits)
        self.codebook = codebook
        self.storage: dict[str, tuple[int, str]] = dict(storage or {})   # module key -> (K, codebook)

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
        """Per-module K and codebook from the checkpoint headers (a local directory)."""
        if not model_name or not os.path.isdir(model_name):
            logger.info("exl3: %r is not a local directory; using the declared bits/codebook", model_name)
            return
        man = load_manifest(model_name)
        for key, m in man.matrices.items():
            if m.bits.is_half:
                raise NotImplementedError(f"{key}: half-integer K={m.bits.value} is not supported by the kernels")
            self.storage[module_key(key)] = (int(m.bits.value), m.codebook.value)
        logger.info("exl3: %d EXL3 modules from the checkpoint headers", len(self.storage))

    def _format_of(self, prefix: str) -> tuple[int, str] | None:
        parts = prefix.split(".")
        if "visual" in parts or "vision_tower" in parts:
            return None
        key = module_key(prefix)
        if not self.storage:
            if key.endswith("in_proj_ba"):
                return None
            return (self.head_bits if key == "lm_head" else int(self.bits)), self.codebook
        base, _, leaf = key.rpartition(".")
        names = [f"{base}.{m}" if base else m for m in FUSED.get(leaf, [leaf])]
        found = [self.storage.get(n) for n in names]
        if all(f is None for f in found):
            return None
        if any(f != found[0] for f in found):
            raise ValueError(f"exl3: fused module {prefix} mixes formats {found}")
        return found[0]

    def get_quant_method(self, layer: torch.nn.Module, prefix: str):
        if isinstance(layer, VLLM.LinearBase) or isinstance(layer, VLLM.ParallelLMHead):
            fmt = self._format_of(prefix)
            if fmt is None:
                return VLLM.UnquantizedLinearMethod() if isinstance(layer, VLLM.LinearBase) else None
            return Exl3LinearMethod(self, *fmt)
        return None


class Exl3LinearMethod(VLLM.LinearMethodBase):
    def __init__(self, config: Exl3Config, bits: int, codebook: str | None = None):
        self.config = config
        self.K = int(bits)
        self.codebook = codebook or config.codebook
        self.cb = CODEBOOK_ID[self.codebook]

    def create_weights(self, layer, input_size_per_partition, output_partition_sizes, input_size, output_size,
                       params_dtype, **extra_weight_attrs):
        k, n = input_size_per_partition, sum(output_partition_sizes)
        if k != input_size or (n != output_size and not isinstance(layer, VLLM.ParallelLMHead)):
            raise NotImplementedError("exl3: tensor-parallel sharding is not supported (one GPU per model)")
        if k % 128 or any(s % 128 for s in output_partition_sizes):
            raise ValueError(f"exl3: dims must be multiples of 128 (k={k}, n={list(output_partition_sizes)})")
        layer.exl3_sizes = list(output_partition_sizes)
        layer.exl3_offsets = [0]
        for s in output_partition_sizes:
            layer.exl3_offsets.append(layer.exl3_offsets[-1] + s)
        layer.exl3_groups = set()

        def param(name, tensor, loader):
            p = torch.nn.Parameter(tensor, requires_grad=False)
            p.weight_loader = loader
            layer.register_parameter(name, p)

        param("trellis", torch.empty((k // 16, n // 16, 16 * self.K), dtype=torch.int16), self._trellis_loader(layer))
        param("suh", torch.empty((len(output_partition_sizes), k), dtype=torch.float16), self._suh_loader(layer))
        param("svh", torch.empty((n,), dtype=torch.float16), self._svh_loader(layer))
        if self.codebook != "3inst":
            param(self.codebook, torch.empty((), dtype=torch.int32), lambda p, w, *a, **kw: p.data.copy_(w))

    @staticmethod
    def _partitions(layer, loaded, shard_id) -> list[int]:
        sid = getattr(loaded, "shard_id", None) if shard_id is None else shard_id
        if sid is None:
            return list(range(len(layer.exl3_sizes)))
        if isinstance(sid, str):
            return [QKV_INDEX[sid]]
        if isinstance(sid, int):
            return [sid]
        return [QKV_INDEX.get(s, s) for s in sid]

    def _span(self, layer, loaded, shard_id):
        parts = self._partitions(layer, loaded, shard_id)
        if parts != list(range(parts[0], parts[-1] + 1)):
            raise ValueError(f"exl3: shard partitions {parts} are not contiguous")
        return parts, layer.exl3_offsets[parts[0]], layer.exl3_offsets[parts[-1] + 1]

    def _trellis_loader(self, layer):
        def load(param, w, shard_id=None):
            parts, a, b = self._span(layer, w, shard_id)
            if w.dtype != torch.int16 or w.shape[-1] != param.shape[-1]:
                raise ValueError(f"exl3: trellis {tuple(w.shape)} {w.dtype} does not match K={self.K} "
                                 f"({tuple(param.shape)})")
            if w.shape[0] != param.shape[0] or w.shape[1] * 16 != b - a:
                raise ValueError(f"exl3: trellis {tuple(w.shape)} does not fit columns [{a}, {b})")
            param.data[:, a // 16: b // 16].copy_(w)
            layer.exl3_groups.add(tuple(parts))
        return load

    def _suh_loader(self, layer):
        def load(param, w, shard_id=None):
            parts, _, _ = self._span(layer, w, shard_id)
            for p in parts:
                param.data[p].copy_(w)
        return load

    def _svh_loader(self, layer):
        def load(param, w, shard_id=None):
            _, a, b = self._span(layer, w, shard_id)
            param.data[a:b].copy_(w)
        return load

    def process_weights_after_loading(self, layer) -> None:
        groups = sorted(layer.exl3_groups) or [tuple(range(len(layer.exl3_sizes)))]
        if [p for g in groups for p in g] != list(range(len(layer.exl3_sizes))):
            raise ValueError(f"exl3: incomplete shards {groups}")
        cb = 1 if hasattr(layer, "mcg") else 2 if hasattr(layer, "mul1") else self.cb
        dev = layer.trellis.device if layer.trellis.is_cuda else target_device()
        trs, suhs, svhs, widths = [], [], [], []
        for g in groups:
            a, b = layer.exl3_offsets[g[0]], layer.exl3_offsets[g[-1] + 1]
            trs.append(layer.trellis.data[:, a // 16: b // 16].to(dev).contiguous())
            suhs.append(layer.suh.data[g[0]].to(dev).contiguous())
            svhs.append(layer.svh.data[a:b].to(dev).contiguous())
            widths.append(b - a)
        for name in ("trellis", "suh", "svh"):
            delattr(layer, name)
        for i, (t, su, sv) in enumerate(zip(trs, suhs, svhs)):
            layer.register_buffer(f"exl3_trellis_{i}", t, persistent=False)
            layer.register_buffer(f"exl3_suh_{i}", su, persistent=False)
            layer.register_buffer(f"exl3_svh_{i}", sv, persistent=False)
        layer.exl3_count, layer.exl3_cb, layer.exl3_widths = len(groups), cb, widths
        layer.exl3_runs = launch_runs([self.K] * len(groups), [cb] * len(groups), widths, widths)
        if dev.type == "cuda":
            from .. import ops
            ops.init_device(dev.index if dev.index is not None else torch.cuda.current_device())

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        n = layer.exl3_count
        y = fused_forward(x, [getattr(layer, f"exl3_trellis_{i}") for i in range(n)],
                          [getattr(layer, f"exl3_suh_{i}") for i in range(n)],
                          [getattr(layer, f"exl3_svh_{i}") for i in range(n)],
                          [layer.exl3_cb] * n, layer.exl3_widths, layer.exl3_runs)
        return y if bias is None else y + bias

    def embedding(self, layer, input_):
        raise NotImplementedError("exl3: quantized input embeddings are not supported")


def register() -> None:
    """The `vllm.general_plugins` entry point: importing this module registers "exl3"."""
    return None
