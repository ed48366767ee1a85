"""The EXL3 linear method both engines run, apart from the engine base class it is registered under.

Engine calls (the contract of cuda/src/sglang_exl3/sglang_glue/linear.py:66-197 and
xpu/exl3xpu/vllm_plugin.py:150-261):
  create_weights   a placeholder parameter per checkpoint suffix, so the model's unmodified `load_weights` delivers
                   `<layer>.<suffix>` (+ shard id) into the layer's TensorStash; tensor parallelism and bias raise
                   NotImplementedError.
  process_weights_after_loading
                   one checked Exl3Matrix per source matrix (ordered by output partition), installed in resident form.
  apply            x fp16|bf16 [..., k] -> [..., sum of output widths] in x's dtype.
The trellis stays in its stored layout (the kernels read it directly; the BLOCKS layout of `ops.repack_trellis`
measures the same, so nothing is copied at load) and nothing is pre-decoded.

What a source matrix must look like comes from the checkpoint headers (`infos`, one MatrixInfo per source in output
order) or, for a vLLM model whose directory is not local, from the declared bitrate only (`declared_bits`): the
shapes then follow the layer, the codebook the checkpoint's marker tensors.
"""
from __future__ import annotations

import functools
import logging

import torch

from .engine import target_device
from .resident import ResidentLinear
from .stash import (SUFFIXES, MatrixInfo, TensorStash, attach_placeholders, detach_placeholders,
                    shard_partitions)

logger = logging.getLogger(__name__)


def _deliver(stash: TensorStash, suffix: str, param, loaded_weight, loaded_shard_id=None, *args, **kwargs) -> None:
    """The placeholders' weight_loader: the engine's (param, tensor, shard id) call, stashed by partitions."""
    stash.put(shard_partitions(loaded_shard_id), suffix, loaded_weight)


def _dense_weight_ignored(param, loaded_weight, *args, **kwargs) -> None:
    logger.warning("EXL3: a dense .weight for a quantized layer was ignored (shape %s)", tuple(loaded_weight.shape))


class Exl3LinearCore:
    """Mixed into the engine's LinearMethodBase; a subclass sets `set_weight_attrs` to the engine's."""

    set_weight_attrs = staticmethod(lambda param, attrs: None)

    def __init__(self, prefix: str, infos: list | None = None, declared_bits: int | None = None):
        if infos is None and declared_bits is None:
            raise ValueError(f"{prefix}: an EXL3 linear needs header entries or a declared bitrate")
        self.prefix = prefix
        self.infos = None if infos is None else [MatrixInfo(*i) for i in infos]
        self.declared_bits = declared_bits

    def create_weights(self, layer, input_size_per_partition, output_partition_sizes, input_size, output_size,
                       params_dtype, **extra_weight_attrs):
        if (input_size_per_partition, sum(output_partition_sizes)) != (input_size, output_size):
            raise NotImplementedError(f"{self.prefix}: tensor-parallel EXL3 is not implemented (one GPU per model)")
        if self.infos is not None and any(i.has_bias for i in self.infos):
            raise NotImplementedError(f"{self.prefix}: EXL3 linears with bias are not implemented")
        layer.exl3_in_size = input_size
        layer.exl3_out_sizes = list(output_partition_sizes)
        layer.exl3_stash = TensorStash(self.prefix, target_device())
        set_attrs = self.set_weight_attrs
        attach_placeholders(layer, SUFFIXES, lambda s: functools.partial(_deliver, layer.exl3_stash, s), set_attrs)
        if not hasattr(layer, "weight"):
            # lm_head: the engine reads `.weight` (vocabulary rows) and slices rows of it for a draft's hot-token
            # head; a zero-width placeholder serves both (linear.py:80-88)
            w = torch.nn.Parameter(torch.empty((sum(output_partition_sizes), 0), dtype=params_dtype),
                                   requires_grad=False)
            set_attrs(w, {"weight_loader": _dense_weight_ignored, "exl3_placeholder": True})
            layer.register_parameter("weight", w)

    def _check_declared(self, layer, key, m) -> None:
        sizes = layer.exl3_out_sizes
        width = sum(sizes[p] for p in key) if key else sum(sizes)
        if m.k != layer.exl3_in_size or m.n < width or m.n - width >= 128:
            raise ValueError(f"{self.prefix}: shard {key!r} is {m.k} x {m.n}, the layer expects {layer.exl3_in_size} "
                             f"x {width} (stored widths pad to 128)")
        if m.bits != self.declared_bits:
            raise ValueError(f"{self.prefix}: shard {key!r} holds K={m.bits}, the model config declares "
                             f"K={self.declared_bits}")

    def process_weights_after_loading(self, layer) -> None:
        stash: TensorStash = layer.exl3_stash
        sizes = layer.exl3_out_sizes
        keys = sorted(stash.keys(), key=lambda parts: parts or (0,))
        if self.infos is not None:
            if keys and len(keys) != len(self.infos):
                raise ValueError(f"{self.prefix}: expected {len(self.infos)} EXL3 matrices, the checkpoint delivered "
                                 f"{len(keys)} (partitions {keys})")
            matrices = [stash.matrix(key, info) for key, info in zip(keys, self.infos)]
        else:
            matrices = [stash.matrix(key) for key in keys]
            for key, m in zip(keys, matrices):
                self._check_declared(layer, key, m)
        widths = [sum(sizes[p] for p in key) if key else sum(sizes) for key in keys]
        if keys and sum(widths) != sum(sizes):
            raise ValueError(f"{self.prefix}: the matrices cover {sum(widths)} of {sum(sizes)} output columns")
        detach_placeholders(layer, SUFFIXES)
        stash.clear()
        del layer.exl3_stash
        if not keys:
            # a draft model's own lm_head, replaced by the target's and never loaded (linear.py:110-113)
            logger.warning("%s: no EXL3 tensors were delivered; the layer stays empty", self.prefix)
            layer.exl3_count = 0
            return
        ResidentLinear.install(layer, matrices, widths)

    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        if not getattr(layer, "exl3_count", 0):
            raise RuntimeError(f"{self.prefix}: EXL3 layer has no weights (never loaded)")
        y = ResidentLinear.forward(layer, x)
        return y if bias is None else y + bias
