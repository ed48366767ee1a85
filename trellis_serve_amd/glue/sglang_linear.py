"""`Exl3LinearMethod` for SGLang linears and ParallelLMHead, running on this library.

Contract of cuda/src/sglang_exl3/sglang_glue/linear.py:66-197:
  create_weights        registers a 0-byte uint8 placeholder per checkpoint suffix (trellis, suh, svh, su, sv, mcg,
                        mul1) with a `weight_loader`, so the model's unmodified `load_weights` routes
                        `<layer>.<suffix>` (+ shard id) here; TP or bias raise NotImplementedError (74-77).
  weight_loader         keeps each loaded tensor whole, per shard id, on the current device; a second load of the
                        same (suffix, shard) raises ValueError (97-105).
  process_weights_after_loading
                        orders the shards, checks shape / K / codebook against the header scan (126-128), converts
                        legacy sign bits (120-122), registers `exl3_{trellis,suh,svh}_{i}` buffers (145-152).
  apply(layer, x, bias) x fp16|bf16 [..., k] -> [..., sum of output widths] in x's dtype (185-197).
No repack: the kernels read the stored trellis directly, so the trellis buffers are the only resident copy and stay
in place (pointers are taken per call).
"""
from __future__ import annotations

import logging

import torch

from .common import CODEBOOK_ID, SUFFIXES, fused_forward, launch_runs, partitions, unpack_signs
from .engine import SGLANG, target_device

logger = logging.getLogger(__name__)


def _shard_order(sid):
    p = partitions(sid)
    return p if p else (0,)


class Exl3LinearMethod(SGLANG.LinearMethodBase):
    def __init__(self, prefix: str, infos: list[tuple]):
        self.prefix = prefix
        self.infos = list(infos)   # per source matrix: (k, n, 2K, codebook, has_bias, legacy_signs)

    # ---- weights
    def create_weights(self, layer, input_size_per_partition, output_partition_sizes, input_size, output_size,
                       params_dtype, **extra_weight_attrs):
        if input_size_per_partition != input_size or sum(output_partition_sizes) != output_size:
            raise NotImplementedError(f"{self.prefix}: tensor-parallel EXL3 is not implemented (one GPU per model)")
        if any(info[4] for info in self.infos):
            raise NotImplementedError(f"{self.prefix}: EXL3 linears with bias are not implemented")
        layer.exl3_out_sizes = list(output_partition_sizes)
        layer.exl3_in_size = input_size
        layer.exl3_shards = {s: {} for s in SUFFIXES}
        for suffix in SUFFIXES:
            p = torch.nn.Parameter(torch.empty(0, dtype=torch.uint8), requires_grad=False)
            SGLANG.set_weight_attrs(p, {"weight_loader": self._loader(layer, suffix), "exl3_placeholder": True})
            layer.register_parameter(suffix, p)
        if not hasattr(layer, "weight"):
            # an lm_head: engines read `.weight` (rows = vocabulary); a zero-width placeholder satisfies them
            w = torch.nn.Parameter(torch.empty((sum(output_partition_sizes), 0), dtype=params_dtype),
                                   requires_grad=False)
            SGLANG.set_weight_attrs(w, {"weight_loader": self._ignore, "exl3_placeholder": True})
            layer.register_parameter("weight", w)

    @staticmethod
    def _ignore(param, loaded_weight, *args, **kwargs):
        logger.warning("EXL3: a dense .weight for a quantized layer was ignored (shape %s)", tuple(loaded_weight.shape))

    def _loader(self, layer, suffix: str):
        def load(param, loaded_weight, loaded_shard_id=None, *args, **kwargs):
            store = layer.exl3_shards[suffix]
            sid = tuple(loaded_shard_id) if isinstance(loaded_shard_id, list) else loaded_shard_id
            if sid in store:
                raise ValueError(f"{self.prefix}.{suffix}: shard {sid!r} loaded twice")
            store[sid] = loaded_weight.detach().to(target_device(), copy=True)
        return load

    def process_weights_after_loading(self, layer) -> None:
        got = layer.exl3_shards
        ids = sorted(got["trellis"], key=_shard_order)
        if not ids:
            logger.warning("%s: no EXL3 tensors were delivered; the layer stays empty", self.prefix)
            layer.exl3_count = 0
            return
        if len(ids) != len(self.infos):
            raise ValueError(f"{self.prefix}: expected {len(self.infos)} EXL3 matrices, the checkpoint delivered "
                             f"{len(ids)} ({ids})")
        codebooks, bits, widths, ns = [], [], [], []
        for i, sid in enumerate(ids):
            suh, svh = got["suh"].get(sid), got["svh"].get(sid)
            if suh is None and sid in got["su"] and sid in got["sv"]:
                suh, svh = unpack_signs(got["su"][sid]), unpack_signs(got["sv"][sid])
            if suh is None or svh is None:
                raise ValueError(f"{self.prefix}: shard {sid!r} has a trellis but no scale vectors")
            cb = "mcg" if sid in got["mcg"] else "mul1" if sid in got["mul1"] else "3inst"
            tr = got["trellis"][sid].contiguous()
            k, n, twice, declared = self.infos[i][:4]
            found = (tr.shape[0] * 16, tr.shape[1] * 16, tr.shape[2] // 8, cb)
            if found != (k, n, twice, declared):
                raise ValueError(f"{self.prefix}: shard {sid!r} {tuple(tr.shape)}/{cb} does not match the header scan "
                                 f"{(k, n, twice, declared)}")
            if twice % 2:
                raise NotImplementedError(f"{self.prefix}: half-integer K={twice / 2} is not supported by the kernels")
            parts = partitions(sid)
            widths.append(sum(layer.exl3_out_sizes[p] for p in parts) if parts else sum(layer.exl3_out_sizes))
            ns.append(n)
            bits.append(twice // 2)
            codebooks.append(CODEBOOK_ID[cb])
            layer.register_buffer(f"exl3_trellis_{i}", tr, persistent=False)
            layer.register_buffer(f"exl3_suh_{i}", suh.to(torch.float16).contiguous(), persistent=False)
            layer.register_buffer(f"exl3_svh_{i}", svh.to(torch.float16).contiguous(), persistent=False)
        if sum(widths) != sum(layer.exl3_out_sizes):
            raise ValueError(f"{self.prefix}: the shards cover {sum(widths)} of {sum(layer.exl3_out_sizes)} output "
                             f"columns")
        for suffix in SUFFIXES:
            delattr(layer, suffix)
        del layer.exl3_shards
        layer.exl3_count, layer.exl3_codebooks, layer.exl3_bits, layer.exl3_widths = len(ids), codebooks, bits, widths
        layer.exl3_runs = launch_runs(bits, codebooks, widths, ns)
        dev = layer.exl3_trellis_0.device
        if dev.type == "cuda":
            from .. import ops
            ops.init_device(dev.index if dev.index is not None else torch.cuda.current_device())

    # ---- forward
    def apply(self, layer, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        n = getattr(layer, "exl3_count", 0)
        if n == 0:
            raise RuntimeError(f"{self.prefix}: EXL3 layer has no weights (never loaded)")
        y = fused_forward(x, [getattr(layer, f"exl3_trellis_{i}") for i in range(n)],
                          [getattr(layer, f"exl3_suh_{i}") for i in range(n)],
                          [getattr(layer, f"exl3_svh_{i}") for i in range(n)],
                          layer.exl3_codebooks, layer.exl3_widths, layer.exl3_runs)
        return y if bias is None else y + bias


class Exl3Dense(torch.nn.Module):
    """Stand-in for a plain nn.Linear whose checkpoint tensors are EXL3 (e.g. an MTP head's `fc`), the reference's
    Exl3Dense (linear.py:200-215)."""

    def __init__(self, in_features: int, out_features: int, info: tuple, prefix: str,
                 params_dtype: torch.dtype = torch.bfloat16):
        super().__init__()
        self.method = Exl3LinearMethod(prefix, [info])
        self.method.create_weights(self, in_features, [out_features], in_features, out_features, params_dtype)

    def process_weights_after_loading(self) -> None:
        self.method.process_weights_after_loading(self)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.method.apply(self, x)
