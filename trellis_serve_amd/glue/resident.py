"""The resident form of an EXL3 layer: what the engines' `process_weights_after_loading` leaves on a layer and what
their `apply` runs, the same for SGLang and vLLM.

Dense (fused) linears keep one trellis, suh and svh buffer per source matrix, registered on the layer as
`exl3_{trellis,suh,svh}_{i}` (the buffers the reference registers, cuda/src/sglang_exl3/sglang_glue/linear.py:
145-152).  They are the only copy: the kernels read the stored layout (the load-time BLOCKS layout of
`ops.repack_trellis` measures the same, so no copy is made at load) and pointers are taken per call.  Consecutive source matrices with one bitrate and codebook run as one launch (up to EXL3_MAX_SHARDS), the
fused-group launch of cuda/csrc/exl3_marlin.cu:507-527.

Routed experts keep the stacked [E, ...] tensors `exl3_moe_forward` reads.

Both reserve their per-device workspaces at load for the engine's largest batch (`EXL3_MI355X_MAX_ROWS`, default
8192 rows or tokens), so `apply` never allocates one, also under graph capture (the reference reserves its scratch
at load, cuda/src/sglang_exl3/kernels/marlin.py:24-33).
"""
from __future__ import annotations

import os

import torch

from .stash import Exl3Matrix

MAX_LAUNCH_SHARDS = 4
MAX_ROWS = int(os.environ.get("EXL3_MI355X_MAX_ROWS", "8192"))


def launch_runs(bits: list[int], codebooks: list[int], widths: list[int], ns: list[int]) -> list[tuple[int, int]]:
    """Half-open index ranges of source matrices that share one launch: equal bitrate and codebook, no trimmed
    (padded) output columns, at most MAX_LAUNCH_SHARDS matrices."""
    runs: list[tuple[int, int]] = []
    for i, key in enumerate(zip(bits, codebooks)):
        padded = widths[i] != ns[i]
        if runs and not padded and i - runs[-1][0] < MAX_LAUNCH_SHARDS and runs[-1][2] == key and not runs[-1][3]:
            runs[-1] = (runs[-1][0], i + 1, key, False)
        else:
            runs.append((i, i + 1, key, padded))
    return [(a, b) for a, b, _, _ in runs]


def _device_index(dev: torch.device) -> int:
    return dev.index if dev.index is not None else torch.cuda.current_device()


class ResidentLinear:
    """Installs and runs the resident form of one (fused) EXL3 linear on a layer."""

    @staticmethod
    def install(layer: torch.nn.Module, matrices: list[Exl3Matrix], widths: list[int]) -> None:
        for i, m in enumerate(matrices):
            layer.register_buffer(f"exl3_trellis_{i}", m.trellis, persistent=False)
            layer.register_buffer(f"exl3_suh_{i}", m.suh, persistent=False)
            layer.register_buffer(f"exl3_svh_{i}", m.svh, persistent=False)
        layer.exl3_count = len(matrices)
        layer.exl3_codebooks = [m.codebook_id for m in matrices]
        layer.exl3_bits = [m.bits for m in matrices]
        layer.exl3_widths = list(widths)
        layer.exl3_runs = launch_runs(layer.exl3_bits, layer.exl3_codebooks, layer.exl3_widths,
                                      [m.n for m in matrices])
        dev = matrices[0].trellis.device
        if dev.type == "cuda":
            ResidentLinear.reserve(layer, dev)

    @staticmethod
    def reserve(layer: torch.nn.Module, dev: torch.device) -> None:
        """Workspaces of every launch of this layer: the decode-GEMV below the prefill switch point, the decode-GEMM
        up to MAX_ROWS rows."""
        from .. import ops
        from ..runtime.ops import PREFILL_ROWS
        ops.init_device(_device_index(dev))
        for a, b in layer.exl3_runs:
            k = getattr(layer, f"exl3_trellis_{a}").shape[0] * 16
            n_total = sum(getattr(layer, f"exl3_trellis_{i}").shape[1] * 16 for i in range(a, b))
            ops.reserve_linear(dev, PREFILL_ROWS - 1, k, n_total, layer.exl3_bits[a])
            ops.reserve_prefill(dev, MAX_ROWS, k, n_total, b - a)

    @staticmethod
    def forward(layer: torch.nn.Module, x: torch.Tensor) -> torch.Tensor:
        """y [..., sum(widths)] in x's dtype: one custom-op call per launch run (torch.ops.exl3_mi355x.linear picks
        the decode-GEMV or the decode-GEMM by rows), padded output columns trimmed."""
        from ..runtime import ops  # noqa: F401  (registers torch.ops.exl3_mi355x)
        parts = []
        for a, b in layer.exl3_runs:
            trellis = [getattr(layer, f"exl3_trellis_{i}") for i in range(a, b)]
            y = torch.ops.exl3_mi355x.linear(x, trellis, [getattr(layer, f"exl3_suh_{i}") for i in range(a, b)],
                                             [getattr(layer, f"exl3_svh_{i}") for i in range(a, b)],
                                             layer.exl3_codebooks[a])
            want = sum(layer.exl3_widths[a:b])
            parts.append(y if y.shape[-1] == want else y[..., :want])
        return parts[0] if len(parts) == 1 else torch.cat(parts, dim=-1)


MOE_ROLES = ("gate", "up", "down")


class ResidentExperts:
    """Installs and runs the stacked routed experts of one MoE layer."""

    @staticmethod
    def install(layer: torch.nn.Module, per_role: dict[str, list[Exl3Matrix]], top_k: int,
                device: torch.device) -> None:
        for role in MOE_ROLES:
            mats = per_role[role]
            for part in ("trellis", "suh", "svh"):
                stacked = torch.stack([getattr(m, part) for m in mats]).to(device).contiguous()
                layer.register_buffer(f"exl3_{role}_{part}", stacked, persistent=False)
        layer.exl3_codebook = per_role["gate"][0].codebook_id
        layer.exl3_bits = {role: per_role[role][0].bits for role in MOE_ROLES}
        if device.type == "cuda":
            from .. import ops
            ops.init_device(_device_index(device))
            g = layer.exl3_gate_trellis
            ops.reserve_moe(device, MAX_ROWS, top_k, g.shape[0], g.shape[1] * 16, g.shape[2] * 16,
                            layer.exl3_bits["gate"], layer.exl3_bits["down"])

    @staticmethod
    def tensors(layer: torch.nn.Module) -> dict[str, torch.Tensor]:
        from ..ops import MOE_TENSORS
        return {name: getattr(layer, f"exl3_{name}") for name in MOE_TENSORS}

    @staticmethod
    def forward(layer: torch.nn.Module, x: torch.Tensor, topk_ids: torch.Tensor,
                topk_weights: torch.Tensor) -> torch.Tensor:
        from .. import ops
        if x.shape[0] == 0:
            return torch.empty_like(x)
        return ops.moe_forward(x.contiguous(), topk_ids, topk_weights, ResidentExperts.tensors(layer),
                               layer.exl3_codebook)
