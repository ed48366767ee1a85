"""Pieces shared by the SGLang and vLLM method classes: checkpoint suffixes, legacy sign unpacking, shard ordering,
grouping of a fused module's matrices into launches, and the forward call."""
from __future__ import annotations

import torch

SUFFIXES = ("trellis", "suh", "svh", "su", "sv", "mcg", "mul1")
CODEBOOK_ID = {"3inst": 0, "mcg": 1, "mul1": 2}
QKV_INDEX = {"q": 0, "k": 1, "v": 2}
MAX_SHARDS_PER_LAUNCH = 4


def unpack_signs(packed: torch.Tensor) -> torch.Tensor:
    """Legacy su / sv: int16 words of sign bits, bit i of word w -> element 16 w + i, value 1 - 2 bit, fp16
    (cuda/src/sglang_exl3/sglang_glue/linear.py:61-63)."""
    words = packed.reshape(-1).to(torch.int32) & 0xFFFF
    bits = (words.unsqueeze(1) >> torch.arange(16, device=packed.device, dtype=torch.int32)) & 1
    return (1 - 2 * bits.reshape(-1)).to(torch.float16)


def partitions(shard_id) -> tuple[int, ...]:
    """The output partitions a loaded shard id covers: None -> all, "q"/"k"/"v" -> 0/1/2, ints, tuples of ints."""
    if shard_id is None:
        return ()
    if isinstance(shard_id, (tuple, list)):
        return tuple(QKV_INDEX.get(s, s) for s in shard_id)
    return (QKV_INDEX.get(shard_id, shard_id),)


def launch_runs(bits: list[int], codebooks: list[int], widths: list[int], ns: list[int]) -> list[tuple[int, int]]:
    """[start, end) runs of consecutive shards one fused launch serves: equal K and codebook, no trimmed padding,
    at most 4 shards (exl3_linear / exl3_linear_prefill take up to EXL3_MAX_SHARDS)."""
    runs, start = [], 0
    for i in range(1, len(bits) + 1):
        joinable = (i < len(bits) and i - start < MAX_SHARDS_PER_LAUNCH and (bits[i], codebooks[i]) ==
                    (bits[start], codebooks[start]) and widths[i] == ns[i] and widths[start] == ns[start])
        if not joinable:
            runs.append((start, i))
            start = i
    return runs


def fused_forward(x: torch.Tensor, trellis: list[torch.Tensor], suh: list[torch.Tensor], svh: list[torch.Tensor],
                  codebooks: list[int], widths: list[int], runs: list[tuple[int, int]]) -> torch.Tensor:
    """y [..., sum(widths)] in x's dtype: one custom-op call per launch run (torch.ops.exl3_mi355x.linear, which
    picks the decode-GEMV or the decode-GEMM by rows), padded output columns trimmed."""
    from ..runtime import ops  # noqa: F401  (registers torch.ops.exl3_mi355x)
    outs = []
    for s, e in runs:
        y = torch.ops.exl3_mi355x.linear(x, trellis[s:e], suh[s:e], svh[s:e], codebooks[s])
        full = sum(t.shape[1] * 16 for t in trellis[s:e])
        want = sum(widths[s:e])
        if want != full:  # a single padded shard (runs never join padded shards)
            y = y[..., :want]
        outs.append(y)
    return outs[0] if len(outs) == 1 else torch.cat(outs, dim=-1)
