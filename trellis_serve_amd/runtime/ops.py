"""Custom ops, one opaque op per layer kind, as in the reference (cuda/src/sglang_exl3/runtime/ops.py:1-137):
row-count dispatch, dtype handling and output allocation live inside the op so a tracing engine sees one node.

`torch.ops.exl3_mi355x.linear(x, trellis[], suh[], svh[], codebook)` -> y [..., sum n_s] in x's dtype.
Dispatch (the reference's `_linear`, runtime/ops.py:62-126, with MI355X switch points):
  rows < PREFILL_ROWS  -> fused decode-GEMV (exl3_linear, up to 64 rows per launch)
  rows >= PREFILL_ROWS -> fused decode-GEMM (exl3_linear_prefill)
PREFILL_ROWS comes from measured crossovers on the 27B shapes: the GEMV streams the weights once per 32 or 64 rows
(two or four 16-row MFMA groups per decoded tile), the fused GEMM once for up to 256 rows.  At 64 rows the layer set
is faster on the GEMV (q/k/v 39.3 vs 49.6 us, o 37.4 vs 51.6, gate/up 104.3 vs 96.5, down 74.3 vs 74.6), at 96 rows
on the GEMM (382 vs 308 us).
"""
from __future__ import annotations

import os

import torch

from .. import ops as _kernels

PREFILL_ROWS = int(os.environ.get("EXL3_MI355X_PREFILL_ROWS", "65"))

_lib = torch.library.Library("exl3_mi355x", "FRAGMENT")  # must stay alive at module scope


def _linear(x: torch.Tensor, trellis: list[torch.Tensor], suh: list[torch.Tensor], svh: list[torch.Tensor],
            codebook: int) -> torch.Tensor:
    rows = x.reshape(-1, x.shape[-1])
    n_total = sum(t.shape[1] * 16 for t in trellis)
    if rows.dtype not in (torch.float16, torch.bfloat16):   # an fp32 caller: explicit cast, as the reference does
        y = _linear(rows.to(torch.float16), trellis, suh, svh, codebook)
        return y.to(x.dtype).view(*x.shape[:-1], n_total)
    fn = _kernels.linear_prefill if rows.shape[0] >= PREFILL_ROWS else _kernels.linear
    y = fn(rows.contiguous(), trellis, suh, svh, codebook)
    return y.view(*x.shape[:-1], n_total)


def _linear_fake(x, trellis, suh, svh, codebook):
    return x.new_empty((*x.shape[:-1], sum(t.shape[1] * 16 for t in trellis)))


_lib.define("linear(Tensor x, Tensor[] trellis, Tensor[] suh, Tensor[] svh, int codebook) -> Tensor")
_lib.impl("linear", _linear, "CUDA")
torch.library.register_fake("exl3_mi355x::linear", _linear_fake, lib=_lib)

linear = torch.ops.exl3_mi355x.linear
