"""Custom ops, one opaque op per layer kind, as in the reference (cuda/src/sglang_exl3/runtime/ops.py:1-137):
row-count dispatch, dtype handling and output allocation live inside the op so a tracing engine sees one node.

`torch.ops.exl3_mi355x.linear(x, trellis[], suh[], svh[], codebook)` -> y [..., sum n_s] in x's dtype.
Dispatch (the reference's `_linear`, runtime/ops.py:62-126, with MI355X switch points):
  rows < PREFILL_ROWS  -> fused decode-GEMV (exl3_linear, up to 32 rows per launch)
  rows >= PREFILL_ROWS -> fused decode-GEMM (exl3_linear_prefill)
PREFILL_ROWS comes from measured crossovers on the 27B shapes: the GEMV streams the weights once per 32 rows (two
16-row MFMA groups per decoded tile), the fused GEMM once for up to 256 rows.  Up to 48 rows the GEMV is faster on
every layer of the set; at 64 rows (two GEMV launches) only gate/up is faster on the GEMM and the set as a whole is
still faster on the GEMV (q/k/v 47.5 vs 50.3 us, o 42.0 vs 51.9, gate/up 102.5 vs 95.6, down 73.5 vs 74.9).
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
