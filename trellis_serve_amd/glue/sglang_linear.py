"""`Exl3LinearMethod` for SGLang linears and ParallelLMHead (cuda/src/sglang_exl3/sglang_glue/linear.py:66-197), and
`Exl3Dense` for a model's plain linear whose checkpoint tensors are EXL3 (linear.py:200-215).  The method itself is
`Exl3LinearCore` on SGLang's LinearMethodBase."""
from __future__ import annotations

import torch

from .engine import SGLANG
from .linear_method import Exl3LinearCore


class Exl3LinearMethod(Exl3LinearCore, SGLANG.LinearMethodBase):
    set_weight_attrs = staticmethod(SGLANG.set_weight_attrs)

    def __init__(self, prefix: str, infos: list):
        super().__init__(prefix, infos)


class Exl3Dense(torch.nn.Module):
    """An nn.Linear-like module over one EXL3 matrix (an MTP head's `fc`)."""

    def __init__(self, in_features: int, out_features: int, info, prefix: str,
                 params_dtype: torch.dtype = torch.bfloat16):
        super().__init__()
        self.method = Exl3LinearMethod(prefix, [info])
        self.method.create_weights(self, in_features, [out_features], in_features, out_features, params_dtype)

    def process_weights_after_loading(self) -> None:
        self.method.process_weights_after_loading(self)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.method.apply(self, x)
