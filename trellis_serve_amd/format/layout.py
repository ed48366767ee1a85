"""Fused runtime modules as ordered groups of stored EXL3 linears.

Same API as core/src/trellis_core/format/layout.py:1-76 (`LogicalMatrix`, `FusionKind`, `FusedLayout`,
`make_layout`).  Engines fuse q/k/v or gate/up into one module; in EXL3 every source matrix keeps its own suh and
may have its own K and codebook, so a fused module is a list of matrices sharing the input and writing adjacent
output spans.  `exl3_linear` / `exl3_linear_prefill` run up to 4 such matrices in one launch when they share K and
the codebook (their n may differ); other groups run one launch per run of equal (K, codebook).
"""
from __future__ import annotations

import enum
from dataclasses import dataclass
from typing import Hashable, Sequence

from .spec import MatrixSpec


@dataclass(frozen=True)
class LogicalMatrix:
    shard_id: Hashable   # the engine's id of this source: "q" / "k" / "v", 0 / 1, or None
    spec: MatrixSpec
    out_width: int       # output columns this source contributes (spec.n minus trailing padding)


class FusionKind(enum.Enum):
    SINGLE = "single"
    UNIFORM = "uniform"         # equal shapes, K and codebook
    SHARD_MAP = "shard_map"     # shared input width, per-shard n / K / codebook
    SEQUENTIAL = "sequential"   # one launch per matrix into slices of one output


@dataclass(frozen=True)
class FusedLayout:
    matrices: tuple[LogicalMatrix, ...]

    def __post_init__(self):
        if not self.matrices:
            raise ValueError("a fused layout needs at least one matrix")
        ks = sorted({m.spec.k for m in self.matrices})
        if len(ks) != 1:
            raise ValueError(f"fused matrices must share their input width, got {ks}")
        for m in self.matrices:
            if m.out_width <= 0 or m.out_width > m.spec.n:
                raise ValueError(f"{m.spec.key}: out_width {m.out_width} does not fit stored width {m.spec.n}")

    @property
    def in_width(self) -> int:
        return self.matrices[0].spec.k

    @property
    def out_width(self) -> int:
        return sum(m.out_width for m in self.matrices)

    def spans(self) -> list[tuple[int, int]]:
        """(offset, width) of every matrix in the fused output, in order."""
        spans, at = [], 0
        for m in self.matrices:
            spans.append((at, m.out_width))
            at += m.out_width
        return spans

    @property
    def best_fusion(self) -> FusionKind:
        if len(self.matrices) == 1:
            return FusionKind.SINGLE
        first = self.matrices[0].spec
        if all(m.spec.same_kernel_class(first) and m.out_width == m.spec.n for m in self.matrices):
            return FusionKind.UNIFORM
        return FusionKind.SHARD_MAP

    def launch_runs(self) -> list[tuple[int, int]]:
        """[start, end) index runs of consecutive matrices that one `exl3_linear` launch can serve: equal K and
        codebook, no trimmed padding, at most 4 per run."""
        runs, start = [], 0
        for i in range(1, len(self.matrices) + 1):
            if i == len(self.matrices) or i - start == 4 or not self._joinable(start, i):
                runs.append((start, i))
                start = i
        return runs

    def _joinable(self, start: int, i: int) -> bool:
        a, b = self.matrices[start], self.matrices[i]
        full = all(m.out_width == m.spec.n for m in (a, b))
        return full and (a.spec.bits, a.spec.codebook) == (b.spec.bits, b.spec.codebook)


def make_layout(shard_ids: Sequence[Hashable], specs: Sequence[MatrixSpec], out_widths: Sequence[int]) -> FusedLayout:
    if not len(shard_ids) == len(specs) == len(out_widths):
        raise ValueError("shard_ids, specs and out_widths must have the same length")
    return FusedLayout(tuple(LogicalMatrix(s, m, int(w)) for s, m, w in zip(shard_ids, specs, out_widths)))
