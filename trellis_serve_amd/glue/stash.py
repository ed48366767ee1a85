"""Staging of checkpoint tensors between an engine's `load_weights` and `process_weights_after_loading`.

An engine hands a layer its checkpoint tensors one at a time, through the `weight_loader` of a placeholder parameter
named like the checkpoint suffix, with a shard id (a fused linear's partition, or an MoE projection and expert).
Nothing can be checked until every tensor of a matrix is in, so a `TensorStash` keeps them keyed by
(matrix key, suffix) and `matrix()` assembles one matrix once loading is over:

  * the +-1 sign vectors come stored (`suh` / `svh`) or as legacy sign words (`su` / `sv`, bit i of word w is
    element 16 w + i, value 1 - 2 bit);
  * the codebook is named by a marker tensor (`mcg` / `mul1`; none means 3INST);
  * shape, bitrate and codebook are checked against what the checkpoint's headers declared for that matrix.

This is the loading contract of the reference's engine glue (cuda/src/sglang_exl3/sglang_glue/linear.py:93-128,
moe.py:95-160); the code here is organised around the stash instead of per-engine copies.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Hashable, NamedTuple

import torch

SUFFIXES = ("trellis", "suh", "svh", "su", "sv", "mcg", "mul1")
CODEBOOK_ID = {"3inst": 0, "mcg": 1, "mul1": 2}


class MatrixInfo(NamedTuple):
    """What the checkpoint headers say about one EXL3 matrix (a tuple, as the header scan stores it)."""
    k: int
    n: int
    twice_bits: int       # 2K: the format allows half-integer K (MUL1 only)
    codebook: str
    has_bias: bool = False
    legacy_signs: bool = False


@dataclass
class Exl3Matrix:
    """One decoded-to-be EXL3 matrix: trellis int16 [k/16, n/16, 16K], suh fp16 [k], svh fp16 [n]."""
    trellis: torch.Tensor
    suh: torch.Tensor
    svh: torch.Tensor
    codebook: str

    @property
    def k(self) -> int:
        return self.trellis.shape[0] * 16

    @property
    def n(self) -> int:
        return self.trellis.shape[1] * 16

    @property
    def bits(self) -> int:
        return self.trellis.shape[2] // 16

    @property
    def codebook_id(self) -> int:
        return CODEBOOK_ID[self.codebook]

    def describe(self) -> tuple:
        return (self.k, self.n, self.trellis.shape[2] // 8, self.codebook)


QKV_PARTITION = {"q": 0, "k": 1, "v": 2}


def shard_partitions(shard_id) -> tuple[int, ...]:
    """The output partitions of a fused linear that one loaded shard fills, as the stash key of its matrix: None ->
    () (the whole layer), 'q' / 'k' / 'v' -> 0 / 1 / 2, an int, or a sequence of those (a checkpoint matrix that
    spans several partitions, e.g. GDN in_proj_qkv) (cuda/src/sglang_exl3/sglang_glue/linear.py:48-53)."""
    if shard_id is None:
        return ()
    items = shard_id if isinstance(shard_id, (tuple, list)) else (shard_id,)
    return tuple(int(QKV_PARTITION.get(s, s)) for s in items)


def attach_placeholders(layer: torch.nn.Module, names, loader_of, set_weight_attrs) -> None:
    """Registers a 0-byte uint8 parameter per name whose `weight_loader` is `loader_of(name)`: the engine's
    unmodified `load_weights` then hands each checkpoint tensor `<layer>.<name>` to that loader
    (linear.py:84-88, moe.py:89-93)."""
    for name in names:
        p = torch.nn.Parameter(torch.empty(0, dtype=torch.uint8), requires_grad=False)
        set_weight_attrs(p, {"weight_loader": loader_of(name), "exl3_placeholder": True})
        layer.register_parameter(name, p)


def detach_placeholders(layer: torch.nn.Module, names) -> None:
    for name in names:
        if hasattr(layer, name):
            delattr(layer, name)


def unpack_signs(words: torch.Tensor) -> torch.Tensor:
    """Legacy sign words (int16, bit i of word w = element 16 w + i) -> fp16 +-1 (1 - 2 bit)
    (cuda/src/sglang_exl3/sglang_glue/linear.py:61-63)."""
    w = words.reshape(-1).to(torch.int32) & 0xFFFF
    shifts = torch.arange(16, dtype=torch.int32, device=words.device)
    bit = (w[:, None] >> shifts) & 1
    return (1 - 2 * bit).reshape(-1).to(torch.float16)


class TensorStash:
    """Checkpoint tensors of one layer, by (matrix key, suffix), until the layer is complete.

    `where` places each delivered tensor (the GPU the layer runs on, or the CPU for experts that are stacked later);
    `owner` names the layer in error messages."""

    def __init__(self, owner: str, where: torch.device | str):
        self.owner = owner
        self.where = torch.device(where)
        self._held: dict[tuple[Hashable, str], torch.Tensor] = {}

    def put(self, key: Hashable, suffix: str, tensor: torch.Tensor) -> None:
        if suffix not in SUFFIXES:
            raise ValueError(f"{self.owner}: {suffix!r} is not an EXL3 checkpoint suffix")
        if (key, suffix) in self._held:
            raise ValueError(f"{self.owner}.{suffix}: a second tensor for shard {key!r}")
        self._held[(key, suffix)] = tensor.detach().to(self.where, copy=True)

    def keys(self) -> list:
        """Matrix keys that received a trellis."""
        return [key for key, suffix in self._held if suffix == "trellis"]

    def has(self, key: Hashable, suffix: str) -> bool:
        return (key, suffix) in self._held

    def matrix(self, key: Hashable, declared: MatrixInfo | tuple | None = None) -> Exl3Matrix:
        """The matrix under `key`, checked against the header scan's `declared` (k, n, 2K, codebook, ...)."""
        get = self._held.get
        trellis = get((key, "trellis"))
        if trellis is None:
            raise ValueError(f"{self.owner}: no trellis arrived for {key!r}")
        suh, svh = get((key, "suh")), get((key, "svh"))
        if suh is None and svh is None and get((key, "su")) is not None and get((key, "sv")) is not None:
            suh, svh = unpack_signs(get((key, "su"))), unpack_signs(get((key, "sv")))
        if suh is None or svh is None:
            raise ValueError(f"{self.owner}: shard {key!r}: trellis without suh/svh (or legacy su/sv) sign vectors")
        codebook = "mcg" if self.has(key, "mcg") else "mul1" if self.has(key, "mul1") else "3inst"
        m = Exl3Matrix(trellis.contiguous(), suh.to(torch.float16).contiguous(), svh.to(torch.float16).contiguous(),
                       codebook)
        if declared is not None and m.describe() != tuple(declared[:4]):
            raise ValueError(f"{self.owner}: shard {key!r} arrived as {m.describe()} (k, n, 2K, codebook), the "
                             f"checkpoint header declares {tuple(declared[:4])}")
        if m.suh.numel() != m.k or m.svh.numel() != m.n:
            raise ValueError(f"{self.owner}: shard {key!r} sign vectors hold {m.suh.numel()} / {m.svh.numel()} "
                             f"values for a {m.k} x {m.n} matrix")
        if m.trellis.shape[2] % 16:
            raise NotImplementedError(f"{self.owner}: half-integer K={m.trellis.shape[2] / 16} is not supported by "
                                      f"the kernels")
        return m

    def clear(self) -> None:
        self._held.clear()
