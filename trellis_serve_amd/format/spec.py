"""EXL3 on-disk format at the level of one quantized linear, derived from tensor names, dtypes and shapes only.

Same API as the reference's format layer (core/src/trellis_core/format/spec.py:1-160: `FormatError`, `Codebook`,
`BitsK`, `TensorInfo`, `MatrixSpec`, `build_matrix_spec`), so a loader written against it runs unchanged.  Pure
Python; nothing here touches tensor data or the GPU.

A quantized linear stored under module key `<key>` owns exactly these tensors (`<key>.<suffix>`):
  trellis  int16 [k/16, n/16, 8 * 2K]     packed codes, input dim first (spec.py:140-143)
  suh/svh  fp16 [k] / [n]                  sign * scale vectors, or the legacy packed sign bits su/sv int16
                                           [k/16] / [n/16] (spec.py:145-151)
  mcg|mul1 int32 scalar marker             codebook; neither means 3INST (spec.py:133-138)
  bias     fp16|fp32 [n]                   optional
k and n are multiples of the 128-wide Hadamard block.  K is the trellis last dim / 16 for integer bitrates; 1.5,
2.5 and 3.5 exist only with the MUL1 codebook (spec.py:52-67).
"""
from __future__ import annotations

import enum
from dataclasses import dataclass, field
from typing import Mapping

BLOCK = 128   # Hadamard block: both stored dims are multiples of it
TILE = 16     # trellis tile edge (256 weights per tile)

REQUIRED_TRELLIS = "trellis"
INPUT_SCALE = ("suh", "su")
OUTPUT_SCALE = ("svh", "sv")
MARKERS = ("mcg", "mul1")
KNOWN_SUFFIXES = frozenset((REQUIRED_TRELLIS, "bias") + INPUT_SCALE + OUTPUT_SCALE + MARKERS)


class FormatError(ValueError):
    """The tensors under a key do not form an EXL3 linear this library runs (spec.py:29-30)."""


class Codebook(enum.Enum):
    INST3 = "3inst"
    MCG = "mcg"
    MUL1 = "mul1"

    @property
    def abi_id(self) -> int:
        """The codebook argument of the C-ABI (include/exl3_mi355x.h): 0 = 3INST, 1 = MCG, 2 = MUL1."""
        return ("3inst", "mcg", "mul1").index(self.value)


@dataclass(frozen=True, order=True)
class BitsK:
    """Bits per weight K, kept doubled (`twice`) so the half-integer rates stay exact."""
    twice: int

    @property
    def value(self) -> float:
        return self.twice / 2

    @property
    def is_half(self) -> bool:
        return bool(self.twice & 1)

    @property
    def trellis_words(self) -> int:
        """int16 words per 16 x 16 tile: 16 K."""
        return 8 * self.twice

    @classmethod
    def from_trellis_words(cls, words: int, codebook: Codebook) -> "BitsK":
        twice, rem = divmod(int(words), 8)
        if rem or twice < 2 or twice > 16:
            raise FormatError(f"trellis last dim {words} is not a valid EXL3 bitrate (8 * 2K words, K in 1..8)")
        bits = cls(twice)
        if bits.is_half:
            if twice not in (3, 5, 7):
                raise FormatError(f"half-integer K={bits.value} is not defined (only 1.5, 2.5 and 3.5 exist)")
            if codebook is not Codebook.MUL1:
                raise FormatError(f"half-integer K={bits.value} requires the mul1 codebook, not {codebook.value}")
        return bits

    def __str__(self) -> str:
        return f"{self.value:g}"


@dataclass(frozen=True)
class TensorInfo:
    """One tensor of a safetensors shard: name, safetensors dtype string ("I16", "F16", ...), shape, the shard file,
    its byte size, and (this library's addition) the absolute byte offset of its data in that file (-1: unknown)."""
    name: str
    dtype: str
    shape: tuple[int, ...]
    file: str = ""
    nbytes: int = 0
    offset: int = -1


@dataclass(frozen=True)
class MatrixSpec:
    """One stored EXL3 linear: y = Had(Had(x * suh) @ W_inner) * svh (+ bias), k / n the stored (128-padded) widths."""
    key: str
    k: int
    n: int
    bits: BitsK
    codebook: Codebook
    has_bias: bool = False
    legacy_signs: bool = False
    tensors: Mapping[str, TensorInfo] = field(default_factory=dict, compare=False, repr=False)

    @property
    def nbytes(self) -> int:
        return sum(t.nbytes for t in self.tensors.values())

    def same_kernel_class(self, other: "MatrixSpec") -> bool:
        """Both can run in one grouped launch (same shape, bitrate and codebook)."""
        return (self.k, self.n, self.bits, self.codebook) == (other.k, other.n, other.bits, other.codebook)


def _expect(info: TensorInfo, dtype: str | tuple[str, ...], shapes: tuple[tuple[int, ...], ...]) -> None:
    dtypes = (dtype,) if isinstance(dtype, str) else dtype
    if info.dtype not in dtypes or tuple(info.shape) not in shapes:
        want = "/".join(dtypes)
        raise FormatError(f"{info.name}: expected {want} {' or '.join(map(str, shapes))}, got {info.dtype} "
                          f"{tuple(info.shape)}")


def _exactly_one(tensors: Mapping[str, TensorInfo], choices: tuple[str, str], key: str) -> str:
    found = [c for c in choices if c in tensors]
    if len(found) != 1:
        raise FormatError(f"{key}: expected exactly one of {choices}, found {found if found else 'none'}")
    return found[0]


def build_matrix_spec(key: str, tensors: Mapping[str, TensorInfo]) -> MatrixSpec:
    """Validates the tensors stored under `key` (suffix -> TensorInfo) and describes the linear.

    Rejects anything outside the stock structure (unknown suffixes, nested derivatives, wrong dtypes or shapes),
    never on a declared version number (spec.py:109-160)."""
    extra = sorted(set(tensors) - KNOWN_SUFFIXES)
    if extra:
        raise FormatError(f"{key}: unknown tensors {extra} under an EXL3 linear (a derivative or newer format)")
    if REQUIRED_TRELLIS not in tensors:
        raise FormatError(f"{key}: no .trellis tensor")
    tr = tensors[REQUIRED_TRELLIS]
    if tr.dtype != "I16" or len(tr.shape) != 3:
        raise FormatError(f"{key}.trellis: expected a 3-D I16 tensor, got {tr.dtype} {tuple(tr.shape)}")

    markers = [m for m in MARKERS if m in tensors]
    if len(markers) > 1:
        raise FormatError(f"{key}: both .mcg and .mul1 markers present")
    for m in markers:
        _expect(tensors[m], "I32", ((), (1,)))
    codebook = Codebook(markers[0]) if markers else Codebook.INST3

    k, n = tr.shape[0] * TILE, tr.shape[1] * TILE
    if k % BLOCK or n % BLOCK:
        raise FormatError(f"{key}: stored dims ({k}, {n}) are not multiples of {BLOCK}")
    bits = BitsK.from_trellis_words(tr.shape[2], codebook)

    sin = _exactly_one(tensors, INPUT_SCALE, key)
    sout = _exactly_one(tensors, OUTPUT_SCALE, key)
    if (sin == "su") != (sout == "sv"):
        raise FormatError(f"{key}: mixed legacy/modern scale tensors ({sin}, {sout})")
    legacy = sin == "su"
    if legacy:
        _expect(tensors["su"], "I16", ((k // TILE,),))
        _expect(tensors["sv"], "I16", ((n // TILE,),))
    else:
        _expect(tensors["suh"], "F16", ((k,),))
        _expect(tensors["svh"], "F16", ((n,),))
    if "bias" in tensors:
        _expect(tensors["bias"], ("F16", "F32"), ((n,),))
    return MatrixSpec(key=key, k=k, n=n, bits=bits, codebook=codebook, has_bias="bias" in tensors,
                      legacy_signs=legacy, tensors=dict(tensors))
