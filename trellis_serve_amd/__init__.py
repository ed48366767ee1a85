"""MI355X-native (gfx950) EXL3 hot path: trellis decode, fused decode-GEMV/GEMM, Hadamard rotations, MoE and
quantized-KV decode attention, behind the reference's plugin surface (0xSero/trellis-serve)."""
from ._lib import ExtensionMissing, Exl3Error  # noqa: F401

__version__ = "0.1.0"
