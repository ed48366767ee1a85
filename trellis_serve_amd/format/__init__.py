"""EXL3 checkpoint format: tensor specs, safetensors headers, manifest, fused layouts.  Pure Python (numpy only for
`read_tensor`); the API of the reference's trellis_core.format (core/src/trellis_core/format/__init__.py:1-9), minus
the tensor-parallel slicing helpers (geometry.py), which no single-GPU path uses."""
from .layout import FusedLayout, FusionKind, LogicalMatrix, make_layout
from .manifest import Manifest, build_manifest, load_manifest
from .safetensors_header import ShardHeader, parse_header, read_header, read_tensor
from .spec import BitsK, Codebook, FormatError, MatrixSpec, TensorInfo, build_matrix_spec

__all__ = ["BitsK", "Codebook", "FormatError", "FusedLayout", "FusionKind", "LogicalMatrix", "Manifest",
           "MatrixSpec", "ShardHeader", "TensorInfo", "build_manifest", "build_matrix_spec", "load_manifest",
           "make_layout", "parse_header", "read_header", "read_tensor"]
