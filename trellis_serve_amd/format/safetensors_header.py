"""safetensors header reader and raw tensor-data reader.

Header: same API as core/src/trellis_core/format/safetensors_header.py:1-54 (`ShardHeader`, `parse_header`,
`read_header`).  A shard is an 8-byte little-endian header length, a JSON header (name -> dtype, shape, data_offsets
relative to the end of the header, plus an optional `__metadata__` map) and the raw data; the header alone describes
every tensor, so a manifest of a very large checkpoint costs only header reads.

Data: `read_tensor` maps one tensor's byte range with numpy (no pickle, nothing executed from the file).
"""
from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass

import numpy as np

from .spec import FormatError, TensorInfo

MAX_HEADER_BYTES = 1 << 30
_NUMPY_DTYPE = {"I8": np.int8, "U8": np.uint8, "I16": np.int16, "U16": np.uint16, "I32": np.int32,
                "U32": np.uint32, "I64": np.int64, "F16": np.float16, "F32": np.float32, "F64": np.float64,
                "BF16": np.uint16, "BOOL": np.bool_}


@dataclass(frozen=True)
class ShardHeader:
    file: str
    metadata: dict[str, str]
    tensors: dict[str, TensorInfo]


def parse_header(raw: bytes, file: str = "", data_start: int = -1) -> ShardHeader:
    """Parses the JSON header bytes of one shard.  `data_start` (the file offset of the data section, 8 + header
    length) makes each TensorInfo carry its absolute data offset; -1 leaves the offsets unknown."""
    try:
        doc = json.loads(raw)
    except ValueError as e:
        raise FormatError(f"{file}: safetensors header is not valid JSON: {e}") from None
    if not isinstance(doc, dict):
        raise FormatError(f"{file}: safetensors header is not a JSON object")
    metadata = doc.pop("__metadata__", None) or {}
    tensors: dict[str, TensorInfo] = {}
    for name, entry in doc.items():
        try:
            begin, end = (int(v) for v in entry["data_offsets"])
            dtype, shape = entry["dtype"], tuple(int(d) for d in entry["shape"])
        except (KeyError, TypeError, ValueError):
            raise FormatError(f"{file}: {name}: malformed header entry {entry!r}") from None
        if end < begin:
            raise FormatError(f"{file}: {name}: data_offsets [{begin}, {end}) is reversed")
        tensors[name] = TensorInfo(name=name, dtype=dtype, shape=shape, file=file, nbytes=end - begin,
                                   offset=data_start + begin if data_start >= 0 else -1)
    return ShardHeader(file=file, metadata=dict(metadata), tensors=tensors)


def read_header(path: str | os.PathLike) -> ShardHeader:
    """Reads and parses the header of the shard at `path`; TensorInfo.file is the file's base name."""
    path = os.fspath(path)
    with open(path, "rb") as f:
        head = f.read(8)
        if len(head) != 8:
            raise FormatError(f"{path}: too short to be a safetensors file")
        (length,) = struct.unpack("<Q", head)
        if length < 2 or length > MAX_HEADER_BYTES:
            raise FormatError(f"{path}: implausible safetensors header length {length}")
        raw = f.read(length)
    if len(raw) != length:
        raise FormatError(f"{path}: truncated safetensors header")
    return parse_header(raw, file=os.path.basename(path), data_start=8 + length)


def read_tensor(model_dir: str | os.PathLike, info: TensorInfo) -> np.ndarray:
    """The data of one tensor as a read-only numpy array (memory-mapped; BF16 comes back as its uint16 bits)."""
    if info.offset < 0:
        raise FormatError(f"{info.name}: header parsed without data offsets")
    dtype = _NUMPY_DTYPE.get(info.dtype)
    if dtype is None:
        raise FormatError(f"{info.name}: unsupported dtype {info.dtype}")
    count = int(np.prod(info.shape, dtype=np.int64)) if info.shape else 1
    if count * np.dtype(dtype).itemsize != info.nbytes:
        raise FormatError(f"{info.name}: {info.nbytes} bytes do not hold {info.dtype} {info.shape}")
    path = os.path.join(os.fspath(model_dir), info.file)
    if count == 0:
        return np.empty(info.shape, dtype=dtype)
    return np.memmap(path, dtype=dtype, mode="r", offset=info.offset, shape=info.shape or (1,)).reshape(info.shape)
