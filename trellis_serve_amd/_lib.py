"""ctypes binding of libexl3_mi355x.so (the C-ABI declared in include/exl3_mi355x.h).

The library is the product path: if it is missing, every op raises ExtensionMissing -- there is no CPU or
PyTorch fallback.  Build it with `python -m trellis_serve_amd.build` (or `__graft_entry__.build()`).
"""
from __future__ import annotations

import ctypes
import os
import re
import threading

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("EXL3_MI355X_LIB") or os.path.join(PKG, "libexl3_mi355x.so")   # env: another build
HEADER = os.path.join(os.path.dirname(PKG), "include", "exl3_mi355x.h")

EXL3_OK, EXL3_ERR_INVALID, EXL3_ERR_HIP, EXL3_ERR_UNSUPPORTED = 0, 1, 2, 3
MAX_SHARDS = 4
MAX_MOE_CLASSES = 2


class ExtensionMissing(RuntimeError):
    """The HIP library is not built / not loadable: the hot path has no fallback."""


class Exl3Error(RuntimeError):
    """A C-ABI call returned an error status (the reference raised RuntimeError via TORCH_CHECK)."""

    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


LAYOUT_STORED, LAYOUT_BLOCKS = 0, 1


class Exl3Shard(ctypes.Structure):
    _fields_ = [("trellis", ctypes.c_void_p), ("suh", ctypes.c_void_p), ("svh", ctypes.c_void_p),
                ("n", ctypes.c_int), ("layout", ctypes.c_int)]


class Exl3MoeWeights(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in ("gate_trellis", "up_trellis", "down_trellis", "gate_suh",
                                                      "gate_svh", "up_suh", "up_svh", "down_suh", "down_svh")]


class Exl3MoeClass(ctypes.Structure):
    _fields_ = [("weights", Exl3MoeWeights), ("expert_map", ctypes.c_void_p), ("num_local", ctypes.c_int),
                ("K_gate_up", ctypes.c_int), ("K_down", ctypes.c_int)]


_P, _I, _SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
_SIGNATURES: dict[str, tuple] = {
    "exl3_abi_version": (_I, []),
    "exl3_last_error": (ctypes.c_char_p, []),
    "exl3_init_device": (_I, [_I]),
    "exl3_xcd_local_chains": (_I, []),
    "exl3_reconstruct": (_I, [_P, _I, _I, _I, _I, _P, _P]),
    "exl3_repack_trellis": (_I, [_P, _I, _I, _I, _P, _P]),
    "exl3_unpack_trellis": (_I, [_P, _I, _I, _I, _P, _P]),
    "exl3_had_in_group": (_I, [_P, _I, _I, _I, _P, _I, _P, _P]),
    "exl3_had_out_into": (_I, [_P, _I, _I, _P, _P, _I, _I, _I, _P]),
    "exl3_linear_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "exl3_linear": (_I, [_P, _I, _I, _I, ctypes.POINTER(Exl3Shard), _I, _I, _I, _P, _I, _P, _SZ, _P]),
    "exl3_gemm_rotated_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "exl3_gemm_rotated": (_I, [_P, _I, _I, _P, _I, _I, _I, _P, _P, _SZ, _P]),
    "exl3_linear_noalloc_max_bytes": (_SZ, []),
    "exl3_linear_noalloc": (_I, [_P, _I, _I, _I, ctypes.POINTER(Exl3Shard), _I, _I, _I, _P, _I, _P]),
    "exl3_prefill_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "exl3_linear_prefill": (_I, [_P, _I, _I, _I, ctypes.POINTER(Exl3Shard), _I, _I, _I, _P, _I, _P, _SZ, _P]),
    "exl3_moe_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I, _I, _I]),
    "exl3_moe_forward": (_I, [_P, _I, _I, _I, _P, _P, _I, _I, _I, ctypes.POINTER(Exl3MoeWeights), _I, _I, _I, _P,
                              _I, _P, _SZ, _P]),
    "exl3_moe_classes_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I, _I, ctypes.POINTER(Exl3MoeClass)]),
    "exl3_moe_forward_classes": (_I, [_P, _I, _I, _I, _P, _P, _I, _I, _I, ctypes.POINTER(Exl3MoeClass), _I, _I, _P,
                                      _I, _P, _SZ, _P]),
    "exl3_moe_align": (_I, [_P, _I, _I, _P, _I, _P, _I, _P, _I, _P, _P]),
    "exl3_moe_align_classes": (_I, [_P, _I, _I, _I, ctypes.POINTER(_P), ctypes.POINTER(_I), ctypes.POINTER(_P),
                                    ctypes.POINTER(_I), ctypes.POINTER(_P), ctypes.POINTER(_I), ctypes.POINTER(_P),
                                    _P]),
    "exl3_moe_had_in": (_I, [_P, _I, _I, _I, _P, _I, _I, ctypes.POINTER(_P), _I, _P, _P]),
    "exl3_moe_gemm_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I]),
    "exl3_moe_gemm": (_I, [_P, _I, _I, ctypes.POINTER(_P), ctypes.POINTER(_P), _I, _I, _P, _P, _P, _I, _I, _I, _I, _I,
                           _P, _P, _SZ, _P]),
    "exl3_moe_glu_had_in": (_I, [_P, _I, _I, _P, _I, _P, _P, _P, _P]),
    "exl3_moe_combine": (_I, [_P, _P, _P, _I, _I, _I, _I, _P, _I, _P]),
    "exl3_kv_decode_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "exl3_kv_decode_attention": (_I, [_P, _P, _P, _P, _P, _I, _P, _I, _P, _I, _I, _I, _I, _I, _I, ctypes.c_float, _P,
                                      _P, _SZ, _P]),
}

_lib = None
_lock = threading.Lock()


def header_symbols() -> list[str]:
    """Function names declared in include/exl3_mi355x.h."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s*(exl3_[a-z0-9_]+)\s*\(", text, flags=re.M)


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(path):
                raise ExtensionMissing(f"{path} is not built; run `python -m trellis_serve_amd.build`")
            try:
                lib = ctypes.CDLL(path)
            except OSError as e:
                raise ExtensionMissing(f"cannot load {path}: {e}") from e
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype, fn.argtypes = res, args
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc != EXL3_OK:
        msg = load().exl3_last_error()
        raise Exl3Error(rc, f"{what}: {msg.decode() if msg else 'error ' + str(rc)}")
