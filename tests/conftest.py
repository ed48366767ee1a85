import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden", "exl3_golden.npz")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def coracle():
    """The C restatement (oracle/exl3_oracle.c), built on demand."""
    so = os.path.join(ROOT, "oracle", "_build", "libexl3_oracle.so")
    if not os.path.exists(so):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    lib = ctypes.CDLL(so)
    lib.exl3_oracle_codebook.restype = ctypes.c_uint16
    lib.exl3_oracle_codebook.argtypes = [ctypes.c_int, ctypes.c_uint32]
    lib.exl3_oracle_f64_to_f16.restype = ctypes.c_uint16
    lib.exl3_oracle_f64_to_f16.argtypes = [ctypes.c_double]
    lib.exl3_oracle_codebook_lut.argtypes = [ctypes.c_int, ctypes.c_void_p]
    lib.exl3_oracle_decode_tile.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    lib.exl3_oracle_perm.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.exl3_oracle_reconstruct.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_void_p]
    return lib


def c_reconstruct(lib, trellis: np.ndarray, K: int, cb: int) -> np.ndarray:
    tr = np.ascontiguousarray(trellis, dtype=np.int16)
    tk, tn, _ = tr.shape
    out = np.empty((16 * tk, 16 * tn), dtype=np.uint16)
    lib.exl3_oracle_reconstruct(tr.ctypes.data, tk, tn, K, cb, out.ctypes.data)
    return out.view(np.float16)
