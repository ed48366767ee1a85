"""The C-ABI library without a GPU: it loads, exports every symbol include/exl3_mi355x.h declares, and rejects bad
arguments before any device work (the reference's TORCH_CHECK paths, cuda/csrc/exl3_marlin.cu:132,189,195)."""
import ctypes

import pytest

from trellis_serve_amd import _lib


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    declared = _lib.header_symbols()
    assert len(declared) >= 9
    for name in declared:
        assert hasattr(lib, name), name
        assert name in _lib._SIGNATURES, f"{name} declared in the header but not bound in _lib"
    assert set(_lib._SIGNATURES) <= set(declared)


def test_abi_version(lib):
    assert lib.exl3_abi_version() == 4


def test_workspace_size_is_deterministic_and_zero_for_bad_shapes(lib):
    a = lib.exl3_linear_workspace_bytes(1, 4096, 4096, 4)
    assert a > 0 and a == lib.exl3_linear_workspace_bytes(1, 4096, 4096, 4)
    assert lib.exl3_linear_workspace_bytes(16, 4096, 4096, 4) >= a
    assert lib.exl3_linear_workspace_bytes(0, 4096, 4096, 4) == 0
    assert lib.exl3_linear_workspace_bytes(1, 4000, 4096, 4) == 0


@pytest.mark.parametrize("call, msg", [
    (lambda l: l.exl3_reconstruct(None, 256, 256, 3, 1, None, None), "null"),
    (lambda l: l.exl3_reconstruct(1, 256, 256, 7, 1, 1, None), "K = 7"),
    (lambda l: l.exl3_reconstruct(1, 256, 256, 3, 5, 1, None), "codebook = 5"),
    (lambda l: l.exl3_repack_trellis(None, 256, 256, 3, 1, None), "null"),
    (lambda l: l.exl3_repack_trellis(1, 256, 256, 7, 2, None), "K = 7"),
    (lambda l: l.exl3_unpack_trellis(1, 250, 256, 3, 2, None), "k = 250"),
    (lambda l: l.exl3_had_in_group(1, 0, 4, 100, 1, 1, 1, None), "k = 100"),
    (lambda l: l.exl3_had_in_group(1, 0, 4, 128, 1, 5, 1, None), "shards = 5"),
    (lambda l: l.exl3_had_out_into(1, 4, 128, 1, 1, 0, 64, 0, None), "ld_out"),
    (lambda l: l.exl3_gemm_rotated(1, 4, 128, 1, 100, 3, 1, 1, 1, 1 << 20, None), "n = 100"),
    (lambda l: l.exl3_kv_decode_attention(1, 1, 1, 1, 1, 4, 1, 4, 1, 2, 40, 8, 64, 16, 8, 0.1, 1, 1, 1 << 20, None),
     "head_dim = 64"),
    (lambda l: l.exl3_kv_decode_attention(1, 1, 1, 1, 1, 4, 1, 4, 1, 2, 40, 8, 128, 16, 3, 0.1, 1, 1, 1 << 20, None),
     "bits = 3"),
    (lambda l: l.exl3_kv_decode_attention(1, 1, 1, 1, 1, 4, 1, 4, 1, 2, 40, 2, 128, 16, 8, 0.1, 1, 1, 1 << 20, None),
     "group <= 16"),
    (lambda l: l.exl3_kv_decode_attention(1, 1, 1, 1, 1, 4, 1, 4, 1, 2, 40, 8, 128, 16, 8, 0.1, 1, 1, 8, None),
     "workspace"),
    (lambda l: l.exl3_kv_decode_attention(1, None, 1, 1, 1, 4, 1, 4, 1, 2, 40, 8, 128, 16, 8, 0.1, 1, 1, 1 << 20,
                                          None), "null"),
])
def test_invalid_arguments_are_rejected_without_launching(lib, call, msg):
    assert call(lib) == _lib.EXL3_ERR_INVALID
    assert msg in lib.exl3_last_error().decode()


def test_linear_rejects_bad_shards_and_small_workspace(lib):
    arr = (_lib.Exl3Shard * 1)(_lib.Exl3Shard(1, 1, 1, 100))
    assert lib.exl3_linear(1, 0, 1, 128, arr, 1, 3, 1, 1, 0, 1, 1 << 20, None) == _lib.EXL3_ERR_INVALID
    assert "multiple of 128" in lib.exl3_last_error().decode()
    assert lib.exl3_linear(1, 0, 1, 128, arr, 5, 3, 1, 1, 0, 1, 1 << 20, None) == _lib.EXL3_ERR_INVALID
    arr = (_lib.Exl3Shard * 1)(_lib.Exl3Shard(1, 1, 1, 128))
    assert lib.exl3_linear(1, 0, 1, 128, arr, 1, 3, 1, 1, 0, 1, 4, None) == _lib.EXL3_ERR_INVALID
    assert "workspace" in lib.exl3_last_error().decode()


def test_check_raises_with_the_library_message(lib):
    lib.exl3_reconstruct(None, 256, 256, 3, 1, None, None)
    with pytest.raises(_lib.Exl3Error, match="null pointer"):
        _lib.check(_lib.EXL3_ERR_INVALID, "reconstruct")


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(_lib.ExtensionMissing):
        _lib.load(str(tmp_path / "nope.so"))


def test_shard_struct_layout():
    assert ctypes.sizeof(_lib.Exl3Shard) == 32
