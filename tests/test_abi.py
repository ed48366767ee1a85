"""The C-ABI library without a GPU: it loads, exports every symbol include/exl3_mi355x.h declares, and rejects bad
arguments before any device work (the reference's TORCH_CHECK paths, cuda/csrc/exl3_marlin.cu:132,189,195)."""
import ctypes

import pytest
import torch

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
    assert lib.exl3_abi_version() == 6


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
    assert _lib.Exl3Shard.layout.offset == 28   # in the padding after n: zero-initialised callers get STORED


def test_unknown_layout_and_aliased_repack_are_rejected_without_launching(lib):
    arr = (_lib.Exl3Shard * 1)(_lib.Exl3Shard(1, 1, 1, 128, 2))
    assert lib.exl3_linear(1, 0, 1, 128, arr, 1, 3, 1, 1, 0, 1, 1 << 20, None) == _lib.EXL3_ERR_INVALID
    assert "layout" in lib.exl3_last_error().decode()
    assert lib.exl3_linear_prefill(1, 0, 1, 128, arr, 1, 3, 1, 1, 0, 1, 1 << 30, None) == _lib.EXL3_ERR_INVALID
    assert "layout" in lib.exl3_last_error().decode()
    assert lib.exl3_repack_trellis(16, 128, 128, 3, 16, None) == _lib.EXL3_ERR_INVALID   # out aliases the input
    assert lib.exl3_unpack_trellis(16, 128, 64, 3, 32, None) == _lib.EXL3_ERR_INVALID    # n not a multiple of 128


def test_noalloc_rejects_calls_beyond_the_scratch(lib):
    """A call whose workspace would exceed the scratch is refused before any launch (no device pointer is used)."""
    k, n, rows = 8192, 131072, 16
    assert lib.exl3_linear_workspace_bytes(rows, k, n, 3) > lib.exl3_linear_noalloc_max_bytes()
    arr = (_lib.Exl3Shard * 1)(_lib.Exl3Shard(1, 1, 1, n))
    assert lib.exl3_linear_noalloc(1, 0, rows, k, arr, 1, 3, 1, 1, 0, None) == _lib.EXL3_ERR_INVALID
    assert "scratch" in lib.exl3_last_error().decode()


@pytest.mark.skipif(torch.cuda.is_available(), reason="passes placeholder pointers: only where no GPU can run them")
def test_reported_workspace_sizes_cover_every_launch_plan(lib):
    """Each entry point checks its workspace against the split plans of exactly the launches it is about to make,
    before any HIP call.  With no GPU present a call that passes that check fails at its first launch (EXL3_ERR_HIP),
    one that does not returns EXL3_ERR_INVALID: so over a grid of shapes and every row count up to 64 (and a few
    prefill row counts) the size each size function reports must get past the check, and 256 bytes less must not."""
    P = 0x1000   # placeholder device pointer: never dereferenced on this path
    ks = (128, 1280, 4096, 11008, 17408)
    ns = (128, 1024, 5120, 17408, 34816)
    for K in (2, 3, 8):
        for k in ks:
            for n in ns:
                for rows in list(range(1, 65)) + [65, 130, 600]:
                    need = lib.exl3_gemm_rotated_workspace_bytes(rows, k, n, K)
                    assert need > 0
                    assert lib.exl3_gemm_rotated(P, rows, k, P, n, K, 0, P, P, need, None) == _lib.EXL3_ERR_HIP, \
                        (K, k, n, rows, lib.exl3_last_error())
                    assert lib.exl3_gemm_rotated(P, rows, k, P, n, K, 0, P, P, need - 256, None) == \
                        _lib.EXL3_ERR_INVALID, (K, k, n, rows)
                    if rows > 64:
                        continue
                    arr = (_lib.Exl3Shard * 1)(_lib.Exl3Shard(P, P, P, n))
                    need = lib.exl3_linear_workspace_bytes(rows, k, n, K)
                    assert lib.exl3_linear(P, 0, rows, k, arr, 1, K, 1, P, 0, P, need, None) == _lib.EXL3_ERR_HIP, \
                        (K, k, n, rows, lib.exl3_last_error())
                    assert lib.exl3_linear(P, 0, rows, k, arr, 1, K, 1, P, 0, P, need - 256, None) == \
                        _lib.EXL3_ERR_INVALID, (K, k, n, rows)


def test_kv_workspace_reserved_for_the_largest_batch_covers_every_smaller_call(lib):
    """A smaller batch can split each sequence into more page chunks, so the KV workspace is not monotone in the
    batch: the reservation takes the maximum over batch sizes 1..max_batch at the reserved page count, and that must
    cover every call with fewer sequences or fewer pages (a captured graph keeps the reserved buffer)."""
    for hkv, hq in ((1, 1), (2, 32), (4, 16), (8, 40), (8, 64)):
        for max_batch in (1, 3, 16, 33):
            for max_pages in (1, 7, 64, 256, 2048):
                reserved = max(lib.exl3_kv_decode_workspace_bytes(b, hq, hkv, max_pages)
                               for b in range(1, max_batch + 1))
                for b in range(1, max_batch + 1):
                    for p in sorted({1, 2, 5, 8, 9, 63, 100, max_pages // 2, max_pages - 1, max_pages}):
                        if 1 <= p <= max_pages:
                            need = lib.exl3_kv_decode_workspace_bytes(b, hq, hkv, p)
                            assert 0 < need <= reserved, (hkv, hq, max_batch, max_pages, b, p)


def test_zero_rows_launch_nothing_and_accept_null_data_pointers(lib):
    """Every entry point called with zero rows / tokens / slots / sequences returns EXL3_OK before any HIP call, with
    its activation, output and routing pointers NULL (weights and caches still given): an empty batch is a no-op,
    so these run without a GPU.  Bad shapes at zero size are still rejected."""
    P, N = 0x1000, None
    shard = (_lib.Exl3Shard * 1)(_lib.Exl3Shard(P, P, P, 256))
    ok = _lib.EXL3_OK
    assert lib.exl3_linear(N, 0, 0, 256, shard, 1, 3, 1, N, 0, N, 0, None) == ok, lib.exl3_last_error()
    assert lib.exl3_linear_noalloc(N, 0, 0, 256, shard, 1, 3, 1, N, 0, None) == ok, lib.exl3_last_error()
    assert lib.exl3_linear_prefill(N, 0, 0, 256, shard, 1, 3, 1, N, 0, N, 0, None) == ok, lib.exl3_last_error()
    assert lib.exl3_gemm_rotated(N, 0, 256, P, 256, 3, 1, N, N, 0, None) == ok, lib.exl3_last_error()
    assert lib.exl3_had_in_group(N, 0, 0, 256, P, 1, N, None) == ok, lib.exl3_last_error()
    assert lib.exl3_had_out_into(N, 0, 256, P, N, 0, 256, 0, None) == ok, lib.exl3_last_error()
    wts = _lib.Exl3MoeWeights(*([P] * 9))
    assert lib.exl3_moe_forward(N, 0, 0, 256, N, N, 8, 16, 128, ctypes.byref(wts), 3, 3, 1, N, 0, N, 0, None) == ok, \
        lib.exl3_last_error()
    assert lib.exl3_moe_combine(N, N, N, 0, 8, 256, 16, N, 0, None) == ok, lib.exl3_last_error()
    suh = (ctypes.c_void_p * 2)(P, P)
    assert lib.exl3_moe_had_in(N, 0, 0, 256, N, 8, 16, suh, 2, N, None) == ok, lib.exl3_last_error()
    tr = (ctypes.c_void_p * 1)(P)
    assert lib.exl3_moe_gemm(N, 0, 256, tr, None, 1, 256, N, N, N, 4, 16, 16, 3, 1, N, N, 0, None) == ok, \
        lib.exl3_last_error()
    assert lib.exl3_moe_glu_had_in(N, 0, 256, N, 16, P, N, N, None) == ok, lib.exl3_last_error()
    assert lib.exl3_kv_decode_attention(N, P, P, P, P, 4, N, 4, N, 0, 40, 8, 128, 16, 8, 0.1, N, N, 0, None) == ok, \
        lib.exl3_last_error()
    # zero size does not excuse bad shapes or missing weights
    assert lib.exl3_linear(N, 0, 0, 200, shard, 1, 3, 1, N, 0, N, 0, None) == _lib.EXL3_ERR_INVALID
    assert lib.exl3_gemm_rotated(N, 0, 256, N, 256, 3, 1, N, N, 0, None) == _lib.EXL3_ERR_INVALID
    assert lib.exl3_kv_decode_attention(N, N, P, P, P, 4, N, 4, N, 0, 40, 8, 128, 16, 8, 0.1, N, N, 0, None) == \
        _lib.EXL3_ERR_INVALID


def test_one_group_split_plan_fills_its_last_round(lib):
    """The decode-GEMV split plan at the configs[1] shapes, read back through the reported workspace size (counter
    region + splits x rows x n x 4 bytes of partials, 256-byte aligned): the longest equal split of 40 / 32 / 24 tile
    rows (5 / 4 / 3 blocks of 128 rows) with >= 448 workgroups, unless that needs more than one round of 1024
    workgroups -- then the split whose last round is fullest.  A plan derived here independently of the library."""
    counters = 256 * 1024
    slots = 1024

    def plan_splits(k, n):
        kb, nblk = k // 128, n // 128
        best = None
        for nt in (40, 32, 24):
            nbc = nt // 8
            splits = -(-kb // nbc)
            if splits * nbc * 50 > kb * 51 or nblk * splits < 448:
                continue
            rounds = nblk * splits / slots
            if best is None and rounds <= 1:
                return splits
            fill = 1.0 if rounds <= 1 else rounds / -(-rounds // 1)
            if best is None or fill > best[0] + 1e-9:
                best = (fill, splits)
        return best[1]

    expect = {(5120, 8192): 8, (6144, 5120): 12, (5120, 34816): 10, (17408, 5120): 46}
    for (k, n), splits in expect.items():
        assert plan_splits(k, n) == splits, (k, n)
        for rows in (1, 4, 7):
            want = counters + ((splits * rows * n * 4 + 255) & ~255)
            assert lib.exl3_linear_workspace_bytes(rows, k, n, 3) == want, (k, n, rows)


def test_kv_chunk_plan_aims_at_one_workgroup_per_cu(lib):
    """The KV decode plan, read back through the reported workspace size (batch x kv heads x chunks x group query
    heads x (128 + 2) fp32): 8-wave workgroups and about 256 of them (one per CU), or 4 waves and about 1024 when the
    8-wave LDS merge of the group would pass 64 KB (16-head groups); chunk pages a multiple of the wave count.  At the
    measured configuration (16 sequences, 40 / 8 heads) that is 2 chunks at 4k and 32k.  A plan derived here
    independently of the library."""
    def chunks(batch, hq, hkv, max_pages):
        g = hq // hkv
        waves = 8 if 8 * g * 131 * 4 <= 65536 else 4
        target = 256 if waves == 8 else 1024
        pairs = batch * hkv
        want = max(1, min(-(-max_pages // waves), -(-target // pairs)))
        cp = -(-max_pages // want)
        cp = -(-cp // waves) * waves
        return -(-max_pages // cp)

    assert chunks(16, 40, 8, 256) == 2 and chunks(16, 40, 8, 2048) == 2
    assert chunks(1, 64, 4, 2048) == 256 and chunks(64, 32, 8, 100) == 1   # 16-head groups: 4 waves, ~1024
    for batch in (1, 2, 5, 16, 33, 128):
        for hq, hkv in ((8, 8), (40, 8), (60, 4), (32, 2), (64, 4), (16, 1)):
            for max_pages in (1, 7, 8, 9, 64, 256, 1000, 2048):
                g = hq // hkv
                want = batch * hkv * chunks(batch, hq, hkv, max_pages) * g * 130 * 4
                assert lib.exl3_kv_decode_workspace_bytes(batch, hq, hkv, max_pages) == want, \
                    (batch, hq, hkv, max_pages)


def test_mixed_moe_entry_points_reject_bad_class_counts(lib):
    P, I = ctypes.c_void_p, ctypes.c_int
    maps, blocks = (P * 3)(1, 1, 1), (I * 3)(16, 16, 16)
    outs, caps = (P * 3)(1, 1, 1), (I * 3)(1 << 20, 1 << 20, 1 << 20)
    assert lib.exl3_moe_align_classes(1, 8, 16, 3, maps, blocks, outs, caps, outs, caps, outs, None) == \
        _lib.EXL3_ERR_INVALID
    assert "nclasses = 3" in lib.exl3_last_error().decode()
    maps = (P * 2)(1, None)
    assert lib.exl3_moe_align_classes(1, 8, 16, 2, maps, blocks, outs, caps, outs, caps, outs, None) == \
        _lib.EXL3_ERR_INVALID
    assert "expert map" in lib.exl3_last_error().decode()
    cls = (_lib.Exl3MoeClass * 1)()
    assert lib.exl3_moe_forward_classes(1, 0, 1, 256, 1, 1, 8, 16, 256, cls, 0, 1, 1, 0, 1, 1 << 20, None) == \
        _lib.EXL3_ERR_INVALID
    assert lib.exl3_moe_classes_workspace_bytes(4, 8, 16, 256, 256, 3, cls) == 0
    cls = (_lib.Exl3MoeClass * 2)()
    for c in range(2):
        cls[c].weights = _lib.Exl3MoeWeights(*([1] * 9))
        cls[c].num_local, cls[c].K_gate_up, cls[c].K_down = 8, 3, 4
    cls[1].expert_map = 1
    assert lib.exl3_moe_forward_classes(1, 0, 1, 256, 1, 1, 8, 16, 256, cls, 2, 1, 1, 0, 1, 1 << 20, None) == \
        _lib.EXL3_ERR_INVALID
    assert "no expert map" in lib.exl3_last_error().decode()
    assert lib.exl3_moe_classes_workspace_bytes(4, 8, 16, 256, 256, 2, cls) > 0
