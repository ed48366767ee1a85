"""GPU parity of the dense EXL3 path (decode, rotations, fused decode-GEMV) against the CPU oracle.

Decoded weights are compared bit for bit (reconstruct and the one-hot readout through the GEMV kernel, the method of
cuda/src/sglang_exl3/parity/marlin_parity.py:149-159 and xpu/tests/test_bitexact_xpu.py:46-102); layer outputs
against the float64 evaluation of had(had(x*suh) @ W) * svh (parity/l1_linear.py:28-36) with the north-star gate:
norm-relative and max-relative error <= 2e-3.
"""
import numpy as np
import pytest
import torch

from conftest import c_reconstruct
from oracle import exl3_oracle as orc

pytestmark = pytest.mark.gpu

KS = (2, 3, 4, 5, 6, 8)
CBS = (0, 1, 2)
TOL = 2e-3


def _ops():
    from trellis_serve_amd import ops
    return ops


def _trellis(rng, k, n, K):
    return rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * K), dtype=np.int16)


def _signs(rng, n):
    return np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16)


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def blocks_layout(tr):
    """The EXL3_LAYOUT_BLOCKS order of a stored trellis [k/16, n/16, 16K] (include/exl3_mi355x.h): tile (i, j) at tile
    position ((j / 8) (k / 128) + i / 8) 64 + (j % 8) 8 + i % 8, returned in the stored array's shape."""
    tk, tn, w = tr.shape
    units = tr.reshape(tk // 8, 8, tn // 8, 8, w)           # [kb][i%8][cb][j%8][w]
    return np.ascontiguousarray(units.transpose(2, 0, 3, 1, 4)).reshape(tk, tn, w)  # [cb][kb][j%8][i%8][w]


def _errs(y, ref):
    y = y.astype(np.float64)
    ref = ref.astype(np.float64)
    return (np.linalg.norm(y - ref) / np.linalg.norm(ref), np.abs(y - ref).max() / np.abs(ref).max())


@pytest.mark.parametrize("K", KS)
@pytest.mark.parametrize("cb", CBS)
def test_reconstruct_is_bit_exact(coracle, K, cb):
    rng = np.random.default_rng(1000 + 10 * K + cb)
    tr = _trellis(rng, 128, 384, K)
    w = _ops().reconstruct(_dev(tr), cb).cpu().numpy()
    np.testing.assert_array_equal(w.view(np.uint16), c_reconstruct(coracle, tr, K, cb).view(np.uint16))


@pytest.mark.parametrize("K", KS)
@pytest.mark.parametrize("cb", CBS)
def test_reconstruct_matches_reference_golden(golden, K, cb):
    w = _ops().reconstruct(_dev(golden[f"recon_in_K{K}_cb{cb}"]), cb).cpu().numpy()
    np.testing.assert_array_equal(w.view(np.uint16), golden[f"recon_out_K{K}_cb{cb}"])


@pytest.mark.parametrize("cb", CBS)
def test_reconstruct_covers_every_state(cb):
    """K = 8: the state of element t is (byte[t-1] << 8) | byte[t]; 512 tiles with bytes (a, i + 128 h) put every
    16-bit state at an odd stream position once.  Checked against the closed-form codebook."""
    K = 8
    tiles = np.zeros((512, 256), dtype=np.uint8)
    for a in range(256):
        for h in range(2):
            tiles[2 * a + h, 0::2] = a
            tiles[2 * a + h, 1::2] = np.arange(128) + 128 * h
    # stream bytes MSB-first per little-endian dword -> int16 storage
    words = tiles.reshape(512, 64, 4)
    u32 = (words[..., 0].astype(np.uint32) << 24) | (words[..., 1].astype(np.uint32) << 16) | \
          (words[..., 2].astype(np.uint32) << 8) | words[..., 3].astype(np.uint32)
    tr = u32.view(np.uint16).reshape(512, 128).view(np.int16).reshape(32, 16, 128)
    w = _ops().reconstruct(_dev(tr), cb).cpu().numpy()
    np.testing.assert_array_equal(w.view(np.uint16), orc.reconstruct_inner(tr, K, cb).view(np.uint16))
    perm = orc.tensor_core_perm()
    lut = orc.codebook_lut(cb).view(np.uint16)
    tiles_w = w.reshape(32, 16, 16, 16).transpose(0, 2, 1, 3).reshape(512, 256)[:, perm]
    odd_states = (tiles[:, 0::2].astype(np.int64) << 8) | tiles[:, 1::2]
    np.testing.assert_array_equal(tiles_w.view(np.uint16)[:, 1::2], lut[odd_states])
    assert np.unique(odd_states).size == 65536


@pytest.mark.parametrize("K", KS)
@pytest.mark.parametrize("cb", CBS)
def test_gemm_rotated_one_hot_readout_is_exact(coracle, K, cb):
    """256 identity rows go through the prefill decode-GEMM (65 rows and more), 64 at a time through the decode-GEMV
    (16-row launches, two decoded tiles per MFMA): both read W_inner back bit for bit."""
    rng = np.random.default_rng(2000 + 10 * K + cb)
    k, n = 256, 256
    tr = _trellis(rng, k, n, K)
    dtr = _dev(tr)
    ref = c_reconstruct(coracle, tr, K, cb).view(np.uint16)
    xh = torch.eye(k, dtype=torch.float16, device="cuda")
    w = _ops().gemm_rotated(xh, dtr, cb).cpu().numpy()
    np.testing.assert_array_equal(w.view(np.uint16), ref)
    w = torch.cat([_ops().gemm_rotated(xh[r0:r0 + 64].contiguous(), dtr, cb) for r0 in range(0, k, 64)])
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint16), ref)


def _halves_sum_lut(cb):
    """lo + hi of every state's masked hash, unrounded (float64): the weight a kernel would use if it added the two
    fp16 halves in the matrix core instead of rounding their sum to fp16 first (codebook.cuh:56-75 rounds, __hadd)."""
    s = np.arange(65536, dtype=np.uint64)
    x = (s * orc.MCG_MULT) if cb == 1 else (s * orc.INST3_MULT + orc.INST3_ADD)
    x = ((x & 0xFFFFFFFF) & 0x8FFF8FFF) ^ 0x3B603B60
    lo = (x & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (x >> 16).astype(np.uint16).view(np.float16).astype(np.float64)
    return lo + hi


@pytest.mark.parametrize("cb", (0, 1))
@pytest.mark.parametrize("K", (2, 3, 4))
def test_gemv_multiplies_by_rounded_weights(K, cb):
    """Rows x = e_i + e_j give fp16(w_i + w_j) per column.  With trellis_core's rounded weights w = fp16(lo + hi)
    (reference.py:52-73) the sum of the two products is exact in fp32 and rounds once; a kernel that fed the matrix
    core the unsummed halves would return fp16((lo_i + hi_i) + (lo_j + hi_j)) instead.  The pairs are chosen where the
    two differ, so this fails for the unsummed form; checked through the decode-GEMV (16 rows) and the decode-GEMM
    (80 rows).  Columns where a weight is below 2^-10 (its fp32 sum with the other could round) are left out."""
    rng = np.random.default_rng(2700 + 10 * K + cb)
    k, n = 512, 256
    tr = _trellis(rng, k, n, K)
    states = orc.decode_states(tr.reshape(-1, 16 * K), K)            # [tiles, 256] stream order
    perm = orc.tensor_core_perm()
    w_rnd = orc.codebook_lut(cb).astype(np.float64)[states]
    w_sum = _halves_sum_lut(cb)[states]

    def inner(v):   # stream order -> [k, n] as reconstruct_inner places it
        t = np.empty_like(v)
        t[:, perm] = v
        return t.reshape(k // 16, n // 16, 16, 16).transpose(0, 2, 1, 3).reshape(k, n)

    W, E = inner(w_rnd), inner(w_sum)
    pairs = []
    for c in range(n):
        if len(pairs) == 80:
            break
        good = np.abs(W[:, c]) >= 2.0 ** -10
        for i in rng.permutation(np.flatnonzero(good))[:64]:
            js = np.flatnonzero(good & (np.arange(k) != i))
            want = (W[i, c] + W[js, c]).astype(np.float16)
            halves = (E[i, c] + E[js, c]).astype(np.float16)
            bad = js[want != halves]
            if bad.size:
                pairs.append((i, bad[0]))
                break
    assert len(pairs) == 80, len(pairs)
    x = np.zeros((80, k), dtype=np.float16)
    for r, (i, j) in enumerate(pairs):
        x[r, i] = x[r, j] = 1
    ii, jj = np.array(pairs).T
    want = (W[ii] + W[jj]).astype(np.float16)
    halves = (E[ii] + E[jj]).astype(np.float16)
    keep = (np.abs(W[ii]) >= 2.0 ** -10) & (np.abs(W[jj]) >= 2.0 ** -10)
    dtr = _dev(tr)
    for rows in (16, 80):
        got = torch.cat([_ops().gemm_rotated(_dev(x[r0:r0 + rows]), dtr, cb) for r0 in range(0, 80, rows)])
        got = got.cpu().numpy()
        assert np.array_equal(got.view(np.uint16)[keep], want.view(np.uint16)[keep]), rows
        assert (got != halves).any(axis=1).all(), rows   # every row differs from the unsummed-halves result


def test_gemm_rotated_17_to_31_rows_in_its_reported_workspace(coracle):
    """gemm_rotated serves 17-31 rows as 16-row GEMV launches; their split plan (one row group) takes more fp32
    partials than exl3_linear's plan of the same row count, so the workspace is sized and checked for its own launches
    (the shape once overflowed: k = 11008, n = 5120, K = 2, 3INST).  One-hot rows read W_inner back exactly."""
    ops = _ops()
    ops.release_workspaces()
    rng = np.random.default_rng(2800)
    k, n, K, cb = 11008, 5120, 2, 0
    tr = _trellis(rng, k, n, K)
    dtr = _dev(tr)
    ref = c_reconstruct(coracle, tr, K, cb).view(np.uint16)
    eye = torch.eye(k, dtype=torch.float16, device="cuda")
    for rows, r0 in ((17, 0), (23, 4000), (31, k - 31)):
        got = ops.gemm_rotated(eye[r0:r0 + rows].contiguous(), dtr, cb).cpu().numpy()
        np.testing.assert_array_equal(got.view(np.uint16), ref[r0:r0 + rows], err_msg=str(rows))


def test_row_counts_either_side_of_the_row_group_switch_agree(coracle):
    """16 rows run one row group (two tiles per 16x16x32 MFMA), 17 rows two groups (16x16x16 MFMAs per tile): both
    multiply by the same rounded weights, so a row's output differs only by fp32 summation order -- well inside the
    layer tolerance, and both meet the oracle."""
    rng = np.random.default_rng(2900)
    k, n, K, cb = 4096, 2048, 3, 1
    tr, suh, svh = _trellis(rng, k, n, K), _signs(rng, k), _signs(rng, n)
    args = ([_dev(tr)], [_dev(suh)], [_dev(svh)], cb)
    x = rng.standard_normal((17, k)).astype(np.float16)
    y17 = _ops().linear(_dev(x), *args).cpu().numpy().astype(np.float64)
    y16 = _ops().linear(_dev(x[:16]), *args).cpu().numpy().astype(np.float64)
    d = np.linalg.norm(y17[:16] - y16) / np.linalg.norm(y16)
    assert d <= 2e-4, d
    ref = orc.linear_forward(x, tr, suh, svh, K, cb, w_inner=c_reconstruct(coracle, tr, K, cb), dtype=np.float64)
    for y, r in ((y16, ref[:16]), (y17, ref)):
        nrel, mrel = _errs(y, r)
        assert nrel <= TOL and mrel <= TOL, (nrel, mrel)


@pytest.mark.parametrize("K", KS)
def test_repack_is_lossless_and_the_kernels_read_it(coracle, K):
    """repack writes the BLOCKS layout (each (128-column block, 128-row block) unit of 64 tiles one run, the 8 tiles of
    a tile column adjacent inside it) bit for bit as blocks_layout restates it; unpack returns the stored trellis bit
    for bit (the invertibility check of cuda/src/sglang_exl3/parity/marlin_parity.py:173); an in-place repack is
    refused; and the GEMV and the prefill decode-GEMM read the repacked form to the same bits as the stored one."""
    rng = np.random.default_rng(500 + K)
    tr = _trellis(rng, 256, 384, K)
    t = torch.from_numpy(tr).cuda()
    ops = _ops()
    packed = ops.repack_trellis(t)
    np.testing.assert_array_equal(packed.cpu().numpy(), blocks_layout(tr))
    np.testing.assert_array_equal(ops.unpack_trellis(packed).cpu().numpy(), tr)
    with pytest.raises(ValueError):
        ops.repack_trellis(t, out=t)
    su, sv = _dev(_signs(rng, 256)), _dev(_signs(rng, 384))
    for rows, fn in ((1, ops.linear), (5, ops.linear), (40, ops.linear), (300, ops.linear_prefill)):
        x = _dev(rng.standard_normal((rows, 256)).astype(np.float16))
        y0 = fn(x, [t], [su], [sv], 1)
        y1 = fn(x, [packed], [su], [sv], 1, layout=1)
        assert torch.equal(y0, y1), (rows, fn.__name__)


@pytest.mark.parametrize("K", (2, 3, 4))
@pytest.mark.parametrize("cb", CBS)
def test_one_hot_readout_through_the_split_k_gemv_is_exact(coracle, K, cb):
    """The decode-GEMV (split-K: every k split of a 128-column block writes fp32 partials, the last arrival sums
    them) read back with one-hot rows: each row of W_inner comes back bit for bit, 4 rows per call and once with a
    single row.  1280 x 16384 has 10 k blocks and 128 column blocks."""
    rng = np.random.default_rng(2500 + 10 * K + cb)
    k, n = 1280, 16384
    tr = _trellis(rng, k, n, K)
    dtr = _dev(tr)
    ref = c_reconstruct(coracle, tr, K, cb).view(np.uint16)
    eye = torch.eye(k, dtype=torch.float16, device="cuda")
    got = np.concatenate([_ops().gemm_rotated(eye[r0:r0 + 4].contiguous(), dtr, cb).cpu().numpy()
                          for r0 in range(0, k, 4)])
    np.testing.assert_array_equal(got.view(np.uint16), ref)
    one = _ops().gemm_rotated(eye[37:38].contiguous(), dtr, cb).cpu().numpy()
    np.testing.assert_array_equal(one.view(np.uint16), ref[37:38])


@pytest.mark.parametrize("M", [1, 3])
@pytest.mark.parametrize("cb", CBS)
def test_gemv_shards_of_uneven_widths(coracle, M, cb):
    """A 3-shard group of uneven widths (23, 10 and 20 column blocks): column blocks of different shards in one launch
    rotate their activations with their own suh and their outputs with their own svh.  Against the float64 oracle."""
    rng = np.random.default_rng(3500 + 10 * M + cb)
    k, ns, K = 4096, (2944, 1280, 2560), 3
    trs = [_trellis(rng, k, n, K) for n in ns]
    suhs = [_signs(rng, k) for _ in ns]
    svhs = [_signs(rng, n) for n in ns]
    x = (rng.standard_normal((M, k)) * 0.5).astype(np.float16)
    y = _ops().linear(_dev(x), [_dev(t) for t in trs], [_dev(s) for s in suhs], [_dev(s) for s in svhs],
                      cb).cpu().numpy()
    ref = np.concatenate([orc.linear_forward(x, t, a, b, K, cb, w_inner=c_reconstruct(coracle, t, K, cb),
                                             dtype=np.float64) for t, a, b in zip(trs, suhs, svhs)], axis=1)
    nrel, mrel = _errs(y, ref)
    assert nrel <= TOL and mrel <= TOL, (nrel, mrel)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 16, 17, 24, 32, 45, 64, 80])
@pytest.mark.parametrize("K,cb", [(2, 1), (3, 1), (4, 0), (5, 2), (6, 1), (8, 0)])
def test_linear_matches_float64_oracle(coracle, M, K, cb):
    """Up to 16 rows one MFMA row group per decoded tile, 17-32 two groups and 33-64 four groups in one launch (rows
    padded with zeros to a multiple of 16), past 64 rows another launch for the rest."""
    rng = np.random.default_rng(3000 + 100 * M + 10 * K + cb)
    k, n = 768, 640
    tr, suh, svh = _trellis(rng, k, n, K), _signs(rng, k), _signs(rng, n)
    x = rng.standard_normal((M, k)).astype(np.float16)
    y = _ops().linear(_dev(x), [_dev(tr)], [_dev(suh)], [_dev(svh)], cb).cpu().numpy()
    ref = orc.linear_forward(x, tr, suh, svh, K, cb, w_inner=c_reconstruct(coracle, tr, K, cb), dtype=np.float64)
    nrel, mrel = _errs(y, ref)
    assert nrel <= TOL and mrel <= TOL, (nrel, mrel)


def test_linear_c1_shape_4096(coracle):
    """4096 -> 4096, K = 4, 3INST, M = 1."""
    rng = np.random.default_rng(4096)
    k = n = 4096
    K, cb = 4, 0
    tr, suh, svh = _trellis(rng, k, n, K), _signs(rng, k), _signs(rng, n)
    x = rng.standard_normal((1, k)).astype(np.float16)
    y = _ops().linear(_dev(x), [_dev(tr)], [_dev(suh)], [_dev(svh)], cb).cpu().numpy()
    ref = orc.linear_forward(x, tr, suh, svh, K, cb, w_inner=c_reconstruct(coracle, tr, K, cb), dtype=np.float64)
    nrel, mrel = _errs(y, ref)
    assert nrel <= TOL and mrel <= TOL, (nrel, mrel)


@pytest.mark.parametrize("rows,k,n", [(4, 512, 384), (16, 4096, 16384), (29, 4096, 16384), (20, 512, 384)])
def test_linear_bf16_boundary_equals_fp16_casts(rows, k, n):
    """run(x_bf16) == run(x_bf16.half()).bfloat16() bit for bit (cuda/src/sglang_exl3/parity/marlin_parity.py:98-111);
    16 rows of a 4096 -> 16384 linear take the path that rotates the input once per shard before the GEMV."""
    rng = np.random.default_rng(5)
    K, cb = 3, 1
    tr, suh, svh = _dev(_trellis(rng, k, n, K)), _dev(_signs(rng, k)), _dev(_signs(rng, n))
    x = torch.from_numpy(rng.standard_normal((rows, k)).astype(np.float32)).cuda().bfloat16()
    y_bf = _ops().linear(x, [tr], [suh], [svh], cb)
    y_h = _ops().linear(x.half(), [tr], [suh], [svh], cb)
    assert y_bf.dtype == torch.bfloat16
    assert torch.equal(y_bf, y_h.bfloat16())


def test_linear_rows_rotated_once_match_rows_rotated_per_workgroup():
    """With 8+ rows and enough column blocks x rows x k-blocks (here 128 x 16 x 32), the input rotation runs once per
    shard (fragment-order rows) before the GEMV; a 16-row call must agree with 4-row calls (rotation inside every
    workgroup) to rounding: the split-K reduce groups its fp32 partials by row count (16 rows: one sequential sum;
    4 rows: 4 interleaved sums, then their sum), so results are bit-identical per shape, not across row counts."""
    rng = np.random.default_rng(6)
    k, K, cb = 4096, 3, 1
    ns = (8192, 8192)
    cases = [(_dev(_trellis(rng, k, n, K)), _dev(_signs(rng, k)), _dev(_signs(rng, n))) for n in ns]
    args = ([c[0] for c in cases], [c[1] for c in cases], [c[2] for c in cases], cb)
    x = torch.from_numpy((rng.standard_normal((16, k)) * 0.5).astype(np.float16)).cuda()
    y16 = _ops().linear(x, *args)
    y4 = torch.cat([_ops().linear(x[r:r + 4].contiguous(), *args) for r in range(0, 16, 4)])
    d = (y16.float() - y4.float()).norm() / y4.float().norm()
    assert d.item() <= 1e-4, d.item()
    assert torch.equal(_ops().linear(x, *args), y16)


def test_linear_fused_group_matches_oracle_per_shard(coracle):
    """q/k/v-style group: 3 shards with their own suh/svh share x and fill adjacent column spans."""
    rng = np.random.default_rng(6)
    k, K, cb = 512, 3, 1
    ns = (512, 128, 256)
    trs = [_trellis(rng, k, n, K) for n in ns]
    suhs = [_signs(rng, k) for _ in ns]
    svhs = [_signs(rng, n) for n in ns]
    x = rng.standard_normal((5, k)).astype(np.float16)
    y = _ops().linear(_dev(x), [_dev(t) for t in trs], [_dev(s) for s in suhs], [_dev(s) for s in svhs], cb)
    y = y.cpu().numpy()
    col = 0
    for t, su, sv, n in zip(trs, suhs, svhs, ns):
        ref = orc.linear_forward(x, t, su, sv, K, cb, w_inner=c_reconstruct(coracle, t, K, cb), dtype=np.float64)
        nrel, mrel = _errs(y[:, col:col + n], ref)
        assert nrel <= TOL and mrel <= TOL, (n, nrel, mrel)
        col += n


@pytest.mark.parametrize("K", KS)
@pytest.mark.parametrize("cb", CBS)
def test_repacked_group_matches_oracle(coracle, K, cb):
    """A 3-shard group in the repacked (BLOCKS) layout, each shard a different number of 128-column blocks, through
    the decode-GEMV (1 and 16 rows) and the prefill decode-GEMM (80 rows), against the float64 oracle of the stored
    trellis."""
    rng = np.random.default_rng(900 + 10 * K + cb)
    k, ns = 384, (256, 128, 384)
    trs = [_trellis(rng, k, n, K) for n in ns]
    suhs, svhs = [_signs(rng, k) for _ in ns], [_signs(rng, n) for n in ns]
    ops = _ops()
    packed = [ops.repack_trellis(_dev(t)) for t in trs]
    for rows, fn in ((1, ops.linear), (16, ops.linear), (80, ops.linear_prefill)):
        x = rng.standard_normal((rows, k)).astype(np.float16)
        y = fn(_dev(x), packed, [_dev(v) for v in suhs], [_dev(v) for v in svhs], cb, layout=1).cpu().numpy()
        col = 0
        for t, su, sv, n in zip(trs, suhs, svhs, ns):
            ref = orc.linear_forward(x, t, su, sv, K, cb, w_inner=c_reconstruct(coracle, t, K, cb), dtype=np.float64)
            nrel, mrel = _errs(y[:, col:col + n], ref)
            assert nrel <= TOL and mrel <= TOL, (rows, n, nrel, mrel)
            col += n


def test_xcd_probe_enables_local_chains_on_a_whole_mi355x():
    """exl3_init_device's probe: on a device with all 256 CUs (8 XCDs), workgroups whose ids agree mod 8 share an XCD,
    so split-K chains of launches with a multiple of 8 column blocks stay in one XCD's L2."""
    from trellis_serve_amd import _lib
    _ops().init_device(0)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if cus != 256:
        pytest.skip(f"{cus} CUs: not a whole MI355X")
    assert _lib.load().exl3_xcd_local_chains() == 1


def test_linear_is_deterministic():
    rng = np.random.default_rng(7)
    k, n, K, cb = 2048, 1024, 3, 1
    args = ([_dev(_trellis(rng, k, n, K))], [_dev(_signs(rng, k))], [_dev(_signs(rng, n))], cb)
    x = _dev(rng.standard_normal((3, k)).astype(np.float16))
    first = _ops().linear(x, *args)
    for _ in range(20):
        assert torch.equal(_ops().linear(x, *args), first)


def test_had_in_group_matches_fp16_oracle():
    rng = np.random.default_rng(8)
    rows, k = 6, 1024
    x = (rng.standard_normal((rows, k)) * 3).astype(np.float16)
    suh = np.stack([_signs(rng, k), (rng.random(k) + 0.5).astype(np.float16)])
    xh = _ops().had_in_group(_dev(x), _dev(suh)).cpu().numpy()
    for s in range(2):
        want = orc.had_in_fp16(x, suh[s])
        got = xh[s * rows:(s + 1) * rows]
        ulp = np.abs(got.view(np.int16).astype(np.int32) - want.view(np.int16).astype(np.int32))
        assert ulp.max() <= 1 and (ulp == 0).mean() > 0.99


def test_had_out_into_writes_its_column_span():
    rng = np.random.default_rng(9)
    rows, n = 3, 256
    y = rng.standard_normal((rows, n)).astype(np.float16)
    svh = _signs(rng, n)
    out = torch.zeros((rows, 640), dtype=torch.float16, device="cuda")
    _ops().had_out_into(_dev(y), _dev(svh), out, 128)
    o = out.cpu().numpy()
    assert not o[:, :128].any() and not o[:, 384:].any()
    want = (orc.had_rows(y.astype(np.float32), np.float64).astype(np.float32).astype(np.float16)
            * svh).astype(np.float16)
    ulp = np.abs(o[:, 128:384].view(np.int16).astype(np.int32) - want.view(np.int16).astype(np.int32))
    assert ulp.max() <= 1


def test_invalid_shapes_raise():
    ops = _ops()
    t = torch.zeros((8, 8, 48), dtype=torch.int16, device="cuda")
    with pytest.raises(ValueError):
        ops.linear(torch.zeros((1, 64), dtype=torch.float16, device="cuda"), [t],
                   [torch.ones(128, dtype=torch.float16, device="cuda")],
                   [torch.ones(128, dtype=torch.float16, device="cuda")], 1)


def test_workspace_shared_by_calls_of_different_shapes(coracle):
    """One workspace serves calls of any shapes: a call with many k-splits leaves fp32 partials behind its counters;
    a later call with more output column blocks must still see zero counters (they sit in a fixed region)."""
    ops = _ops()
    ops.release_workspaces()
    rng = np.random.default_rng(10)
    K, cb = 3, 1
    for k, n, M in ((8192, 128, 16), (256, 12800, 1), (1024, 4096, 3), (8192, 128, 16)):
        tr, suh, svh = _trellis(rng, k, n, K), _signs(rng, k), _signs(rng, n)
        x = rng.standard_normal((M, k)).astype(np.float16)
        y = ops.linear(_dev(x), [_dev(tr)], [_dev(suh)], [_dev(svh)], cb).cpu().numpy()
        ref = orc.linear_forward(x, tr, suh, svh, K, cb, w_inner=c_reconstruct(coracle, tr, K, cb), dtype=np.float64)
        nrel, mrel = _errs(y, ref)
        assert nrel <= TOL and mrel <= TOL, (k, n, M, nrel, mrel)


@pytest.mark.parametrize("rows", [17, 32, 50, 64])
def test_two_row_groups_match_oracle_with_prepared_rows(coracle, rows):
    """Two 16-row groups share each decoded tile: at 17 rows every workgroup rotates its rows, at 32 rows (64 column
    blocks x 32 rows x 32 k-blocks) the input is rotated once per shard before the GEMV; both shards against the
    float64 oracle, repeatable bit for bit."""
    rng = np.random.default_rng(70 + rows)
    k, K, cb = 4096, 3, 1
    ns = (4096, 4096)
    cases = [(_trellis(rng, k, n, K), _signs(rng, k), _signs(rng, n)) for n in ns]
    args = ([_dev(c[0]) for c in cases], [_dev(c[1]) for c in cases], [_dev(c[2]) for c in cases], cb)
    x = (rng.standard_normal((rows, k)) * 0.5).astype(np.float16)
    y = _ops().linear(_dev(x), *args)
    col = 0
    for (tr, suh, svh), n in zip(cases, ns):
        w = c_reconstruct(coracle, tr[:, :64], K, cb)   # the first 1024 columns of the shard
        ref = orc.linear_forward(x, tr[:, :64], suh, svh[:1024], K, cb, w_inner=w, dtype=np.float64)
        nrel, mrel = _errs(y[:, col:col + 1024].cpu().numpy(), ref)
        assert nrel <= TOL and mrel <= TOL, (n, nrel, mrel)
        col += n
    assert torch.equal(_ops().linear(_dev(x), *args), y)


@pytest.mark.parametrize("rows", [40, 64])
def test_wide_layer_rows_past_32_take_two_group_launches(coracle, rows):
    """A wide layer (256 column blocks) at 33-64 rows runs as launches of 32 rows with two row groups (four groups
    would need more LDS than a launch gets by default); the first and last 1024 columns against the oracle."""
    rng = np.random.default_rng(90 + rows)
    k, n, K, cb = 2048, 32768, 3, 1
    tr, suh, svh = _trellis(rng, k, n, K), _signs(rng, k), _signs(rng, n)
    x = (rng.standard_normal((rows, k)) * 0.5).astype(np.float16)
    y = _ops().linear(_dev(x), [_dev(tr)], [_dev(suh)], [_dev(svh)], cb).cpu().numpy()
    for c0 in (0, n - 1024):
        t = tr[:, c0 // 16:(c0 + 1024) // 16]
        ref = orc.linear_forward(x, t, suh, svh[c0:c0 + 1024], K, cb, w_inner=c_reconstruct(coracle, t, K, cb),
                                 dtype=np.float64)
        nrel, mrel = _errs(y[:, c0:c0 + 1024], ref)
        assert nrel <= TOL and mrel <= TOL, (c0, nrel, mrel)
