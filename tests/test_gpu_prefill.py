"""GPU parity of the fused prefill decode-GEMM (exl3_linear_prefill) against the float64 oracle, and against the
decode-GEMV path on the same inputs.  Gate: norm-relative and max-relative error <= 2e-3."""
import numpy as np
import pytest
import torch

from conftest import c_reconstruct
from oracle import exl3_oracle as orc

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _ops():
    from trellis_serve_amd import ops
    return ops


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _case(rng, k, n, K):
    tr = rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * K), dtype=np.int16)
    suh = np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16)
    svh = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16)
    return tr, suh, svh


def _errs(y, ref):
    y = y.astype(np.float64)
    return np.linalg.norm(y - ref) / np.linalg.norm(ref), np.abs(y - ref).max() / np.abs(ref).max()


@pytest.mark.parametrize("M", [1, 37, 256, 300])
@pytest.mark.parametrize("K,cb", [(2, 0), (3, 1), (4, 2), (5, 1), (6, 0), (8, 2)])
def test_prefill_matches_float64_oracle(coracle, M, K, cb):
    rng = np.random.default_rng(7000 + 10 * K + cb + M)
    k, n = 512, 384
    tr, suh, svh = _case(rng, k, n, K)
    x = (rng.standard_normal((M, k)) * 0.5).astype(np.float16)
    y = _ops().linear_prefill(_dev(x), [_dev(tr)], [_dev(suh)], [_dev(svh)], cb).cpu().numpy()
    ref = orc.linear_forward(x, tr, suh, svh, K, cb, w_inner=c_reconstruct(coracle, tr, K, cb), dtype=np.float64)
    nrel, mrel = _errs(y, ref)
    assert nrel <= TOL and mrel <= TOL, (nrel, mrel)


def test_prefill_fused_group_and_bf16(coracle):
    rng = np.random.default_rng(11)
    k, K, cb, M = 640, 3, 1, 300
    ns = (512, 128, 256)
    cases = [_case(rng, k, n, K) for n in ns]
    x = (rng.standard_normal((M, k)) * 0.5).astype(np.float16)
    args = ([_dev(c[0]) for c in cases], [_dev(c[1]) for c in cases], [_dev(c[2]) for c in cases], cb)
    y = _ops().linear_prefill(_dev(x), *args).cpu().numpy()
    col = 0
    for (tr, suh, svh), n in zip(cases, ns):
        ref = orc.linear_forward(x, tr, suh, svh, K, cb, w_inner=c_reconstruct(coracle, tr, K, cb), dtype=np.float64)
        nrel, mrel = _errs(y[:, col:col + n], ref)
        assert nrel <= TOL and mrel <= TOL, (n, nrel, mrel)
        col += n
    xb = _dev(x).bfloat16()
    yb = _ops().linear_prefill(xb, *args)
    assert yb.dtype == torch.bfloat16
    assert torch.equal(yb, _ops().linear_prefill(xb.half(), *args).bfloat16())


def test_prefill_agrees_with_gemv_path():
    rng = np.random.default_rng(12)
    k, n, K, cb, M = 1024, 1024, 4, 1, 64
    tr, suh, svh = (_dev(a) for a in _case(rng, k, n, K))
    x = torch.randn((M, k), device="cuda").half()
    a = _ops().linear_prefill(x, [tr], [suh], [svh], cb).float()
    b = _ops().linear(x, [tr], [suh], [svh], cb).float()
    assert ((a - b).norm() / b.norm()).item() < 1e-3


def test_prefill_is_deterministic():
    rng = np.random.default_rng(13)
    k, n, K, cb, M = 1024, 512, 3, 1, 513
    args = ([_dev(a) for a in _case(rng, k, n, K)[:1]], [_dev(_case(rng, k, n, K)[1])], [_dev(_case(rng, k, n, K)[2])], cb)
    x = torch.randn((M, k), device="cuda").half()
    first = _ops().linear_prefill(x, *args)
    for _ in range(5):
        assert torch.equal(_ops().linear_prefill(x, *args), first)


def test_prefill_split_tail_tiles_match_oracle(coracle):
    """More tiles than one round of the machine holds: the tiles past the last whole round run as k-split items whose
    fp32 partials are summed in split order.  The tail (last row block, last column blocks) and a data-parallel tile
    are checked against the float64 oracle, and repeated calls are bit-identical."""
    slots = torch.cuda.get_device_properties(0).multi_processor_count  # one 256 x 256 tile per CU at a time
    M, k, K, cb = 768, 1024, 3, 1
    cbk = (slots + 28 + 2) // 3  # 3 row blocks x cbk 256-column tiles = slots + ~28 tail tiles
    n = 256 * cbk
    rng = np.random.default_rng(14)
    tr, suh, svh = _case(rng, k, n, K)
    x = (rng.standard_normal((M, k)) * 0.5).astype(np.float16)
    args = ([_dev(tr)], [_dev(suh)], [_dev(svh)], cb)
    y = _ops().linear_prefill(_dev(x), *args)
    tail = 3 * cbk - slots
    c0 = (cbk - tail) * 256  # first column of the tail tiles in the last row block
    for rows, cols in ((slice(512, 768), slice(c0, n)), (slice(0, 256), slice(0, 512))):
        t = tr[:, cols.start // 16:cols.stop // 16]
        ref = orc.linear_forward(x[rows], t, suh, svh[cols], K, cb, w_inner=c_reconstruct(coracle, t, K, cb),
                                 dtype=np.float64)
        nrel, mrel = _errs(y[rows, cols].cpu().numpy(), ref)
        assert nrel <= TOL and mrel <= TOL, (rows, cols, nrel, mrel)
    for _ in range(3):
        assert torch.equal(_ops().linear_prefill(_dev(x), *args), y)


@pytest.mark.parametrize("M", [1, 16, 40, 255])
@pytest.mark.parametrize("n", [512, 384])
def test_prefill_few_rows_many_contributors(coracle, M, n):
    """Under 256 rows with only 1-2 column tiles and a long k: every tile is shared out over many stream-K workgroups
    (tens of fp32 partials per tile, each holding only the row blocks below M; the MFMAs of row blocks past M are
    skipped).  Against the float64 oracle and repeatable bit for bit."""
    rng = np.random.default_rng(300 + M + n)
    k, K, cb = 6144, 3, 1
    tr, suh, svh = _case(rng, k, n, K)
    x = (rng.standard_normal((M, k)) * 0.5).astype(np.float16)
    args = ([_dev(tr)], [_dev(suh)], [_dev(svh)], cb)
    y = _ops().linear_prefill(_dev(x), *args)
    ref = orc.linear_forward(x, tr, suh, svh, K, cb, w_inner=c_reconstruct(coracle, tr, K, cb), dtype=np.float64)
    nrel, mrel = _errs(y.cpu().numpy(), ref)
    assert nrel <= TOL and mrel <= TOL, (nrel, mrel)
    for _ in range(2):
        assert torch.equal(_ops().linear_prefill(_dev(x), *args), y)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("rows,k,ns", [(1, 128, (128,)), (5, 384, (256, 128)), (37, 512, (256,)), (333, 1280, (128, 128, 384, 256)),
                                        (2200, 640, (512, 128, 256)), (8200, 2048, (128,))])
def test_prefill_rotation_layouts_bit_identical(bf16, rows, k, ns):
    """The input rotation has two kernels: 16 lanes per 128-value unit with 16-byte loads (x and every suh 16-byte
    aligned) and 32 lanes with 8-byte loads (otherwise).  Both run the butterfly's stages in the same order on the
    same pairs, so the whole prefill output must be bit-identical.  An input viewed 8 bytes into a buffer takes the
    second kernel.  The shapes reach 1, 2 and 4 units per lane group of the first (below 2^15, from 2^15, from 2^17
    units)."""
    rng = np.random.default_rng(9100 + rows + int(bf16))
    K, cb = 3, 1
    cases = [_case(rng, k, n, K) for n in ns]
    args = ([_dev(c[0]) for c in cases], [_dev(c[1]) for c in cases], [_dev(c[2]) for c in cases], cb)
    dt = torch.bfloat16 if bf16 else torch.float16
    x = torch.from_numpy(rng.standard_normal((rows, k)).astype(np.float32) * 0.5).to(dt).cuda()
    buf = torch.empty(rows * k + 8, dtype=dt, device="cuda")
    x_off = buf[4:4 + rows * k].view(rows, k)
    x_off.copy_(x)
    assert x.data_ptr() % 16 == 0 and x_off.data_ptr() % 16 == 8
    y16 = _ops().linear_prefill(x, *args)
    y8 = _ops().linear_prefill(x_off, *args)
    torch.cuda.synchronize()
    assert torch.equal(y16.view(torch.int16), y8.view(torch.int16))
    assert torch.isfinite(y16.float()).all()
