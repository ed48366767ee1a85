"""The fused kernels at the benchmark's own shapes (BASELINE configs[1] and [2]), where the split plans, tail tiles
and shard maps take the forms the small parity shapes never reach.  The reference output is built on the GPU from
pieces pinned elsewhere: the bit-exact reconstruct (W_inner), the input rotation (1-ulp fp16 agreement with the
oracle) and an fp32 matmul, then the output rotation; the fused result must agree within the north-star tolerance
(norm-relative and max-relative 2e-3)."""
import pytest
import torch

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _ops():
    from trellis_serve_amd import ops
    return ops


def _layer(g, k, ns, K):
    trs = [torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16, generator=g).cuda() for n in ns]
    suhs = [(torch.randint(0, 2, (k,), generator=g) * 2 - 1).half().cuda() for _ in ns]
    svhs = [(torch.randint(0, 2, (n,), generator=g) * 2 - 1).half().cuda() for n in ns]
    return trs, suhs, svhs


def _reference(x, trs, suhs, svhs, cb):
    """had(had(x * suh) @ W_inner) * svh per shard: rotation kernels + reconstruct + fp32 matmul."""
    ops = _ops()
    M = x.shape[0]
    out = torch.empty((M, sum(t.shape[1] * 16 for t in trs)), dtype=torch.float16, device=x.device)
    col = 0
    for tr, suh, svh in zip(trs, suhs, svhs):
        xh = ops.had_in_group(x, suh)
        w = ops.reconstruct(tr, cb)
        y = (xh.float() @ w.float()).half()
        ops.had_out_into(y, svh, out, col)
        col += w.shape[1]
        del w
    return out


def _check(y, ref):
    y, ref = y.float(), ref.float()
    nrel = ((y - ref).norm() / ref.norm()).item()
    mrel = ((y - ref).abs().max() / ref.abs().max()).item()
    assert nrel <= TOL and mrel <= TOL, (nrel, mrel)


C2_LAYERS = {"qkv": (5120, [6144, 1024, 1024]), "o": (6144, [5120]), "gate_up": (5120, [17408, 17408]),
             "down": (17408, [5120])}


@pytest.mark.parametrize("M", [1, 4, 16])
@pytest.mark.parametrize("name", list(C2_LAYERS))
def test_gemv_c2_layer_set_shapes(name, M):
    """the four fused K = 3 MCG linears of the 27B-class layer set at M = 1, 4 and 16."""
    g = torch.Generator(device="cpu").manual_seed(100 + M)
    k, ns = C2_LAYERS[name]
    trs, suhs, svhs = _layer(g, k, ns, 3)
    x = torch.randn((M, k), generator=g).half().cuda()
    _check(_ops().linear(x, trs, suhs, svhs, 1), _reference(x, trs, suhs, svhs, 1))


@pytest.mark.parametrize("name", list(C2_LAYERS))
def test_c2_layer_set_shapes_read_the_repacked_layout_bit_identically(name):
    """configs[1] at M = 1 with the trellis repacked to the BLOCKS layout: the decode-GEMV gives the same bits as on
    the stored layout (the split-K chain runs in one XCD's L2 here: every layer has a multiple of 8 column blocks)."""
    g = torch.Generator(device="cpu").manual_seed(7)
    k, ns = C2_LAYERS[name]
    trs, suhs, svhs = _layer(g, k, ns, 3)
    ops = _ops()
    packed = [ops.repack_trellis(t) for t in trs]
    x = torch.randn((1, k), generator=g).half().cuda()
    assert torch.equal(ops.linear(x, trs, suhs, svhs, 1), ops.linear(x, packed, suhs, svhs, 1, layout=1))


@pytest.mark.parametrize("K,cb,M", [(3, 1, 2048), (2, 0, 512), (8, 2, 512), (3, 1, 8192), (4, 2, 2048), (5, 1, 2048),
                                    (6, 0, 2048), (2, 0, 2048), (8, 2, 2048)])
def test_prefill_c3_shape(K, cb, M):
    """the 5120 -> 17408 prefill decode-GEMM (68 column tiles, split-K tail items) at the benchmark's K,
    codebook and row counts."""
    g = torch.Generator(device="cpu").manual_seed(200 + K)
    trs, suhs, svhs = _layer(g, 5120, [17408], K)
    x = (torch.randn((M, 5120), generator=g) * 0.5).half().cuda()
    _check(_ops().linear_prefill(x, trs, suhs, svhs, cb), _reference(x, trs, suhs, svhs, cb))


@pytest.mark.parametrize("name,M,K,cb,fn", [("gate_up", 1, 3, 1, "linear"), ("down", 4, 3, 1, "linear"),
                                            ("c3", 2048, 3, 1, "linear_prefill"), ("c3", 8192, 5, 2, "linear_prefill")])
def test_full_shape_column_slices_against_the_oracle(coracle, name, M, K, cb, fn):
    """The full-shape outputs, checked on sampled 128-column blocks and rows against the float64 oracle built from the
    C restatement's decode (the output rotation works per 128-column block, so a block of columns is a complete
    smaller layer): full-size parity that does not rest on this library's own reconstruct and rotation kernels."""
    import numpy as np
    from conftest import c_reconstruct
    from oracle import exl3_oracle as orc
    k, ns = (5120, [17408]) if name == "c3" else C2_LAYERS[name]
    g = torch.Generator(device="cpu").manual_seed(300 + M + K)
    trs, suhs, svhs = _layer(g, k, ns, K)
    x = (torch.randn((M, k), generator=g) * 0.5).half().cuda()
    y = getattr(_ops(), fn)(x, trs, suhs, svhs, cb).float().cpu().numpy()
    rng = np.random.default_rng(M)
    rows = np.sort(rng.choice(M, size=min(M, 48), replace=False))
    xs = x.cpu().numpy()[rows]
    col = 0
    for tr, suh, svh in zip(trs, suhs, svhs):
        tn = tr.shape[1]
        trn = tr.cpu().numpy()
        for cbk in rng.choice(tn // 8, size=min(3, tn // 8), replace=False):
            sl = trn[:, 8 * cbk:8 * cbk + 8]
            w = c_reconstruct(coracle, sl, K, cb)
            sv = svh.cpu().numpy()[128 * cbk:128 * cbk + 128]
            ref = orc.linear_forward(xs, sl, suh.cpu().numpy(), sv, K, cb, w_inner=w, dtype=np.float64)
            got = y[rows][:, col + 128 * cbk:col + 128 * cbk + 128].astype(np.float64)
            nrel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
            mrel = np.abs(got - ref).max() / np.abs(ref).max()
            assert nrel <= TOL and mrel <= TOL, (cbk, nrel, mrel)
        col += tn * 16


@pytest.mark.parametrize("K", (2, 3, 4, 5, 6, 8))
@pytest.mark.parametrize("cb", (0, 1, 2))
def test_prefill_gemm_one_hot_readout_on_c3_column_slices(coracle, K, cb):
    """The decoded weights of the prefill decode-GEMM read back bit for bit (the method of
    cuda/src/sglang_exl3/parity/marlin_parity.py:149-159): 5120 identity rows through exl3_gemm_rotated take the
    decode-GEMM (no rotations), on two column slices of a C3 (5120 -> 17408) trellis -- 768 columns from the start
    (three 256-column tiles) and 640 from the end (the last a half tile) -- against the C restatement's decode.  With
    20 row blocks the launch shares tiles out by k-step runs, so partial tiles are summed too (zeros but one term)."""
    import numpy as np
    from conftest import c_reconstruct
    rng = np.random.default_rng(400 + 10 * K + cb)
    k, n = 5120, 17408
    tr = rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * K), dtype=np.int16)
    eye = torch.eye(k, dtype=torch.float16, device="cuda")
    for c0, c1 in ((0, 768), (n - 640, n)):
        sl = np.ascontiguousarray(tr[:, c0 // 16:c1 // 16])
        got = _ops().gemm_rotated(eye, torch.from_numpy(sl).cuda(), cb).cpu().numpy()
        np.testing.assert_array_equal(got.view(np.uint16), c_reconstruct(coracle, sl, K, cb).view(np.uint16),
                                      err_msg=f"columns {c0}:{c1}")
