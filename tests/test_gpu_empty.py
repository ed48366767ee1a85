"""Empty batches through every torch-facing entry point: zero rows (tokens, sequences) launch nothing and return an
empty output of the right shape and dtype, the same as the reference's wrappers do for an empty batch; the calls right
after them, on the same workspaces, still give their usual results."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

K, CB = 3, 1


def _ops():
    from trellis_serve_amd import ops
    return ops


def _linear_layer(g, k, ns):
    trs = [torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), generator=g, dtype=torch.int32)
           .to(torch.int16).cuda() for n in ns]
    suhs = [(torch.randint(0, 2, (k,), generator=g) * 2 - 1).half().cuda() for _ in ns]
    svhs = [(torch.randint(0, 2, (n,), generator=g) * 2 - 1).half().cuda() for n in ns]
    return trs, suhs, svhs


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
def test_empty_rows_through_the_linear_paths(dtype):
    ops = _ops()
    g = torch.Generator().manual_seed(3)
    k, ns = 256, [256, 128]
    trs, suhs, svhs = _linear_layer(g, k, ns)
    x0 = torch.empty((0, k), dtype=dtype, device="cuda")
    for fn in (ops.linear, ops.linear_prefill):
        y = fn(x0, trs, suhs, svhs, CB)
        assert y.shape == (0, sum(ns)) and y.dtype == dtype
    y = ops.gemm_rotated(torch.empty((0, k), dtype=torch.float16, device="cuda"), trs[0], CB)
    assert y.shape == (0, ns[0])
    x = torch.randn((3, k), generator=g).to(dtype).cuda()
    assert torch.equal(ops.linear(x, trs, suhs, svhs, CB), ops.linear(x.clone(), trs, suhs, svhs, CB))


def test_empty_batch_through_moe_and_kv():
    ops = _ops()
    rng = np.random.default_rng(4)
    E, H, I, top_k = 8, 256, 128, 2
    st = {}
    for proj, (kk, nn) in (("gate", (H, I)), ("up", (H, I)), ("down", (I, H))):
        st[f"{proj}_trellis"] = torch.from_numpy(
            rng.integers(-32768, 32768, size=(E, kk // 16, nn // 16, 16 * K), dtype=np.int16)).cuda()
        st[f"{proj}_suh"] = torch.from_numpy(np.where(rng.random((E, kk)) < 0.5, -1.0, 1.0).astype(np.float16)).cuda()
        st[f"{proj}_svh"] = torch.from_numpy(np.where(rng.random((E, nn)) < 0.5, -1.0, 1.0).astype(np.float16)).cuda()
    x0 = torch.empty((0, H), dtype=torch.float16, device="cuda")
    ids0 = torch.empty((0, top_k), dtype=torch.int32, device="cuda")
    w0 = torch.empty((0, top_k), dtype=torch.float32, device="cuda")
    y = ops.moe_forward(x0, ids0, w0, st, CB)
    assert y.shape == (0, H) and y.dtype == torch.float16
    yc = ops.moe_combine(torch.empty((0, H), dtype=torch.float16, device="cuda"), w0, ids0, E)
    assert yc.shape == (0, H)
    x = torch.from_numpy((rng.standard_normal((2, H)) * 0.5).astype(np.float16)).cuda()
    ids = torch.tensor([[1, 5], [0, 7]], dtype=torch.int32, device="cuda")
    w = torch.tensor([[0.6, 0.4], [0.3, 0.7]], dtype=torch.float32, device="cuda")
    assert torch.equal(ops.moe_forward(x, ids, w, st, CB), ops.moe_forward(x.clone(), ids, w, st, CB))

    P, Hkv, Hq = 4, 2, 4
    kc = torch.zeros((P, Hkv, 16, 128), dtype=torch.int8, device="cuda")
    sc = torch.ones((P, Hkv), dtype=torch.float16, device="cuda")
    q0 = torch.empty((0, Hq, 128), dtype=torch.float16, device="cuda")
    table0 = torch.empty((0, 2), dtype=torch.int32, device="cuda")
    lens0 = torch.empty((0,), dtype=torch.int32, device="cuda")
    o = ops.kv_decode_attention(q0, kc, kc, sc, sc, table0, lens0, 8)
    assert o.shape == (0, Hq, 128)
