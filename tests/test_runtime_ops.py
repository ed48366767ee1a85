"""The custom op surface (torch.ops.exl3_mi355x.linear): schema, fake impl for tracing (CPU), and on the GPU the row
dispatch (GEMV below the switch point, fused GEMM above) against the float64 oracle."""
import numpy as np
import pytest
import torch


def test_op_is_registered_with_fake_impl():
    from trellis_serve_amd.runtime import ops
    assert hasattr(torch.ops.exl3_mi355x, "linear")
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        x = torch.empty((3, 5, 256), dtype=torch.float16)
        tr = [torch.empty((16, 8, 48), dtype=torch.int16), torch.empty((16, 4, 48), dtype=torch.int16)]
        su = [torch.empty(256, dtype=torch.float16)] * 2
        sv = [torch.empty(128, dtype=torch.float16), torch.empty(64, dtype=torch.float16)]
        y = ops.linear(x, tr, su, sv, 1)
        assert y.shape == (3, 5, 192) and y.dtype == torch.float16


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [1, 33, 64, 65, 600])
def test_op_dispatch_matches_oracle(coracle, rows):
    from conftest import c_reconstruct
    from oracle import exl3_oracle as orc
    from trellis_serve_amd.runtime import ops
    rng = np.random.default_rng(rows)
    k, n, K, cb = 512, 256, 3, 1
    tr = rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * K), dtype=np.int16)
    suh = np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16)
    svh = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16)
    x = (rng.standard_normal((rows, k)) * 0.5).astype(np.float16)
    d = lambda a: torch.from_numpy(a).cuda()  # noqa: E731
    y = ops.linear(d(x).view(1, rows, k), [d(tr)], [d(suh)], [d(svh)], cb).view(rows, n).cpu().numpy()
    ref = orc.linear_forward(x, tr, suh, svh, K, cb, w_inner=c_reconstruct(coracle, tr, K, cb), dtype=np.float64)
    nrel = np.linalg.norm(y.astype(np.float64) - ref) / np.linalg.norm(ref)
    mrel = np.abs(y.astype(np.float64) - ref).max() / np.abs(ref).max()
    assert nrel <= 2e-3 and mrel <= 2e-3, (nrel, mrel)
