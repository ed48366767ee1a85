"""The allocation-free entry point exl3_linear_noalloc against exl3_linear, through the C-ABI.

exl3_linear_noalloc runs the same kernels on a scratch array the library holds per GPU instead of a caller's
workspace, so its outputs must equal exl3_linear's bit for bit on the same inputs.  Two calls in a row, the second
smaller, check that the scratch the first call leaves behind (its partials; its counters, which every call resets)
does not leak into the next.  The oracle pins the result as well.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import exl3_oracle as orc

pytestmark = pytest.mark.gpu


def _group(rng, k, ns, K):
    tr = [rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * K), dtype=np.int16) for n in ns]
    suh = [np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16) for _ in ns]
    svh = [np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16) for n in ns]
    return tr, suh, svh


def _shards(dev_tr, dev_suh, dev_svh):
    arr = (_lib().Exl3Shard * len(dev_tr))()
    for i, (t, a, b) in enumerate(zip(dev_tr, dev_suh, dev_svh)):
        arr[i] = _lib().Exl3Shard(t.data_ptr(), a.data_ptr(), b.data_ptr(), t.shape[1] * 16)
    return arr


def _lib():
    from trellis_serve_amd import _lib
    return _lib


def _both(x, arr, K, cb, n_total):
    """(noalloc output, workspace output) of the same call, both on torch's current stream."""
    lib = _lib().load()
    rows, k = x.shape
    stream = torch.cuda.current_stream().cuda_stream
    y0 = torch.full((rows, n_total), float("nan"), dtype=torch.float16, device=x.device)
    y1 = torch.full((rows, n_total), float("nan"), dtype=torch.float16, device=x.device)
    _lib().check(lib.exl3_linear_noalloc(x.data_ptr(), 0, rows, k, arr, len(arr), K, cb, y0.data_ptr(), 0, stream),
                 "exl3_linear_noalloc")
    need = lib.exl3_linear_workspace_bytes(rows, k, n_total, K)
    ws = torch.zeros(need, dtype=torch.uint8, device=x.device)
    _lib().check(lib.exl3_linear(x.data_ptr(), 0, rows, k, arr, len(arr), K, cb, y1.data_ptr(), 0, ws.data_ptr(),
                                 ws.numel(), stream), "exl3_linear")
    torch.cuda.synchronize()
    return y0, y1


@pytest.mark.parametrize("K, cb", [(3, 1), (4, 0), (2, 2)])
def test_noalloc_equals_workspace_entry_on_two_calls(K, cb):
    """A 3-shard group at 16 rows (the rotated-rows pre-pass and 16-row split plan), then a single-shard call of one
    row on a smaller matrix: bit-identical to exl3_linear each time, and within the oracle's tolerance."""
    rng = np.random.default_rng(900 + 10 * K + cb)
    cases = ((2048, (1024, 256, 256), 16), (512, (384,), 1))
    for k, ns, rows in cases:
        tr, suh, svh = _group(rng, k, ns, K)
        d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
        dtr, dsuh, dsvh = [d(t) for t in tr], [d(s) for s in suh], [d(s) for s in svh]
        x = (rng.standard_normal((rows, k))).astype(np.float16)
        y0, y1 = _both(d(x), _shards(dtr, dsuh, dsvh), K, cb, sum(ns))
        assert torch.equal(y0, y1), (k, ns, rows)
        col = 0
        for t, a, b, n in zip(tr, suh, svh, ns):
            ref = orc.linear_forward(x, t, a, b, K, cb, dtype=np.float64)
            got = y0[:, col:col + n].cpu().numpy().astype(np.float64)
            assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 2e-3
            col += n
