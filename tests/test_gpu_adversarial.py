"""Adversarial activations through the decode-GEMV, the prefill decode-GEMM and the MoE layer: all-zero rows, rows near
the top of the fp16 range, fp16 subnormal rows and batches that mix all of them.  Rows are independent, so every row
is checked against its own float64 evaluation (zero rows must come back exactly zero).  Subnormal rows are compared
with the kernels' rounding points applied (the fp16 rotated input, the fp16 output): below 2^-14 an fp16 value keeps
only the bits above 2^-24, so the bar there is a few units of 2^-24 plus the usual 2e-3 of the largest output rather than a relative error
per row -- the reference's kernels round at the same points (cuda/csrc/exl3_had.cuh:20-84)."""
import numpy as np
import pytest
import torch

from conftest import c_reconstruct
from oracle import exl3_oracle as orc

pytestmark = pytest.mark.gpu
TOL = 2e-3
SUB_ULP = 2.0 ** -24


def _ops():
    from trellis_serve_amd import ops
    return ops


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _matrix(seed, k, n, K):
    rng = np.random.default_rng(seed)
    tr = rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * K), dtype=np.int16)
    suh = np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16)
    svh = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16)
    return tr, suh, svh


def _rows(rng, k, kinds):
    """One activation row per kind: 'zero', 'normal' (N(0, 0.5)), 'huge' (one spike of 4000 plus N(0, 50): outputs
    reach ~2e4, a third of fp16's 65504), 'tiny' (N(0, 1e-3)), 'subnormal' (|x| < 2^-14, fp16 subnormals)."""
    out = np.zeros((len(kinds), k), dtype=np.float32)
    for i, kind in enumerate(kinds):
        if kind == "normal":
            out[i] = rng.standard_normal(k) * 0.5
        elif kind == "huge":
            out[i] = rng.standard_normal(k) * 50
            out[i, rng.integers(k)] = 4000
        elif kind == "tiny":
            out[i] = rng.standard_normal(k) * 1e-3
        elif kind == "subnormal":
            out[i] = rng.standard_normal(k) * 1e-6
    return out.astype(np.float16)


def _check_rows(y, x, kinds, tr, suh, svh, K, cb, w):
    assert np.isfinite(y).all()
    exact = orc.linear_forward(x, tr, suh, svh, K, cb, w_inner=w, dtype=np.float64)
    # the same layer with the kernels' rounding points: fp16 rotated input, fp16 output
    xh = orc.had_in_fp16(x, suh).astype(np.float64)
    rounded = (orc.had_rows(xh @ w.astype(np.float64), np.float64) * svh.astype(np.float64)).astype(np.float16)
    for i, kind in enumerate(kinds):
        yi = y[i].astype(np.float64)
        if kind == "zero":
            assert not yi.any(), "a zero row must give an exactly zero output"
        elif kind == "subnormal":
            ri = rounded[i].astype(np.float64)
            err = np.abs(yi - ri).max()
            assert err <= 4 * SUB_ULP + TOL * np.abs(ri).max(), (kind, err / SUB_ULP)
            assert np.abs(yi).max() > 0, "subnormal activations were flushed to zero"
        else:
            ref = exact[i]
            nrel = np.linalg.norm(yi - ref) / np.linalg.norm(ref)
            mrel = np.abs(yi - ref).max() / np.abs(ref).max()
            assert nrel <= TOL and mrel <= TOL, (kind, nrel, mrel)


GEMV_BATCHES = [["zero"], ["huge"], ["subnormal"], ["tiny"],
                ["huge", "tiny", "zero", "normal"],
                ["subnormal", "huge", "normal", "zero", "tiny", "normal", "zero", "huge"] * 2]


@pytest.mark.parametrize("kinds", GEMV_BATCHES, ids=lambda k: "-".join(k[:8]) + ("x2" if len(k) > 8 else ""))
@pytest.mark.parametrize("K,cb", [(3, 1), (4, 0), (2, 2)])
def test_gemv_adversarial_rows(coracle, kinds, K, cb):
    k, n = 2048, 1280
    tr, suh, svh = _matrix(40 + K, k, n, K)
    w = c_reconstruct(coracle, tr, K, cb)
    x = _rows(np.random.default_rng(len(kinds) + K), k, kinds)
    y = _ops().linear(_dev(x), [_dev(tr)], [_dev(suh)], [_dev(svh)], cb).cpu().numpy()
    _check_rows(y, x, kinds, tr, suh, svh, K, cb, w)


@pytest.mark.parametrize("K,cb", [(3, 1), (5, 2)])
def test_prefill_adversarial_rows(coracle, K, cb):
    """The decode-GEMM at 160 rows of every kind, interleaved (tiles of 16 rows mix kinds)."""
    k, n = 2048, 1280
    tr, suh, svh = _matrix(60 + K, k, n, K)
    w = c_reconstruct(coracle, tr, K, cb)
    kinds = ["zero", "huge", "subnormal", "tiny", "normal"] * 32
    x = _rows(np.random.default_rng(9 + K), k, kinds)
    y = _ops().linear_prefill(_dev(x), [_dev(tr)], [_dev(suh)], [_dev(svh)], cb).cpu().numpy()
    _check_rows(y, x, kinds, tr, suh, svh, K, cb, w)


def test_moe_adversarial_tokens():
    """Zero tokens, tiny tokens and large tokens in one batch, with a zero routing weight among the choices: each
    token against its own exact layer.  The layer is quadratic in x (SiLU(g) * u) and keeps fp16 intermediates as the
    reference kernels do, so "large" is x ~ N(0, 1) here: per-expert down outputs then reach ~1.6e4, a quarter of
    fp16's 65504 (at N(0, 4) they overflow, in the reference kernels as well)."""
    from test_gpu_moe import _experts, _stack
    rng = np.random.default_rng(77)
    E, H, I, K, top_k = 8, 256, 256, 3, 2
    ex = _experts(rng, E, H, I, K)
    scales = [0.0, 1e-3, 0.5, 1.0, 0.0, 1.0]
    x = np.stack([rng.standard_normal(H) * s for s in scales]).astype(np.float16)
    T = len(scales)
    ids = np.stack([rng.choice(E, top_k, replace=False) for _ in range(T)]).astype(np.int32)
    w = np.full((T, top_k), 0.5, np.float32)
    w[3, 1] = 0.0
    y = _ops().moe_forward(_dev(x), _dev(ids), _dev(w), _stack(ex), 1).cpu().numpy()
    ref = orc.moe_forward(x, ids, w, ex, K, 1)
    assert np.isfinite(y).all()
    for t, s in enumerate(scales):
        if s == 0.0:
            assert not y[t].astype(np.float64).any()
            continue
        yt, rt = y[t].astype(np.float64), ref[t]
        nrel = np.linalg.norm(yt - rt) / np.linalg.norm(rt)
        assert nrel <= TOL, (t, s, nrel)
