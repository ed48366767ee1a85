"""GPU parity of the EXL3 MoE layer (exl3_moe_forward) against the oracle's float64 routed-expert forward
(oracle.moe_forward, the exact layer of cuda/src/sglang_exl3/tools/moe_parity_sm86.py:76-89).  The kernel keeps the
reference kernels' fp16 intermediates (gate/up outputs, the SiLU product, down outputs), so its error against the
exact layer is the fp16 rounding of those values, not of the weights."""
import numpy as np
import pytest
import torch

from oracle import exl3_oracle as orc

pytestmark = pytest.mark.gpu


def _experts(rng, E, H, I, K):
    def mat(k, n):
        return (rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * K), dtype=np.int16),
                np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16),
                np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16))
    return [dict(gate=mat(H, I), up=mat(H, I), down=mat(I, H)) for _ in range(E)]


def _stack(ex):
    d = {}
    for proj in ("gate", "up", "down"):
        for i, part in enumerate(("trellis", "suh", "svh")):
            d[f"{proj}_{part}"] = torch.from_numpy(np.stack([e[proj][i] for e in ex])).cuda()
    return d


def _errs(y, ref):
    y = y.astype(np.float64)
    return np.linalg.norm(y - ref) / np.linalg.norm(ref), np.abs(y - ref).max() / np.abs(ref).max()


@pytest.mark.parametrize("T,cb", [(1, 1), (5, 0), (64, 2)])
def test_moe_matches_exact_layer(T, cb):
    rng = np.random.default_rng(100 + T)
    E, H, I, K, top_k = 16, 256, 256, 3, 4
    ex = _experts(rng, E, H, I, K)
    x = (rng.standard_normal((T, H)) * 0.5).astype(np.float16)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    ids = np.argsort(-logits, axis=1)[:, :top_k].astype(np.int32)
    sel = np.take_along_axis(logits, ids, 1)
    w = (np.exp(sel - sel.max(1, keepdims=True)) / np.exp(sel - sel.max(1, keepdims=True)).sum(1, keepdims=True))
    w = w.astype(np.float32)
    if T > 1:
        ids[1, 2] = -1  # an unrouted slot is skipped
    from trellis_serve_amd import ops
    y = ops.moe_forward(torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(),
                        _stack(ex), cb).cpu().numpy()
    ref = orc.moe_forward(x, ids, w, ex, K, cb)
    nrel, mrel = _errs(y, ref)
    print(f"T={T} cb={cb}: norm-rel {nrel:.2e} max-rel {mrel:.2e}")
    assert nrel <= 2e-3 and mrel <= 2e-3, (nrel, mrel)


def test_moe_bf16_and_determinism():
    rng = np.random.default_rng(9)
    E, H, I, K, top_k, T = 8, 256, 128, 3, 2, 7
    ex = _experts(rng, E, H, I, K)
    st = _stack(ex)
    x = torch.from_numpy((rng.standard_normal((T, H)) * 0.5).astype(np.float32)).cuda().bfloat16()
    ids = torch.from_numpy(rng.integers(0, E, size=(T, top_k)).astype(np.int32)).cuda()
    w = torch.rand((T, top_k), device="cuda")
    from trellis_serve_amd import ops
    yb = ops.moe_forward(x, ids, w, st, 1)
    assert yb.dtype == torch.bfloat16
    first = ops.moe_forward(x.half(), ids, w, st, 1)
    # the combine rounds its fp32 sum once to the output dtype (exl3_marlin_moe.cu:262-292): bf16 out is that sum
    # rounded to bf16, fp16 out the same sum rounded to fp16, so they agree to bf16's half-ulp
    diff = (yb.float() - first.float()).abs()
    assert (diff <= first.float().abs() * 2.0 ** -8 + 1e-6).all()
    for _ in range(5):
        assert torch.equal(ops.moe_forward(x.half(), ids, w, st, 1), first)
        assert torch.equal(ops.moe_forward(x, ids, w, st, 1), yb)


def test_moe_workspace_shared_by_calls_of_different_shapes():
    """A call with many slots, then calls with fewer slots and another layer shape, on one workspace: the split
    counters sit in a fixed region, so no call reads an earlier call's rows or partials as counters."""
    from trellis_serve_amd import ops
    ops._moe_ws.clear()
    rng = np.random.default_rng(11)
    for E, H, I, T, top_k in ((16, 256, 256, 64, 4), (16, 256, 256, 1, 4), (8, 512, 128, 3, 2), (16, 256, 256, 9, 4)):
        ex = _experts(rng, E, H, I, 3)
        x = (rng.standard_normal((T, H)) * 0.5).astype(np.float16)
        ids = np.stack([rng.permutation(E)[:top_k] for _ in range(T)]).astype(np.int32)
        w = rng.random((T, top_k)).astype(np.float32)
        y = ops.moe_forward(torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(),
                            _stack(ex), 1).cpu().numpy()
        nrel, mrel = _errs(y, orc.moe_forward(x, ids, w, ex, 3, 1))
        assert nrel <= 2e-3 and mrel <= 2e-3, (E, H, I, T, nrel, mrel)


def test_moe_single_token_slot_mode_with_repeated_and_unrouted_ids():
    """One token runs its top-k slots directly (no routing launch); a repeated expert id and an unrouted slot (-1)
    in that token must give the exact layer's result (split counters index slots, not experts)."""
    from trellis_serve_amd import ops
    rng = np.random.default_rng(12)
    E, H, I, K, top_k = 8, 256, 128, 3, 4
    ex = _experts(rng, E, H, I, K)
    x = (rng.standard_normal((1, H)) * 0.5).astype(np.float16)
    ids = np.array([[3, 3, -1, 6]], dtype=np.int32)
    w = np.array([[0.4, 0.3, 0.2, 0.1]], dtype=np.float32)
    for cb in (0, 1):
        y = ops.moe_forward(torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(),
                            _stack(ex), cb).cpu().numpy()
        nrel, mrel = _errs(y, orc.moe_forward(x, ids, w, ex, K, cb))
        assert nrel <= 2e-3 and mrel <= 2e-3, (cb, nrel, mrel)
