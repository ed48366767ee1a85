"""GPU parity of the EXL3 MoE layer (exl3_moe_forward) against the oracle's float64 routed-expert forward
(oracle.moe_forward, the exact layer of cuda/src/sglang_exl3/tools/moe_parity_sm86.py:76-89).  The kernel keeps the
reference kernels' fp16 intermediates (gate/up outputs, the SiLU product, down outputs), so its error against the
exact layer is the fp16 rounding of those values, not of the weights."""
import numpy as np
import pytest
import torch

from oracle import exl3_oracle as orc

pytestmark = pytest.mark.gpu


def _experts(rng, E, H, I, K, K_down=None):
    def mat(k, n, bits):
        return (rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * bits), dtype=np.int16),
                np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16),
                np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16))
    return [dict(gate=mat(H, I, K), up=mat(H, I, K), down=mat(I, H, K_down or K)) for _ in range(E)]


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
    ops.release_workspaces()
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


def test_moe_combine_edge_rows():
    """Unrouted slots, a repeated id and a token whose ids are all unrouted (its row is exactly zero, written into an
    output pre-filled with NaN), top_k = 10 (two chunks of the combine, the second partial): the exact layer's result."""
    from trellis_serve_amd import ops
    rng = np.random.default_rng(46)
    E, H, I, K, top_k, T = 16, 256, 128, 3, 10, 6
    ex = _experts(rng, E, H, I, K)
    x = (rng.standard_normal((T, H)) * 0.5).astype(np.float16)
    ids = np.stack([rng.permutation(E)[:top_k] for _ in range(T)]).astype(np.int32)
    ids[0, 1] = -1
    ids[1, :] = -1
    ids[2, 9] = ids[2, 0]
    ids[3, 8] = E
    w = rng.random((T, top_k)).astype(np.float32)
    y = torch.full((T, H), float("nan"), dtype=torch.float16, device="cuda")
    ops.moe_forward(torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(), _stack(ex),
                    1, out=y)
    assert (y[1] == 0).all()
    nrel, mrel = _errs(y.cpu().numpy(), orc.moe_forward(x, ids, w, ex, K, 1))
    assert nrel <= 2e-3 and mrel <= 2e-3, (nrel, mrel)

def test_moe_single_token_all_unrouted_is_zero():
    from trellis_serve_amd import ops
    rng = np.random.default_rng(41)
    E, H, I, K = 8, 256, 128, 3
    st = _stack(_experts(rng, E, H, I, K))
    x = torch.randn((1, H), device="cuda").half()
    ids = torch.full((1, 4), -1, dtype=torch.int32, device="cuda")
    ids[0, 2] = E  # out of range too
    w = torch.rand((1, 4), device="cuda")
    y = torch.full((1, H), float("nan"), dtype=torch.float16, device="cuda")
    ops.moe_forward(x, ids, w, st, 1, out=y)
    assert (y == 0).all()


@pytest.mark.parametrize("top_k", [4, 64])
def test_moe_single_token_top_k_range_bf16_and_repeat(top_k):
    """A single token up to the largest top-k (64; one grid row per slot): against the exact layer, bf16 out equal to
    fp16 out to bf16's half-ulp (one rounding of the same fp32 sum), repeat calls bit-identical, one unrouted slot
    skipped."""
    from trellis_serve_amd import ops
    rng = np.random.default_rng(50 + top_k)
    E, H, I, K = 128, 256, 128, 3
    ex = _experts(rng, E, H, I, K)
    st = _stack(ex)
    x = (rng.standard_normal((1, H)) * 0.5).astype(np.float16)
    ids = rng.permutation(E)[:top_k].astype(np.int32)[None]
    ids[0, top_k // 2] = -1
    w = (rng.random((1, top_k)) / top_k).astype(np.float32)
    xd, idd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    y = ops.moe_forward(xd, idd, wd, st, 1)
    nrel, mrel = _errs(y.cpu().numpy(), orc.moe_forward(x, ids, w, ex, K, 1))
    assert nrel <= 2e-3 and mrel <= 2e-3, (nrel, mrel)
    yb = ops.moe_forward(xd.bfloat16(), idd, wd, st, 1)
    assert yb.dtype == torch.bfloat16
    yh = ops.moe_forward(xd.bfloat16(), idd, wd, st, 1, out=torch.empty((1, H), dtype=torch.float16, device="cuda"))
    assert ((yb.float() - yh.float()).abs() <= yh.float().abs() * 2.0 ** -8 + 1e-6).all()
    for _ in range(3):
        assert torch.equal(ops.moe_forward(xd, idd, wd, st, 1), y)


def test_moe_many_slots_use_the_routing_launch():
    """2080 slots over 8 experts (260 per expert: passes of 64 slots, the last one partial); both ends of the token
    range against the exact layer, and a repeat is bit-identical."""
    from trellis_serve_amd import ops
    rng = np.random.default_rng(47)
    E, H, I, K, top_k, T = 8, 128, 128, 3, 8, 260  # 2080 slots
    ex = _experts(rng, E, H, I, K)
    x = (rng.standard_normal((T, H)) * 0.5).astype(np.float16)
    ids = np.stack([rng.permutation(E)[:top_k] for _ in range(T)]).astype(np.int32)
    ids[5, 3] = -1
    w = rng.random((T, top_k)).astype(np.float32)
    args = (torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(), _stack(ex), 2)
    y = ops.moe_forward(*args)
    for sl in (slice(0, 8), slice(T - 4, T)):
        nrel, mrel = _errs(y[sl].cpu().numpy(), orc.moe_forward(x[sl], ids[sl], w[sl], ex, K, 2))
        assert nrel <= 2e-3 and mrel <= 2e-3, (sl, nrel, mrel)
    assert torch.equal(ops.moe_forward(*args), y)


def test_moe_full_shape_batched_tokens_match_single_token(coracle):
    """BASELINE configs[3] shape (128 experts, top-8, hidden 2048, inter 768, K = 3 MCG): every k-split plan covers
    all input rows.  One token against the exact layer (C reconstruct); batches of 16 and 256 tokens (other k-split
    plans, other modes: only fp32 summation order differs) within 1e-3 of per-token calls, and sampled tokens of both
    batches against the exact layer."""
    from conftest import c_reconstruct
    from trellis_serve_amd import ops
    rng = np.random.default_rng(48)
    E, H, I, K, top_k, cb = 128, 2048, 768, 3, 8, 1
    st = {}
    for proj, (kk, nn) in (("gate", (H, I)), ("up", (H, I)), ("down", (I, H))):
        st[f"{proj}_trellis"] = torch.from_numpy(
            rng.integers(-32768, 32768, size=(E, kk // 16, nn // 16, 16 * K), dtype=np.int16)).cuda()
        st[f"{proj}_suh"] = torch.from_numpy(np.where(rng.random((E, kk)) < 0.5, -1.0, 1.0).astype(np.float16)).cuda()
        st[f"{proj}_svh"] = torch.from_numpy(np.where(rng.random((E, nn)) < 0.5, -1.0, 1.0).astype(np.float16)).cuda()
    T = 256
    # scaled so that the fp16 intermediates of 2048- and 768-long sums of unit-size weights stay finite
    x = torch.from_numpy((rng.standard_normal((T, H)) * 0.05).astype(np.float16)).cuda()
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32))
    wsel, ids = torch.topk(logits, top_k, dim=1)
    ids, w = ids.to(torch.int32).cuda(), torch.softmax(wsel, dim=1).cuda()

    # one token against the exact layer
    ids0 = ids[:1].cpu().numpy()
    ex, cache = [None] * E, {}  # indexed by expert id (the oracle skips ids outside [0, len))
    for e in set(ids0[0].tolist()):
        ex[e] = {p: tuple(st[f"{p}_{part}"][e].cpu().numpy() for part in ("trellis", "suh", "svh"))
                 for p in ("gate", "up", "down")}
        for p in ("gate", "up", "down"):
            cache[(e, p)] = c_reconstruct(coracle, ex[e][p][0], K, cb)
    single = [ops.moe_forward(x[t:t + 1], ids[t:t + 1], w[t:t + 1], st, cb) for t in range(16)]
    ref = orc.moe_forward(x[:1].cpu().numpy(), ids0, w[:1].cpu().numpy(), ex, K, cb, w_cache=cache)
    nrel, mrel = _errs(single[0].cpu().numpy(), ref)
    assert nrel <= 2e-3 and mrel <= 2e-3, (nrel, mrel)

    y16 = ops.moe_forward(x[:16], ids[:16], w[:16], st, cb).float()
    y256 = ops.moe_forward(x, ids, w, st, cb).float()
    for t in range(16):
        for y in (y16, y256):
            d = (y[t] - single[t].float()).norm() / single[t].float().norm()
            assert d.item() <= 1e-3, (t, y.shape[0], d.item())
    for t in (100, 255):
        one = ops.moe_forward(x[t:t + 1], ids[t:t + 1], w[t:t + 1], st, cb).float()
        d = (y256[t] - one[0]).norm() / one[0].norm()
        assert d.item() <= 1e-3, (t, d.item())

    # the batched calls themselves (the benchmark's T = 16 and T = 256 launches) against the exact layer on sampled
    # tokens, each touched expert decoded by the C restatement
    xs, ids_np, w_np = x.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy()
    for y, toks in ((y16, (3, 9, 15)), (y256, (0, 37, 81, 128, 199, 255))):
        for t in toks:
            for e in set(ids_np[t].tolist()):
                if ex[e] is None:
                    ex[e] = {p: tuple(st[f"{p}_{part}"][e].cpu().numpy() for part in ("trellis", "suh", "svh"))
                             for p in ("gate", "up", "down")}
                    for p in ("gate", "up", "down"):
                        cache[(e, p)] = c_reconstruct(coracle, ex[e][p][0], K, cb)
            ref = orc.moe_forward(xs[t:t + 1], ids_np[t:t + 1], w_np[t:t + 1], ex, K, cb, w_cache=cache)
            nrel, mrel = _errs(y[t:t + 1].cpu().numpy(), ref)
            assert nrel <= 2e-3 and mrel <= 2e-3, (y.shape[0], t, nrel, mrel)


@pytest.mark.parametrize("T", [3, 20, 40, 300])
def test_moe_slot_groups_and_passes_match_exact_layer(T):
    """Several tokens: routing + input rotation launch, up to 16 P slots sharing each decoded tile, the GLU folded into
    the gate/up reducer.  3 / 20 / 40 / 300 tokens over 8 experts run P = 1 / 2 / 4 / 4 groups (40 tokens: one pass of 40 slots per
    expert in 3 groups; 300 tokens: 300 slots per expert, several passes).  Every token against the exact layer, and
    two tokens against their single-token calls (slot mode: other k-split plan) within 1e-3."""
    from trellis_serve_amd import ops
    rng = np.random.default_rng(60 + T)
    E, H, I, K, top_k = 8, 256, 256, 3, 8
    ex = _experts(rng, E, H, I, K)
    st = _stack(ex)
    x = (rng.standard_normal((T, H)) * 0.5).astype(np.float16)
    ids = np.stack([rng.permutation(E)[:top_k] for _ in range(T)]).astype(np.int32)
    ids[0, 2] = -1
    w = rng.random((T, top_k)).astype(np.float32)
    xd, idd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda()
    y = ops.moe_forward(xd, idd, wd, st, 1)
    nrel, mrel = _errs(y.cpu().numpy(), orc.moe_forward(x, ids, w, ex, K, 1))
    assert nrel <= 2e-3 and mrel <= 2e-3, (nrel, mrel)
    for t in (0, T - 1):
        one = ops.moe_forward(xd[t:t + 1], idd[t:t + 1], wd[t:t + 1], st, 1).float()[0]
        assert ((y[t].float() - one).norm() / one.norm()).item() <= 1e-3, t
    assert torch.equal(ops.moe_forward(xd, idd, wd, st, 1), y)

def _moe_cases(seed, count):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        E = int(rng.integers(2, 17))
        out.append((E, 128 * int(rng.integers(1, 5)), 128 * int(rng.integers(1, 5)), int(rng.choice([2, 3, 4, 5, 6, 8])),
                    int(rng.integers(0, 3)), int(rng.integers(1, 49)), int(rng.integers(1, min(8, E) + 1))))
    return out


MOE_CASES = _moe_cases(2028, 12)


@pytest.mark.parametrize("case", MOE_CASES, ids=[f"E{c[0]}-H{c[1]}-I{c[2]}-K{c[3]}-cb{c[4]}-T{c[5]}-top{c[6]}"
                                                  for c in MOE_CASES])
def test_moe_random_shapes_match_exact_layer(case):
    """Seeded random MoE layers: experts 2-16, hidden and inter 128-512, every bit width and codebook, 1-48 tokens,
    top-k 1-8 with about one id in ten unrouted (-1), against the float64 exact layer."""
    from trellis_serve_amd import ops
    E, H, I, K, cb, T, top_k = case
    rng = np.random.default_rng(abs(hash(case)) % (1 << 32))
    ex = _experts(rng, E, H, I, K)
    x = (rng.standard_normal((T, H)) * 0.5).astype(np.float16)
    ids = np.stack([rng.permutation(E)[:top_k] for _ in range(T)]).astype(np.int32)
    ids[rng.random(ids.shape) < 0.1] = -1
    w = rng.random((T, top_k)).astype(np.float32)
    y = ops.moe_forward(torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(),
                        _stack(ex), cb).cpu().numpy()
    ref = orc.moe_forward(x, ids, w, ex, K, cb)
    if not np.abs(ref).max() > 0:  # every slot unrouted: a zero row
        assert (y == 0).all()
        return
    nrel, mrel = _errs(y, ref)
    assert nrel <= 2e-3 and mrel <= 2e-3, (case, nrel, mrel)


@pytest.mark.parametrize("K, K_down", [(3, 4), (4, 3), (2, 6)])
@pytest.mark.parametrize("T", [1, 5, 40])
def test_moe_down_bitrate_differs_from_gate_up(K, K_down, T):
    """A checkpoint may store down_proj at another bitrate than gate_proj / up_proj (the reference requires only gate
    K == up K, cuda/src/sglang_exl3/sglang_glue/moe.py:148-152, and runs bits_gate_up and bits_down separately,
    kernels/reference.py:123-149).  Single token (slot mode), a few tokens (P = 1) and 40 tokens (P = 2, the GLU
    folded into the gate/up reducer) against the float64 exact layer, every codebook."""
    from trellis_serve_amd import ops
    rng = np.random.default_rng(7000 + 10 * K + K_down + T)
    E, H, I, top_k = 8, 256, 384, 4
    ex = _experts(rng, E, H, I, K, K_down)
    st = _stack(ex)
    assert st["down_trellis"].shape[-1] == 16 * K_down and st["gate_trellis"].shape[-1] == 16 * K
    x = (rng.standard_normal((T, H)) * 0.5).astype(np.float16)
    ids = np.stack([rng.permutation(E)[:top_k] for _ in range(T)]).astype(np.int32)
    w = rng.random((T, top_k)).astype(np.float32)
    for cb in (0, 1, 2):
        y = ops.moe_forward(torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(), st,
                            cb).cpu().numpy()
        nrel, mrel = _errs(y, orc.moe_forward(x, ids, w, ex, None, cb))
        assert nrel <= 2e-3 and mrel <= 2e-3, (K, K_down, T, cb, nrel, mrel)


def test_moe_full_shape_single_token_mixed_bitrates(coracle):
    """BASELINE configs[3] shape (128 experts, top-8, hidden 2048, inter 768, MCG) with gate/up at K = 3 and down at
    K = 4: one token against the exact layer (C reconstruct of every touched expert)."""
    from conftest import c_reconstruct
    from trellis_serve_amd import ops
    rng = np.random.default_rng(49)
    E, H, I, top_k, cb = 128, 2048, 768, 8, 1
    bits = {"gate": 3, "up": 3, "down": 4}
    st = {}
    for proj, (kk, nn) in (("gate", (H, I)), ("up", (H, I)), ("down", (I, H))):
        st[f"{proj}_trellis"] = torch.from_numpy(
            rng.integers(-32768, 32768, size=(E, kk // 16, nn // 16, 16 * bits[proj]), dtype=np.int16)).cuda()
        st[f"{proj}_suh"] = torch.from_numpy(np.where(rng.random((E, kk)) < 0.5, -1.0, 1.0).astype(np.float16)).cuda()
        st[f"{proj}_svh"] = torch.from_numpy(np.where(rng.random((E, nn)) < 0.5, -1.0, 1.0).astype(np.float16)).cuda()
    x = (rng.standard_normal((1, H)) * 0.05).astype(np.float16)
    ids = rng.permutation(E)[:top_k].astype(np.int32)[None]
    w = rng.random((1, top_k)).astype(np.float32)
    ex, cache = [None] * E, {}
    for e in ids[0].tolist():
        ex[e] = {p: tuple(st[f"{p}_{part}"][e].cpu().numpy() for part in ("trellis", "suh", "svh"))
                 for p in ("gate", "up", "down")}
        for p in ("gate", "up", "down"):
            cache[(e, p)] = c_reconstruct(coracle, ex[e][p][0], bits[p], cb)
    y = ops.moe_forward(torch.from_numpy(x).cuda(), torch.from_numpy(ids).cuda(), torch.from_numpy(w).cuda(), st, cb)
    nrel, mrel = _errs(y.cpu().numpy(), orc.moe_forward(x, ids, w, ex, None, cb, w_cache=cache))
    assert nrel <= 2e-3 and mrel <= 2e-3, (nrel, mrel)
