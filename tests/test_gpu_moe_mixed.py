"""GPU parity of mixed-K MoE layers: experts in two K classes (the reference's MixedPack, e.g. 192 experts at K = 3 plus
64 at K = 4; cuda/src/sglang_exl3/kernels/marlin_moe.py:135-170), served by one routing plus per-class expert launches
(exl3_moe_forward_classes; the reference's run_mixed, marlin_moe.py:247-272) or by the per-launch stages with the
one-launch two-class align (exl3_moe_align_classes; moe_align_decode, cuda/csrc/exl3_marlin_moe.cu:532-618).
Against the float64 exact layer (oracle.moe_forward reads each projection's bitrate from its trellis) with every
touched expert decoded by the C restatement, and against the single-class path where the classes share one K."""
import numpy as np
import pytest
import torch

from conftest import c_reconstruct
from oracle import exl3_oracle as orc
from test_gpu_moe import _errs
from test_gpu_moe_stages import _runs

pytestmark = pytest.mark.gpu

E, H, I, TOP_K, CB = 128, 2048, 768, 8, 1


def _ops():
    from trellis_serve_amd import ops
    return ops


def _layer(seed, ks=(3, 4), split=96):
    """Global experts 0..E-1; a random `split` of them in class 0 (K = ks[0]), the rest in class 1 (K = ks[1])."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)
    members = [np.sort(perm[:split]), np.sort(perm[split:])]
    ex = [None] * E
    classes = []
    for c, mem in enumerate(members):
        K = ks[c]
        st = {}
        for proj, (kk, nn) in (("gate", (H, I)), ("up", (H, I)), ("down", (I, H))):
            st[f"{proj}_trellis"] = rng.integers(-32768, 32768, size=(len(mem), kk // 16, nn // 16, 16 * K),
                                                 dtype=np.int16)
            st[f"{proj}_suh"] = np.where(rng.random((len(mem), kk)) < 0.5, -1.0, 1.0).astype(np.float16)
            st[f"{proj}_svh"] = np.where(rng.random((len(mem), nn)) < 0.5, -1.0, 1.0).astype(np.float16)
        for li, g in enumerate(mem):
            ex[g] = {p: tuple(st[f"{p}_{part}"][li] for part in ("trellis", "suh", "svh"))
                     for p in ("gate", "up", "down")}
        emap = np.full(E, -1, dtype=np.int32)
        emap[mem] = np.arange(len(mem), dtype=np.int32)
        classes.append(({k: torch.from_numpy(v).cuda() for k, v in st.items()}, torch.from_numpy(emap).cuda()))
    return rng, ex, classes


def _routing(rng, T):
    logits = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32))
    wsel, ids = torch.topk(logits, TOP_K, dim=1)
    return ids.to(torch.int32).cuda(), torch.softmax(wsel, dim=1).cuda()


def _exact(coracle, ex, cache, x, ids, w, toks):
    for t in toks:
        for e in set(ids[t].tolist()):
            for p in ("gate", "up", "down"):
                if (e, p) not in cache:
                    tr = ex[e][p][0]
                    cache[(e, p)] = c_reconstruct(coracle, tr, tr.shape[-1] // 16, CB)
    return {t: orc.moe_forward(x[t:t + 1], ids[t:t + 1], w[t:t + 1], ex, None, CB, w_cache=cache)[0] for t in toks}


@pytest.fixture(scope="module")
def layer():
    return _layer(5100)


@pytest.mark.parametrize("T,toks", [(1, (0,)), (16, (0, 7, 15)), (256, (0, 101, 255))])
def test_mixed_classes_match_exact_layer(coracle, layer, T, toks):
    """The C4 shape with 96 experts at K = 3 and 32 at K = 4 (MCG): single token (slot mode), 16 and 256 tokens
    (routing launch, per-class expert launches), sampled tokens against the float64 exact layer."""
    rng, ex, classes = layer
    x = torch.from_numpy((np.random.default_rng(T).standard_normal((T, H)) * 0.05).astype(np.float16)).cuda()
    ids, w = _routing(np.random.default_rng(T + 1), T)
    y = _ops().moe_forward_classes(x, ids, w, classes, E, CB).cpu().numpy()
    ref = _exact(coracle, ex, {}, x.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy(), toks)
    for t in toks:
        nrel, mrel = _errs(y[t:t + 1], ref[t][None])
        assert nrel <= 2e-3 and mrel <= 2e-3, (T, t, nrel, mrel)
    assert torch.equal(_ops().moe_forward_classes(x, ids, w, classes, E, CB).cpu(), torch.from_numpy(y))


@pytest.mark.parametrize("T", [1, 24])
def test_two_classes_of_one_bitrate_equal_the_single_class_layer(T):
    """Both classes at K = 3: the per-class launches compute exactly what one launch over the global stack computes
    (same plan, same expert rows, same split order), so the outputs are bit-identical."""
    rng, ex, classes = _layer(5200 + T, ks=(3, 3), split=80)
    glob = {}
    for name in classes[0][0]:
        glob[name] = torch.from_numpy(np.stack([ex[e][name.split("_")[0]][("trellis", "suh", "svh").index(
            name.split("_")[1])] for e in range(E)])).cuda()
    x = torch.from_numpy((rng.standard_normal((T, H)) * 0.05).astype(np.float16)).cuda()
    ids, w = _routing(rng, T)
    y_cls = _ops().moe_forward_classes(x, ids, w, classes, E, CB)
    y_one = _ops().moe_forward(x, ids, w, glob, CB)
    assert torch.equal(y_cls, y_one)


def test_align_classes_matches_per_class_contract(layer):
    """One launch, two classes: each class's (sorted_ids, expert_ids, num_post_padded) is moe_align_block_size's
    layout for that class's slots only, with local expert ids (oracle restatement of the contract)."""
    rng, ex, classes = layer
    ids, _ = _routing(np.random.default_rng(77), 40)
    maps = [c[1] for c in classes]
    blocks = [16, 32]
    got = _ops().moe_align_classes(ids, E, maps, blocks)
    ids_np = ids.cpu().numpy()
    for (s, e, p), emap, block in zip(got, maps, blocks):
        emap = emap.cpu().numpy()
        kept = np.where(emap[ids_np] >= 0, ids_np, -1)
        ws, we, wp = orc.moe_align(kept, block, E)
        s, e, p = s.cpu().numpy(), e.cpu().numpy(), int(p.item())
        assert p == wp
        np.testing.assert_array_equal(e[:p // block], emap[we])
        assert (e[p // block:] == -1).all() and (s[p:] == ids_np.size).all()
        got_runs, want_runs = _runs(s, e, p, block), _runs(ws, emap[we], wp, block)
        assert got_runs.keys() == want_runs.keys()
        for le, run in want_runs.items():
            n = sum(1 for v in run if v != ids_np.size)
            assert sorted(got_runs[le][:n]) == sorted(run[:n]), le   # the expert's slots, any order
            assert all(v == ids_np.size for v in got_runs[le][n:]), le


def test_mixed_stage_chain_matches_exact_layer(coracle, layer):
    """The reference's run_mixed with the per-launch stages: one two-class align, the input rotation with the union
    suh stacks in global order, each class's grouped GEMM (gate | up, then down) into the shared slabs, one GLU, one
    combine."""
    rng, ex, classes = layer
    T = 12
    ops = _ops()
    x = torch.from_numpy((np.random.default_rng(12).standard_normal((T, H)) * 0.05).astype(np.float16)).cuda()
    ids, w = _routing(np.random.default_rng(13), T)
    suh = {p: torch.from_numpy(np.stack([ex[e][p][1] for e in range(E)])).cuda() for p in ("gate", "up", "down")}
    blocks = [16, 16]
    routes = ops.moe_align_classes(ids, E, [c[1] for c in classes], blocks)
    xh = ops.moe_had_in(x, [suh["gate"], suh["up"]], ids)
    slots = T * TOP_K
    gu = torch.empty((slots, 2 * I), dtype=torch.float16, device="cuda")
    for (st, _), (s, e, p), b in zip(classes, routes, blocks):
        ops.moe_gemm(xh, [st["gate_trellis"], st["up_trellis"]], [st["gate_svh"], st["up_svh"]], s, e, p, b, CB,
                     out=gu)
    _, xd = ops.moe_glu_had_in(gu, suh["down"], ids)
    yd = torch.empty((slots, H), dtype=torch.float16, device="cuda")
    for (st, _), (s, e, p), b in zip(classes, routes, blocks):
        ops.moe_gemm(xd, [st["down_trellis"]], [st["down_svh"]], s, e, p, b, CB, out=yd)
    y = ops.moe_combine(yd, w, ids, E).cpu().numpy()
    toks = (0, 5, 11)
    ref = _exact(coracle, ex, {}, x.cpu().numpy(), ids.cpu().numpy(), w.cpu().numpy(), toks)
    for t in toks:
        nrel, mrel = _errs(y[t:t + 1], ref[t][None])
        assert nrel <= 2e-3 and mrel <= 2e-3, (t, nrel, mrel)
    fused = ops.moe_forward_classes(x, ids, w, classes, E, CB).cpu().numpy().astype(np.float64)
    assert np.abs(y - fused).max() <= 2e-3 * np.abs(fused).max()
