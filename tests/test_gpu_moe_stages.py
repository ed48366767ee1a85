"""GPU parity of the MoE per-launch stages (exl3_moe_align / _had_in / _gemm / _glu_had_in / _combine), the launches of
the reference's unfused path (cuda/csrc/exl3_marlin_moe.cu:376-618, run order cuda/src/sglang_exl3/kernels/
marlin_moe.py:272-294).  The align layout is checked against the moe_align_block_size contract the oracle restates;
the grouped GEMM reads rows back bit for bit through one-hot inputs (the method of
cuda/src/sglang_exl3/tools/moe_parity_sm86.py:158-229: each output row is then one decoded weight row of the routed
expert); the chained stages against the float64 exact layer and against exl3_moe_forward."""
import numpy as np
import pytest
import torch

from conftest import c_reconstruct
from oracle import exl3_oracle as orc
from test_gpu_moe import _experts, _stack

pytestmark = pytest.mark.gpu


def _ops():
    from trellis_serve_amd import ops
    return ops


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _topk(rng, T, E, top_k, invalid=0):
    ids = np.stack([rng.choice(E, top_k, replace=False) for _ in range(T)]).astype(np.int32)
    for _ in range(invalid):
        ids[rng.integers(T), rng.integers(top_k)] = rng.choice([-1, E])
    return ids


def _runs(sorted_ids, expert_ids, post, block):
    """expert -> the slot run of that expert (in stored order) and its padded length."""
    out = {}
    for b in range(post // block):
        out.setdefault(int(expert_ids[b]), []).extend(sorted_ids[b * block:(b + 1) * block].tolist())
    return out


@pytest.mark.parametrize("T,E,top_k,block", [(1, 8, 2, 16), (7, 128, 8, 16), (300, 64, 4, 64), (33, 16, 8, 8),
                                             (5, 1000, 8, 32)])
def test_align_matches_the_moe_align_contract(T, E, top_k, block):
    rng = np.random.default_rng(T + E + block)
    ids = _topk(rng, T, E, top_k, invalid=min(3, T))
    sorted_ids, expert_ids, post = _ops().moe_align(_dev(ids), E, block)
    s, e, p = sorted_ids.cpu().numpy(), expert_ids.cpu().numpy(), int(post.item())
    ws, we, wp = orc.moe_align(ids, block, E)
    assert p == wp
    np.testing.assert_array_equal(e[:p // block], we)
    assert (e[p // block:] == -1).all() and (s[p:] == ids.size).all()
    got, want = _runs(s, e, p, block), _runs(ws, we, wp, block)
    assert got.keys() == want.keys()
    for ex, run in want.items():
        n = sum(1 for v in run if v != ids.size)
        assert sorted(got[ex][:n]) == run[:n], ex          # the expert's slots, any order
        assert all(v == ids.size for v in got[ex][n:]), ex  # then the padding sentinels


def test_align_with_an_expert_map():
    """Expert parallelism's local ids: even experts map to e / 2, odd ones are not served here (-1) and drop out."""
    rng = np.random.default_rng(3)
    E, block = 32, 16
    ids = _topk(rng, 40, E, 4)
    emap = np.array([e // 2 if e % 2 == 0 else -1 for e in range(E)], dtype=np.int32)
    sorted_ids, expert_ids, post = _ops().moe_align(_dev(ids), E, block, expert_map=_dev(emap))
    s, e, p = sorted_ids.cpu().numpy(), expert_ids.cpu().numpy(), int(post.item())
    kept = np.where(emap[np.clip(ids, 0, E - 1)] >= 0, ids, -1)
    ws, we, wp = orc.moe_align(kept, block, E)
    assert p == wp
    np.testing.assert_array_equal(e[:p // block], emap[we])
    got, want = _runs(s, e, p, block), _runs(ws, emap[we], wp, block)
    for ex, run in want.items():
        n = sum(1 for v in run if v != ids.size)
        assert sorted(got[ex][:n]) == run[:n]


@pytest.mark.parametrize("x_dtype", [torch.float16, torch.bfloat16])
def test_had_in_matches_fp16_oracle(x_dtype):
    rng = np.random.default_rng(11)
    T, k, E, top_k = 6, 512, 8, 3
    ids = _topk(rng, T, E, top_k, invalid=2)
    x = torch.from_numpy(rng.standard_normal((T, k)).astype(np.float32) * 2).to(x_dtype).cuda()
    suh = [np.where(rng.random((E, k)) < 0.5, -1.0, 1.0).astype(np.float16) for _ in range(2)]
    xh = _ops().moe_had_in(x, [_dev(s) for s in suh], _dev(ids)).cpu().numpy()
    xf = x.float().cpu().numpy().astype(np.float16)   # the kernel's fp16 input (bf16 widened exactly, then rounded)
    for sh in range(2):
        for slot in range(T * top_k):
            e = ids.reshape(-1)[slot]
            if not 0 <= e < E:
                continue
            want = orc.had_in_fp16(xf[slot // top_k:slot // top_k + 1], suh[sh][e])[0]
            got = xh[sh * T * top_k + slot]
            ulp = np.abs(got.view(np.int16).astype(np.int32) - want.view(np.int16).astype(np.int32))
            assert ulp.max() <= 1, (sh, slot)


@pytest.mark.parametrize("K,cb", [(2, 0), (3, 1), (4, 2), (6, 1)])
@pytest.mark.parametrize("block", [16, 64])
def test_gemm_one_hot_readout_is_bit_exact(coracle, K, cb, block):
    """No output transform, one-hot rows: row r of c is the decoded weight row kidx(r) of the expert the align blocks
    route it to, bit for bit, for gate and up side by side (two shards)."""
    rng = np.random.default_rng(100 * K + cb + block)
    E, k, n, T, top_k = 6, 256, 384, 9, 2
    stacks = [rng.integers(-32768, 32768, size=(E, k // 16, n // 16, 16 * K), dtype=np.int16) for _ in range(2)]
    ids = _topk(rng, T, E, top_k, invalid=1)
    slots = T * top_k
    kidx = rng.integers(0, k, size=(2, slots))
    a = np.zeros((2 * slots, k), dtype=np.float16)
    for sh in range(2):
        a[sh * slots + np.arange(slots), kidx[sh]] = 1.0
    ops = _ops()
    sorted_ids, expert_ids, post = ops.moe_align(_dev(ids), E, block)
    c = ops.moe_gemm(_dev(a), [_dev(s) for s in stacks], None, sorted_ids, expert_ids, post, block, cb)
    c = c.cpu().numpy()
    w = {(sh, e): c_reconstruct(coracle, stacks[sh][e], K, cb) for sh in range(2) for e in range(E)}
    for slot in range(slots):
        e = ids.reshape(-1)[slot]
        if not 0 <= e < E:
            continue
        for sh in range(2):
            np.testing.assert_array_equal(c[slot, sh * n:(sh + 1) * n].view(np.uint16),
                                          w[(sh, e)][kidx[sh, slot]].view(np.uint16))


@pytest.mark.parametrize("T,cb,K_down,block", [(1, 1, 3, 16), (5, 0, 4, 16), (64, 2, 2, 32), (40, 1, 3, 64)])
def test_chained_stages_match_exact_layer_and_fused_forward(T, cb, K_down, block):
    """moe_align -> moe_had_in -> moe_gemm (gate | up, output transform) -> moe_glu_had_in -> moe_gemm (down) ->
    moe_combine, as the reference's run_tensors chains them, against the float64 exact layer and exl3_moe_forward."""
    rng = np.random.default_rng(700 + T + cb)
    E, H, I, K, top_k = 16, 256, 384, 3, 4
    ex = _experts(rng, E, H, I, K, K_down)
    d = _stack(ex)
    x = (rng.standard_normal((T, H)) * 0.5).astype(np.float16)
    ids = _topk(rng, T, E, top_k, invalid=1 if T > 1 else 0)
    logits = rng.standard_normal((T, top_k)).astype(np.float32)
    w = (np.exp(logits) / np.exp(logits).sum(1, keepdims=True)).astype(np.float32)
    ops = _ops()
    xt, it, wt = _dev(x), _dev(ids), _dev(w)
    sorted_ids, expert_ids, post = ops.moe_align(it, E, block)
    xh = ops.moe_had_in(xt, [d["gate_suh"], d["up_suh"]], it)
    gu = ops.moe_gemm(xh, [d["gate_trellis"], d["up_trellis"]], [d["gate_svh"], d["up_svh"]], sorted_ids, expert_ids,
                      post, block, cb)
    act, xd = ops.moe_glu_had_in(gu, d["down_suh"], it)
    yd = ops.moe_gemm(xd, [d["down_trellis"]], [d["down_svh"]], sorted_ids, expert_ids, post, block, cb)
    y = ops.moe_combine(yd, wt, it, E).cpu().numpy()
    ref = orc.moe_forward(x, ids, w, ex, None, cb)
    nrel = np.linalg.norm(y.astype(np.float64) - ref) / np.linalg.norm(ref)
    mrel = np.abs(y.astype(np.float64) - ref).max() / np.abs(ref).max()
    print(f"T={T} cb={cb} K_down={K_down} block={block}: norm-rel {nrel:.2e} max-rel {mrel:.2e}")
    assert nrel <= 2e-3 and mrel <= 2e-3, (nrel, mrel)
    fused = ops.moe_forward(xt, it, wt, d, cb).cpu().numpy().astype(np.float64)
    assert np.abs(y - fused).max() <= 2e-3 * np.abs(fused).max()
    # the GLU stage's own outputs: act = fp16(silu(g) * u) from the fp16 g|u rows
    valid = (ids.reshape(-1) >= 0) & (ids.reshape(-1) < E)   # unrouted slots hold no defined g|u rows
    guf = gu.float().cpu().numpy()[valid]
    g, u = guf[:, :I], guf[:, I:]
    want_act = (orc.silu32(g) * u).astype(np.float16)
    got_act = act.cpu().numpy()[valid].view(np.int16).astype(np.int32)
    assert np.abs(got_act - want_act.view(np.int16).astype(np.int32)).max() <= 1   # fp32 exp within an ulp


def test_combine_skips_unrouted_slots_and_rounds_once():
    rng = np.random.default_rng(21)
    T, top_k, H, E = 4, 3, 256, 8
    yd = rng.standard_normal((T * top_k, H)).astype(np.float16)
    w = rng.random((T, top_k)).astype(np.float32)
    ids = rng.integers(0, E, size=(T, top_k)).astype(np.int32)
    ids[1, 2], ids[3, 0] = -1, E
    y = _ops().moe_combine(_dev(yd), _dev(w), _dev(ids), E).cpu().numpy()
    use = (ids >= 0) & (ids < E)
    want = np.zeros((T, H), dtype=np.float32)
    for t in range(T):
        for j in range(top_k):
            if use[t, j]:
                want[t] = want[t] + w[t, j] * yd[t * top_k + j].astype(np.float32)
    np.testing.assert_allclose(y.astype(np.float32), want.astype(np.float16).astype(np.float32), rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("block", [1, 16])
def test_gemm_over_more_align_blocks_than_one_launch_counts(block):
    """Every (align block, column block) of a launch has its own split counter in the 256 KiB counter region (65536
    counters): 4096 slots in blocks of 1 over 32 column blocks need 131072, so the align blocks go out in two
    launches (block 16: 4500 slots, 337 blocks, one launch).  Rows against fp32 matmuls of each expert's decoded weights
    (no output transform), to the layer tolerance."""
    rng = np.random.default_rng(900 + block)
    E, k, n, K, cb = 8, 256, 4096, 2, 1
    slots = 4096 if block == 1 else 4500
    stack = torch.from_numpy(rng.integers(-32768, 32768, size=(E, k // 16, n // 16, 16 * K), dtype=np.int16)).cuda()
    ids = torch.from_numpy(rng.integers(0, E, size=(slots, 1)).astype(np.int32)).cuda()
    a = torch.from_numpy((rng.standard_normal((slots, k)) * 0.5).astype(np.float16)).cuda()
    ops = _ops()
    sorted_ids, expert_ids, post = ops.moe_align(ids, E, block)
    assert expert_ids.numel() * n // 128 > 65536 or block == 16
    c = ops.moe_gemm(a, [stack], None, sorted_ids, expert_ids, post, block, cb).float()
    ref = torch.empty_like(c)
    flat = ids.reshape(-1)
    for e in range(E):
        rows = (flat == e).nonzero().flatten()
        ref[rows] = (a[rows].float() @ ops.reconstruct(stack[e], cb).float()).half().float()
    d = (c - ref).norm() / ref.norm()
    assert d.item() <= 2e-3, d.item()
    assert ((c - ref).abs().max() / ref.abs().max()).item() <= 2e-3


def test_stage_chain_replays_from_a_graph_after_reservation():
    """The chained stages captured in one HIP graph after reserve_moe_stage (the library's workspaces do not grow in the
    capture; every buffer is the caller's), and every replay, with eager work and synchronizations between replays,
    equals the eager chain bit for bit."""
    rng = np.random.default_rng(950)
    E, H, I, K, top_k, T, block, cb = 16, 256, 384, 3, 4, 24, 16, 1
    d = _stack(_experts(rng, E, H, I, K))
    ops = _ops()
    x = _dev((rng.standard_normal((T, H)) * 0.5).astype(np.float16))
    it = _dev(_topk(rng, T, E, top_k))
    logits = rng.standard_normal((T, top_k)).astype(np.float32)
    wt = _dev((np.exp(logits) / np.exp(logits).sum(1, keepdims=True)).astype(np.float32))
    slots = T * top_k
    ops.reserve_moe_stage(x.device, slots, H, I, 2, E, block)
    ops.reserve_moe_stage(x.device, slots, I, H, 1, E, block)
    cap, max_blocks = ops.moe_align_capacity(slots, E, block)
    st = dict(sorted=torch.empty(cap, dtype=torch.int32, device="cuda"),
              eids=torch.empty(max_blocks, dtype=torch.int32, device="cuda"),
              post=torch.empty(1, dtype=torch.int32, device="cuda"),
              xh=torch.empty((2 * slots, H), dtype=torch.float16, device="cuda"),
              gu=torch.empty((slots, 2 * I), dtype=torch.float16, device="cuda"),
              act=torch.empty((slots, I), dtype=torch.float16, device="cuda"),
              xd=torch.empty((slots, I), dtype=torch.float16, device="cuda"),
              yd=torch.empty((slots, H), dtype=torch.float16, device="cuda"),
              y=torch.empty((T, H), dtype=torch.float16, device="cuda"))
    lib = ops._lib.load()

    def chain():
        ops._lib.check(lib.exl3_moe_align(it.data_ptr(), slots, E, None, block, st["sorted"].data_ptr(), cap,
                                          st["eids"].data_ptr(), max_blocks, st["post"].data_ptr(),
                                          ops._stream(x.device)), "moe_align")
        ops.moe_had_in(x, [d["gate_suh"], d["up_suh"]], it, out=st["xh"])
        ops.moe_gemm(st["xh"], [d["gate_trellis"], d["up_trellis"]], [d["gate_svh"], d["up_svh"]], st["sorted"],
                     st["eids"], st["post"], block, cb, out=st["gu"])
        ops.moe_glu_had_in(st["gu"], d["down_suh"], it, act=st["act"], out=st["xd"])
        ops.moe_gemm(st["xd"], [d["down_trellis"]], [d["down_svh"]], st["sorted"], st["eids"], st["post"], block, cb,
                     out=st["yd"])
        ops.moe_combine(st["yd"], wt, it, E, out=st["y"])

    chain()
    torch.cuda.synchronize()
    eager = st["y"].clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        chain()   # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        chain()
    for r in range(4):
        st["y"].zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(st["y"], eager), r
        chain()   # eager work between replays
        torch.cuda.synchronize()
