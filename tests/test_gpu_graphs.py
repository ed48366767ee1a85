"""HIP-graph capture of every op after its workspace was reserved: the serving path of an engine that reserves at load
and captures decode graphs (the reference reserves its scratch at load, cuda/src/sglang_exl3/kernels/marlin.py:24-33,
and its engines capture the decode step).  Each test captures a small call, then alternates eager calls of other
shapes (larger ones included) with replays on new inputs, and checks every replay bit for bit against an eager call
on the same inputs; the reserved workspace must keep its address throughout, and a capture that needs more than
was reserved must raise instead of allocating."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ops():
    from trellis_serve_amd import ops
    return ops


@pytest.fixture(autouse=True)
def fresh_workspaces():
    _ops().release_workspaces()
    yield
    torch.cuda.synchronize()
    _ops().release_workspaces()


def _capture(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def _group(g, k, ns, K):
    trs = [torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16, generator=g).cuda() for n in ns]
    suhs = [(torch.randint(0, 2, (k,), generator=g) * 2 - 1).half().cuda() for _ in ns]
    svhs = [(torch.randint(0, 2, (n,), generator=g) * 2 - 1).half().cuda() for n in ns]
    return trs, suhs, svhs


def _ws_ptr(kind):
    return _ops().workspace(torch.device("cuda"), 0, kind).data_ptr()


@pytest.mark.parametrize("M", [1, 4, 24, 48])   # one row group; two; four (a narrow layer)
def test_linear_graph_after_reservation(M):
    ops = _ops()
    g = torch.Generator().manual_seed(31 + M)
    k, ns, K, cb = 2048, [1024, 512, 512], 3, 1
    trs, suhs, svhs = _group(g, k, ns, K)
    ops.reserve_linear(torch.device("cuda"), max(16, M), k, sum(ns), K)
    ptr = _ws_ptr("linear")
    x = torch.randn((M, k), generator=g).half().cuda()
    out = torch.empty((M, sum(ns)), dtype=torch.float16, device="cuda")
    graph = _capture(lambda: ops.linear(x, trs, suhs, svhs, cb, out=out))
    for i in range(4):
        other = torch.randn((16 if i % 2 else 7, k), generator=g).half().cuda()
        ops.linear(other, trs, suhs, svhs, cb)                       # eager, other shapes, same workspace
        ops.linear(torch.randn((80, k), generator=g).half().cuda(), trs, suhs, svhs, cb)   # beyond the reservation
        x.copy_(torch.randn((M, k), generator=g).half().cuda())
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ops.linear(x, trs, suhs, svhs, cb)), i
    assert _ws_ptr("linear") == ptr


def test_prefill_graph_after_reservation():
    ops = _ops()
    g = torch.Generator().manual_seed(41)
    k, ns, K, cb = 2048, [1280, 768], 4, 2
    trs, suhs, svhs = _group(g, k, ns, K)
    ops.reserve_prefill(torch.device("cuda"), 512, k, sum(ns), len(ns))
    ptr = _ws_ptr("prefill")
    x = torch.randn((200, k), generator=g).half().cuda()
    out = torch.empty((200, sum(ns)), dtype=torch.float16, device="cuda")
    graph = _capture(lambda: ops.linear_prefill(x, trs, suhs, svhs, cb, out=out))
    for i in range(3):
        ops.linear_prefill(torch.randn((512 if i else 130, k), generator=g).half().cuda(), trs, suhs, svhs, cb)
        x.copy_(torch.randn((200, k), generator=g).half().cuda())
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ops.linear_prefill(x, trs, suhs, svhs, cb)), i
    assert _ws_ptr("prefill") == ptr


def test_moe_graph_after_reservation():
    ops = _ops()
    g = torch.Generator().manual_seed(51)
    E, H, I, K, K_dn, top_k = 16, 512, 256, 3, 4, 4
    experts = {}
    for proj, (k, n, bits) in {"gate": (H, I, K), "up": (H, I, K), "down": (I, H, K_dn)}.items():
        experts[f"{proj}_trellis"] = torch.randint(-32768, 32768, (E, k // 16, n // 16, 16 * bits), dtype=torch.int16,
                                                   generator=g).cuda()
        experts[f"{proj}_suh"] = (torch.randint(0, 2, (E, k), generator=g) * 2 - 1).half().cuda()
        experts[f"{proj}_svh"] = (torch.randint(0, 2, (E, n), generator=g) * 2 - 1).half().cuda()

    def routing(T):
        ids = torch.stack([torch.randperm(E, generator=g)[:top_k] for _ in range(T)]).to(torch.int32).cuda()
        w = torch.softmax(torch.randn((T, top_k), generator=g), -1).cuda()
        return ids, w

    ops.reserve_moe(torch.device("cuda"), 64, top_k, E, H, I, K, K_dn)
    ptr = _ws_ptr("moe")
    T = 2
    x = torch.randn((T, H), generator=g).half().cuda()
    ids, w = routing(T)
    out = torch.empty((T, H), dtype=torch.float16, device="cuda")
    graph = _capture(lambda: ops.moe_forward(x, ids, w, experts, 1, out=out))
    for i in range(3):
        ops.moe_forward(torch.randn((64, H), generator=g).half().cuda(), *routing(64), experts, 1)
        x.copy_(torch.randn((T, H), generator=g).half().cuda())
        new_ids, new_w = routing(T)
        ids.copy_(new_ids)
        w.copy_(new_w)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ops.moe_forward(x, ids, w, experts, 1)), i
    assert _ws_ptr("moe") == ptr


@pytest.mark.parametrize("max_pages", [64, 4])   # 8 chunks and a merge launch / one chunk, no merge launch
def test_kv_graph_after_reservation(max_pages):
    ops = _ops()
    g = torch.Generator().manual_seed(61 + max_pages)
    B, Hq, Hkv, D = 4, 16, 4, 128
    P = B * max_pages
    kc = torch.randint(-128, 128, (P, Hkv, 16, D), dtype=torch.int8, generator=g).cuda()
    vc = torch.randint(-128, 128, (P, Hkv, 16, D), dtype=torch.int8, generator=g).cuda()
    ks = (torch.rand((P, Hkv), generator=g) * 0.02 + 0.01).half().cuda()
    vs = (torch.rand((P, Hkv), generator=g) * 0.02 + 0.01).half().cuda()
    table = torch.randperm(P, generator=g).to(torch.int32).view(B, max_pages).cuda()
    lens = torch.tensor([1000, 17, 512, 1], dtype=torch.int32).cuda()
    ops.reserve_kv(torch.device("cuda"), B, Hq, Hkv, max_pages)
    ptr = _ws_ptr("kv")
    q = torch.randn((B, Hq, D), generator=g).half().cuda()
    out = torch.empty((B, Hq, D), dtype=torch.float16, device="cuda")
    graph = _capture(lambda: ops.kv_decode_attention(q, kc, vc, ks, vs, table, lens, 8, out=out))
    for i in range(3):
        ops.kv_decode_attention(torch.randn((2, Hq, D), generator=g).half().cuda(), kc, vc, ks, vs, table[:2],
                                lens[:2], 8)
        q.copy_(torch.randn((B, Hq, D), generator=g).half().cuda())
        lens.copy_(torch.randint(1, 16 * max_pages + 1, (B,), generator=g).to(torch.int32).cuda())
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ops.kv_decode_attention(q, kc, vc, ks, vs, table, lens, 8)), i
    assert _ws_ptr("kv") == ptr


def test_capture_beyond_the_reservation_raises():
    ops = _ops()
    g = torch.Generator().manual_seed(71)
    k, ns, K = 1024, [512], 3
    trs, suhs, svhs = _group(g, k, ns, K)
    ops.reserve_linear(torch.device("cuda"), 1, k, sum(ns), K)
    x = torch.randn((16, k), generator=g).half().cuda()
    need = __import__("trellis_serve_amd._lib", fromlist=["load"]).load().exl3_linear_workspace_bytes(16, k, 512, K)
    if need <= ops.workspace(torch.device("cuda"), 0, "linear").numel():
        pytest.skip("the 16-row plan fits the 1-row reservation on this device")
    ops.linear(x, trs, suhs, svhs, 1)   # warm-up outside capture (a one-off buffer)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(ops.WorkspaceTooSmall):
        with torch.cuda.graph(graph):
            ops.linear(x, trs, suhs, svhs, 1)
