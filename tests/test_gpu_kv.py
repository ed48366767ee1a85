"""GPU parity of the quantized-KV paged decode attention (exl3_kv_decode_attention) against the oracle's float64
closed form (oracle.kv_decode_attention: dequantize code * scale, softmax attention per query head).

The reference has no quantized-KV decode kernel (its nearest relative is the paged fp8 attention with log-sum-exp merge
of xpu/exl3xpu/fp8kv_prefill.py:73-117), so this path is "parity unpinned" against the reference itself; the oracle
is pinned by tests/test_oracle.py against a contiguous-cache evaluation.  Bar: norm-rel and max-rel (max abs error over
max |ref|) <= 2e-3 -- the kernel's own roundings are the fp16 probabilities (p * v_scale) and the fp16 output."""
import numpy as np
import pytest
import torch

from oracle import exl3_oracle as orc

pytestmark = pytest.mark.gpu

D, PAGE = 128, 16


def _cache(rng, num_pages, Hkv, bits):
    kf = rng.standard_normal((num_pages, Hkv, PAGE, D)).astype(np.float16)
    vf = rng.standard_normal((num_pages, Hkv, PAGE, D)).astype(np.float16)
    kq, ks = orc.kv_quantize(kf, bits)
    vq, vs = orc.kv_quantize(vf, bits)
    if bits == 4:
        return orc.kv_pack4(kq), orc.kv_pack4(vq), ks, vs
    return kq, vq, ks, vs


def _table(rng, lens, max_pages, num_pages):
    """Each sequence gets distinct physical pages in a random order; unused entries hold -1 (never read)."""
    perm = rng.permutation(num_pages)
    table = np.full((len(lens), max_pages), -1, dtype=np.int32)
    off = 0
    for b, L in enumerate(lens):
        n = -(-L // PAGE)
        table[b, :n] = perm[off:off + n]
        off += n
    assert off <= num_pages
    return table


def _run(q, kc, vc, ks, vs, table, lens, bits, sm_scale):
    from trellis_serve_amd import ops
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return ops.kv_decode_attention(t(q), t(kc), t(vc), t(ks), t(vs), t(table), t(np.asarray(lens, np.int32)), bits,
                                   sm_scale)


def _errs(y, ref):
    y = y.astype(np.float64)
    return np.linalg.norm(y - ref) / np.linalg.norm(ref), np.abs(y - ref).max() / np.abs(ref).max()


def _case(seed, lens, Hq, Hkv, bits, max_pages=None, extra_pages=3):
    rng = np.random.default_rng(seed)
    npg = sum(-(-L // PAGE) for L in lens)
    num_pages = npg + extra_pages
    max_pages = max_pages or max(1, max(-(-L // PAGE) for L in lens))
    kc, vc, ks, vs = _cache(rng, num_pages, Hkv, bits)
    table = _table(rng, lens, max_pages, num_pages)
    q = rng.standard_normal((len(lens), Hq, D)).astype(np.float16)
    return q, kc, vc, ks, vs, table


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("lens,Hq,Hkv", [([1, 17, 300], 40, 8), ([16, 33, 1000, 64], 8, 8), ([255, 4], 32, 2),
                                         ([2049], 40, 8), ([1, 40, 64], 40, 8)])   # the last: one chunk, no merge
def test_kv_decode_matches_closed_form(bits, lens, Hq, Hkv):
    q, kc, vc, ks, vs, table = _case(7 + len(lens) + bits, lens, Hq, Hkv, bits)
    sm = D ** -0.5
    y = _run(q, kc, vc, ks, vs, table, lens, bits, sm).cpu().numpy()
    ref = orc.kv_decode_attention(q, kc, vc, ks, vs, table, np.asarray(lens, np.int32), bits, sm)
    nrel, mrel = _errs(y, ref)
    print(f"bits={bits} lens={lens} heads {Hq}/{Hkv}: norm-rel {nrel:.2e} max-rel {mrel:.2e}")
    assert nrel <= 2e-3 and mrel <= 2e-3, (nrel, mrel)


@pytest.mark.parametrize("bits", [8, 4])
def test_kv_decode_c5_4k_batch16(bits):
    """The measured configuration at 4k context: B = 16, 40 / 8 heads, random page order."""
    lens = [4096] * 15 + [4000]
    q, kc, vc, ks, vs, table = _case(40 + bits, lens, 40, 8, bits, extra_pages=0)
    sm = D ** -0.5
    y = _run(q, kc, vc, ks, vs, table, lens, bits, sm).cpu().numpy()
    ref = orc.kv_decode_attention(q, kc, vc, ks, vs, table, np.asarray(lens, np.int32), bits, sm)
    nrel, mrel = _errs(y, ref)
    print(f"C5 4k bits={bits}: norm-rel {nrel:.2e} max-rel {mrel:.2e}")
    assert nrel <= 2e-3 and mrel <= 2e-3, (nrel, mrel)


def test_kv_decode_32k():
    lens = [32768, 32768 - 5]
    q, kc, vc, ks, vs, table = _case(32, lens, 40, 8, 8, extra_pages=0)
    # a sharp query: logits of a few keys dominate (the running max moves across chunks)
    q = (q.astype(np.float32) * 4).astype(np.float16)
    sm = D ** -0.5
    y = _run(q, kc, vc, ks, vs, table, lens, 8, sm).cpu().numpy()
    ref = orc.kv_decode_attention(q, kc, vc, ks, vs, table, np.asarray(lens, np.int32), 8, sm)
    nrel, mrel = _errs(y, ref)
    print(f"32k: norm-rel {nrel:.2e} max-rel {mrel:.2e}")
    assert nrel <= 2e-3 and mrel <= 2e-3, (nrel, mrel)


def test_kv_decode_c5_32k_4bit_batch16():
    """The measured configuration at 32k context and 4-bit codes: B = 16, 40 / 8 heads, random page order."""
    rng = np.random.default_rng(324)
    lens = [32768] * 15 + [32768 - 9]
    P = 16 * 2048
    # random packed codes and scales straight away (quantizing 5e8 normal values on the host would take minutes)
    kc, vc = (rng.integers(0, 256, size=(P, 8, PAGE, D // 2), dtype=np.uint8) for _ in range(2))
    ks, vs = ((rng.random((P, 8)) * 0.02 + 0.01).astype(np.float16) for _ in range(2))
    table = _table(rng, lens, 2048, P)
    q = rng.standard_normal((16, 40, D)).astype(np.float16)
    sm = D ** -0.5
    y = _run(q, kc, vc, ks, vs, table, lens, 4, sm).cpu().numpy()
    ref = orc.kv_decode_attention(q, kc, vc, ks, vs, table, np.asarray(lens, np.int32), 4, sm)
    nrel, mrel = _errs(y, ref)
    print(f"C5 32k 4-bit B=16: norm-rel {nrel:.2e} max-rel {mrel:.2e}")
    assert nrel <= 2e-3 and mrel <= 2e-3, (nrel, mrel)


def test_kv_decode_c5_32k_8bit_batch16():
    """The measured configuration at 32k context and 8-bit codes: B = 16, 40 / 8 heads, random page order."""
    rng = np.random.default_rng(328)
    lens = [32768] * 15 + [32768 - 3]
    P = 16 * 2048
    kc, vc = (rng.integers(-128, 128, size=(P, 8, PAGE, D), dtype=np.int8) for _ in range(2))
    ks, vs = ((rng.random((P, 8)) * 0.01 + 0.004).astype(np.float16) for _ in range(2))
    table = _table(rng, lens, 2048, P)
    q = rng.standard_normal((16, 40, D)).astype(np.float16)
    sm = D ** -0.5
    y = _run(q, kc, vc, ks, vs, table, lens, 8, sm).cpu().numpy()
    ref = orc.kv_decode_attention(q, kc, vc, ks, vs, table, np.asarray(lens, np.int32), 8, sm)
    nrel, mrel = _errs(y, ref)
    print(f"C5 32k 8-bit B=16: norm-rel {nrel:.2e} max-rel {mrel:.2e}")
    assert nrel <= 2e-3 and mrel <= 2e-3, (nrel, mrel)


@pytest.mark.parametrize("bits", [8, 4])
def test_kv_decode_uniform_keys_give_mean_of_values(bits):
    """All-zero K codes: every logit is 0, so each head's output is the plain mean of its V rows (closed form)."""
    lens = [50, 16, 1]
    q, kc, vc, ks, vs, table = _case(5, lens, 16, 4, bits)
    kc[:] = 0
    y = _run(q, kc, vc, ks, vs, table, lens, bits, 0.1).cpu().numpy().astype(np.float64)
    vcodes = orc.kv_unpack4(vc) if bits == 4 else vc
    for b, L in enumerate(lens):
        pages = table[b, :-(-L // PAGE)]
        vals = (vcodes[pages].astype(np.float32) * vs[pages].astype(np.float32)[:, :, None, None])  # [n, Hkv, 16, D]
        vals = vals.transpose(1, 0, 2, 3).reshape(4, -1, D)[:, :L].astype(np.float64)
        mean = vals.mean(axis=1)
        for h in range(16):
            np.testing.assert_allclose(y[b, h], mean[h // 4], rtol=2e-3, atol=2e-3 * np.abs(mean).max())


def test_kv_decode_page_order_and_padding_invariance():
    """Moving a sequence's pages to other physical slots, and widening the page table, changes nothing (bit-exact);
    a zero-length sequence gives zeros; repeated calls are bit-identical."""
    lens = [700, 0, 129]
    q, kc, vc, ks, vs, table = _case(11, lens, 40, 8, 8, max_pages=44, extra_pages=60)
    first = _run(q, kc, vc, ks, vs, table, lens, 8, 0.08)
    rng = np.random.default_rng(3)
    P = kc.shape[0]
    perm = rng.permutation(P)          # physical page p moves to slot perm[p]
    kc2, vc2, ks2, vs2 = (np.empty_like(a) for a in (kc, vc, ks, vs))
    for a2, a in ((kc2, kc), (vc2, vc), (ks2, ks), (vs2, vs)):
        a2[perm] = a
    table2 = np.where(table >= 0, perm[np.maximum(table, 0)], -1).astype(np.int32)
    table2 = np.concatenate([table2, np.full((3, 20), -1, np.int32)], axis=1)
    second = _run(q, kc2, vc2, ks2, vs2, table2, lens, 8, 0.08)
    assert torch.equal(first[0], second[0]) and torch.equal(first[2], second[2])
    assert not first[1].any() and not second[1].any()
    for _ in range(3):
        assert torch.equal(_run(q, kc, vc, ks, vs, table, lens, 8, 0.08), first)


def test_kv_decode_shapes_on_one_workspace_and_repeatable():
    """Calls of different batch / head / length shapes on one workspace, each against the closed form, a
    zero-length sequence in the batch (its rows are zero), and repeated calls bit-identical."""
    from trellis_serve_amd import ops
    ops.release_workspaces()
    sm = D ** -0.5
    for seed, lens, Hq, Hkv, bits in ((81, [4096, 0, 700], 40, 8, 8), (82, [33], 8, 2, 4), (83, [1500, 2049], 16, 4, 8)):
        q, kc, vc, ks, vs, table = _case(seed, lens, Hq, Hkv, bits)
        first = _run(q, kc, vc, ks, vs, table, lens, bits, sm)
        live = [b for b, L in enumerate(lens) if L > 0]
        ref = orc.kv_decode_attention(q[live], kc, vc, ks, vs, table[live], np.asarray(lens, np.int32)[live], bits, sm)
        y = first.cpu().numpy()
        nrel, mrel = _errs(y[live], ref)
        assert nrel <= 2e-3 and mrel <= 2e-3, (lens, nrel, mrel)
        assert all((y[b] == 0).all() for b, L in enumerate(lens) if L == 0)
        for _ in range(3):
            assert torch.equal(_run(q, kc, vc, ks, vs, table, lens, bits, sm), first)


def _kv_cases(seed, count):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        Hkv = int(rng.choice([1, 2, 4, 8]))
        G = int(rng.integers(1, 17))
        B = int(rng.integers(1, 9))
        lens = tuple(int(v) for v in rng.integers(1, 3000, size=B))
        out.append((lens, G * Hkv, Hkv, int(rng.choice([4, 8])), int(rng.integers(0, 3))))
    return out


KV_CASES = _kv_cases(2029, 12)


@pytest.mark.parametrize("case", KV_CASES, ids=[f"B{len(c[0])}-L{max(c[0])}-q{c[1]}-kv{c[2]}-b{c[3]}" for c in KV_CASES])
def test_kv_decode_random_shapes(case):
    """Seeded random batches: 1-8 sequences of 1 … 2999 tokens, 1 / 2 / 4 / 8 KV heads with GQA groups of 1-16, 4 or
    8 bits, 0-2 spare table columns, against the float64 closed form."""
    lens, Hq, Hkv, bits, spare = case
    max_pages = max(-(-L // PAGE) for L in lens) + spare
    q, kc, vc, ks, vs, table = _case(abs(hash(case)) % (1 << 32), list(lens), Hq, Hkv, bits, max_pages=max_pages)
    sm = D ** -0.5
    y = _run(q, kc, vc, ks, vs, table, lens, bits, sm).cpu().numpy()
    ref = orc.kv_decode_attention(q, kc, vc, ks, vs, table, np.asarray(lens, np.int32), bits, sm)
    nrel, mrel = _errs(y, ref)
    assert nrel <= 2e-3 and mrel <= 2e-3, (case, nrel, mrel)
