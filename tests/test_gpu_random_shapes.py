"""Seeded random shapes through the fused linear (GEMV rows 1..16) and the prefill decode-GEMM (17..600 rows): k and
per-shard n of 128..5120 and 1..4 shards, every bit width and codebook, fp16 or bf16 input.  The split plans, shard
maps, tail tiles and half tiles take forms here that the fixed shapes of the other tests do not.  The reference is
built on the GPU from pieces pinned elsewhere -- the bit-exact reconstruct (W_inner), the input rotation of every
shard and an fp32 matmul, then the output rotation -- and the fused result must agree within the north-star
tolerance (norm-relative and max-relative 2e-3).  Outputs are fp16 (a bf16 input still gives an fp16 output)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _cases(seed, count, rows_lo, rows_hi, k_hi, n_hi):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        K = int(rng.choice([2, 3, 4, 5, 6, 8]))
        cb = int(rng.integers(0, 3))
        k = 128 * int(rng.integers(1, k_hi // 128 + 1))
        shards = int(rng.integers(1, 5))
        ns = [128 * int(rng.integers(1, n_hi // 128 + 1)) for _ in range(shards)]
        M = int(rng.integers(rows_lo, rows_hi + 1))
        bf = bool(rng.random() < 0.3)
        out.append((K, cb, k, tuple(ns), M, bf))
    return out


GEMV_CASES = _cases(2026, 24, 1, 16, 5120, 3072)
PREFILL_CASES = _cases(2027, 10, 17, 600, 2048, 2048)


def _ids(cases):
    return [f"K{K}-cb{cb}-k{k}-n{'+'.join(map(str, ns))}-M{M}{'-bf16' if bf else ''}" for K, cb, k, ns, M, bf in cases]


def _run(case, prefill):
    from trellis_serve_amd import ops
    K, cb, k, ns, M, bf = case
    g = torch.Generator(device="cpu").manual_seed(hash(case) & 0xFFFFFFFF)
    trs = [torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16, generator=g).cuda() for n in ns]
    suhs = [(torch.randint(0, 2, (k,), generator=g) * 2 - 1).half().cuda() for _ in ns]
    svhs = [(torch.randint(0, 2, (n,), generator=g) * 2 - 1).half().cuda() for n in ns]
    x = (torch.randn((M, k), generator=g) * 0.5).cuda()
    x = x.bfloat16() if bf else x.half()
    out = torch.empty((M, sum(ns)), dtype=torch.float16, device="cuda")
    fn = ops.linear_prefill if prefill else ops.linear
    y = fn(x, trs, suhs, svhs, cb, out=out).float()
    ref = torch.empty((M, sum(ns)), dtype=torch.float16, device="cuda")
    col = 0
    for tr, suh, svh in zip(trs, suhs, svhs):
        xh = ops.had_in_group(x, suh)
        w = ops.reconstruct(tr, cb)
        ops.had_out_into((xh.float() @ w.float()).half(), svh, ref, col)
        col += w.shape[1]
    ref = ref.float()
    nrel = ((y - ref).norm() / ref.norm()).item()
    mrel = ((y - ref).abs().max() / ref.abs().max()).item()
    assert nrel <= TOL and mrel <= TOL, (case, nrel, mrel)


@pytest.mark.parametrize("case", GEMV_CASES, ids=_ids(GEMV_CASES))
def test_random_gemv_shapes(case):
    _run(case, prefill=False)


@pytest.mark.parametrize("case", PREFILL_CASES, ids=_ids(PREFILL_CASES))
def test_random_prefill_shapes(case):
    _run(case, prefill=True)
