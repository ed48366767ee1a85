"""Benchmark of the EXL3 hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Workload: the dense 27B-class decoder layer set at K = 3 bpw, MCG codebook, seeded random
packed codes and +-1 sign vectors: q/k/v 5120 -> 6144+1024+1024 (one fused 3-shard group), o_proj 6144 -> 5120,
gate/up 5120 -> 17408+17408 (one fused 2-shard group), down 17408 -> 5120, fp16 activations N(0,1) at M = 1.
One step = the four fused linears (decode-GEMV + rotations) over one batch of M rows.  Inputs are resident in HBM
before timing starts; R rotating copies of the layer set (>= 512 MB, twice the 256 MB MALL) keep the weights cold.

Prints one JSON line: metric/value = algorithmic HBM GB/s of the layer set at M = 1 (trellis + sign vectors +
activations in/out: 128,174,080 B per step), plus the roofline of the dominant kernel (the fused
decode-GEMV), the CPU baseline (the oracle's decode + matmul on up to 16 host cores, on a bounded sample), the
M = 4 / 16 rates, and the other configs as reported fields: the single 4096 x 4096 linear of configs[0] (K = 4,
3INST, M = 1), the prefill decode-GEMM TFLOPS (configs[2], `decode_gemm_tflops_m2048` is the second half of the
metric), the MoE layer and the quantized-KV decode attention.  For scale: the warm (single copy) layer-set rate, the trellis-only
weight-stream rate, hipBLASLt's fp16 8192^3 GEMM, and the reference's prefill design (W decoded to HBM, then the vendor
GEMM) rebuilt on this box at configs[2] M = 2048.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
LAYERS = {  # name: (k, [n per shard])
    "qkv": (5120, [6144, 1024, 1024]),
    "o": (6144, [5120]),
    "gate_up": (5120, [17408, 17408]),
    "down": (17408, [5120]),
}
K_BITS, CODEBOOK = 3, 1  # 3 bpw, MCG
# trellis bytes of one step (the reference's weight-stream figure, xpu/bench/linear_budget.py:83-88)
TRELLIS_BYTES_PER_STEP = sum(k * sum(ns) * K_BITS // 8 for k, ns in LAYERS.values())


def alg_bytes(k: int, ns: list[int], M: int, K: int) -> int:
    """Trellis + suh per shard + svh + x in + y out (fp16): the algorithmic bytes of one fused linear."""
    n = sum(ns)
    return k * n * K // 8 + 2 * k * len(ns) + 2 * n + 2 * M * k + 2 * M * n


def make_layer_set(torch, rng_seed: int, device, names=None):
    g = torch.Generator(device="cpu").manual_seed(rng_seed)
    out = {}
    for name, (k, ns) in LAYERS.items():
        if names is not None and name not in names:
            continue
        trs, suhs, svhs = [], [], []
        for n in ns:
            t = torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K_BITS), dtype=torch.int16, generator=g)
            trs.append(t.to(device))
            suhs.append((torch.randint(0, 2, (k,), generator=g) * 2 - 1).half().to(device))
            svhs.append((torch.randint(0, 2, (n,), generator=g) * 2 - 1).half().to(device))
        out[name] = (trs, suhs, svhs)
    return out


def _capture(torch, fn):
    """HIP graph of fn() (the reference times its decode path by CUDA-graph replay, decode_microbench.py:27-41)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # first call outside capture: allocates outputs and workspace
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


# steps per graph: a serving engine replays one graph per decode step holding every layer (hundreds of launches), so
# the few microseconds between two replays are spread over many launches there; 20 layer sets per graph keep that
# share near what serving pays (5 per graph: +1.7 us per step)
GRAPH_STEPS = 20
SPINUP_S = 0.3   # untimed GPU work before the first timed replay (clock ramp after the idle layer-set build)


def time_layer_set(torch, ops, sets, xs, steps: int, warmup: int, layout: int = 0):
    """One graph holds S steps, rounds of the R copies (step i: the 4 fused linears on copy i mod R), S = R x up to
    GRAPH_STEPS // R rounds, no more than the steps asked for allow.  Replays it ceil(steps / S) times after
    ceil(warmup / S) untimed replays; returns (steps timed, ms per step, per-layer us per launch).  Per-layer times
    come from a graph of S launches of that layer alone, timed the same way (same warmup)."""
    R = len(sets)
    S = R * max(1, min(GRAPH_STEPS // R, steps // R))
    names = list(LAYERS)
    outs = {nm: torch.empty((xs[nm].shape[0], sum(LAYERS[nm][1])), dtype=torch.float16, device=xs[nm].device)
            for nm in names}

    def run(copies, layer_names):
        for r in copies:
            for nm in layer_names:
                trs, suhs, svhs = sets[r][nm]
                ops.linear(xs[nm], trs, suhs, svhs, CODEBOOK, out=outs[nm], layout=layout)

    def timed(g, reps, warm):
        for _ in range(warm):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    order = [i % R for i in range(S)]
    g_all = _capture(torch, lambda: run(order, names))
    reps = -(-steps // S)
    total = timed(g_all, reps, -(-warmup // S))
    per_layer = {}
    for nm in names:
        g = _capture(torch, lambda nm=nm: run(order, [nm]))
        lreps = max(4, reps // 2)
        per_layer[nm] = timed(g, lreps, -(-warmup // S)) / (lreps * S)
    return reps * S, total / (reps * S), per_layer


def _cpu_threads() -> int:
    """Host threads for the CPU baseline: the cores this process may run on, at most 16 (the box's CPU share)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_s(fn, runs: int) -> float:
    times = []
    for _ in range(runs):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return float(np.median(times))


MOE_SHAPE = (128, 2048, 768, 3, 8)  # E, H, I, K, top_k
KV_SHAPE = (16, 40, 8, 128)         # B, Hq, Hkv, head_dim


def cpu_table(runs: int = 3, sample_tiles: int = 8192) -> dict:
    """The CPU baseline: the reference's CPU path (trellis_core reference.py:80-153) restated
    in torch (oracle/torch_cpu.py) on the host's cores, median of `runs` runs, decode and matmul timed apart:
      C1  4096 x 4096, K = 4, 3INST, M = 1: the whole path (all 65536 tiles decoded);
      C2  the 27B layer set at M = 1 (K = 3, MCG), per layer, each source matrix as the reference runs it;
      C3  5120 -> 17408 at M = 512, one K per codebook (K = 3 MCG, K = 2 3INST, K = 4 MUL1);
      C4  the MoE layer at T = 1 (8 experts x gate, up, down), SiLU-gated;
      C5  quantized-KV attention at 4k context: closed-form dequant of the pages + fp32 attention, 8 and 4 bits.
    Decode of C2-C4 is timed on the first `sample_tiles` tiles of each matrix (decode time is linear in tiles) and
    scaled to the whole matrix; matmuls (fp32 Hadamards + GEMM) run at full size on a same-shaped fp32 W."""
    import torch

    from oracle import torch_cpu as tc
    threads = _cpu_threads()
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(7)

    def trellis(tiles, K):
        return torch.randint(-32768, 32768, (1, tiles, 16 * K), dtype=torch.int16, generator=g)

    def signs(n):
        return (torch.randint(0, 2, (n,), generator=g) * 2 - 1).half()

    def decode_s(k, n, K, cb, full=False):
        tiles = (k // 16) * (n // 16)
        take = tiles if full else min(tiles, sample_tiles)
        tr = trellis(take, K)
        return _median_s(lambda: tc.reconstruct_inner(tr, K, cb), runs) * tiles / take

    def matmul_s(M, k, n):
        w, x, suh, svh = torch.randn((k, n), generator=g), torch.randn((M, k), generator=g), signs(k), signs(n)
        return _median_s(lambda: tc.linear_from_inner(x, w, suh, svh), runs)

    def entry(dec, mm, nbytes=None, flops=None):
        e = {"decode_us": round(dec * 1e6, 1), "matmul_us": round(mm * 1e6, 1), "total_us": round((dec + mm) * 1e6, 1)}
        if nbytes is not None:
            e["GB/s"] = round(nbytes / (dec + mm) / 1e9, 4)
        if flops is not None:
            e["TFLOPS"] = round(flops / (dec + mm) / 1e12, 5)
        return e

    t0 = time.perf_counter()
    table = {}
    # C1: the real pipeline on one matrix, parity-checked against the numpy oracle
    from oracle import exl3_oracle as orc
    tr = torch.randint(-32768, 32768, (256, 256, 64), dtype=torch.int16, generator=g)
    suh, svh, x = signs(4096), signs(4096), torch.randn((1, 4096), generator=g).half()
    w_inner = tc.reconstruct_inner(tr, 4, 0)
    y = tc.linear_from_inner(x, w_inner, suh, svh).numpy()
    ref = orc.linear_forward(x.numpy(), tr.numpy(), suh.numpy(), svh.numpy(), 4, 0, w_inner=w_inner.numpy())
    rel = float(np.linalg.norm(y - ref) / np.linalg.norm(ref))
    assert rel < 1e-5, f"torch CPU path disagrees with the oracle: {rel}"
    dec = _median_s(lambda: tc.reconstruct_inner(tr, 4, 0), runs)
    mm = _median_s(lambda: tc.linear_from_inner(x, w_inner, suh, svh), runs)
    table["C1_4096_K4_3inst_M1"] = entry(dec, mm, alg_bytes(4096, [4096], 1, 4))
    # C2: the layer set at M = 1
    per_layer, tot_dec, tot_mm = {}, 0.0, 0.0
    for name, (k, ns) in LAYERS.items():
        dec = sum(decode_s(k, n, K_BITS, CODEBOOK) for n in ns)
        mm = sum(matmul_s(1, k, n) for n in ns)
        per_layer[name] = entry(dec, mm)
        tot_dec, tot_mm = tot_dec + dec, tot_mm + mm
    c2_bytes = sum(alg_bytes(k, ns, 1, K_BITS) for k, ns in LAYERS.values())
    table["C2_layer_set_M1"] = dict(entry(tot_dec, tot_mm, c2_bytes), per_layer=per_layer)
    # C3: M = 512, one K per codebook; the matmul does not depend on the codebook
    mm = matmul_s(512, 5120, 17408)
    for K, cb, tag in ((3, 1, "K3_mcg"), (2, 0, "K2_3inst"), (4, 2, "K4_mul1")):
        table[f"C3_5120x17408_{tag}_M512"] = entry(decode_s(5120, 17408, K, cb), mm, flops=2 * 512 * 5120 * 17408)
    # C4: the MoE layer at one token: 8 experts, each gate and up (H -> I), SiLU(g) * u, down (I -> H)
    E, H, I, K, top_k = MOE_SHAPE
    dec = top_k * (2 * decode_s(H, I, K, CODEBOOK) + decode_s(I, H, K, CODEBOOK))
    ws = [(torch.randn((H, I), generator=g), torch.randn((H, I), generator=g), torch.randn((I, H), generator=g))
          for _ in range(top_k)]
    xs, sH, sI = torch.randn((1, H), generator=g), signs(H), signs(I)

    def moe_token():
        y = torch.zeros((1, H))
        for wg, wu, wd in ws:
            h = torch.nn.functional.silu(tc.linear_from_inner(xs, wg, sH, sI)) * tc.linear_from_inner(xs, wu, sH, sI)
            y += tc.linear_from_inner(h, wd, sI, sH) / top_k
        return y
    moe_bytes = top_k * (2 * H * I + I * H) * K // 8
    table["C4_moe_T1"] = entry(dec, _median_s(moe_token, runs), moe_bytes)
    # C5: 4k context, batch 16, 40 / 8 heads
    B, Hq, Hkv, D = KV_SHAPE
    L = 4096
    npg = L // 16
    P = B * npg
    for bits in (8, 4):
        row = D if bits == 8 else D // 2
        kc = torch.randint(-128, 128, (P, Hkv, 16, row), dtype=torch.int8, generator=g)
        vc = torch.randint(-128, 128, (P, Hkv, 16, row), dtype=torch.int8, generator=g)
        ks, vs = torch.rand((P, Hkv), generator=g).half(), torch.rand((P, Hkv), generator=g).half()
        table_pages = torch.randperm(P, generator=g).to(torch.int32).view(B, npg)
        q = torch.randn((B, Hq, D), generator=g).half()
        dec = _median_s(lambda: (tc.kv_dequant(kc, ks, bits), tc.kv_dequant(vc, vs, bits)), runs)
        kd, vd = tc.kv_dequant(kc, ks, bits), tc.kv_dequant(vc, vs, bits)
        att = _median_s(lambda: tc.decode_attention(q, kd, vd, table_pages, D ** -0.5), runs)
        nbytes = 2 * B * Hkv * L * row + 2 * 2 * P * Hkv + 4 * B * npg + 2 * 2 * B * Hq * D
        table[f"C5_L4k_{bits}bit_B16"] = entry(dec, att, nbytes)
        del kc, vc, kd, vd
    c2 = table["C2_layer_set_M1"]
    return {"value": c2["GB/s"], "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"trellis_core's CPU path (reference.py:80-153) restated in torch, {threads} threads, median of "
                      f"{runs} runs: C2 layer set at M = 1, decode of each matrix timed on its first {sample_tiles} "
                      f"tiles and scaled, fp32 Hadamards + GEMV at full size; C1 parity vs the numpy oracle "
                      f"{rel:.1e}",
            "cpu_model": _cpu_model(), "torch": torch.__version__, "runs": runs,
            "wall_s": round(time.perf_counter() - t0, 1), "table": table}


def cpu_baseline() -> dict:
    out = cpu_table()
    out["c_restatement"] = cpu_c_restatement()
    return out


def cpu_c_restatement(seconds_target: float = 6.0) -> dict:
    """The oracle's decode + matmul on the host cores (trellis_core's CPU path restated: reference.py:102-153): the
    o_proj linear (6144 -> 5120, K = 3, MCG) at M = 1.  The k range is cut into one slice of tile rows per thread;
    each thread decodes its slice with the C restatement (oracle/exl3_oracle.c, ctypes releases the GIL) and multiplies
    it with its part of the rotated input (numpy, one BLAS thread each); the partial rows are summed and rotated.
    Checked once against the numpy oracle; repeated until ~seconds_target of wall time."""
    import ctypes
    from concurrent.futures import ThreadPoolExecutor

    from threadpoolctl import threadpool_limits

    from oracle import exl3_oracle as orc
    so = os.path.join(ROOT, "oracle", "_build", "libexl3_oracle.so")
    if not os.path.exists(so):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    lib = ctypes.CDLL(so)
    lib.exl3_oracle_reconstruct.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_void_p]
    rng = np.random.default_rng(1)
    k, n = 6144, 5120
    tr = rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * K_BITS), dtype=np.int16)
    suh = np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16)
    svh = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16)
    x = rng.standard_normal((1, k)).astype(np.float16)
    nt = _cpu_threads()
    tk = k // 16
    bounds = [(tk * i // nt, tk * (i + 1) // nt) for i in range(nt)]

    def part(xh, i0, i1):
        w = np.empty((16 * (i1 - i0), n), dtype=np.uint16)
        lib.exl3_oracle_reconstruct(tr[i0:i1].ctypes.data, i1 - i0, n // 16, K_BITS, CODEBOOK, w.ctypes.data)
        return xh[:, 16 * i0:16 * i1] @ w.view(np.float16).astype(np.float32)

    def forward(pool):
        xh = orc.had_rows(x.astype(np.float32) * suh.astype(np.float32))
        y = sum(pool.map(lambda b: part(xh, *b), bounds))
        return orc.had_rows(y) * svh.astype(np.float32)

    w0 = np.empty((16, n), dtype=np.uint16)  # fills the decoder's lookup table once, before any concurrent call
    lib.exl3_oracle_reconstruct(tr[:1].ctypes.data, 1, n // 16, K_BITS, CODEBOOK, w0.ctypes.data)
    with threadpool_limits(limits=1), ThreadPoolExecutor(nt) as pool:
        y = forward(pool)
        ref = orc.linear_forward(x, tr, suh, svh, K_BITS, CODEBOOK)
        rel = float(np.linalg.norm(y - ref) / np.linalg.norm(ref))
        assert rel < 1e-4, f"CPU baseline disagrees with the oracle: {rel}"
        reps, t_total = 0, 0.0
        while t_total < seconds_target and reps < 200:
            t = time.perf_counter()
            forward(pool)
            t_total += time.perf_counter() - t
            reps += 1
    per = t_total / reps
    b = alg_bytes(k, [n], 1, K_BITS)
    return {"GB/s": round(b / per / 1e9, 4), "threads": nt,
            "what": f"oracle decode (C restatement) + fp32 matmul of o_proj 6144->5120 K=3 MCG M=1 over {nt} "
                      f"threads (k cut in {nt} slices), {reps} reps, {per * 1e3:.1f} ms each; agrees with the numpy "
                      f"oracle to {rel:.1e}"}


DOMINANT = "gate_up"  # the largest fused linear: its gemv_kernel instance is the dominant kernel of a step
MFMA_F16_PEAK_TFLOPS = 2500.0


def _graph_us(torch, fn, calls: int, reps: int = 3, warm_s: float = 0.05) -> float:
    """Mean device time of fn() in microseconds: a graph of `calls` back-to-back calls, replayed `reps` times after
    untimed replays for at least `warm_s` seconds (the inputs of each secondary line are generated on the host first,
    which leaves the GPU idle long enough for its clock to drop: one warm replay read the prefill ~7 % slow)."""
    g = _capture(torch, lambda: [fn(i) for i in range(calls)])
    t_end = time.perf_counter() + warm_s
    g.replay()
    torch.cuda.synchronize()
    while time.perf_counter() < t_end:
        g.replay()
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (calls * reps)


def bench_c1(torch, ops, dev) -> dict:
    """one 4096 -> 4096 linear, K = 4, 3INST, M = 1 (x fp16 N(0,1)): decode-GEMV with both
    rotations.  64 rotating copies (537 MB > 2 x the 256 MB MALL) keep the weights cold; the graph replays one call per
    copy.  Bytes = 8,421,376 per call (trellis + suh + svh + x + y)."""
    k = n = 4096
    K, cb, copies = 4, 0, 64
    g = torch.Generator(device="cpu").manual_seed(14)
    sets = []
    for _ in range(copies):
        tr = torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16, generator=g).to(dev)
        suh = (torch.randint(0, 2, (k,), generator=g) * 2 - 1).half().to(dev)
        svh = (torch.randint(0, 2, (n,), generator=g) * 2 - 1).half().to(dev)
        sets.append((tr, suh, svh))
    x = torch.randn((1, k), generator=g).half().to(dev)
    y = torch.empty((1, n), dtype=torch.float16, device=dev)
    us = _graph_us(torch, lambda i: ops.linear(x, [sets[i % copies][0]], [sets[i % copies][1]], [sets[i % copies][2]],
                                               cb, out=y), copies, reps=4)
    nbytes = alg_bytes(k, [n], 1, K)
    gbs = nbytes / (us * 1e-6) / 1e9
    print(f"[bench] C1 4096x4096 K=4 3inst M=1: {us:.2f} us, {gbs:.0f} GB/s", file=sys.stderr, flush=True)
    del sets
    return {"us": round(us, 2), "GB/s": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
            "bytes": nbytes}


def bench_prefill(torch, ops, dev) -> dict:
    """one 5120 -> 17408 linear, fp16 x ~ N(0,1) * 0.5, the fused decode-GEMM
    (exl3_linear_prefill).  M in {512, 2048, 8192} at K = 3 MCG, and M = 2048 over K in {2,4,5,6,8} cycling the three
    codebooks.  TFLOPS = 2 M k n / device time."""
    k, n = 5120, 17408
    g = torch.Generator(device="cpu").manual_seed(11)
    cases = [(3, 1, 512), (3, 1, 2048), (3, 1, 8192), (2, 0, 2048), (4, 2, 2048), (5, 1, 2048), (6, 0, 2048),
             (8, 2, 2048)]
    ops.reserve_prefill(dev, max(M for _, _, M in cases), k, n, 1)
    names = {0: "3inst", 1: "mcg", 2: "mul1"}
    out = {}
    for K, cb, M in cases:
        tr = torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16, generator=g).to(dev)
        suh = (torch.randint(0, 2, (k,), generator=g) * 2 - 1).half().to(dev)
        svh = (torch.randint(0, 2, (n,), generator=g) * 2 - 1).half().to(dev)
        x = (torch.randn((M, k), generator=g) * 0.5).half().to(dev)
        y = torch.empty((M, n), dtype=torch.float16, device=dev)
        us = _graph_us(torch, lambda i: ops.linear_prefill(x, [tr], [suh], [svh], cb, out=y), 5)
        tf = 2.0 * M * k * n / (us * 1e-6) / 1e12
        out[f"K{K}_{names[cb]}_M{M}"] = {"us": round(us, 1), "TFLOPS": round(tf, 1),
                                        "pct_mfma_peak": round(100 * tf / MFMA_F16_PEAK_TFLOPS, 2)}
        print(f"[bench] prefill K={K} {names[cb]} M={M}: {us:.1f} us, {tf:.0f} TFLOPS", file=sys.stderr, flush=True)
    return out


def _eager_us(torch, fn, reps: int = 10, warm: int = 3) -> float:
    """Mean device time of fn() in microseconds over back-to-back eager calls (HIP events on the current stream);
    for library calls that stay out of graphs."""
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def bench_vendor(torch, ops, dev) -> dict:
    """The vendor fp16 GEMM on the same box, for scale: (1) torch.mm (hipBLASLt) on 8192^3 fp16, the practical MFMA
    ceiling of a plain GEMM; (2) the reference's own prefill design (decode W_inner to HBM, vendor GEMM, output
    rotation: kernels/reference.py:71-104, runtime/ops.py:36-59) rebuilt from this library's had_in / reconstruct /
    had_out kernels around torch.mm, at BASELINE configs[2] M = 2048, K = 3 MCG, against the fused decode-GEMM on the
    same inputs.  Eager launches (each >= tens of us), HIP events."""
    out = {}
    g = torch.Generator(device="cpu").manual_seed(21)
    a = torch.randn((8192, 8192), generator=g).half().to(dev)
    b = torch.randn((8192, 8192), generator=g).half().to(dev)
    c = torch.empty((8192, 8192), dtype=torch.float16, device=dev)
    us = _eager_us(torch, lambda: torch.mm(a, b, out=c))
    tf = 2.0 * 8192 ** 3 / (us * 1e-6) / 1e12
    out["hipblaslt_fp16_8192cube"] = {"us": round(us, 1), "TFLOPS": round(tf, 1),
                                      "pct_mfma_peak": round(100 * tf / MFMA_F16_PEAK_TFLOPS, 2)}
    print(f"[bench] hipBLASLt fp16 8192^3: {us:.1f} us, {tf:.0f} TFLOPS", file=sys.stderr, flush=True)
    del a, b, c
    k, n, M, K, cb = 5120, 17408, 2048, 3, 1
    tr = torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16, generator=g).to(dev)
    suh = (torch.randint(0, 2, (k,), generator=g) * 2 - 1).half().to(dev)
    svh = (torch.randint(0, 2, (n,), generator=g) * 2 - 1).half().to(dev)
    x = (torch.randn((M, k), generator=g) * 0.5).half().to(dev)
    xh = torch.empty((M, k), dtype=torch.float16, device=dev)
    w = torch.empty((k, n), dtype=torch.float16, device=dev)
    yr = torch.empty((M, n), dtype=torch.float16, device=dev)
    y = torch.empty((M, n), dtype=torch.float16, device=dev)
    yf = torch.empty((M, n), dtype=torch.float16, device=dev)

    def reference_design():
        ops.had_in_group(x, suh, xh)
        ops.reconstruct(tr, cb, out=w)
        torch.mm(xh, w, out=yr)
        ops.had_out_into(yr, svh, y, 0)

    flops = 2.0 * M * k * n
    parts = {"reconstruct": lambda: ops.reconstruct(tr, cb, out=w), "gemm": lambda: torch.mm(xh, w, out=yr)}
    res = {"total": _eager_us(torch, reference_design)}
    for nm, fn in parts.items():
        res[nm] = _eager_us(torch, fn)
    fused = _eager_us(torch, lambda: ops.linear_prefill(x, [tr], [suh], [svh], cb, out=yf))
    same = (yf.float() - y.float()).norm().item() / max(y.float().norm().item(), 1e-30)
    out["reference_design_prefill_M2048_K3_mcg"] = {
        "us": round(res["total"], 1), "TFLOPS": round(flops / (res["total"] * 1e-6) / 1e12, 1),
        "reconstruct_us": round(res["reconstruct"], 1), "hipblaslt_gemm_us": round(res["gemm"], 1),
        "hipblaslt_gemm_TFLOPS": round(flops / (res["gemm"] * 1e-6) / 1e12, 1),
        "fused_decode_gemm_us": round(fused, 1), "fused_TFLOPS": round(flops / (fused * 1e-6) / 1e12, 1),
        "speedup_fused_vs_reference_design": round(res["total"] / fused, 3),
        "norm_rel_diff_fused_vs_reference_design": float(f"{same:.3g}")}
    print(f"[bench] reference design prefill M=2048: {res['total']:.1f} us (reconstruct {res['reconstruct']:.1f}, "
          f"hipBLASLt {res['gemm']:.1f}); fused {fused:.1f} us; rel diff {same:.2e}", file=sys.stderr, flush=True)
    return out


def bench_moe(torch, ops, dev) -> dict:
    """128 experts, top-8, hidden 2048, intermediate 768, K = 3 MCG; router logits fp32 N(0,1),
    top-8 ids and softmax weights over the selected logits.  Three rotating copies of the experts, a new routing per
    call.  Bytes = touched experts x 1,786,368 (trellis + sign vectors) + T x (8192 + 64)."""
    from trellis_serve_amd.ops import MOE_TENSORS
    E, H, I, K, top_k, copies = 128, 2048, 768, 3, 8, 3
    g = torch.Generator(device="cpu").manual_seed(12)

    def experts():
        d = {}
        for proj, (kk, nn) in (("gate", (H, I)), ("up", (H, I)), ("down", (I, H))):
            d[f"{proj}_trellis"] = torch.randint(-32768, 32768, (E, kk // 16, nn // 16, 16 * K), dtype=torch.int16,
                                                 generator=g).to(dev)
            d[f"{proj}_suh"] = (torch.randint(0, 2, (E, kk), generator=g) * 2 - 1).half().to(dev)
            d[f"{proj}_svh"] = (torch.randint(0, 2, (E, nn), generator=g) * 2 - 1).half().to(dev)
        assert set(d) == set(MOE_TENSORS)
        return d

    sets = [experts() for _ in range(copies)]
    ops.reserve_moe(dev, 256, top_k, E, H, I, K, K)
    out = {}
    for T in (1, 16, 256):
        routes = []
        touched = 0
        for r in range(copies):
            logits = torch.randn((T, E), generator=g)
            w, ids = torch.topk(logits, top_k, dim=1)
            routes.append((ids.to(torch.int32).to(dev), torch.softmax(w, dim=1).to(dev)))
            touched += len(torch.unique(ids))
        x = torch.randn((T, H), generator=g).half().to(dev)
        y = torch.empty((T, H), dtype=torch.float16, device=dev)
        us = _graph_us(torch, lambda i: ops.moe_forward(x, routes[i % copies][0], routes[i % copies][1],
                                                       sets[i % copies], 1, out=y), copies * 4)
        nbytes = touched / copies * 1786368 + T * (8192 + 64)
        out[f"T{T}"] = {"us": round(us, 1), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
                        "experts_touched": round(touched / copies, 1),
                        "TFLOPS": round(T * 75497472 / (us * 1e-6) / 1e12, 2)}
        print(f"[bench] moe T={T}: {us:.1f} us, {out[f'T{T}']['GB/s']} GB/s", file=sys.stderr, flush=True)
    return out


def bench_kv(torch, ops, dev) -> dict:
    """quantized-KV decode attention, 40 query / 8 KV heads, head_dim 128, batch 16, context 4k
    and 32k, 16-token pages in a random page order, 8- and 4-bit codes with per-(page, head) fp16 scales.  Rotating
    cache copies keep >= 512 MB in play at 4k.  Bytes = codes + scales + page table + q/out."""
    B, Hq, Hkv, D = 16, 40, 8, 128
    g = torch.Generator(device="cpu").manual_seed(13)
    ops.reserve_kv(dev, B, Hq, Hkv, 32768 // 16)
    out = {}
    for L in (4096, 32768):
        for bits in (8, 4):
            npg = L // 16
            P = B * npg
            row = D if bits == 8 else D // 2
            copies = 4 if L == 4096 else 1
            sets = []
            for _ in range(copies):
                kc = torch.randint(-128, 128, (P, Hkv, 16, row), dtype=torch.int8, device=dev)
                vc = torch.randint(-128, 128, (P, Hkv, 16, row), dtype=torch.int8, device=dev)
                ks = (torch.rand((P, Hkv), device=dev) * 0.02 + 0.01).half()
                vs = (torch.rand((P, Hkv), device=dev) * 0.02 + 0.01).half()
                table = torch.randperm(P, generator=g).to(torch.int32).view(B, npg).to(dev)
                sets.append((kc, vc, ks, vs, table))
            q = torch.randn((B, Hq, D), generator=g).half().to(dev)
            lens = torch.full((B,), L, dtype=torch.int32, device=dev)
            o = torch.empty((B, Hq, D), dtype=torch.float16, device=dev)
            us = _graph_us(torch, lambda i: ops.kv_decode_attention(q, *sets[i % copies][:4], sets[i % copies][4],
                                                                    lens, bits, out=o), copies * 8)
            nbytes = 2 * B * Hkv * L * row + 2 * 2 * P * Hkv + 4 * B * npg + 2 * 2 * B * Hq * D
            gbs = nbytes / (us * 1e-6) / 1e9
            out[f"L{L // 1024}k_{bits}bit"] = {"us": round(us, 1), "GB/s": round(gbs, 1),
                                               "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2)}
            print(f"[bench] kv L={L} bits={bits}: {us:.1f} us, {gbs:.0f} GB/s", file=sys.stderr, flush=True)
            del sets
    torch.cuda.empty_cache()
    return out


def _under_profiler() -> bool:
    return any(k.startswith(("ROCPROF_", "ROCPROFILER_")) for k in os.environ)


def probe(kind: str, launches: int) -> int:
    """Short GPU programs for counter passes: `gate_up` launches the dominant GEMV kernel `launches` times over five
    rotating copies of the layer; `prefill` the configs[2] decode-GEMM (5120 -> 17408, K = 3 MCG, M = 2048); `kv8` /
    `kv4` the configs[4] KV decode attention at 4k context (B = 16, 40 / 8 heads, 8- / 4-bit codes, four rotating
    caches in a random page order); `copy` runs a plain 512 MiB device copy (the calibration of FETCH_SIZE /
    WRITE_SIZE)."""
    import torch

    from trellis_serve_amd import ops
    dev = torch.device("cuda", 0)
    if kind == "prefill":
        g = torch.Generator(device="cpu").manual_seed(5)
        tr = torch.randint(-32768, 32768, (5120 // 16, 17408 // 16, 16 * K_BITS), dtype=torch.int16, generator=g).to(dev)
        suh = (torch.randint(0, 2, (5120,), generator=g) * 2 - 1).half().to(dev)
        svh = (torch.randint(0, 2, (17408,), generator=g) * 2 - 1).half().to(dev)
        x = (torch.randn((2048, 5120), generator=g) * 0.5).half().to(dev)
        y = ops.linear_prefill(x, [tr], [suh], [svh], CODEBOOK)
        for _ in range(launches):
            ops.linear_prefill(x, [tr], [suh], [svh], CODEBOOK, out=y)
    elif kind in ("kv8", "kv4"):
        bits, B, Hq, Hkv, D, L = int(kind[2:]), 16, 40, 8, 128, 4096
        g = torch.Generator(device="cpu").manual_seed(13)
        P, row = B * L // 16, D if bits == 8 else D // 2
        sets = [(torch.randint(-128, 128, (P, Hkv, 16, row), dtype=torch.int8, device=dev),
                 torch.randint(-128, 128, (P, Hkv, 16, row), dtype=torch.int8, device=dev),
                 (torch.rand((P, Hkv), device=dev) * 0.02 + 0.01).half(),
                 (torch.rand((P, Hkv), device=dev) * 0.02 + 0.01).half(),
                 torch.randperm(P, generator=g).to(torch.int32).view(B, L // 16).to(dev)) for _ in range(4)]
        q = torch.randn((B, Hq, D), generator=g).half().to(dev)
        lens = torch.full((B,), L, dtype=torch.int32, device=dev)
        o = torch.empty((B, Hq, D), dtype=torch.float16, device=dev)
        for i in range(launches):
            ops.kv_decode_attention(q, *sets[i % 4][:4], sets[i % 4][4], lens, bits, out=o)
    elif kind == "copy":
        src = torch.empty(128 << 20, dtype=torch.float32, device=dev).uniform_()
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
    else:
        # five copies of the layer (5 x 67 MB > the 256 MB MALL), rotated as the timed step rotates its copies, so the
        # counters see weights coming from HBM rather than from the MALL
        k, ns = LAYERS[kind]
        copies = [make_layer_set(torch, 99 + r, dev, names=(kind,))[kind] for r in range(5)]
        x = torch.randn((1, k), dtype=torch.float16, device=dev)
        out = ops.linear(x, *copies[0], CODEBOOK)
        for i in range(launches):
            ops.linear(x, *copies[i % len(copies)], CODEBOOK, out=out)
    torch.cuda.synchronize()
    return 0


def _pmc_pass(counter: str, kind: str, name_filter: str) -> float | None:
    """Mean per-dispatch value of `counter` over the dispatches whose kernel name contains `name_filter` (the
    largest-valued dispatch for the copy probe), from `rocprofv3 --pmc` on `bench.py --probe kind`."""
    with tempfile.TemporaryDirectory() as d:
        cmd = ["timeout", "-s", "KILL", "120", "rocprofv3", "--pmc", counter, "--output-format", "csv", "-d", d,
               "-o", "pmc", "--", sys.executable, os.path.abspath(__file__), "--probe", kind]
        r = subprocess.run(cmd, capture_output=True, text=True)
        files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        if r.returncode != 0 or not files:
            print(f"[bench] counter pass {counter}/{kind} failed (rc {r.returncode}): {r.stderr[-400:]}",
                  file=sys.stderr, flush=True)
            return None
        vals = [float(row["Counter_Value"]) for row in csv.DictReader(open(files[0]))
                if row["Counter_Name"] == counter and name_filter in row["Kernel_Name"]]
    if not vals:
        return None
    return max(vals) if kind == "copy" else sum(vals) / len(vals)


def measure_traffic() -> dict | None:
    """HBM bytes per launch of the dominant GEMV kernel from FETCH_SIZE and WRITE_SIZE (KiB per dispatch), each scaled
    by what the same counter reads for a plain copy of 512 MiB."""
    copy_bytes = 512 << 20
    got = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        kern = _pmc_pass(counter, DOMINANT, "gemv_kernel")
        cal = _pmc_pass(counter, "copy", "")
        if kern is None or not cal:
            return None
        got[counter] = (kern, cal, copy_bytes / (cal * 1024.0))
    fetch = got["FETCH_SIZE"][0] * 1024.0 * got["FETCH_SIZE"][2]
    write = got["WRITE_SIZE"][0] * 1024.0 * got["WRITE_SIZE"][2]
    return {"bytes": fetch + write, "fetch_bytes": fetch, "write_bytes": write,
            "fetch_kib_raw": got["FETCH_SIZE"][0], "write_kib_raw": got["WRITE_SIZE"][0],
            "fetch_scale": got["FETCH_SIZE"][2], "write_scale": got["WRITE_SIZE"][2]}


def _lib_xcd_local() -> int:
    from trellis_serve_amd import _lib
    return _lib.load().exl3_xcd_local_chains()


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--rows", type=int, default=1)
    ap.add_argument("--copies", type=int, default=5, help="rotating copies of the layer set (cold HBM)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--extra-rows", default="4,16,32,64",
                    help="also report these M (comma list, '' for none; past 16 rows the GEMV takes 2 or 4 row groups)")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 counter passes")
    ap.add_argument("--no-secondary", action="store_true", help="skip the prefill / MoE / KV-attention lines")
    ap.add_argument("--probe", choices=["gate_up", "prefill", "kv8", "kv4", "copy"], help=argparse.SUPPRESS)
    ap.add_argument("--probe-launches", type=int, default=20, help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.probe:
        return probe(args.probe, args.probe_launches)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (--gpus {args.gpus} requested). "
              "The value is one GPU's throughput; run with --gpus 1.", file=sys.stderr)
        return 2

    traffic = None
    if not args.no_traffic and not _under_profiler():
        print("[bench] counter passes (FETCH_SIZE, WRITE_SIZE) on the dominant kernel", file=sys.stderr, flush=True)
        traffic = measure_traffic()

    import torch

    from trellis_serve_amd import ops
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    ops.init_device(0)
    print(f"[bench] building {args.copies} copies of the K={K_BITS} MCG layer set", file=sys.stderr, flush=True)
    sets = [make_layer_set(torch, 1234 + r, dev) for r in range(args.copies)]
    g = torch.Generator(device="cpu").manual_seed(7)

    def xs_for(M):
        return {nm: torch.randn((M, k), generator=g).half().to(dev) for nm, (k, _) in LAYERS.items()}

    # the headline row count is timed last: a single timed replay (the driver's --steps 20) right after the layer-set
    # build and the counter passes read up to ~10 % slow against the same graph timed after other GPU work
    row_list = [int(v) for v in args.extra_rows.split(",") if v and int(v) != args.rows] + [args.rows]
    # load-time reservation, as an engine does before capturing graphs: one workspace per kind and device, sized for
    # the largest call, so no captured graph ever holds a buffer that a larger call would replace
    for k, ns in LAYERS.values():
        ops.reserve_linear(dev, max(row_list), k, sum(ns), K_BITS)
    # GPU clock spin-up: the layer-set build leaves the GPU idle for seconds, and the first graph replay timed after it
    # read up to ~10 % slow at the driver's settings (one timed replay of 20 steps).  The layer set's own launches run
    # untimed for SPINUP_S first (not counted as warmup steps; reported as clock_spinup_s).
    xs1 = xs_for(args.rows)
    t_end = time.perf_counter() + SPINUP_S
    while time.perf_counter() < t_end:
        for st in sets:
            for nm, (trs, suhs, svhs) in st.items():
                ops.linear(xs1[nm], trs, suhs, svhs, CODEBOOK)
        torch.cuda.synchronize()
    results = {}
    for M in row_list:
        xs = xs_for(M)
        steps = args.steps if M == args.rows else max(20, args.steps // 4)
        steps, ms_step, per_layer = time_layer_set(torch, ops, sets, xs, steps, args.warmup)
        step_bytes = sum(alg_bytes(k, ns, M, K_BITS) for k, ns in LAYERS.values())
        results[M] = dict(ms_per_step=ms_step, gbs=step_bytes / (ms_step * 1e-3) / 1e9,
                          per_layer=per_layer, step_bytes=step_bytes, steps=steps)
        print(f"[bench] M={M}: {ms_step * 1e3:.1f} us/step, {results[M]['gbs']:.0f} GB/s "
              f"per layer us {({k: round(v * 1e3, 1) for k, v in per_layer.items()})}", file=sys.stderr, flush=True)

    main_r = results[args.rows]
    # warm secondary: one copy of the layer set (128 MB, inside the 256 MB MALL) replayed back to back
    _, warm_ms, _ = time_layer_set(torch, ops, sets[:1], xs_for(args.rows), max(20, args.steps // 4), args.warmup)
    print(f"[bench] M={args.rows} warm (one copy): {warm_ms * 1e3:.1f} us/step", file=sys.stderr, flush=True)
    # the same step on the load-time BLOCKS layout (exl3_repack_trellis), same process and copies, timed like the
    # headline; the stored-layout figures it is compared with are the headline's own
    blocks_sets = [{nm: ([ops.repack_trellis(t) for t in trs], suhs, svhs) for nm, (trs, suhs, svhs) in st.items()}
                   for st in sets]
    _, blk_ms, blk_layer = time_layer_set(torch, ops, blocks_sets, xs_for(args.rows), main_r["steps"], args.warmup,
                                          layout=1)
    del blocks_sets
    print(f"[bench] M={args.rows} BLOCKS layout: {blk_ms * 1e3:.1f} us/step per layer us "
          f"{({k: round(v * 1e3, 1) for k, v in blk_layer.items()})}", file=sys.stderr, flush=True)
    # dominant kernel: the gate_up fused linear (one gemv_kernel launch); its per-launch time comes from HIP events
    # around graph replays of that layer alone
    kd, nd = LAYERS[DOMINANT]
    dom_bytes = alg_bytes(kd, nd, args.rows, K_BITS)
    dom_ms = main_r["per_layer"][DOMINANT]
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    all_ms = sum(main_r["per_layer"].values())
    line = {
        "metric": "EXL3 GEMV HBM GB/s (% peak) at M=1; decode-GEMM TFLOPS at M=2048",
        "value": round(main_r["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": main_r["steps"],
        "warmup": args.warmup,
        "clock_spinup_s": SPINUP_S,
        "ms_per_step": round(main_r["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded uniform int16 trellis codes, +-1 fp16 signs, N(0,1) fp16 activations)",
        "config": {"workload": "27B-class dense layer set, K=3 bpw, MCG (BASELINE configs[1])",
                   "rows": args.rows, "layers": {k: [kk, ns] for k, (kk, ns) in LAYERS.items()},
                   "copies": args.copies, "bytes_per_step": main_r["step_bytes"],
                   "xcd_local_chains": bool(_lib_xcd_local())},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None if traffic is None else round(traffic["bytes"]),
                     "kernel": f"gemv_kernel<{K_BITS}, MCG, rotate, NT> of the {DOMINANT} linear "
                               f"({kd}->{'+'.join(map(str, nd))}), {dom_bytes} algorithmic bytes per launch",
                     "us_per_launch": round(dom_ms * 1e3, 2)},
        "pct_hbm_peak": round(100 * main_r["gbs"] / HBM_PEAK_GBS, 2),
        "us_per_layer": {k: round(v * 1e3, 2) for k, v in main_r["per_layer"].items()},
        "gemv_kernels_gbs": round(main_r["step_bytes"] / (all_ms * 1e-3) / 1e9, 2),
        "weight_stream_gbs": round(TRELLIS_BYTES_PER_STEP / (main_r["ms_per_step"] * 1e-3) / 1e9, 2),
        "warm_single_copy": {"GB/s": round(main_r["step_bytes"] / (warm_ms * 1e-3) / 1e9, 1),
                             "us_per_step": round(warm_ms * 1e3, 2)},
        "other_rows": {str(M): {"GB/s": round(r["gbs"], 1), "us_per_step": round(r["ms_per_step"] * 1e3, 2)}
                       for M, r in results.items() if M != args.rows},
        "blocks_layout": {"GB/s": round(main_r["step_bytes"] / (blk_ms * 1e-3) / 1e9, 1),
                          "us_per_step": round(blk_ms * 1e3, 2),
                          "us_per_layer": {k: round(v * 1e3, 2) for k, v in blk_layer.items()},
                          "what": "the headline step on the trellis repacked to EXL3_LAYOUT_BLOCKS at load, same "
                                  "process; the stored-layout figures are value / us_per_layer"},
    }
    if not args.no_secondary:
        del sets
        torch.cuda.empty_cache()
        line["c1_linear_4096_k4_3inst"] = bench_c1(torch, ops, dev)
        line["prefill_decode_gemm"] = bench_prefill(torch, ops, dev)
        line["decode_gemm_tflops_m2048"] = line["prefill_decode_gemm"]["K3_mcg_M2048"]["TFLOPS"]
        line["vendor_gemm"] = bench_vendor(torch, ops, dev)
        line["moe_layer"] = bench_moe(torch, ops, dev)
        line["kv_decode_attention"] = bench_kv(torch, ops, dev)
    if traffic is not None:
        line["roofline"]["traffic_detail"] = {k: (round(v, 4) if isinstance(v, float) else v)
                                              for k, v in traffic.items()}
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
