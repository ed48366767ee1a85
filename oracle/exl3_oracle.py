"""CPU oracle for the EXL3 hot path -- TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may import this module, and
only as the checker (or the timed CPU baseline).  The product path (`trellis_serve_amd`) never imports it.

This is a numpy restatement of the reference decoder `core/src/trellis_core/reference.py` (trellis_core,
the ground truth of the reference repository), plus the pieces of the reference's kernels whose numerics
the tests must follow.  Every function cites the reference lines it restates.

Pinning (how each function is checked independently of this file; the tests named here do it):
  codebook_lut          golden fixture (sha256 of the full 65536-entry LUT written by trellis_core itself),
                        reference KAT points + moments (core/tests/test_reference.py:19-30), the C restatement
                        (oracle/exl3_oracle.c) over all 65536 states.        tests/test_oracle.py
  tensor_core_perm      golden fixture; the independent row/col closed form of xpu/csrc/exl3_esimd.h:6-8.
  decode_states         golden fixture (states of one tile per K); the shift-register invariant
                        state[t+1] = ((state[t] << K) | new) & 0xFFFF; the low K bits of the states,
                        concatenated, reproduce the bit stream; the C restatement (funnel-shift form).
  reconstruct_inner     golden fixture for every (K, codebook); the C restatement; brute force on 1 tile.
  hadamard128/had_rows  scipy.linalg.hadamard (textbook Sylvester); H @ H = I; golden fixture.
  weight_orig/linear_forward   golden fixture (k=256, n=128, K=3, mul1); float64 evaluation.
  moe_forward           restates cuda/csrc/exl3_marlin_moe.cu:210-292 numerics; checked against a float64
                        per-expert evaluation (tools/moe_parity_sm86.py:76-89 form).  The fp16 rounding points
                        are this build's; "parity unpinned" against the reference MoE kernels (no GPU build of
                        them can run here).
  kv_decode_attention   closed-form dequant + fp32 softmax attention.  The reference has no quantized-KV decode
                        kernel (its nearest relative is xpu/exl3xpu/fp8kv_prefill.py:73-117), so this function is
                        "parity unpinned" against the reference; it is checked against a float64 evaluation.
"""
from __future__ import annotations

import math
from functools import lru_cache

import numpy as np

MCG_MULT = 0xCBAC1FED
MUL1_MULT = 0x83DCD12D
INST3_MULT = 89226354
INST3_ADD = 64248484
CB_3INST, CB_MCG, CB_MUL1 = 0, 1, 2
HAD_SCALE = 0.088388347648  # 1/sqrt(128) as the reference kernels write it (cuda/csrc/exl3_marlin.cu:251)


# ---------------------------------------------------------------------------------------------------------------
# Tile order, codebooks, bit windows (reference.py:30-115)

@lru_cache
def tensor_core_perm() -> np.ndarray:
    """Stream position t (0..255) -> tile position row*16+col.  Restates reference.py:30-45."""
    perm = np.zeros(256, dtype=np.int64)
    for thread in range(32):
        r0 = (thread % 4) * 2
        c0 = thread // 4
        rows = (r0, r0 + 1, r0 + 8, r0 + 9)
        for j in range(8):
            r = rows[j % 4]
            c = c0 + (8 if j >= 4 else 0)
            perm[thread * 8 + j] = r * 16 + c
    return perm


def _f16_from_bits(u) -> np.ndarray:
    return np.asarray(u).astype(np.uint16).view(np.float16)


@lru_cache
def codebook_lut(cb: int) -> np.ndarray:
    """fp16 value of every 16-bit trellis state.  Restates reference.py:52-73 (itself codebook.cuh:56-90)."""
    s = np.arange(65536, dtype=np.uint64)
    if cb == CB_MUL1:
        x = (s * MUL1_MULT) & 0xFFFFFFFF
        bsum = (x & 0xFF) + ((x >> 8) & 0xFF) + ((x >> 16) & 0xFF) + ((x >> 24) & 0xFF)
        h = (1024 + bsum).astype(np.float64)                  # fp16 bits 0x6400 + bsum are exactly 1024 + bsum
        inv = float(_f16_from_bits(0x1EEE))
        bias = float(_f16_from_bits(0xC931))
        val = (h * inv + bias).astype(np.float16)             # exact in float64, then ONE rounding (hfma)
    else:
        if cb == CB_3INST:
            x = (s * INST3_MULT + INST3_ADD) & 0xFFFFFFFF
        elif cb == CB_MCG:
            x = (s * MCG_MULT) & 0xFFFFFFFF
        else:
            raise ValueError(f"unknown codebook {cb}")
        x = (x & 0x8FFF8FFF) ^ 0x3B603B60
        lo = _f16_from_bits(x & 0xFFFF).astype(np.float64)
        hi = _f16_from_bits(x >> 16).astype(np.float64)
        val = (lo + hi).astype(np.float16)                    # exact sum, ONE rounding (hadd)
    val.setflags(write=False)
    return val


def codebook_of(mcg: bool, mul1: bool) -> int:
    """reference.py:76-77."""
    return CB_MCG if mcg else (CB_MUL1 if mul1 else CB_3INST)


@lru_cache
def state_index(K: int) -> np.ndarray:
    """[256, 16] bit positions (MSB first) of each state's window in the 256*K-bit tile.  reference.py:80-87."""
    nbits = 256 * K
    t = np.arange(256)
    b0 = (t * K + K - 16 + nbits) % nbits
    pos = (b0[:, None] + np.arange(16)[None, :]) % nbits
    return pos.astype(np.int64)


def decode_states(trellis: np.ndarray, K: int) -> np.ndarray:
    """int16 [..., 16K] -> uint32 states [..., 256] in stream order.  Restates reference.py:90-99:
    words = little-endian int16 pairs (h[2m] | h[2m+1] << 16), bits MSB first, gathered windows."""
    t16 = trellis.astype(np.int64) & 0xFFFF
    words = (t16[..., 0::2] | (t16[..., 1::2] << 16)).astype(np.uint32)   # [..., 8K]
    shifts = np.arange(31, -1, -1, dtype=np.uint32)
    bits = ((words[..., None] >> shifts) & 1).astype(np.uint8)
    bits = bits.reshape(*words.shape[:-1], 32 * words.shape[-1])          # [..., 256K] MSB first
    win = bits[..., state_index(K)]                                       # [..., 256, 16]
    weights = (1 << np.arange(15, -1, -1)).astype(np.uint32)
    return (win.astype(np.uint32) * weights).sum(-1).astype(np.uint32)


def reconstruct_inner(trellis: np.ndarray, K: int, cb: int, chunk_tiles: int = 1 << 13) -> np.ndarray:
    """int16 [k/16, n/16, 16K] -> W_inner fp16 [k, n] (Hadamard domain).  Restates reference.py:102-115."""
    tk, tn, words = trellis.shape
    if words != 16 * K:
        raise ValueError(f"trellis last dim {words} != 16*K for K={K}")
    lut = codebook_lut(cb)
    perm = tensor_core_perm()
    flat = trellis.reshape(tk * tn, 16 * K)
    out = np.empty((tk * tn, 256), dtype=np.float16)
    for s in range(0, tk * tn, chunk_tiles):
        st = decode_states(flat[s:s + chunk_tiles], K)
        vals = lut[st]
        tile = np.empty_like(vals)
        tile[:, perm] = vals
        out[s:s + chunk_tiles] = tile
    return out.reshape(tk, tn, 16, 16).transpose(0, 2, 1, 3).reshape(tk * 16, tn * 16)


# ---------------------------------------------------------------------------------------------------------------
# Hadamard and the forward (reference.py:118-153)

@lru_cache
def hadamard128() -> np.ndarray:
    """Normalised Sylvester H128 (float64).  reference.py:118-123."""
    h = np.ones((1, 1), dtype=np.float64)
    while h.shape[0] < 128:
        h = np.block([[h, h], [h, -h]])
    return h / math.sqrt(128)


def had_rows(x: np.ndarray, dtype=np.float32) -> np.ndarray:
    """H128 on the last dim in blocks of 128 (x @ H).  reference.py:126-130 (fp32 by default, float64 on request)."""
    shp = x.shape
    h = hadamard128().astype(dtype)
    return (x.astype(dtype).reshape(-1, 128) @ h).reshape(shp)


def weight_orig(trellis, suh, svh, K, cb) -> np.ndarray:
    """Original-basis fp32 weight [k, n] = diag(suh) H W_inner H diag(svh).  reference.py:133-142."""
    w = reconstruct_inner(trellis, K, cb).astype(np.float32)
    k, n = w.shape
    h = hadamard128().astype(np.float32)
    w = np.einsum("ij,bjn->bin", h, w.reshape(k // 128, 128, n)).reshape(k, n)
    w = w * suh.astype(np.float32)[:, None]
    w = (w.reshape(k, n // 128, 128) @ h).reshape(k, n)
    return w * svh.astype(np.float32)[None, :]


def linear_forward(x, trellis, suh, svh, K, cb, bias=None, w_inner=None, dtype=np.float32) -> np.ndarray:
    """y = had(had(x*suh) @ W_inner) * svh (+ bias), accumulated in fp32.  reference.py:145-153.
    `w_inner` may be passed to skip the decode; dtype=float64 gives the exact evaluation used as a tolerance anchor
    (cuda/src/sglang_exl3/parity/l1_linear.py:28-36)."""
    w = (reconstruct_inner(trellis, K, cb) if w_inner is None else w_inner).astype(dtype)
    xh = had_rows(x.astype(dtype) * suh.astype(dtype), dtype)
    y = xh @ w
    y = had_rows(y, dtype) * svh.astype(dtype)
    if bias is not None:
        y = y + bias.astype(dtype)
    return y


# ---------------------------------------------------------------------------------------------------------------
# fp16 kernel-class numerics (what a fused kernel may round) -- used for tolerances, not for bit equality

def had_in_fp16(x: np.ndarray, suh: np.ndarray) -> np.ndarray:
    """xh = fp16(Had128(fp16(fp16(x) * suh)) ): the input transform with the rounding points of
    cuda/csrc/exl3_had.cuh:20-84 (fp16 pre-scale product, fp32 butterfly, one rounding to fp16)."""
    xs = (x.astype(np.float16) * suh.astype(np.float16)).astype(np.float16)
    return had_rows(xs.astype(np.float32), np.float64).astype(np.float32).astype(np.float16)


# ---------------------------------------------------------------------------------------------------------------
# MoE layer (cuda/csrc/exl3_marlin_moe.cu:1-12, 210-292; kernels/marlin_moe.py:272-294)

def silu32(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.float32)
    return x / (np.float32(1.0) + np.exp(-x))


def moe_forward(x, topk_ids, topk_w, experts, K, cb, dtype=np.float64, w_cache=None):
    """Routed SiLU-gated MoE: for each slot (token t, choice j) with expert e:
        g = linear(x_t, gate_e), u = linear(x_t, up_e), a = silu(g) * u, d = linear(a, down_e)
        y_t = sum_j w[t, j] * d_slot   (slot order, as exl3_marlin_moe.cu:262-292)
    `experts[e]` = dict(gate=(trellis, suh, svh), up=(...), down=(...)).  Evaluated in `dtype` (float64 = the
    exact layer of tools/moe_parity_sm86.py:76-89).  Slots whose id is outside [0, E) are skipped
    (exl3_marlin_moe.cu:274).  Each projection runs at its own bitrate, read from its trellis (16K int16 per tile;
    the reference's gate/up and down bitrates, cuda/src/sglang_exl3/kernels/reference.py:123-149); `K`, when not
    None, must agree with every projection."""
    tokens, hidden = x.shape
    top_k = topk_ids.shape[1]
    y = np.zeros((tokens, hidden), dtype=dtype)
    w_cache = {} if w_cache is None else w_cache

    def bits(e, proj):
        kp = experts[e][proj][0].shape[-1] // 16
        assert K is None or K == kp, f"expert {e} {proj}: trellis holds K = {kp}, caller said {K}"
        return kp

    def w_of(e, proj):
        key = (e, proj)
        if key not in w_cache:
            t, _, _ = experts[e][proj]
            w_cache[key] = reconstruct_inner(t, bits(e, proj), cb)
        return w_cache[key]

    for t in range(tokens):
        for j in range(top_k):
            e = int(topk_ids[t, j])
            if e < 0 or e >= len(experts):
                continue
            xt = x[t:t + 1].astype(dtype)
            g = linear_forward(xt, *experts[e]["gate"], bits(e, "gate"), cb, w_inner=w_of(e, "gate"), dtype=dtype)
            u = linear_forward(xt, *experts[e]["up"], bits(e, "up"), cb, w_inner=w_of(e, "up"), dtype=dtype)
            a = (g / (1.0 + np.exp(-g))) * u
            d = linear_forward(a, *experts[e]["down"], bits(e, "down"), cb, w_inner=w_of(e, "down"), dtype=dtype)
            y[t] += dtype(topk_w[t, j]) * d[0]
    return y


def moe_align(topk_ids: np.ndarray, block: int, num_experts: int):
    """The moe_align_block_size contract (vLLM / SGLang; restated at cuda/csrc/exl3_marlin_moe.cu:532-594):
    slots (t*top_k + j) grouped by expert in ascending expert order, each expert's list padded to a multiple of
    `block` with the sentinel `numel`; one expert id per block; num_post = padded total.  Ids outside [0, E)
    are dropped.  Returns (sorted_ids, expert_ids, num_post)."""
    flat = topk_ids.reshape(-1)
    numel = flat.size
    sorted_ids, expert_ids = [], []
    for e in range(num_experts):
        slots = [s for s in range(numel) if int(flat[s]) == e]
        if not slots:
            continue
        padded = -(-len(slots) // block) * block
        sorted_ids += slots + [numel] * (padded - len(slots))
        expert_ids += [e] * (padded // block)
    return np.array(sorted_ids, dtype=np.int32), np.array(expert_ids, dtype=np.int32), len(sorted_ids)


# ---------------------------------------------------------------------------------------------------------------
# Quantized paged KV cache + decode attention (no reference kernel; nearest: xpu/exl3xpu/fp8kv_prefill.py:73-117)

def kv_quantize(x: np.ndarray, bits: int):
    """Symmetric per-(page, head) quantization of fp16 K or V.
    x: [num_pages, H_kv, page, D] float.  Returns (q, scale): int8 values in [-127, 127] (bits=8) or
    [-7, 7] (bits=4), scale fp16 [num_pages, H_kv] = max|x| / qmax (rounded to fp16; 1 when the block is all 0).
    Codes are q = clip(round(x / scale), -qmax, qmax) with the fp16 scale."""
    qmax = 127 if bits == 8 else 7
    amax = np.abs(x.astype(np.float32)).max(axis=(2, 3))
    scale = (amax / qmax).astype(np.float16)
    scale = np.where(scale == 0, np.float16(1.0), scale).astype(np.float16)
    q = np.clip(np.rint(x.astype(np.float32) / scale.astype(np.float32)[:, :, None, None]), -qmax, qmax)
    return q.astype(np.int8), scale


def kv_pack4(q: np.ndarray) -> np.ndarray:
    """int8 codes in [-8, 7], [..., D] -> uint8 [..., D/2]: element 2i in the low nibble, 2i+1 in the high nibble,
    two's complement."""
    u = (q.astype(np.int16) & 0xF).astype(np.uint8)
    return (u[..., 0::2] | (u[..., 1::2] << 4)).astype(np.uint8)


def kv_unpack4(p: np.ndarray) -> np.ndarray:
    lo = (p & 0xF).astype(np.int16)
    hi = (p >> 4).astype(np.int16)
    lo = np.where(lo >= 8, lo - 16, lo)
    hi = np.where(hi >= 8, hi - 16, hi)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.int8)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out


def kv_decode_attention(q, k_codes, v_codes, k_scale, v_scale, page_table, seq_lens, bits, sm_scale,
                        dtype=np.float64):
    """Single-query decode attention over a quantized paged cache.
    q: [B, Hq, D]; k_codes/v_codes: int8 [P, Hkv, page, D] (bits=8) or packed uint8 [P, Hkv, page, D/2] (bits=4);
    k_scale/v_scale fp16 [P, Hkv]; page_table int32 [B, max_pages]; seq_lens int32 [B].  GQA: q head h reads kv
    head h // (Hq / Hkv).  Returns o [B, Hq, D] in `dtype`.  Dequant: value = code * scale (fp32 product)."""
    B, Hq, D = q.shape
    Hkv = k_codes.shape[1]
    page = k_codes.shape[2]
    group = Hq // Hkv
    kc = kv_unpack4(k_codes) if bits == 4 else k_codes
    vc = kv_unpack4(v_codes) if bits == 4 else v_codes
    out = np.zeros((B, Hq, D), dtype=dtype)
    for b in range(B):
        L = int(seq_lens[b])
        npg = -(-L // page)
        pages = page_table[b, :npg]
        for hk in range(Hkv):
            ks = (kc[pages, hk].astype(np.float32) * k_scale[pages, hk].astype(np.float32)[:, None, None])
            vs = (vc[pages, hk].astype(np.float32) * v_scale[pages, hk].astype(np.float32)[:, None, None])
            ks = ks.reshape(-1, D)[:L].astype(dtype)
            vs = vs.reshape(-1, D)[:L].astype(dtype)
            for g in range(group):
                h = hk * group + g
                s = (ks @ q[b, h].astype(dtype)) * dtype(sm_scale)
                s = s - s.max()
                p = np.exp(s)
                out[b, h] = (p @ vs) / p.sum()
    return out
