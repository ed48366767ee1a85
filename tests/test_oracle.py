"""Pins the CPU oracle (oracle/exl3_oracle.py, oracle/exl3_oracle.c) before anything is checked against it.

Each oracle function is checked against (a) golden vectors written by the reference decoder itself
(tests/golden/make_golden.py), (b) an independent closed form or invariant, and (c) the second restatement.
The `test_planted_*` tests plant a plausible mistake in a copy of the oracle and show that a check catches it.
"""
import hashlib
import struct

import numpy as np
import pytest
import scipy.linalg

from conftest import c_reconstruct
from oracle import exl3_oracle as orc

KS = (2, 3, 4, 5, 6, 8)
CBS = (orc.CB_3INST, orc.CB_MCG, orc.CB_MUL1)


# ---- codebooks -------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("cb", CBS)
def test_codebook_lut_matches_reference_hash_and_samples(golden, cb):
    lut = orc.codebook_lut(cb).view(np.uint16)
    assert hashlib.sha256(lut.tobytes()).digest() == golden[f"lut_sha256_cb{cb}"].tobytes()
    np.testing.assert_array_equal(lut[golden["lut_sample_states"]], golden[f"lut_sample_cb{cb}"])


@pytest.mark.parametrize("cb", CBS)
def test_codebook_lut_equals_c_restatement_on_all_states(coracle, cb):
    c = np.empty(65536, dtype=np.uint16)
    coracle.exl3_oracle_codebook_lut(cb, c.ctypes.data)
    np.testing.assert_array_equal(c, orc.codebook_lut(cb).view(np.uint16))


def _mcg_independent(state: int) -> float:
    """core/tests/test_reference.py:10-16, one state at a time via struct."""
    x = (state * 0xCBAC1FED) & 0xFFFFFFFF
    x = ((x & 0x8FFF8FFF) ^ 0x3B603B60) & 0xFFFFFFFF
    lo = np.frombuffer(struct.pack("<H", x & 0xFFFF), dtype=np.float16)[0]
    hi = np.frombuffer(struct.pack("<H", x >> 16), dtype=np.float16)[0]
    return float(np.float16(np.float64(lo) + np.float64(hi)))


def test_mcg_known_answers():
    lut = orc.codebook_lut(orc.CB_MCG).astype(np.float64)
    for s in (0, 1, 0xB38D, 0x7FFF, 0xFFFF, 12345):
        assert lut[s] == _mcg_independent(s), hex(s)


@pytest.mark.parametrize("cb", CBS)
def test_codebooks_are_bell_shaped_and_centred(cb):
    v = orc.codebook_lut(cb).astype(np.float64)
    assert abs(v.mean()) < 0.05 and 1.0 < v.std() < 1.5      # core/tests/test_reference.py:25-30


def test_c_fp16_rounding_agrees_with_numpy(coracle):
    rng = np.random.default_rng(0)
    vals = np.concatenate([rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 5, 20000),
                           [0.0, -0.0, 65504.0, 65520.0, 65519.99, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                            1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11]])
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([coracle.exl3_oracle_f64_to_f16(float(v)) for v in vals], dtype=np.uint16)
    np.testing.assert_array_equal(got, want)


# ---- tile order ------------------------------------------------------------------------------------------------

def test_perm_matches_reference_and_closed_form(golden, coracle):
    perm = orc.tensor_core_perm()
    np.testing.assert_array_equal(perm, golden["perm"])
    rows = np.empty(256, dtype=np.int32)
    cols = np.empty(256, dtype=np.int32)
    coracle.exl3_oracle_perm(rows.ctypes.data, cols.ctypes.data)
    np.testing.assert_array_equal(perm, rows * 16 + cols)
    assert sorted(perm.tolist()) == list(range(256))


# ---- bit windows -----------------------------------------------------------------------------------------------

@pytest.mark.parametrize("K", KS)
def test_decode_states_matches_reference(golden, K):
    np.testing.assert_array_equal(orc.decode_states(golden[f"states_in_K{K}"], K), golden[f"states_out_K{K}"])


def _stream_bits(tile: np.ndarray) -> np.ndarray:
    """MSB-first bits of the little-endian int16-pair words, written independently of the oracle."""
    u = tile.astype(np.uint16)
    words = [int(u[2 * m]) | (int(u[2 * m + 1]) << 16) for m in range(len(u) // 2)]
    return np.array([(w >> (31 - b)) & 1 for w in words for b in range(32)], dtype=np.uint32)


@pytest.mark.parametrize("K", KS)
def test_decode_states_shift_register_invariants(K):
    rng = np.random.default_rng(K)
    tile = rng.integers(-32768, 32768, size=16 * K, dtype=np.int16)
    st = orc.decode_states(tile, K).astype(np.int64)
    # consecutive states overlap by 16-K bits: a trellis is a K-bit shift register
    nxt = np.roll(st, -1)
    np.testing.assert_array_equal(nxt >> K, st & ((1 << (16 - K)) - 1))
    # the low K bits of the states, in order, are the bit stream itself
    low = np.array([[(s >> (K - 1 - b)) & 1 for b in range(K)] for s in st]).reshape(-1)
    np.testing.assert_array_equal(low, _stream_bits(tile))


@pytest.mark.parametrize("K", KS)
def test_decode_states_equals_c_funnel_form(coracle, K):
    rng = np.random.default_rng(100 + K)
    tiles = rng.integers(-32768, 32768, size=(64, 16 * K), dtype=np.int16)
    want = orc.decode_states(tiles, K)
    got = np.empty(256, dtype=np.uint32)
    for i in range(tiles.shape[0]):
        coracle.exl3_oracle_decode_tile(np.ascontiguousarray(tiles[i]).ctypes.data, K, got.ctypes.data)
        np.testing.assert_array_equal(got, want[i])


# ---- reconstruct -----------------------------------------------------------------------------------------------

@pytest.mark.parametrize("K", KS)
@pytest.mark.parametrize("cb", CBS)
def test_reconstruct_matches_reference(golden, K, cb):
    w = orc.reconstruct_inner(golden[f"recon_in_K{K}_cb{cb}"], K, cb)
    np.testing.assert_array_equal(w.view(np.uint16), golden[f"recon_out_K{K}_cb{cb}"])


@pytest.mark.parametrize("K", KS)
@pytest.mark.parametrize("cb", CBS)
def test_reconstruct_equals_c_restatement(coracle, K, cb):
    rng = np.random.default_rng(K * 10 + cb)
    tr = rng.integers(-32768, 32768, size=(8, 8, 16 * K), dtype=np.int16)
    np.testing.assert_array_equal(orc.reconstruct_inner(tr, K, cb).view(np.uint16),
                                  c_reconstruct(coracle, tr, K, cb).view(np.uint16))


def test_reconstruct_brute_force_one_tile():
    """Element-by-element from the format definition: W[row(t), col(t)] = LUT[window ending at (t+1)K]."""
    K, cb = 3, orc.CB_MCG
    rng = np.random.default_rng(7)
    tile = rng.integers(-32768, 32768, size=(1, 1, 16 * K), dtype=np.int16)
    bits = _stream_bits(tile[0, 0])
    lut = orc.codebook_lut(cb)
    want = np.zeros((16, 16), dtype=np.float16)
    for t in range(256):
        end = (t + 1) * K
        s = 0
        for b in range(end - 16, end):
            s = (s << 1) | int(bits[b % (256 * K)])
        row = 8 * ((t >> 1) & 1) + 2 * ((t >> 3) & 3) + (t & 1)
        col = (t >> 5) + 8 * ((t >> 2) & 1)
        want[row, col] = lut[s]
    np.testing.assert_array_equal(orc.reconstruct_inner(tile, K, cb).view(np.uint16), want.view(np.uint16))


# ---- Hadamard and forward --------------------------------------------------------------------------------------

def test_hadamard_is_textbook_and_involutive(golden):
    h = orc.hadamard128()
    np.testing.assert_array_equal(h * np.sqrt(128), scipy.linalg.hadamard(128))
    np.testing.assert_allclose(h @ h, np.eye(128), atol=1e-12)
    np.testing.assert_allclose(orc.had_rows(golden["had_in"]), golden["had_out"], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("tag", ["lin_a", "lin_b"])
def test_linear_forward_matches_reference(golden, tag):
    k, n, K, cb = golden[f"{tag}_dims"].tolist()
    args = (golden[f"{tag}_x"], golden[f"{tag}_trellis"], golden[f"{tag}_suh"], golden[f"{tag}_svh"], K, cb)
    y = orc.linear_forward(*args)
    ref = golden[f"{tag}_y"]
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()
    y64 = orc.linear_forward(*args, dtype=np.float64)
    assert np.abs(y64 - ref).max() <= 1e-5 * np.abs(ref).max()


def test_weight_orig_matches_reference_and_forward(golden):
    k, n, K, cb = golden["lin_a_dims"].tolist()
    tr, suh, svh, x = (golden[f"lin_a_{s}"] for s in ("trellis", "suh", "svh", "x"))
    w = orc.weight_orig(tr, suh, svh, K, cb)
    np.testing.assert_allclose(w, golden["lin_a_w"], rtol=1e-5, atol=1e-5)
    y = orc.linear_forward(x, tr, suh, svh, K, cb)
    np.testing.assert_allclose(y, x.astype(np.float32) @ w, rtol=2e-4, atol=2e-4)


# ---- MoE and KV-attention restatements -------------------------------------------------------------------------

def _tiny_experts(rng, E, H, I, K, cb, K_down=None):
    def mat(k, n, bits):
        return (rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * bits), dtype=np.int16),
                np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16),
                np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16))
    return [dict(gate=mat(H, I, K), up=mat(H, I, K), down=mat(I, H, K_down or K)) for _ in range(E)]


@pytest.mark.parametrize("K, K_down", [(3, 3), (3, 4), (2, 6)])
def test_moe_forward_equals_original_basis_evaluation(K, K_down):
    """The routed layer against a direct evaluation with the original-basis weights, gate/up and down at their own
    bitrates (the reference runs bits_gate_up and bits_down separately, kernels/reference.py:123-149)."""
    rng = np.random.default_rng(3)
    E, H, I, cb, T, top_k = 4, 128, 128, orc.CB_MCG, 3, 2
    ex = _tiny_experts(rng, E, H, I, K, cb, K_down)
    x = rng.standard_normal((T, H)).astype(np.float16)
    ids = np.array([[0, 2], [3, 0], [1, 2]], dtype=np.int32)
    w = rng.random((T, top_k)).astype(np.float32)
    y = orc.moe_forward(x, ids, w, ex, None, cb)
    if K == K_down:
        assert np.array_equal(y, orc.moe_forward(x, ids, w, ex, K, cb))
    else:
        with pytest.raises(AssertionError):
            orc.moe_forward(x, ids, w, ex, K, cb)
    bits = {"gate": K, "up": K, "down": K_down}
    W = {(e, p): orc.weight_orig(*ex[e][p], bits[p], cb).astype(np.float64) for e in range(E)
         for p in ("gate", "up", "down")}
    want = np.zeros((T, H))
    for t in range(T):
        for j in range(top_k):
            e = ids[t, j]
            g = x[t].astype(np.float64) @ W[e, "gate"]
            u = x[t].astype(np.float64) @ W[e, "up"]
            want[t] += w[t, j] * (((g / (1 + np.exp(-g))) * u) @ W[e, "down"])
    assert np.abs(y - want).max() <= 1e-4 * np.abs(want).max()


def test_moe_align_contract():
    rng = np.random.default_rng(4)
    ids = rng.integers(0, 16, size=(9, 4)).astype(np.int32)
    for block in (1, 4, 8, 16):
        sorted_ids, expert_ids, post = orc.moe_align(ids, block, 16)
        numel = ids.size
        assert post == len(sorted_ids) and post % block == 0 and len(expert_ids) == post // block
        valid = sorted_ids[sorted_ids < numel]
        assert sorted(valid.tolist()) == list(range(numel))
        for i, s in enumerate(sorted_ids):
            if s < numel:
                assert ids.reshape(-1)[s] == expert_ids[i // block]
        assert list(expert_ids) == sorted(expert_ids)


def test_kv_pack4_roundtrip_and_attention_against_contiguous_form():
    rng = np.random.default_rng(5)
    B, Hq, Hkv, D, page, npages = 2, 4, 2, 32, 16, 10
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    kf = rng.standard_normal((npages, Hkv, page, D)).astype(np.float16)
    vf = rng.standard_normal((npages, Hkv, page, D)).astype(np.float16)
    table = np.stack([rng.permutation(npages)[:5] for _ in range(B)]).astype(np.int32)
    lens = np.array([70, 33], dtype=np.int32)
    for bits in (8, 4):
        kq, ks = orc.kv_quantize(kf, bits)
        vq, vs = orc.kv_quantize(vf, bits)
        kc, vc = (orc.kv_pack4(kq), orc.kv_pack4(vq)) if bits == 4 else (kq, vq)
        if bits == 4:
            np.testing.assert_array_equal(orc.kv_unpack4(kc), kq)
        o = orc.kv_decode_attention(q, kc, vc, ks, vs, table, lens, bits, 1 / np.sqrt(D))
        for b in range(B):
            L = lens[b]
            kk = np.concatenate([kq[p].astype(np.float64) * ks[p].astype(np.float64)[:, None, None]
                                 for p in table[b]], axis=1)[:, :L]          # [Hkv, L, D]
            vv = np.concatenate([vq[p].astype(np.float64) * vs[p].astype(np.float64)[:, None, None]
                                 for p in table[b]], axis=1)[:, :L]
            for h in range(Hq):
                s = kk[h // (Hq // Hkv)] @ q[b, h].astype(np.float64) / np.sqrt(D)
                p = np.exp(s - s.max())
                np.testing.assert_allclose(o[b, h], p @ vv[h // (Hq // Hkv)] / p.sum(), rtol=1e-5, atol=1e-6)
        # the quantization is as good as its bit width allows
        err = np.abs(kq.astype(np.float32) * ks.astype(np.float32)[:, :, None, None] - kf).max()
        assert err <= 0.5 * np.abs(kf).max() / (127 if bits == 8 else 7) * 1.01


# ---- the checks catch plausible mistakes -----------------------------------------------------------------------

def test_planted_word_order_mistake_is_caught(golden):
    """int16 pair order reversed (h[2m] << 16 | h[2m+1]) must fail the golden states."""
    t16 = golden["states_in_K4"].copy()
    t16[0::2], t16[1::2] = golden["states_in_K4"][1::2], golden["states_in_K4"][0::2]
    assert not np.array_equal(orc.decode_states(t16, 4), golden["states_out_K4"])


def test_planted_window_end_mistake_is_caught(golden):
    K = 3
    tile = golden["states_in_K3"]
    pos = (orc.state_index(K) + 1) % (256 * K)            # window ending one bit late
    t16 = tile.astype(np.int64) & 0xFFFF
    words = (t16[0::2] | (t16[1::2] << 16)).astype(np.uint32)
    bits = ((words[:, None] >> np.arange(31, -1, -1, dtype=np.uint32)) & 1).reshape(-1)
    wrong = (bits[pos] * (1 << np.arange(15, -1, -1))).sum(-1)
    assert not np.array_equal(wrong, golden["states_out_K3"])


def test_planted_transposed_perm_is_caught(golden):
    perm = orc.tensor_core_perm()
    transposed = (perm % 16) * 16 + perm // 16
    assert not np.array_equal(transposed, golden["perm"])


def test_planted_double_rounding_in_mul1_is_caught(golden):
    s = np.arange(65536, dtype=np.uint64)
    x = (s * orc.MUL1_MULT) & 0xFFFFFFFF
    bsum = (x & 0xFF) + ((x >> 8) & 0xFF) + ((x >> 16) & 0xFF) + ((x >> 24) & 0xFF)
    h = (1024 + bsum).astype(np.float16)
    two_roundings = (h * np.float16(orc._f16_from_bits(0x1EEE))).astype(np.float16) + orc._f16_from_bits(0xC931)
    assert hashlib.sha256(two_roundings.astype(np.float16).view(np.uint16).tobytes()).digest() != \
        golden["lut_sha256_cb2"].tobytes()


# ---- the torch CPU restatement timed as the CPU baseline ---------------------------------------------------------

@pytest.mark.parametrize("K", KS)
@pytest.mark.parametrize("cb", CBS)
def test_torch_cpu_reconstruct_matches_reference(golden, K, cb):
    import torch
    from oracle import torch_cpu
    tr = torch.from_numpy(golden[f"recon_in_K{K}_cb{cb}"])
    w = torch_cpu.reconstruct_inner(tr, K, cb, chunk=3)   # a chunk that does not divide the tile count
    np.testing.assert_array_equal(w.numpy().view(np.uint16), golden[f"recon_out_K{K}_cb{cb}"])


@pytest.mark.parametrize("tag", ["lin_a", "lin_b"])
def test_torch_cpu_linear_forward_matches_reference(golden, tag):
    import torch
    from oracle import torch_cpu
    k, n, K, cb = golden[f"{tag}_dims"].tolist()
    args = [torch.from_numpy(golden[f"{tag}_{p}"]) for p in ("x", "trellis", "suh", "svh")]
    y = torch_cpu.linear_forward(*args, K, cb).numpy()
    ref = golden[f"{tag}_y"]
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("bits", [8, 4])
def test_torch_cpu_kv_attention_matches_oracle(bits):
    import torch
    from oracle import torch_cpu
    rng = np.random.default_rng(bits)
    B, Hq, Hkv, D, npg = 3, 8, 2, 128, 5
    P = B * npg
    kq, ks = orc.kv_quantize(rng.standard_normal((P, Hkv, 16, D)).astype(np.float16), bits)
    vq, vs = orc.kv_quantize(rng.standard_normal((P, Hkv, 16, D)).astype(np.float16), bits)
    if bits == 4:
        kq, vq = orc.kv_pack4(kq), orc.kv_pack4(vq)
    table = rng.permutation(P).astype(np.int32).reshape(B, npg)
    q = rng.standard_normal((B, Hq, D)).astype(np.float16)
    ref = orc.kv_decode_attention(q, kq, vq, ks, vs, table, np.full(B, 16 * npg, np.int32), bits, 0.088)
    T = torch.from_numpy
    k = torch_cpu.kv_dequant(T(kq.view(np.int8)), T(ks), bits)
    v = torch_cpu.kv_dequant(T(vq.view(np.int8)), T(vs), bits)
    got = torch_cpu.decode_attention(T(q), k, v, T(table), 0.088).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)
