"""torch CPU restatement of the reference's CPU path -- TEST INFRASTRUCTURE ONLY (the timed CPU baseline).

Only `tests/` and `bench.py`'s `cpu_baseline` leg may import this module.  It is the CPU path of trellis_core
(core/src/trellis_core/reference.py:80-153) restated step for step in torch, so that its timing on the host cores is
the reference's own CPU algorithm, multithreaded by torch:
  decode_states       bits of the tile's 8K little-endian words expanded MSB first, the 16-bit window of every
                      state gathered and weighted (reference.py:80-99);
  reconstruct_inner   states -> fp16 through the 65536-entry codebook table, scattered into the 16x16 tile order,
                      tiles laid out as the k x n matrix (reference.py:102-115);
  had_rows / linear_forward   fp32 Hadamard matmuls in blocks of 128 and the fp32 GEMM (reference.py:118-153).
The tables (window positions, tile order, codebook values) come from oracle/exl3_oracle.py, where they are pinned
against the reference's golden vectors; tests/test_oracle.py checks every function here against that module.
"""
from __future__ import annotations

from functools import lru_cache

import numpy as np
import torch

from . import exl3_oracle as orc


@lru_cache
def _window_positions(K: int) -> torch.Tensor:
    return torch.from_numpy(orc.state_index(K).astype(np.int64))


@lru_cache
def _tile_order() -> torch.Tensor:
    return torch.from_numpy(orc.tensor_core_perm().astype(np.int64))


@lru_cache
def _codebook(cb: int) -> torch.Tensor:
    return torch.from_numpy(orc.codebook_lut(cb).view(np.float16).copy())


@lru_cache
def _hadamard() -> torch.Tensor:
    return torch.from_numpy(orc.hadamard128().astype(np.float32))


_MSB_FIRST = torch.arange(31, -1, -1, dtype=torch.int64)
_WINDOW_WEIGHTS = torch.tensor([1 << (15 - i) for i in range(16)], dtype=torch.int64)


def decode_states(tiles: torch.Tensor, K: int) -> torch.Tensor:
    """int16 [T, 16K] -> int32 states [T, 256] in stream order."""
    h = tiles.to(torch.int64) & 0xFFFF
    words = h[:, 0::2] | (h[:, 1::2] << 16)                                   # [T, 8K]
    stream = ((words[:, :, None] >> _MSB_FIRST) & 1).reshape(tiles.shape[0], -1)  # [T, 256K] bits
    windows = stream[:, _window_positions(K)]                                  # [T, 256, 16]
    return (windows * _WINDOW_WEIGHTS).sum(-1).to(torch.int32)


def reconstruct_inner(trellis: torch.Tensor, K: int, cb: int, chunk: int = 4096) -> torch.Tensor:
    """int16 [k/16, n/16, 16K] -> W_inner fp16 [k, n]."""
    tk, tn, _ = trellis.shape
    flat = trellis.reshape(tk * tn, 16 * K)
    lut, order = _codebook(cb), _tile_order()
    tiles = torch.empty((tk * tn, 256), dtype=torch.float16)
    for s in range(0, tk * tn, chunk):
        vals = lut[decode_states(flat[s:s + chunk], K).long()]
        tiles[s:s + chunk, order] = vals
    return tiles.view(tk, tn, 16, 16).permute(0, 2, 1, 3).reshape(tk * 16, tn * 16)


def had_rows(x: torch.Tensor) -> torch.Tensor:
    """H128 on the last dim in blocks of 128, fp32."""
    return (x.float().reshape(-1, 128) @ _hadamard()).reshape(x.shape)


def linear_from_inner(x: torch.Tensor, w_inner: torch.Tensor, suh: torch.Tensor, svh: torch.Tensor) -> torch.Tensor:
    """y = had(had(x * suh) @ W_inner) * svh in fp32 (the matmul half of reference.py:145-153)."""
    xh = had_rows(x.float() * suh.float())
    return had_rows(xh @ w_inner.float()) * svh.float()


def linear_forward(x, trellis, suh, svh, K: int, cb: int) -> torch.Tensor:
    return linear_from_inner(x, reconstruct_inner(trellis, K, cb), suh, svh)


def kv_dequant(codes: torch.Tensor, scales: torch.Tensor, bits: int) -> torch.Tensor:
    """Closed-form dequant of a paged cache: int8 codes [P, H, 16, D] (4-bit: two per byte, low nibble first) times
    the per-(page, head) fp16 scale -> fp32 [P, H, 16, D]."""
    if bits == 4:
        lo = ((codes.to(torch.int16) & 0xF) ^ 8) - 8
        hi = (((codes.to(torch.int16) >> 4) & 0xF) ^ 8) - 8
        codes = torch.stack([lo, hi], dim=-1).flatten(-2)
    return codes.float() * scales.float()[:, :, None, None]


def decode_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, page_table: torch.Tensor, sm_scale: float,
                     ) -> torch.Tensor:
    """fp32 single-query attention of every sequence over its pages: q [B, Hq, D], k/v [P, Hkv, 16, D] dequantized,
    page_table [B, pages] (all sequences full length).  GQA: query head h reads kv head h // (Hq / Hkv)."""
    B, Hq, D = q.shape
    Hkv = k.shape[1]
    g = Hq // Hkv
    out = torch.empty((B, Hq, D), dtype=torch.float32)
    for b in range(B):
        kb = k[page_table[b].long()].permute(1, 0, 2, 3).reshape(Hkv, -1, D)   # [Hkv, L, D]
        vb = v[page_table[b].long()].permute(1, 0, 2, 3).reshape(Hkv, -1, D)
        qb = q[b].float().view(Hkv, g, D)
        p = torch.softmax((qb @ kb.transpose(1, 2)) * sm_scale, dim=-1)         # [Hkv, g, L]
        out[b] = (p @ vb).reshape(Hq, D)
    return out
