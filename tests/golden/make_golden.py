"""Writes tests/golden/exl3_golden.npz from the reference decoder itself (trellis_core, imported from the read-only
reference checkout).  Run in the build container only -- the reference never travels:

    python tests/golden/make_golden.py /root/reference/core/src

Inputs are stored explicitly (not seeds), so the fixture does not depend on torch's RNG streams.  What it pins
(functions no closed form in the tests fully pins): decode_states' word/bit order (reference.py:90-99),
reconstruct_inner's permute (102-115), codebook_lut's rounding of every state (52-73, as a sha256 of the full
LUT plus sampled entries), had_rows (126-130), weight_orig / linear_forward (133-153).
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np


def main(src: str) -> None:
    sys.path.insert(0, src)
    import torch
    from trellis_core import reference as ref

    rng = np.random.default_rng(20261201)
    out: dict[str, np.ndarray] = {}

    # codebooks: sha256 of each full LUT + 2048 sampled states
    sample = np.sort(rng.choice(65536, size=2048, replace=False)).astype(np.int64)
    sample[:6] = [0, 1, 0xB38D, 0x7FFF, 0xFFFF, 12345]
    out["lut_sample_states"] = sample
    for cb in (0, 1, 2):
        lut = ref.codebook_lut(cb).numpy().view(np.uint16)
        out[f"lut_sha256_cb{cb}"] = np.frombuffer(hashlib.sha256(lut.tobytes()).digest(), dtype=np.uint8)
        out[f"lut_sample_cb{cb}"] = lut[sample]

    out["perm"] = np.array(ref.tensor_core_perm(), dtype=np.int64)

    # decode_states on one tile per K, and reconstruct_inner on 2x3 tiles per (K, codebook)
    for K in (2, 3, 4, 5, 6, 8):
        tile = rng.integers(-32768, 32768, size=(16 * K,), dtype=np.int16)
        out[f"states_in_K{K}"] = tile
        out[f"states_out_K{K}"] = ref.decode_states(torch.from_numpy(tile.copy()), K).numpy().astype(np.uint32)
        for cb in (0, 1, 2):
            tr = rng.integers(-32768, 32768, size=(2, 3, 16 * K), dtype=np.int16)
            w = ref.reconstruct_inner(torch.from_numpy(tr.copy()), K, cb).numpy()
            out[f"recon_in_K{K}_cb{cb}"] = tr
            out[f"recon_out_K{K}_cb{cb}"] = w.view(np.uint16)

    # Hadamard rows
    xr = rng.standard_normal((3, 256)).astype(np.float32)
    out["had_in"] = xr
    out["had_out"] = ref.had_rows(torch.from_numpy(xr.copy())).numpy()

    # one linear, the shape of core/tests/test_reference.py:33-43 (k=256, n=128, K=3, mul1) and one 3INST K=4
    for tag, (k, n, K, cb) in {"lin_a": (256, 128, 3, 2), "lin_b": (256, 256, 4, 0)}.items():
        tr = rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * K), dtype=np.int16)
        suh = np.where(rng.random(k) < 0.5, -1.0, 1.0).astype(np.float16)
        svh = (rng.standard_normal(n) * 0.1).astype(np.float16)
        x = rng.standard_normal((4, k)).astype(np.float16)
        T = lambda a: torch.from_numpy(a.copy())
        out[f"{tag}_dims"] = np.array([k, n, K, cb], dtype=np.int64)
        out[f"{tag}_trellis"], out[f"{tag}_suh"], out[f"{tag}_svh"], out[f"{tag}_x"] = tr, suh, svh, x
        out[f"{tag}_y"] = ref.linear_forward(T(x), T(tr), T(suh), T(svh), K, cb).numpy()
        if tag == "lin_a":
            out[f"{tag}_w"] = ref.weight_orig(T(tr), T(suh), T(svh), K, cb).numpy()

    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "exl3_golden.npz")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst}: {len(out)} arrays, {os.path.getsize(dst)} bytes")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/core/src")
