"""Synthetic EXL3 checkpoints for the format and glue tests: seeded trellis codes, +-1 sign vectors (or legacy packed
sign bits), codebook markers, written as safetensors shards with an index and config.json.  No checkpoint exists in
this environment, so every checkpoint test runs on these."""
from __future__ import annotations

import json
import os

import numpy as np
from safetensors.numpy import save_file

H, I_DENSE, I_EXPERT, N_EXPERTS, VOCAB = 256, 384, 128, 4, 512
PREFIX = "model.language_model.layers"


def signs(rng, n: int) -> np.ndarray:
    return np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float16)


def pack_signs(s: np.ndarray) -> np.ndarray:
    """fp16 +-1 [16 w] -> legacy int16 words: bit i of word w set when element 16 w + i is -1."""
    bits = (s.reshape(-1, 16) < 0).astype(np.uint32)
    words = (bits << np.arange(16, dtype=np.uint32)).sum(axis=1).astype(np.uint32)
    return words.astype(np.uint16).view(np.int16)


def linear(rng, key: str, k: int, n: int, K: int, codebook: str, legacy: bool = False) -> dict[str, np.ndarray]:
    t = {f"{key}.trellis": rng.integers(-32768, 32768, size=(k // 16, n // 16, 16 * K), dtype=np.int16)}
    suh, svh = signs(rng, k), signs(rng, n)
    if legacy:
        t[f"{key}.su"], t[f"{key}.sv"] = pack_signs(suh), pack_signs(svh)
    else:
        t[f"{key}.suh"], t[f"{key}.svh"] = suh, svh
    if codebook != "3inst":
        t[f"{key}.{codebook}"] = np.array(0, dtype=np.int32)
    return t


def tiny_model(seed: int = 0, K: int = 3, codebook: str = "mcg") -> dict[str, np.ndarray]:
    """Layer 0: attention q/k/v/o (o_proj with legacy signs) and a dense MLP; layer 1: 4 routed experts; an lm_head
    at K = 4 MUL1; unquantized norm and embedding."""
    rng = np.random.default_rng(seed)
    t: dict[str, np.ndarray] = {}
    a = f"{PREFIX}.0.self_attn"
    t |= linear(rng, f"{a}.q_proj", H, 256, K, codebook)
    t |= linear(rng, f"{a}.k_proj", H, 128, K, codebook)
    t |= linear(rng, f"{a}.v_proj", H, 128, K, codebook)
    t |= linear(rng, f"{a}.o_proj", 256, H, K, codebook, legacy=True)
    m = f"{PREFIX}.0.mlp"
    t |= linear(rng, f"{m}.gate_proj", H, I_DENSE, K, codebook)
    t |= linear(rng, f"{m}.up_proj", H, I_DENSE, K, codebook)
    t |= linear(rng, f"{m}.down_proj", I_DENSE, H, K, codebook)
    for e in range(N_EXPERTS):
        x = f"{PREFIX}.1.mlp.experts.{e}"
        t |= linear(rng, f"{x}.gate_proj", H, I_EXPERT, K, codebook)
        t |= linear(rng, f"{x}.up_proj", H, I_EXPERT, K, codebook)
        t |= linear(rng, f"{x}.down_proj", I_EXPERT, H, K, codebook)
    t |= linear(rng, "lm_head", H, VOCAB, 4, "mul1")
    t["model.language_model.norm.weight"] = np.ones(H, dtype=np.float16)
    t["model.language_model.embed_tokens.weight"] = rng.standard_normal((VOCAB, H)).astype(np.float16)
    return t


def write(model_dir: str, tensors: dict[str, np.ndarray], shards: int = 2, quant_config: dict | None = None,
          index: bool = True) -> None:
    """Splits `tensors` over `shards` files (module-sorted, round robin by module key), writes the index and a
    config.json with `quantization_config`."""
    os.makedirs(model_dir, exist_ok=True)
    names = sorted(tensors)
    parts: list[dict[str, np.ndarray]] = [{} for _ in range(shards)]
    modules = sorted({n.rpartition(".")[0] for n in names})
    owner = {mod: i % shards for i, mod in enumerate(modules)}
    for n in names:
        parts[owner[n.rpartition(".")[0]]][n] = np.ascontiguousarray(tensors[n])
    weight_map = {}
    for i, part in enumerate(parts):
        fname = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
        save_file(part, os.path.join(model_dir, fname), metadata={"format": "pt"})
        weight_map.update({n: fname for n in part})
    if index:
        with open(os.path.join(model_dir, "model.safetensors.index.json"), "w") as f:
            json.dump({"metadata": {}, "weight_map": weight_map}, f)
    qc = {"quant_method": "exl3", "version": "0.0.7", "bits": 3.0, "head_bits": 4, "codebook": "mcg"}
    qc.update(quant_config or {})
    with open(os.path.join(model_dir, "config.json"), "w") as f:
        json.dump({"architectures": ["Tiny"], "quantization_config": qc}, f)
