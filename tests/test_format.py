"""The checkpoint format layer (trellis_serve_amd.format): tensor specs, safetensors headers and data, manifest,
fused layouts.  The first five tests restate the reference's own cases (core/tests/test_format.py:21-64) against
this implementation; the rest cover the manifest rules of core/src/trellis_core/format/manifest.py:68-170 on
synthetic checkpoints written with the `safetensors` package."""
import json
import os
import struct

import numpy as np
import pytest

from trellis_serve_amd.format import (BitsK, Codebook, FormatError, FusionKind, TensorInfo, build_matrix_spec,
                                      load_manifest, make_layout, parse_header, read_header, read_tensor)

import exl3_ckpt


def _linear(k, n, words, marker="mul1", legacy=False):
    t = {"trellis": TensorInfo("m.trellis", "I16", (k // 16, n // 16, words))}
    if legacy:
        t["su"], t["sv"] = TensorInfo("m.su", "I16", (k // 16,)), TensorInfo("m.sv", "I16", (n // 16,))
    else:
        t["suh"], t["svh"] = TensorInfo("m.suh", "F16", (k,)), TensorInfo("m.svh", "F16", (n,))
    if marker:
        t[marker] = TensorInfo(f"m.{marker}", "I32", ())
    return t


def test_spec_reads_bits_and_codebook_from_shapes():
    spec = build_matrix_spec("m", _linear(256, 512, 48))
    assert (spec.k, spec.n, spec.bits.value, spec.codebook) == (256, 512, 3.0, Codebook.MUL1)
    assert build_matrix_spec("m", _linear(256, 512, 64, "mcg")).codebook is Codebook.MCG
    assert build_matrix_spec("m", _linear(256, 512, 64, None)).codebook is Codebook.INST3
    assert [c.abi_id for c in (Codebook.INST3, Codebook.MCG, Codebook.MUL1)] == [0, 1, 2]


def test_half_bitrates_need_mul1():
    assert build_matrix_spec("m", _linear(128, 128, 40)).bits == BitsK(5)
    with pytest.raises(FormatError, match="requires the mul1 codebook"):
        build_matrix_spec("m", _linear(128, 128, 40, "mcg"))
    with pytest.raises(FormatError, match="not defined"):
        build_matrix_spec("m", _linear(128, 128, 72))          # K = 4.5
    with pytest.raises(FormatError, match="not a valid EXL3 bitrate"):
        build_matrix_spec("m", _linear(128, 128, 12))


def test_rejects_broken_linears():
    t = _linear(128, 128, 32)
    del t["suh"]
    with pytest.raises(FormatError, match="expected exactly one of"):
        build_matrix_spec("m", t)
    with pytest.raises(FormatError, match="not multiples of 128"):
        build_matrix_spec("m", _linear(144, 128, 32))
    t = _linear(128, 128, 32)
    t["extra"] = TensorInfo("m.extra", "F16", (1,))
    with pytest.raises(FormatError, match="unknown tensors"):
        build_matrix_spec("m", t)


def test_header_parser_reads_names_shapes_and_sizes():
    doc = {"__metadata__": {"format": "pt"},
           "m.trellis": {"dtype": "I16", "shape": [8, 8, 48], "data_offsets": [0, 6144]},
           "m.suh": {"dtype": "F16", "shape": [128], "data_offsets": [6144, 6400]}}
    h = parse_header(json.dumps(doc).encode(), "shard.safetensors")
    assert h.metadata == {"format": "pt"}
    assert h.tensors["m.trellis"].shape == (8, 8, 48) and h.tensors["m.trellis"].nbytes == 6144
    assert struct.calcsize("<Q") == 8


def test_header_parser_rejects_a_reversed_byte_range():
    parsed = parse_header(json.dumps({"w": {"dtype": "F16", "shape": [0], "data_offsets": [4, 4]}}).encode(), "s")
    assert parsed.tensors["w"].nbytes == 0
    with pytest.raises(FormatError, match="reversed"):
        parse_header(json.dumps({"w": {"dtype": "F16", "shape": [2], "data_offsets": [10, 4]}}).encode(), "s")


def test_more_spec_rules():
    spec = build_matrix_spec("m", _linear(256, 128, 32, None, legacy=True))
    assert spec.legacy_signs and spec.bits.value == 2.0
    t = _linear(256, 128, 32, None)
    t["sv"] = TensorInfo("m.sv", "I16", (8,))
    del t["svh"]
    with pytest.raises(FormatError, match="mixed legacy/modern"):
        build_matrix_spec("m", t)
    t = _linear(256, 128, 32, "mcg")
    t["mul1"] = TensorInfo("m.mul1", "I32", ())
    with pytest.raises(FormatError, match="both .mcg and .mul1"):
        build_matrix_spec("m", t)
    t = _linear(256, 128, 32)
    t["svh"] = TensorInfo("m.svh", "F32", (128,))
    with pytest.raises(FormatError, match="expected F16"):
        build_matrix_spec("m", t)
    t = _linear(256, 128, 32)
    t["bias"] = TensorInfo("m.bias", "F32", (128,))
    assert build_matrix_spec("m", t).has_bias
    t["bias"] = TensorInfo("m.bias", "F32", (256,))
    with pytest.raises(FormatError, match="bias"):
        build_matrix_spec("m", t)
    with pytest.raises(FormatError, match="no .trellis"):
        build_matrix_spec("m", {"suh": TensorInfo("m.suh", "F16", (128,))})


def test_header_reader_on_files(tmp_path):
    p = tmp_path / "x.safetensors"
    p.write_bytes(b"\x01")
    with pytest.raises(FormatError, match="too short"):
        read_header(p)
    p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(FormatError, match="implausible"):
        read_header(p)
    p.write_bytes(struct.pack("<Q", 100) + b"{}")
    with pytest.raises(FormatError, match="truncated"):
        read_header(p)
    p.write_bytes(struct.pack("<Q", 3) + b"{x}")
    with pytest.raises(FormatError, match="not valid JSON"):
        read_header(p)


def test_manifest_of_a_synthetic_checkpoint_and_tensor_data(tmp_path):
    tensors = exl3_ckpt.tiny_model(seed=1)
    exl3_ckpt.write(str(tmp_path), tensors, shards=3)
    man = load_manifest(tmp_path)
    q = "model.language_model.layers.0.self_attn.q_proj"
    assert man.is_quantized(q) and not man.is_quantized("model.language_model.norm")
    assert (man.matrices[q].k, man.matrices[q].n, man.matrices[q].bits.value, man.matrices[q].codebook) == \
        (256, 256, 3.0, Codebook.MCG)
    assert man.matrices["lm_head"].codebook is Codebook.MUL1 and man.matrices["lm_head"].bits.value == 4.0
    assert man.matrices["model.language_model.layers.0.self_attn.o_proj"].legacy_signs
    assert len(man.children("model.language_model.layers.1.mlp.experts")) == 3 * exl3_ckpt.N_EXPERTS
    assert set(man.unquantized) == {"model.language_model.norm.weight", "model.language_model.embed_tokens.weight"}
    s = man.summary()
    assert s["quantized_linears"] == 7 + 3 * exl3_ckpt.N_EXPERTS + 1
    assert s["by_bits_codebook"] == {"K=3 mcg": 19, "K=4 mul1": 1} and s["legacy_sign_linears"] == 1
    assert s["declared"]["codebook"] == "mcg"
    assert any("codebook='mcg'" in w for w in man.warnings)          # the lm_head is mul1
    assert s["quantized_bytes"] == sum(v.nbytes for k, v in tensors.items() if ".norm." not in k
                                       and "embed_tokens" not in k)
    # the raw data reader returns exactly what was written
    for name in (f"{q}.trellis", f"{q}.suh", f"{q}.mcg", "model.language_model.layers.0.self_attn.o_proj.su"):
        key, _, suffix = name.rpartition(".")
        info = man.matrices[key].tensors[suffix]
        np.testing.assert_array_equal(read_tensor(tmp_path, info), tensors[name])
    assert read_tensor(tmp_path, man.unquantized["model.language_model.norm.weight"]).dtype == np.float16


def test_manifest_index_rules(tmp_path):
    tensors = exl3_ckpt.tiny_model(seed=2)
    exl3_ckpt.write(str(tmp_path), tensors, shards=2)
    idx = json.loads((tmp_path / "model.safetensors.index.json").read_text())
    # a tensor listed in the index but absent from every shard
    idx2 = dict(idx, weight_map=dict(idx["weight_map"], **{"ghost.weight": "model-00001-of-00002.safetensors"}))
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(idx2))
    with pytest.raises(FormatError, match="in no shard"):
        load_manifest(tmp_path)
    # a tensor present but not in the index: a warning
    wm = dict(idx["weight_map"])
    wm.pop("model.language_model.norm.weight")
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(dict(idx, weight_map=wm)))
    assert any("not in model.safetensors.index.json" in w for w in load_manifest(tmp_path).warnings)


def test_manifest_duplicates_nesting_and_quant_method(tmp_path):
    from safetensors.numpy import save_file
    d = tmp_path / "dup"
    tensors = exl3_ckpt.tiny_model(seed=3)
    exl3_ckpt.write(str(d), tensors, shards=2)
    # the same tensor stored again in a third shard: the index arbitrates
    save_file({"model.language_model.norm.weight": np.zeros(exl3_ckpt.H, np.float16)},
              str(d / "model-extra.safetensors"))
    man = load_manifest(d)
    assert any("more than one shard" in w for w in man.warnings)
    owner = json.loads((d / "model.safetensors.index.json").read_text())["weight_map"][
        "model.language_model.norm.weight"]
    assert man.unquantized["model.language_model.norm.weight"].file == owner
    # nothing may live below a quantized linear
    n = tmp_path / "nested"
    t = exl3_ckpt.linear(np.random.default_rng(0), "m.proj", 128, 128, 3, "mcg")
    t["m.proj.rank0.trellis"] = t["m.proj.trellis"].copy()
    exl3_ckpt.write(str(n), t, shards=1, index=False)
    with pytest.raises(FormatError, match="nested under EXL3 linear"):
        load_manifest(n)
    # config.json must declare exl3 if it declares anything
    w = tmp_path / "wrong"
    exl3_ckpt.write(str(w), exl3_ckpt.linear(np.random.default_rng(0), "m.proj", 128, 128, 3, "mcg"), shards=1,
                    quant_config={"quant_method": "gptq"})
    with pytest.raises(FormatError, match="not 'exl3'"):
        load_manifest(w)
    with pytest.raises(FormatError, match="no .safetensors"):
        load_manifest(tmp_path / "missing_dir_is_empty")


def test_manifest_keeps_ngram_tables_apart(tmp_path):
    from safetensors.numpy import save_file
    exl3_ckpt.write(str(tmp_path), exl3_ckpt.linear(np.random.default_rng(0), "m.proj", 128, 128, 3, "mcg"),
                    shards=1, index=False)
    save_file({"ngram.trellis": np.zeros((4, 48), np.int16)}, str(tmp_path / "ngram.safetensors"),
              metadata={"format": "exl3_ngram_trellis"})
    man = load_manifest(tmp_path)
    assert len(man.ngram_tables) == 1 and man.ngram_tables[0].nbytes == 4 * 48 * 2
    assert list(man.matrices) == ["m.proj"]


def test_fused_layouts(tmp_path):
    exl3_ckpt.write(str(tmp_path), exl3_ckpt.tiny_model(seed=4), shards=1)
    man = load_manifest(tmp_path)
    a = "model.language_model.layers.0.self_attn"
    specs = [man.matrices[f"{a}.{p}_proj"] for p in "qkv"]
    lay = make_layout(["q", "k", "v"], specs, [256, 128, 128])
    assert lay.in_width == 256 and lay.out_width == 512 and lay.spans() == [(0, 256), (256, 128), (384, 128)]
    assert lay.best_fusion is FusionKind.SHARD_MAP and lay.launch_runs() == [(0, 3)]
    m = "model.language_model.layers.0.mlp"
    gu = make_layout([0, 1], [man.matrices[f"{m}.gate_proj"], man.matrices[f"{m}.up_proj"]], [384, 384])
    assert gu.best_fusion is FusionKind.UNIFORM
    assert make_layout([None], [man.matrices["lm_head"]], [500]).launch_runs() == [(0, 1)]
    with pytest.raises(ValueError, match="share their input width"):
        make_layout([0, 1], [man.matrices[f"{m}.gate_proj"], man.matrices[f"{m}.down_proj"]], [384, 256])
    with pytest.raises(ValueError, match="does not fit"):
        make_layout([0], [man.matrices[f"{m}.gate_proj"]], [400])
    assert os.path.isdir(tmp_path)
