"""Engine glue on synthetic checkpoints: SGLang's Exl3Config / Exl3LinearMethod / Exl3MoEMethod and the vLLM
method, with the engines' base classes replaced by the local stand-ins (no engine is installed here).  An engine's
`load_weights` is emulated: each checkpoint tensor goes to the placeholder of its module with the shard id the engine
would pass.  CPU tests cover routing, loading, validation and errors; the `gpu` tests run `apply` through the
library and compare with the oracle (cuda/src/sglang_exl3/sglang_glue/linear.py:66-197, moe.py:54-237,
xpu/exl3xpu/vllm_plugin.py:150-261 define the contracts)."""
import types

import numpy as np
import pytest
import torch

import exl3_ckpt
from trellis_serve_amd.glue import activate, engine, register
from trellis_serve_amd.glue.sglang_config import Exl3Config
from trellis_serve_amd.glue.sglang_linear import Exl3LinearMethod
from trellis_serve_amd.glue.sglang_moe import Exl3MoEMethod
from trellis_serve_amd.glue import vllm_plugin
from trellis_serve_amd.glue.index import CheckpointIndex, module_key
from trellis_serve_amd.glue.stash import MatrixInfo, TensorStash, shard_partitions

SG = engine.SGLANG
L0 = "model.language_model.layers.0"


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    d = tmp_path_factory.mktemp("exl3")
    tensors = exl3_ckpt.tiny_model(seed=5)
    exl3_ckpt.write(str(d), tensors, shards=2)
    return str(d), tensors


def _config(path):
    return Exl3Config.from_config({"hf_config": types.SimpleNamespace(_name_or_path=path)})


def _linear_layer(cfg, prefix, sizes, k, lm_head=False):
    layer = (SG.ParallelLMHead if lm_head else SG.LinearBase)()
    method = cfg.get_quant_method(layer, prefix)
    method.create_weights(layer, k, sizes, k, sum(sizes), torch.float16)
    layer.quant_method = method
    return layer, method


def _feed(layer, tensors, key, shard_id):
    for name, arr in tensors.items():
        if name.rpartition(".")[0] == key:
            suffix = name.rpartition(".")[2]
            param = getattr(layer, suffix)
            param.weight_loader(param, torch.from_numpy(np.array(arr)), shard_id)


def _qkv(cfg, tensors):
    layer, method = _linear_layer(cfg, "model.layers.0.self_attn.qkv_proj", [256, 128, 128], 256)
    for sid in "vqk":   # any delivery order
        _feed(layer, tensors, f"{L0}.self_attn.{sid}_proj", sid)
    method.process_weights_after_loading(layer)
    return layer, method


def test_config_routes_modules(ckpt):
    path, _ = ckpt
    cfg = _config(path)
    assert cfg.get_name() == "exl3" and torch.bfloat16 in cfg.get_supported_act_dtypes()
    assert cfg.override_quantization_method({"quant_method": "exl3"}, None) == "exl3"
    assert cfg.override_quantization_method({"quant_method": "awq"}, None) is None
    m = cfg.get_quant_method(SG.LinearBase(), "model.layers.0.self_attn.qkv_proj")
    assert isinstance(m, Exl3LinearMethod) and [i[:4] for i in m.infos] == [(256, 256, 6, "mcg"), (256, 128, 6, "mcg"),
                                                                             (256, 128, 6, "mcg")]
    assert isinstance(cfg.get_quant_method(SG.LinearBase(), "model.layers.0.self_attn.o_proj"), Exl3LinearMethod)
    assert cfg.index.find("model.layers.0.o_proj") is not None        # `.self_attn.` dropped
    assert isinstance(cfg.get_quant_method(SG.LinearBase(), "model.layers.0.mlp.shared_expert_gate"),
                      SG.UnquantizedLinearMethod)
    head = cfg.get_quant_method(SG.ParallelLMHead(), "lm_head")
    assert isinstance(head, Exl3LinearMethod) and head.infos[0][:4] == (256, 512, 8, "mul1")
    moe = cfg.get_quant_method(SG.FusedMoE(), "model.layers.1.mlp.experts")
    assert isinstance(moe, Exl3MoEMethod) and len(moe.infos) == 3 * exl3_ckpt.N_EXPERTS
    assert cfg.get_quant_method(SG.FusedMoE(), "model.layers.0.mlp.experts") is None
    assert cfg.get_quant_method(torch.nn.LayerNorm(4), "model.norm") is None


def test_linear_loading_and_validation(ckpt):
    path, tensors = ckpt
    cfg = _config(path)
    layer, method = _qkv(cfg, tensors)
    assert layer.exl3_count == 3 and layer.exl3_widths == [256, 128, 128] and layer.exl3_runs == [(0, 3)]
    assert layer.exl3_codebooks == [1, 1, 1] and layer.exl3_bits == [3, 3, 3]
    np.testing.assert_array_equal(layer.exl3_trellis_1.cpu().numpy(), tensors[f"{L0}.self_attn.k_proj.trellis"])
    assert not hasattr(layer, "trellis") and not hasattr(layer, "exl3_stash")
    # legacy packed signs become the +-1 vectors
    o, om = _linear_layer(cfg, "model.layers.0.self_attn.o_proj", [256], 256)
    _feed(o, tensors, f"{L0}.self_attn.o_proj", None)
    om.process_weights_after_loading(o)
    rng_suh = exl3_ckpt.pack_signs(o.exl3_suh_0.cpu().numpy())
    np.testing.assert_array_equal(rng_suh, tensors[f"{L0}.self_attn.o_proj.su"])
    assert set(np.unique(o.exl3_svh_0.cpu().numpy())) <= {-1.0, 1.0}
    # lm_head: a zero-width weight placeholder for the engine
    h, hm = _linear_layer(cfg, "lm_head", [512], 256, lm_head=True)
    assert h.weight.shape == (512, 0)
    _feed(h, tensors, "lm_head", None)
    hm.process_weights_after_loading(h)
    assert h.exl3_codebooks == [2] and h.exl3_bits == [4]


def test_linear_errors(ckpt):
    path, tensors = ckpt
    cfg = _config(path)
    layer, method = _linear_layer(cfg, "model.layers.0.mlp.gate_up_proj", [384, 384], 256)
    _feed(layer, tensors, f"{L0}.mlp.gate_proj", 0)
    with pytest.raises(ValueError, match="a second tensor for shard"):
        _feed(layer, tensors, f"{L0}.mlp.gate_proj", 0)
    with pytest.raises(ValueError, match="expected 2 EXL3 matrices"):
        method.process_weights_after_loading(layer)
    layer, method = _linear_layer(cfg, "model.layers.0.mlp.gate_up_proj", [384, 384], 256)
    _feed(layer, tensors, f"{L0}.mlp.gate_proj", 0)
    _feed(layer, tensors, f"{L0}.mlp.down_proj", 1)       # wrong matrix for shard 1
    with pytest.raises(ValueError, match="the checkpoint header declares"):
        method.process_weights_after_loading(layer)
    with pytest.raises(NotImplementedError, match="tensor-parallel"):
        Exl3LinearMethod("x", [(256, 256, 6, "mcg", False, False)]).create_weights(
            SG.LinearBase(), 128, [256], 256, 256, torch.float16)
    with pytest.raises(NotImplementedError, match="bias"):
        Exl3LinearMethod("x", [(256, 256, 6, "mcg", True, False)]).create_weights(
            SG.LinearBase(), 256, [256], 256, 256, torch.float16)
    with pytest.raises(ValueError, match="mixes EXL3 and unquantized"):
        cfg.index.forget(f"{L0}.mlp.up_proj")
        cfg.get_quant_method(SG.LinearBase(), "model.layers.0.mlp.gate_up_proj")


def _moe_layer(cfg, tensors):
    layer = SG.FusedMoE()
    method = cfg.get_quant_method(layer, "model.layers.1.mlp.experts")
    method.create_weights(layer, exl3_ckpt.N_EXPERTS, exl3_ckpt.H, exl3_ckpt.I_EXPERT, torch.float16)
    method.create_moe_runner(layer, types.SimpleNamespace(activation="silu", is_gated=True,
                                                          apply_router_weight_on_input=False,
                                                          routed_scaling_factor=None, top_k=2))
    for name, arr in tensors.items():
        if ".experts." not in name:
            continue
        key, _, suffix = name.rpartition(".")
        e = int(key.split(".experts.")[1].split(".")[0])
        proj = key.rpartition(".")[2]
        w, sid = ("w2", "w2") if proj == "down_proj" else ("w13", "w1" if proj == "gate_proj" else "w3")
        param = getattr(layer, f"{w}_{suffix}")
        param.weight_loader(param, torch.from_numpy(np.array(arr)), name, shard_id=sid, expert_id=e)
    method.process_weights_after_loading(layer)
    return layer, method


def test_moe_loading(ckpt):
    path, tensors = ckpt
    cfg = _config(path)
    layer, method = _moe_layer(cfg, tensors)
    ex = method.experts(layer)
    E, H, I = exl3_ckpt.N_EXPERTS, exl3_ckpt.H, exl3_ckpt.I_EXPERT
    assert tuple(ex["gate_trellis"].shape) == (E, H // 16, I // 16, 48)
    assert tuple(ex["down_trellis"].shape) == (E, I // 16, H // 16, 48)
    assert tuple(ex["up_suh"].shape) == (E, H) and tuple(ex["down_svh"].shape) == (E, H)
    np.testing.assert_array_equal(ex["up_trellis"][2].cpu().numpy(),
                                  tensors["model.language_model.layers.1.mlp.experts.2.up_proj.trellis"])
    assert layer.exl3_codebook == 1 and layer.exl3_bits == {"gate": 3, "up": 3, "down": 3}
    assert not hasattr(layer, "w13_trellis")
    with pytest.raises(NotImplementedError, match="SiLU"):
        method.create_moe_runner(layer, types.SimpleNamespace(activation="gelu"))
    with pytest.raises(NotImplementedError, match="routed_scaling_factor"):
        method.create_moe_runner(layer, types.SimpleNamespace(activation="silu", routed_scaling_factor=2.5))
    bad = SG.FusedMoE()
    bad.moe_ep_size = 2
    with pytest.raises(NotImplementedError, match="expert-parallel"):
        method.create_weights(bad, E, H, I, torch.float16)
    with pytest.raises(ValueError, match="no EXL3 tensors"):
        method.create_weights(SG.FusedMoE(), E + 1, H, I, torch.float16)


def _vllm_qkv(path, tensors):
    cfg = vllm_plugin.Exl3Config.from_config({"bits": 3, "codebook": "mcg"})
    cfg.maybe_update_config(path)
    layer = engine.VLLM.LinearBase()
    method = cfg.get_quant_method(layer, "model.layers.0.self_attn.qkv_proj")
    method.create_weights(layer, 256, [256, 128, 128], 256, 512, torch.float16)
    for sid in "qkv":
        key = f"{L0}.self_attn.{sid}_proj"
        for suffix in ("trellis", "suh", "svh", "mcg"):
            p = getattr(layer, suffix)
            p.weight_loader(p, torch.from_numpy(np.array(tensors[f"{key}.{suffix}"])), sid)
    method.process_weights_after_loading(layer)
    return layer, method


def test_vllm_method(ckpt):
    path, tensors = ckpt
    layer, method = _vllm_qkv(path, tensors)
    assert layer.exl3_codebooks == [1, 1, 1] and layer.exl3_bits == [3, 3, 3] and layer.exl3_count == 3
    assert layer.exl3_runs == [(0, 3)]
    for i, sid in enumerate("qkv"):
        key = f"{L0}.self_attn.{sid}_proj"
        np.testing.assert_array_equal(getattr(layer, f"exl3_trellis_{i}").cpu().numpy(), tensors[f"{key}.trellis"])
        np.testing.assert_array_equal(getattr(layer, f"exl3_svh_{i}").cpu().numpy(), tensors[f"{key}.svh"])
        assert getattr(layer, f"exl3_trellis_{i}").is_contiguous()
    cfg = vllm_plugin.Exl3Config.from_config({})
    cfg.maybe_update_config(path)
    assert cfg.index.find("lm_head")[:4] == (256, 512, 8, "mul1")
    assert cfg.index.find("language_model.model.layers.0.self_attn.q_proj")[:4] == (256, 256, 6, "mcg")
    assert isinstance(cfg.get_quant_method(engine.VLLM.LinearBase(), "model.layers.0.mlp.foo_proj"),
                      engine.VLLM.UnquantizedLinearMethod)


def test_vllm_declared_format_without_a_local_checkpoint(ckpt):
    """A model directory that is not local: the declared bitrate decides which linears are EXL3 and is checked
    against what arrives; shapes follow the layer, the codebook the checkpoint's marker tensors."""
    path, tensors = ckpt
    cfg = vllm_plugin.Exl3Config.from_config({"bits": 3, "head_bits": 4, "codebook": "mcg"})
    cfg.maybe_update_config("org/not-a-local-dir")
    assert cfg.index is None
    assert cfg.get_quant_method(engine.VLLM.LinearBase(), "model.layers.0.linear_attn.in_proj_ba") is not None
    assert isinstance(cfg.get_quant_method(engine.VLLM.LinearBase(), "model.layers.0.linear_attn.in_proj_ba"),
                      engine.VLLM.UnquantizedLinearMethod)
    assert isinstance(cfg.get_quant_method(engine.VLLM.LinearBase(), "model.visual.blocks.0.attn.qkv"),
                      engine.VLLM.UnquantizedLinearMethod)
    assert cfg.get_quant_method(engine.VLLM.ParallelLMHead(), "lm_head").declared_bits == 4
    layer = engine.VLLM.LinearBase()
    method = cfg.get_quant_method(layer, "model.layers.0.self_attn.qkv_proj")
    assert method.declared_bits == 3 and method.infos is None
    method.create_weights(layer, 256, [256, 128, 128], 256, 512, torch.float16)
    for sid in "qkv":
        key = f"{L0}.self_attn.{sid}_proj"
        for suffix in ("trellis", "suh", "svh", "mcg"):
            p = getattr(layer, suffix)
            p.weight_loader(p, torch.from_numpy(np.array(tensors[f"{key}.{suffix}"])), sid)
    method.process_weights_after_loading(layer)
    assert layer.exl3_codebooks == [1, 1, 1] and layer.exl3_widths == [256, 128, 128]
    # a shard at another bitrate than declared
    cfg4 = vllm_plugin.Exl3Config.from_config({"bits": 4})
    layer = engine.VLLM.LinearBase()
    method = cfg4.get_quant_method(layer, "model.layers.0.self_attn.o_proj")
    method.create_weights(layer, 256, [256], 256, 256, torch.float16)
    for suffix in ("trellis", "su", "sv", "mcg"):
        p = getattr(layer, suffix)
        p.weight_loader(p, torch.from_numpy(np.array(tensors[f"{L0}.self_attn.o_proj.{suffix}"])))
    with pytest.raises(ValueError, match="declares K=4"):
        method.process_weights_after_loading(layer)


def test_checkpoint_index_spellings_and_experts():
    mcg3 = MatrixInfo(256, 256, 6, "mcg")
    idx = CheckpointIndex({
        "model.language_model.layers.2.self_attn.q_proj": mcg3,
        "model.language_model.layers.2.mlp.experts.0.gate_proj": mcg3,
        "model.language_model.layers.2.mlp.experts.0.down_proj": mcg3,
        "model.language_model.layers.2.mlp.experts.11.up_proj": mcg3,
        "mtp.layers.0.mlp.down_proj": mcg3,
        "lm_head": MatrixInfo(256, 512, 8, "mul1"),
    })
    for spelling in ("model.language_model.layers.2.self_attn.q_proj", "model.layers.2.self_attn.q_proj",
                     "model.layers.2.q_proj", "language_model.model.layers.2.self_attn.q_proj"):
        assert idx.find(spelling) == mcg3, spelling
    assert module_key("language_model.model.layers.3.mlp.gate_proj") == "layers.3.mlp.gate_proj"
    assert module_key("model.mtp.layers.0.mlp.up_proj") == "mtp.layers.0.mlp.up_proj"
    assert idx.find("model.layers.0.mlp.down_proj") == mcg3            # a draft's layer 0 is the checkpoint's mtp
    assert idx.find("model.layers.3.q_proj") is None and "lm_head" in idx
    assert idx.find("model.visual.layers.2.q_proj") is None             # towers keep their own prefix
    assert idx.experts("model.layers.2.mlp.experts") == {("gate", 0): mcg3, ("down", 0): mcg3, ("up", 11): mcg3}
    assert idx.linear("model.layers.2.mlp.gate_up_proj") is None
    with pytest.raises(ValueError, match="mixes EXL3 and unquantized"):
        idx.linear("model.layers.2.self_attn.qkv_proj")
    assert idx.linear("model.layers.2.qkv_proj", {"qkv_proj": ["q_proj"]}) == [mcg3]   # the engine's own map
    with pytest.raises(ValueError, match="same module"):
        CheckpointIndex({"model.layers.0.q_proj": mcg3, "model.language_model.layers.0.self_attn.q_proj": mcg3})
    bad = CheckpointIndex({"model.layers.1.mlp.experts.0.w9": mcg3})
    with pytest.raises(ValueError, match="unexpected EXL3 matrix"):
        bad.experts("model.layers.1.mlp.experts")


def test_stash_keys_and_legacy_signs():
    assert shard_partitions(None) == () and shard_partitions("k") == (1,) and shard_partitions([0, "v"]) == (0, 2)
    st = TensorStash("blk", "cpu")
    tr = torch.zeros((16, 8, 48), dtype=torch.int16)
    st.put((1,), "trellis", tr)
    with pytest.raises(ValueError, match="a second tensor"):
        st.put((1,), "trellis", tr)
    with pytest.raises(ValueError, match="not an EXL3 checkpoint suffix"):
        st.put((1,), "weight", tr)
    with pytest.raises(ValueError, match="without suh/svh"):
        st.matrix((1,))
    words = torch.tensor([0x0001, -0x8000], dtype=torch.int16)       # bit 0 of word 0, bit 15 of word 1
    st.put((1,), "su", torch.zeros(16, dtype=torch.int16))
    st.put((1,), "sv", torch.cat([words, torch.zeros(6, dtype=torch.int16)]))
    st.put((1,), "mul1", torch.zeros((), dtype=torch.int32))
    m = st.matrix((1,), MatrixInfo(256, 128, 6, "mul1"))
    assert m.codebook_id == 2 and m.bits == 3 and m.suh.dtype == torch.float16 and bool((m.suh == 1).all())
    sv = m.svh.tolist()
    assert sv[0] == -1 and sv[31] == -1 and sv.count(-1) == 2
    with pytest.raises(ValueError, match="the checkpoint header declares"):
        st.matrix((1,), MatrixInfo(256, 128, 8, "mul1"))


def test_plugin_registration():
    activate()
    register()
    assert engine.SGLANG.QUANTIZATION_METHODS["exl3"] is Exl3Config
    assert engine.VLLM.QUANTIZATION_METHODS["exl3"] is vllm_plugin.Exl3Config


# ------------------------------------------------------------------------------------------------ GPU: apply()

def _rows(rng, n, k):
    return (rng.standard_normal((n, k)) * 0.5).astype(np.float16)


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [1, 7, 160])
def test_sglang_apply_matches_oracle(ckpt, rows):
    from oracle import exl3_oracle as orc
    path, tensors = ckpt
    cfg = _config(path)
    layer, method = _qkv(cfg, tensors)
    x = _rows(np.random.default_rng(rows), rows, 256)
    y = method.apply(layer, torch.from_numpy(x).cuda()).float().cpu().numpy()
    refs = []
    for sid in "qkv":
        key = f"{L0}.self_attn.{sid}_proj"
        refs.append(orc.linear_forward(x, tensors[f"{key}.trellis"], tensors[f"{key}.suh"], tensors[f"{key}.svh"],
                                       3, 1))
    ref = np.concatenate(refs, axis=1).astype(np.float64)
    err = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    print(f"rows={rows}: norm-rel {err:.2e}")
    assert err <= 2e-3 and np.abs(y - ref).max() / np.abs(ref).max() <= 2e-3
    vl, vm = _vllm_qkv(path, tensors)
    assert torch.equal(vm.apply(vl, torch.from_numpy(x).cuda()).cpu(), torch.from_numpy(y).half())


@pytest.mark.gpu
def test_sglang_moe_apply_matches_oracle(ckpt):
    from oracle import exl3_oracle as orc
    path, tensors = ckpt
    cfg = _config(path)
    layer, method = _moe_layer(cfg, tensors)
    T, top_k, E = 6, 2, exl3_ckpt.N_EXPERTS
    rng = np.random.default_rng(8)
    x = _rows(rng, T, exl3_ckpt.H)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    ids = np.argsort(-logits, axis=1)[:, :top_k].astype(np.int32)
    sel = np.take_along_axis(logits, ids, 1)
    w = (np.exp(sel) / np.exp(sel).sum(1, keepdims=True)).astype(np.float32)
    topk = types.SimpleNamespace(topk_ids=torch.from_numpy(ids).cuda(), topk_weights=torch.from_numpy(w).cuda())
    out = method.apply(layer, types.SimpleNamespace(hidden_states=torch.from_numpy(x).cuda(), topk_output=topk))
    y = out.hidden_states.float().cpu().numpy()
    pre = "model.language_model.layers.1.mlp.experts"
    ex = [{p: (tensors[f"{pre}.{e}.{p}_proj.trellis"], tensors[f"{pre}.{e}.{p}_proj.suh"],
               tensors[f"{pre}.{e}.{p}_proj.svh"]) for p in ("gate", "up", "down")} for e in range(E)]
    ref = orc.moe_forward(x, ids, w, ex, 3, 1)
    err = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    print(f"moe via glue: norm-rel {err:.2e}")
    assert err <= 2e-3
