"""`Exl3MoEMethod`: EXL3 routed experts for SGLang's FusedMoE, running on `exl3_moe_forward`.

The engine calls (contract of cuda/src/sglang_exl3/sglang_glue/moe.py:54-237):
  create_weights(layer, num_experts, hidden_size, intermediate_size_per_partition, params_dtype, **extra)
        placeholders `w13_<suffix>` (gate = shard w1, up = shard w3) and `w2_<suffix>` (down) for every checkpoint
        suffix; the model's `load_weights` calls `weight_loader(param, tensor, name, shard_id=, expert_id=)`, which
        stashes the tensor on the CPU under (role, expert).  Tensor / expert parallelism, fused shared experts and
        bias raise NotImplementedError.
  create_moe_runner     SiLU-gated experts only, no routed scaling, router weights not applied on the input.
  process_weights_after_loading
        every expert matrix checked against the headers, then stacked into the [E, ...] tensors the MoE kernel
        reads, moved to the GPU once per layer.
  apply(layer, dispatch_output) -> StandardCombineInput(hidden_states=y); topk_ids [T, top_k] int32|int64,
        topk_weights [T, top_k] fp32.
Gate/up and down may differ in bitrate; gate and up share one (they run as one fused launch).
"""
from __future__ import annotations

import functools
import logging

import torch

from .engine import SGLANG, target_device
from .index import EXPERT_ROLES
from .resident import ResidentExperts
from .stash import SUFFIXES, MatrixInfo, TensorStash, attach_placeholders, detach_placeholders

logger = logging.getLogger(__name__)

ROLE_OF_SHARD = {"w1": "gate", "w3": "up", "w2": "down"}
PLACEHOLDERS = tuple(f"{w}_{s}" for w in ("w13", "w2") for s in SUFFIXES)


def _deliver(stash: TensorStash, name: str, param, loaded_weight, weight_name=None, shard_id=None, expert_id=None,
             *args, **kwargs) -> None:
    """The placeholders' weight_loader: FusedMoE's (param, tensor, name, shard_id, expert_id) call."""
    role = ROLE_OF_SHARD.get(shard_id)
    if role is None or expert_id is None:
        raise ValueError(f"{stash.owner}.{name}: unexpected expert shard {shard_id!r} / expert {expert_id!r}")
    stash.put((role, int(expert_id)), name.partition("_")[2], loaded_weight)


class Exl3MoEMethod(SGLANG.FusedMoEMethodBase):
    def __init__(self, config, prefix: str, experts: dict):
        self.config = config
        self.prefix = prefix
        self.runner = None             # FusedMoE reads quant_method.runner; no MoE runner is used
        self.moe_runner_config = None
        self.infos: dict[tuple[str, int], MatrixInfo] = {key: MatrixInfo(*i) for key, i in experts.items()}

    def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition, params_dtype,
                       **extra_weight_attrs):
        if getattr(layer, "moe_tp_size", 1) != 1 or getattr(layer, "moe_ep_size", 1) != 1:
            raise NotImplementedError(f"{self.prefix}: tensor/expert-parallel EXL3 MoE is not implemented")
        if getattr(layer, "num_fused_shared_experts", 0):
            raise NotImplementedError(f"{self.prefix}: fused shared experts are not supported "
                                      f"(run with --disable-shared-experts-fusion)")
        wanted = [(role, e) for role in EXPERT_ROLES for e in range(num_experts)]
        absent = [w for w in wanted if w not in self.infos]
        if absent:
            raise ValueError(f"{self.prefix}: the checkpoint has no EXL3 tensors for {len(absent)} of {len(wanted)} "
                             f"expert matrices, e.g. {absent[0]}")
        if extra_weight_attrs.get("with_bias") or any(self.infos[w].has_bias for w in wanted):
            raise NotImplementedError(f"{self.prefix}: EXL3 experts with bias are not implemented")
        layer.exl3_geometry = (num_experts, hidden_size, intermediate_size_per_partition)
        # CPU until every expert is in: the GPU receives one stacked tensor per projection and part
        layer.exl3_stash = TensorStash(self.prefix, "cpu")
        attach_placeholders(layer, PLACEHOLDERS, lambda n: functools.partial(_deliver, layer.exl3_stash, n),
                            SGLANG.set_weight_attrs)

    def create_moe_runner(self, layer, moe_runner_config):
        cfg = moe_runner_config
        self.moe_runner_config = cfg
        refused = [
            (getattr(cfg, "activation", "silu") != "silu" or not getattr(cfg, "is_gated", True),
             f"only SiLU-gated experts are implemented (got {getattr(cfg, 'activation', None)})"),
            (getattr(cfg, "apply_router_weight_on_input", False), "apply_router_weight_on_input is not supported"),
            (getattr(cfg, "routed_scaling_factor", None) not in (None, 1.0),
             f"routed_scaling_factor {getattr(cfg, 'routed_scaling_factor', None)} is not supported"),
            (getattr(cfg, "num_fused_shared_experts", 0), "fused shared experts are not supported"),
        ]
        for bad, why in refused:
            if bad:
                raise NotImplementedError(f"{self.prefix}: {why}")

    def process_weights_after_loading(self, layer) -> None:
        E, H, I = layer.exl3_geometry
        stash: TensorStash = layer.exl3_stash
        per_role = {role: [stash.matrix((role, e), self.infos[(role, e)]) for e in range(E)] for role in EXPERT_ROLES}
        for role, mats in per_role.items():
            if len({m.trellis.shape for m in mats}) != 1:
                raise NotImplementedError(f"{self.prefix}: the experts of {role}_proj differ in shape / bitrate")
        codebooks = {m.codebook for mats in per_role.values() for m in mats}
        if len(codebooks) != 1:
            raise NotImplementedError(f"{self.prefix}: mixed codebooks {sorted(codebooks)}")
        gate, up, down = (per_role[r][0] for r in EXPERT_ROLES)
        if gate.bits != up.bits:
            raise NotImplementedError(f"{self.prefix}: gate and up bitrates differ ({gate.bits}, {up.bits})")
        if (gate.k, gate.n, up.k, up.n, down.k, down.n) != (H, I, H, I, I, H):
            raise ValueError(f"{self.prefix}: expert shapes gate {gate.k}x{gate.n}, up {up.k}x{up.n}, down "
                             f"{down.k}x{down.n} do not fit hidden {H}, intermediate {I}")
        detach_placeholders(layer, PLACEHOLDERS)
        stash.clear()
        del layer.exl3_stash
        top_k = getattr(self.moe_runner_config, "top_k", None) or 8
        ResidentExperts.install(layer, per_role, top_k, target_device())
        logger.info("%s: %d experts, K gate/up %d down %d, codebook %s", self.prefix, E, gate.bits, down.bits,
                    gate.codebook)

    def experts(self, layer) -> dict[str, torch.Tensor]:
        return ResidentExperts.tensors(layer)

    def apply(self, layer, dispatch_output):
        x = dispatch_output.hidden_states
        topk = dispatch_output.topk_output
        flat = x.reshape(-1, x.shape[-1])
        y = ResidentExperts.forward(layer, flat, topk.topk_ids.reshape(flat.shape[0], -1),
                                    topk.topk_weights.reshape(flat.shape[0], -1))
        return SGLANG.StandardCombineInput(hidden_states=y.view_as(x))

    def get_triton_quant_info(self, layer):
        raise NotImplementedError("EXL3 experts do not run on the Triton MoE runner")
