"""`Exl3MoEMethod`: EXL3 routed experts for SGLang's FusedMoE, running on `exl3_moe_forward`.

Contract of cuda/src/sglang_exl3/sglang_glue/moe.py:54-237:
  create_weights(layer, num_experts, hidden_size, intermediate_size_per_partition, params_dtype, **extra)
        placeholders `w13_<suffix>` (gate = shard w1, up = shard w3) and `w2_<suffix>` (down) for every checkpoint
        suffix, so the model's `load_weights` calls `weight_loader(param, tensor, name, shard_id=, expert_id=)`;
        TP / EP / fused shared experts / bias raise NotImplementedError (69-93).
  create_moe_runner     SiLU-gated experts only, no routed scaling, weights not applied on the input (109-119).
  process_weights_after_loading
        checks every expert against the header scan, converts legacy signs, then stacks the experts into the
        [E, ...] tensors the grouped kernel reads (the reference's marlin_moe.prepare pack, 170-203).
  apply(layer, dispatch_output) -> StandardCombineInput(hidden_states=y) (231-237); routing input topk_ids
        [T, top_k] int32/int64, topk_weights [T, top_k] fp32.
The stacked tensors are the only resident copy; no align step and no padding are needed (exl3_moe_forward routes
on the device).
"""
from __future__ import annotations

import logging
import re

import torch

from .common import CODEBOOK_ID, SUFFIXES, unpack_signs
from .engine import SGLANG, target_device

logger = logging.getLogger(__name__)
_ROLE = {"w1": "gate", "w3": "up", "w2": "down"}
_EXPERT_KEY = re.compile(r"\.experts\.(\d+)\.(gate|up|down)_proj$")


class Exl3MoEMethod(SGLANG.FusedMoEMethodBase):
    def __init__(self, config, prefix: str, experts: dict[str, tuple]):
        self.config = config
        self.prefix = prefix
        self.runner = None
        self.moe_runner_config = None
        self.infos: dict[tuple[str, int], tuple] = {}
        for key, info in experts.items():
            m = _EXPERT_KEY.search(key)
            if m is None:
                raise ValueError(f"{prefix}: unexpected EXL3 matrix under the experts: {key}")
            self.infos[(m.group(2), int(m.group(1)))] = info

    # ---- weights
    def create_weights(self, layer, num_experts, hidden_size, intermediate_size_per_partition, params_dtype,
                       **extra_weight_attrs):
        if getattr(layer, "moe_tp_size", 1) != 1 or getattr(layer, "moe_ep_size", 1) != 1:
            raise NotImplementedError(f"{self.prefix}: tensor/expert-parallel EXL3 MoE is not implemented")
        if getattr(layer, "num_fused_shared_experts", 0):
            raise NotImplementedError(f"{self.prefix}: fused shared experts are not supported "
                                      f"(run with --disable-shared-experts-fusion)")
        if extra_weight_attrs.get("with_bias"):
            raise NotImplementedError(f"{self.prefix}: EXL3 experts with bias are not implemented")
        wanted = {(r, e) for r in ("gate", "up", "down") for e in range(num_experts)}
        missing = sorted(wanted - set(self.infos))
        if missing:
            raise ValueError(f"{self.prefix}: the checkpoint has no EXL3 tensors for {len(missing)} of "
                             f"{3 * num_experts} expert matrices, e.g. {missing[0]}")
        if any(self.infos[w][4] for w in wanted):
            raise NotImplementedError(f"{self.prefix}: EXL3 experts with bias are not implemented")
        layer.exl3_store = {}
        layer.exl3_num_experts, layer.exl3_hidden, layer.exl3_inter = num_experts, hidden_size, \
            intermediate_size_per_partition
        for w in ("w13", "w2"):
            for suffix in SUFFIXES:
                p = torch.nn.Parameter(torch.empty(0, dtype=torch.uint8), requires_grad=False)
                SGLANG.set_weight_attrs(p, {"weight_loader": self._loader(layer, suffix), "exl3_placeholder": True})
                layer.register_parameter(f"{w}_{suffix}", p)

    def _loader(self, layer, suffix: str):
        def load(param, loaded_weight, weight_name=None, shard_id=None, expert_id=None, *args, **kwargs):
            role = _ROLE.get(shard_id)
            if role is None or expert_id is None:
                raise ValueError(f"{self.prefix}.{suffix}: unexpected expert shard {shard_id!r} / expert {expert_id!r}")
            store = layer.exl3_store.setdefault((role, suffix), {})
            e = int(expert_id)
            if e in store:
                raise ValueError(f"{self.prefix}: {role} {suffix} of expert {e} loaded twice")
            store[e] = loaded_weight.detach().to("cpu", copy=True)   # stacked once all experts are in
        return load

    def create_moe_runner(self, layer, moe_runner_config):
        cfg = moe_runner_config
        self.moe_runner_config = cfg
        if getattr(cfg, "activation", "silu") != "silu" or not getattr(cfg, "is_gated", True):
            raise NotImplementedError(f"{self.prefix}: only SiLU-gated experts are implemented "
                                      f"(got {getattr(cfg, 'activation', None)})")
        if getattr(cfg, "apply_router_weight_on_input", False):
            raise NotImplementedError(f"{self.prefix}: apply_router_weight_on_input is not supported")
        if getattr(cfg, "routed_scaling_factor", None) not in (None, 1.0):
            raise NotImplementedError(f"{self.prefix}: routed_scaling_factor {cfg.routed_scaling_factor} is not "
                                      f"supported")
        if getattr(cfg, "num_fused_shared_experts", 0):
            raise NotImplementedError(f"{self.prefix}: fused shared experts are not supported")

    def process_weights_after_loading(self, layer) -> None:
        store, E = layer.exl3_store, layer.exl3_num_experts
        codebooks, bits, stacked = set(), {}, {}
        for role in ("gate", "up", "down"):
            t = {s: store.get((role, s), {}) for s in SUFFIXES}
            absent = [e for e in range(E) if e not in t["trellis"]]
            if absent:
                raise ValueError(f"{self.prefix}: {role}_proj trellis missing for {len(absent)} experts, "
                                 f"e.g. {absent[0]}")
            trs, suhs, svhs = [], [], []
            for e in range(E):
                tr = t["trellis"][e]
                su, sv = t["suh"].get(e), t["svh"].get(e)
                if su is None and e in t["su"] and e in t["sv"]:
                    su, sv = unpack_signs(t["su"][e]), unpack_signs(t["sv"][e])
                if su is None or sv is None:
                    raise ValueError(f"{self.prefix}: {role}_proj of expert {e} has a trellis but no scale vectors")
                cb = "mcg" if e in t["mcg"] else "mul1" if e in t["mul1"] else "3inst"
                k, n, twice, declared = self.infos[(role, e)][:4]
                if (tr.shape[0] * 16, tr.shape[1] * 16, tr.shape[2] // 8, cb) != (k, n, twice, declared):
                    raise ValueError(f"{self.prefix}: {role}_proj expert {e} {tuple(tr.shape)}/{cb} does not match "
                                     f"the header scan {(k, n, twice, declared)}")
                codebooks.add(cb)
                trs.append(tr)
                suhs.append(su.to(torch.float16))
                svhs.append(sv.to(torch.float16))
            if len({tuple(x.shape) for x in trs}) != 1:
                raise NotImplementedError(f"{self.prefix}: the experts of {role}_proj differ in shape / bitrate")
            bits[role] = trs[0].shape[2] // 16
            stacked[role] = (torch.stack(trs), torch.stack(suhs), torch.stack(svhs))
        if len(codebooks) != 1:
            raise NotImplementedError(f"{self.prefix}: mixed codebooks {sorted(codebooks)}")
        if bits["gate"] != bits["up"]:
            raise NotImplementedError(f"{self.prefix}: gate and up bitrates differ {bits}")
        H, I = layer.exl3_hidden, layer.exl3_inter
        g, d = stacked["gate"][0], stacked["down"][0]
        if (g.shape[1] * 16, g.shape[2] * 16) != (H, I) or (d.shape[1] * 16, d.shape[2] * 16) != (I, H):
            raise ValueError(f"{self.prefix}: expert shapes {tuple(g.shape)} / {tuple(d.shape)} do not fit hidden "
                             f"{H}, intermediate {I}")
        dev = target_device()
        for role in ("gate", "up", "down"):
            for part, tensor in zip(("trellis", "suh", "svh"), stacked[role]):
                layer.register_buffer(f"exl3_{role}_{part}", tensor.to(dev).contiguous(), persistent=False)
        layer.exl3_codebook = CODEBOOK_ID[codebooks.pop()]
        layer.exl3_bits = bits
        store.clear()
        del layer.exl3_store
        for w in ("w13", "w2"):
            for suffix in SUFFIXES:
                delattr(layer, f"{w}_{suffix}")
        if dev.type == "cuda":
            from .. import ops
            ops.init_device(dev.index if dev.index is not None else torch.cuda.current_device())
        logger.info("%s: %d experts, K gate/up %d down %d, codebook %d, stacked for exl3_moe_forward", self.prefix,
                    E, bits["gate"], bits["down"], layer.exl3_codebook)

    def experts(self, layer) -> dict[str, torch.Tensor]:
        from ..ops import MOE_TENSORS
        return {name: getattr(layer, f"exl3_{name}") for name in MOE_TENSORS}

    # ---- forward
    def forward_experts(self, layer, x: torch.Tensor, topk_ids: torch.Tensor,
                        topk_weights: torch.Tensor) -> torch.Tensor:
        from .. import ops
        if x.shape[0] == 0:
            return torch.empty_like(x)
        return ops.moe_forward(x.contiguous(), topk_ids, topk_weights, self.experts(layer), layer.exl3_codebook)

    def apply(self, layer, dispatch_output):
        x = dispatch_output.hidden_states
        topk = dispatch_output.topk_output
        flat = x.reshape(-1, x.shape[-1])
        y = self.forward_experts(layer, flat, topk.topk_ids.reshape(flat.shape[0], -1),
                                 topk.topk_weights.reshape(flat.shape[0], -1))
        return SGLANG.StandardCombineInput(hidden_states=y.view_as(x))
