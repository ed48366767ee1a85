"""Torch-facing wrappers of the C-ABI: device tensors in, device tensors out, every launch on the current stream.

These mirror the building blocks of the reference's Marlin backend (cuda/src/sglang_exl3/kernels/marlin.py:138-190)
and ExLlamaV3's reconstruct (cuda/src/sglang_exl3/kernels/reference.py:71-76), with the same argument meaning.
Nothing here computes on the CPU: a missing library raises ExtensionMissing.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

CODEBOOK_ID = {"3inst": 0, "mcg": 1, "mul1": 2}


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def bits_of(trellis: torch.Tensor) -> int:
    """K from the trellis last dim (16 K int16 per tile; core/src/trellis_core/format/spec.py:58-61)."""
    words = trellis.shape[-1]
    if words % 16:
        raise ValueError(f"trellis last dim {words} is not 16*K")
    return words // 16


def _check_trellis(t: torch.Tensor) -> tuple[int, int, int]:
    if t.dtype != torch.int16 or t.dim() != 3 or not t.is_contiguous() or not t.is_cuda:
        raise ValueError(f"trellis must be a contiguous CUDA int16 [k/16, n/16, 16K] tensor, got {t.dtype} "
                         f"{tuple(t.shape)} on {t.device}")
    return t.shape[0] * 16, t.shape[1] * 16, bits_of(t)


def _half(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.float16 or not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous CUDA fp16 tensor, got {t.dtype} on {t.device}")
    return t


class WorkspaceTooSmall(RuntimeError):
    """A call inside HIP-graph capture needs more workspace than was reserved (nothing may allocate there)."""


class _Workspace:
    """The per-device scratch of one kind of launch (split counters, rotated activations, fp32 partials).

    A workspace only ever grows by replacement while no captured graph can hold its address.  Once it has been used
    inside a graph capture it is never freed or replaced: a later eager call that needs more runs on a temporary
    buffer of its own (as the reference's run does past its reserved rows, cuda/src/sglang_exl3/kernels/marlin.py:
    86-89), and a capture that needs more raises WorkspaceTooSmall.  After `reserve_*` the workspace keeps its
    reserved size the same way, so an engine that reserves for its largest batch at load time never allocates on the
    serving path (cuda/src/sglang_exl3/kernels/base.py:74-76)."""

    def __init__(self, kind: str, zeroed: bool):
        self.kind, self.zeroed = kind, zeroed
        self.buf: torch.Tensor | None = None
        self.reserved = False   # sized by reserve_*: later calls beyond it use a temporary buffer
        self.captured = False   # used inside a graph capture: the address must never change

    def _alloc(self, nbytes: int, device: torch.device) -> torch.Tensor:
        # counters must start at zero (every call leaves them there); the KV workspace holds only fully written data
        make = torch.zeros if self.zeroed else torch.empty
        return make(max(int(nbytes), 256), dtype=torch.uint8, device=device)

    def get(self, device: torch.device, nbytes: int) -> torch.Tensor:
        capturing = torch.cuda.is_current_stream_capturing()
        if self.buf is not None and self.buf.numel() >= nbytes:
            self.captured |= capturing
            return self.buf
        have = 0 if self.buf is None else self.buf.numel()
        if capturing:
            raise WorkspaceTooSmall(f"{self.kind} workspace on {device} holds {have} bytes, a call inside graph capture "
                                    f"needs {nbytes}: call ops.reserve_{self.kind}(...) for the largest shape before "
                                    f"capturing")
        if self.captured or self.reserved:
            return self._alloc(nbytes, device)   # one-off: the reserved buffer keeps its address
        self.buf = self._alloc(nbytes, device)
        return self.buf

    def reserve(self, device: torch.device, nbytes: int) -> None:
        if self.buf is None or self.buf.numel() < nbytes:
            if self.captured:
                raise WorkspaceTooSmall(f"{self.kind} workspace on {device} is held by a captured graph; reserve "
                                        f"{nbytes} bytes before the first capture")
            self.buf = self._alloc(nbytes, device)
        self.reserved = True


_KINDS = {"linear": True, "prefill": True, "moe": True, "moe_stage": True, "kv": False}
_workspaces: dict[tuple[str, int], _Workspace] = {}


def _dev_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


_initialised: set[int] = set()


def _ws(kind: str, device: torch.device) -> _Workspace:
    idx = _dev_index(device)
    if idx not in _initialised and not torch.cuda.is_current_stream_capturing():
        # the device check, and the probe of the workgroup -> XCD assignment that lets split-K chains stay in one
        # XCD's L2 (the reference's init_device, cuda/csrc/exl3_marlin.cu:537); a workspace is first taken (or
        # reserved) before any capture
        init_device(idx)
        _initialised.add(idx)
    key = (kind, idx)
    ws = _workspaces.get(key)
    if ws is None:
        ws = _workspaces[key] = _Workspace(kind, _KINDS[kind])
    return ws


def workspace(device: torch.device, nbytes: int, kind: str = "linear") -> torch.Tensor:
    """The per-device workspace of `kind` ("linear", "prefill", "moe", "kv") holding at least `nbytes`."""
    dev = torch.device("cuda", _dev_index(device))
    return _ws(kind, dev).get(dev, nbytes)


def release_workspaces() -> None:
    """Drops every workspace (tests; an engine that has captured graphs must keep them)."""
    _workspaces.clear()


def _max_need(fn, max_rows: int) -> int:
    """The largest workspace any row count 1..max_rows needs (split plans do not grow monotonically with rows)."""
    return max(fn(r) for r in range(1, max(1, int(max_rows)) + 1))


def reserve_linear(device: torch.device, max_rows: int, k: int, n_total: int, K: int) -> None:
    """Reserves the decode-GEMV workspace for every call of up to `max_rows` rows on a group of input width k and
    n_total output columns at bitrate K (the reference reserves its scratch at load, kernels/marlin.py:24-33)."""
    lib = _lib.load()
    dev = torch.device("cuda", _dev_index(device))
    _ws("linear", dev).reserve(dev, _max_need(lambda r: lib.exl3_linear_workspace_bytes(r, k, n_total, K), max_rows))


def reserve_prefill(device: torch.device, max_rows: int, k: int, n_total: int, nshards: int) -> None:
    """Reserves the decode-GEMM workspace for every call of up to `max_rows` rows."""
    lib = _lib.load()
    dev = torch.device("cuda", _dev_index(device))
    with torch.cuda.device(dev):   # the plan depends on the device's CU count
        need = _max_need(lambda r: lib.exl3_prefill_workspace_bytes(r, k, n_total, nshards), max_rows)
    _ws("prefill", dev).reserve(dev, need)


def reserve_moe(device: torch.device, max_tokens: int, top_k: int, num_experts: int, hidden: int, inter: int,
                K_gate_up: int, K_down: int) -> None:
    """Reserves the MoE workspace for every call of up to `max_tokens` tokens."""
    lib = _lib.load()
    dev = torch.device("cuda", _dev_index(device))
    need = _max_need(lambda t: lib.exl3_moe_workspace_bytes(t, top_k, num_experts, hidden, inter, K_gate_up,
                                                            K_down), max_tokens)
    _ws("moe", dev).reserve(dev, need)


def moe_align_capacity(slots: int, num_experts: int, block: int) -> tuple[int, int]:
    """(sorted_ids entries, expert_ids blocks) that moe_align allocates for `slots` routed slots."""
    cap = slots + num_experts * (block - 1)
    return cap, -(-cap // block)


def reserve_moe_stage(device: torch.device, max_slots: int, k: int, n: int, shards: int, num_experts: int,
                      block: int) -> None:
    """Reserves the grouped-GEMM workspace of the per-launch MoE stages (moe_gemm) for every call of up to `max_slots`
    rows routed by moe_align with `num_experts` experts and this block size, so a captured stage chain never
    allocates."""
    lib = _lib.load()
    dev = torch.device("cuda", _dev_index(device))
    need = _max_need(lambda r: lib.exl3_moe_gemm_workspace_bytes(r, k, n, shards,
                                                                 moe_align_capacity(r, num_experts, block)[1]),
                     max_slots)
    _ws("moe_stage", dev).reserve(dev, need)


def reserve_kv(device: torch.device, max_batch: int, num_q_heads: int, num_kv_heads: int, max_pages: int) -> None:
    """Reserves the KV decode-attention workspace for batches of up to `max_batch` sequences of up to `max_pages`
    pages (a smaller batch can take more page chunks per sequence, so every batch size is sized; fewer pages never
    need more)."""
    lib = _lib.load()
    dev = torch.device("cuda", _dev_index(device))
    _ws("kv", dev).reserve(dev, _max_need(
        lambda b: lib.exl3_kv_decode_workspace_bytes(b, num_q_heads, num_kv_heads, max_pages), max_batch))


def reserve_workspace(device: torch.device, rows: int, k: int, n_total: int, K: int) -> None:
    """Older name of reserve_linear."""
    reserve_linear(device, rows, k, n_total, K)


def _check_out(out: torch.Tensor, shape: tuple, like: torch.Tensor, dtypes=(torch.float16, torch.bfloat16)) -> None:
    """A caller-supplied output must be exactly what the kernels write: the C-ABI only sees a pointer."""
    if tuple(out.shape) != tuple(shape):
        raise ValueError(f"out has shape {tuple(out.shape)}, expected {tuple(shape)}")
    if out.dtype not in dtypes:
        raise ValueError(f"out must be one of {[str(d) for d in dtypes]}, got {out.dtype}")
    if not out.is_contiguous():
        raise ValueError("out must be contiguous")
    if out.device != like.device:
        raise ValueError(f"out is on {out.device}, the inputs on {like.device}")


def init_device(index: int) -> None:
    _lib.check(_lib.load().exl3_init_device(int(index)), "exl3_init_device")


def reconstruct(trellis: torch.Tensor, codebook: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """W_inner fp16 [k, n], bit-identical to trellis_core.reference.reconstruct_inner (reference.py:102-115)."""
    k, n, K = _check_trellis(trellis)
    if out is None:
        out = torch.empty((k, n), dtype=torch.float16, device=trellis.device)
    if out.shape != (k, n) or out.dtype != torch.float16 or not out.is_contiguous():
        raise ValueError("out must be a contiguous fp16 [k, n] tensor")
    _lib.check(_lib.load().exl3_reconstruct(trellis.data_ptr(), k, n, K, int(codebook), out.data_ptr(),
                                            _stream(trellis.device)), "reconstruct")
    return out


def repack_trellis(trellis: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """The trellis in the load-time layout (LAYOUT_BLOCKS; the reference's repack_trellis,
    cuda/csrc/exl3_marlin.cu:344-381): the same bytes per tile, each (128-column block, 128-row block) unit of 64
    tiles one contiguous run.  Same shape and dtype as the stored tensor; `out` must not be the input."""
    return _trellis_relayout(trellis, out, "exl3_repack_trellis")


def unpack_trellis(packed: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Inverse of repack_trellis: the stored layout back, bit for bit (the reference's unpack_trellis,
    exl3_marlin.cu:384-408)."""
    return _trellis_relayout(packed, out, "exl3_unpack_trellis")


def _trellis_relayout(t: torch.Tensor, out: torch.Tensor | None, entry: str) -> torch.Tensor:
    k, n, K = _check_trellis(t)
    if out is None:
        out = torch.empty_like(t)
    if out.shape != t.shape or out.dtype != torch.int16 or not out.is_contiguous() or out.device != t.device:
        raise ValueError(f"out must be a contiguous int16 {tuple(t.shape)} tensor on {t.device}")
    if out.data_ptr() == t.data_ptr():
        raise ValueError(f"{entry}: out must not be the input")
    _lib.check(getattr(_lib.load(), entry)(t.data_ptr(), k, n, K, out.data_ptr(), _stream(t.device)), entry)
    return out


def had_in_group(x: torch.Tensor, suh_cat: torch.Tensor, xh: torch.Tensor | None = None) -> torch.Tensor:
    """xh[s] = fp16(Had128(fp16(x) * suh_cat[s])) for all shards: x fp16|bf16 [rows, k] -> fp16 [shards*rows, k]
    (kernels/marlin.py:138-146)."""
    if x.dtype not in (torch.float16, torch.bfloat16) or x.dim() != 2 or not x.is_contiguous():
        raise ValueError("x must be a contiguous fp16/bf16 [rows, k] tensor")
    rows, k = x.shape
    suh_cat = _half(suh_cat, "suh_cat")
    shards = suh_cat.numel() // k
    if shards * k != suh_cat.numel():
        raise ValueError(f"suh_cat has {suh_cat.numel()} values, not a multiple of k = {k}")
    if xh is None:
        xh = torch.empty((shards * rows, k), dtype=torch.float16, device=x.device)
    _lib.check(_lib.load().exl3_had_in_group(x.data_ptr(), int(x.dtype == torch.bfloat16), rows, k,
                                             suh_cat.data_ptr(), shards, xh.data_ptr(), _stream(x.device)),
               "had_in_group")
    return xh


def had_out_into(y: torch.Tensor, svh: torch.Tensor, out: torch.Tensor, col0: int) -> None:
    """out[:, col0:col0+n] = fp16(Had128(y)) * svh in out's dtype (kernels/marlin.py:149-151)."""
    y = _half(y, "y")
    rows, n = y.shape
    if out.dtype not in (torch.float16, torch.bfloat16) or out.dim() != 2 or out.stride(1) != 1:
        raise ValueError("out must be an fp16/bf16 [rows, N] tensor with unit column stride")
    if out.shape[0] != rows or col0 + n > out.shape[1]:
        raise ValueError(f"out {tuple(out.shape)} cannot hold columns {col0}..{col0 + n} of {rows} rows")
    _lib.check(_lib.load().exl3_had_out_into(y.data_ptr(), rows, n, _half(svh, "svh").data_ptr(), out.data_ptr(),
                                             int(out.dtype == torch.bfloat16), out.stride(0), int(col0),
                                             _stream(y.device)), "had_out_into")


def gemm_rotated(xh: torch.Tensor, trellis: torch.Tensor, codebook: int,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """xh @ W_inner in the rotated basis, fp32 accumulation, fp16 out; identity rows read W_inner out exactly
    (kernels/marlin.py:153-159).  Below 65 rows the decode-GEMV serves the rows, from 65 rows the prefill decode-GEMM,
    as in a linear."""
    k, n, K = _check_trellis(trellis)
    xh = _half(xh, "xh")
    if xh.dim() != 2 or xh.shape[1] != k:
        raise ValueError(f"xh must be [rows, {k}]")
    rows = xh.shape[0]
    if out is None:
        out = torch.empty((rows, n), dtype=torch.float16, device=xh.device)
    _check_out(out, (rows, n), xh, (torch.float16,))
    lib = _lib.load()
    ws = workspace(xh.device, lib.exl3_gemm_rotated_workspace_bytes(rows, k, n, K))
    _lib.check(lib.exl3_gemm_rotated(xh.data_ptr(), rows, k, trellis.data_ptr(), n, K, int(codebook),
                                     out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(xh.device)), "gemm_rotated")
    return out


def _shards(trellis: list[torch.Tensor], suh: list[torch.Tensor], svh: list[torch.Tensor], device: torch.device,
            layout: int = _lib.LAYOUT_STORED):
    if not (1 <= len(trellis) <= _lib.MAX_SHARDS) or not (len(trellis) == len(suh) == len(svh)):
        raise ValueError(f"1..{_lib.MAX_SHARDS} shards with one trellis, suh and svh each")
    arr = (_lib.Exl3Shard * len(trellis))()
    k0 = K0 = None
    for i, (t, su, sv) in enumerate(zip(trellis, suh, svh)):
        k, n, K = _check_trellis(t)
        if k0 is None:
            k0, K0 = k, K
        if (k, K) != (k0, K0):
            raise ValueError("all shards of a group share the input width k and the bitrate K")
        if _half(su, "suh").numel() != k or _half(sv, "svh").numel() != n:
            raise ValueError(f"shard {i}: suh/svh sizes {su.numel()}/{sv.numel()} != {k}/{n}")
        if not (t.device == su.device == sv.device == device):
            raise ValueError(f"shard {i}: tensors on {t.device}/{su.device}/{sv.device}, x on {device}")
        arr[i] = _lib.Exl3Shard(t.data_ptr(), su.data_ptr(), sv.data_ptr(), n, int(layout))
    return arr, k0, K0


def linear(x: torch.Tensor, trellis: list[torch.Tensor], suh: list[torch.Tensor], svh: list[torch.Tensor],
           codebook: int, out: torch.Tensor | None = None, layout: int = _lib.LAYOUT_STORED) -> torch.Tensor:
    """Fused group: y[..., sum n_s] = concat_s(Had(Had(x * suh_s) @ W_s) * svh_s), x fp16|bf16 [..., k], y in x's
    dtype (exl3_linear_marlin_multi_out, cuda/csrc/exl3_marlin.cu:507-527)."""
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"x must be fp16 or bf16, got {x.dtype}")
    arr, k, K = _shards(trellis, suh, svh, x.device, layout)
    rows2d = x.reshape(-1, x.shape[-1]).contiguous()
    if rows2d.shape[1] != k:
        raise ValueError(f"x has {rows2d.shape[1]} features, the group expects {k}")
    rows = rows2d.shape[0]
    n_total = sum(a.n for a in arr)
    if out is None:
        out = torch.empty((rows, n_total), dtype=x.dtype, device=x.device)
    _check_out(out, (rows, n_total), x)
    lib = _lib.load()
    ws = workspace(x.device, lib.exl3_linear_workspace_bytes(rows, k, n_total, K))
    _lib.check(lib.exl3_linear(rows2d.data_ptr(), int(x.dtype == torch.bfloat16), rows, k, arr, len(arr), K,
                               int(codebook), out.data_ptr(), int(out.dtype == torch.bfloat16), ws.data_ptr(),
                               ws.numel(), _stream(x.device)), "linear")
    return out.view(*x.shape[:-1], n_total)


def linear_prefill(x: torch.Tensor, trellis: list[torch.Tensor], suh: list[torch.Tensor], svh: list[torch.Tensor],
                   codebook: int, out: torch.Tensor | None = None, layout: int = _lib.LAYOUT_STORED) -> torch.Tensor:
    """Many-row form of `linear`: input rotations into a per-device workspace, then the fused decode-GEMM (weights
    decoded into LDS, fp16 MFMA).  Same result contract as `linear` (the reference's prefill branch,
    cuda/src/sglang_exl3/runtime/ops.py:87-95)."""
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"x must be fp16 or bf16, got {x.dtype}")
    arr, k, K = _shards(trellis, suh, svh, x.device, layout)
    rows2d = x.reshape(-1, x.shape[-1]).contiguous()
    if rows2d.shape[1] != k:
        raise ValueError(f"x has {rows2d.shape[1]} features, the group expects {k}")
    rows = rows2d.shape[0]
    n_total = sum(a.n for a in arr)
    if out is None:
        out = torch.empty((rows, n_total), dtype=x.dtype, device=x.device)
    _check_out(out, (rows, n_total), x)
    lib = _lib.load()
    with torch.cuda.device(x.device):   # the plan depends on the device's CU count
        need = lib.exl3_prefill_workspace_bytes(rows, k, n_total, len(arr))
    ws = workspace(x.device, need, "prefill")
    _lib.check(lib.exl3_linear_prefill(rows2d.data_ptr(), int(x.dtype == torch.bfloat16), rows, k, arr, len(arr), K,
                                       int(codebook), out.data_ptr(), int(out.dtype == torch.bfloat16), ws.data_ptr(),
                                       ws.numel(), _stream(x.device)), "linear_prefill")
    return out.view(*x.shape[:-1], n_total)


MOE_TENSORS = ("gate_trellis", "up_trellis", "down_trellis", "gate_suh", "gate_svh", "up_suh", "up_svh", "down_suh",
               "down_svh")


def _expert_stacks(experts: dict[str, torch.Tensor], H: int, device: torch.device) -> tuple[int, int, int, int]:
    """Checks one set of stacked expert tensors (MOE_TENSORS); returns (E, inter, K gate/up, K down)."""
    gt, ut, dt = experts["gate_trellis"], experts["up_trellis"], experts["down_trellis"]
    if any(t.dim() != 4 or t.dtype != torch.int16 for t in (gt, ut, dt)):
        raise ValueError("stacked trellis tensors must be int16 [E, k/16, n/16, 16K]")
    E, I = gt.shape[0], gt.shape[2] * 16
    if ut.shape != gt.shape:
        raise ValueError(f"gate {tuple(gt.shape)} and up {tuple(ut.shape)} must have one shape and bitrate")
    if gt.shape[1] * 16 != H or tuple(dt.shape[:3]) != (E, I // 16, H // 16):
        raise ValueError(f"expert shapes {tuple(gt.shape)} / {tuple(dt.shape)} do not match H = {H}")
    sizes = {"gate_suh": H, "up_suh": H, "gate_svh": I, "up_svh": I, "down_suh": I, "down_svh": H}
    for name in MOE_TENSORS:
        t = experts[name]
        if not (t.is_cuda and t.is_contiguous()) or t.shape[0] != E or t.device != device:
            raise ValueError(f"{name} must be a contiguous tensor with {E} experts on {device}")
        if name in sizes and (t.dtype != torch.float16 or tuple(t.shape) != (E, sizes[name])):
            raise ValueError(f"{name} must be fp16 [{E}, {sizes[name]}], got {t.dtype} {tuple(t.shape)}")
    return E, I, bits_of(gt), bits_of(dt)


def _routing(x: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor):
    T = x.shape[0]
    if topk_ids.dim() != 2 or topk_ids.shape[0] != T or tuple(topk_weights.shape) != tuple(topk_ids.shape):
        raise ValueError(f"topk_ids {tuple(topk_ids.shape)} and topk_weights {tuple(topk_weights.shape)} must both be "
                         f"[{T}, top_k]")
    if topk_ids.dtype not in (torch.int32, torch.int64) or topk_ids.device != x.device \
            or topk_weights.device != x.device:
        raise ValueError("topk_ids must be int32/int64 and both routing tensors on x's device")
    return topk_ids.to(torch.int32).contiguous(), topk_weights.to(torch.float32).contiguous()


def moe_forward(x: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor, experts: dict[str, torch.Tensor],
                codebook: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """Routed SiLU-gated EXL3 MoE layer (cuda/src/sglang_exl3/kernels/marlin_moe.py:272-294).
    x fp16|bf16 [T, H]; topk_ids [T, top_k] (int32 or int64); topk_weights fp32 [T, top_k]; `experts` holds the
    stacked tensors named in MOE_TENSORS (trellis int16 [E, k/16, n/16, 16K], scales fp16 [E, k] / [E, n]).
    Gate and up share one bitrate, down may have another (cuda/src/sglang_exl3/kernels/reference.py:123-149)."""
    if x.dtype not in (torch.float16, torch.bfloat16) or x.dim() != 2:
        raise ValueError("x must be a 2-D fp16/bf16 tensor")
    T, H = x.shape
    E, I, K_gu, K_dn = _expert_stacks(experts, H, x.device)
    ids, w = _routing(x, topk_ids, topk_weights)
    top_k = ids.shape[1]
    if out is None:
        out = torch.empty((T, H), dtype=x.dtype, device=x.device)
    _check_out(out, (T, H), x)
    lib = _lib.load()
    ws = workspace(x.device, lib.exl3_moe_workspace_bytes(T, top_k, E, H, I, K_gu, K_dn), "moe")
    wts = _lib.Exl3MoeWeights(*[experts[n].data_ptr() for n in MOE_TENSORS])
    _lib.check(lib.exl3_moe_forward(x.contiguous().data_ptr(), int(x.dtype == torch.bfloat16), T, H, ids.data_ptr(),
                                    w.data_ptr(), top_k, E, I, ctypes.byref(wts), K_gu, K_dn, int(codebook),
                                    out.data_ptr(), int(out.dtype == torch.bfloat16), ws.data_ptr(), ws.numel(),
                                    _stream(x.device)),
               "moe_forward")
    return out


def moe_forward_classes(x: torch.Tensor, topk_ids: torch.Tensor, topk_weights: torch.Tensor,
                        classes: list[tuple[dict[str, torch.Tensor], torch.Tensor]], num_experts: int, codebook: int,
                        out: torch.Tensor | None = None) -> torch.Tensor:
    """moe_forward for a layer whose experts come in up to two K classes (the reference's MixedPack / run_mixed,
    cuda/src/sglang_exl3/kernels/marlin_moe.py:135-170, 247-272): `classes` holds per class its stacked expert tensors
    in LOCAL order and its expert map (int32 [num_experts]: global id -> local id, -1 for the other class's experts).
    topk_ids hold global ids; every id in [0, num_experts) must belong to exactly one class."""
    if x.dtype not in (torch.float16, torch.bfloat16) or x.dim() != 2:
        raise ValueError("x must be a 2-D fp16/bf16 tensor")
    if not 1 <= len(classes) <= _lib.MAX_MOE_CLASSES:
        raise ValueError(f"1..{_lib.MAX_MOE_CLASSES} expert classes")
    T, H = x.shape
    arr = (_lib.Exl3MoeClass * len(classes))()
    I0 = None
    maps = []
    for c, (experts, emap) in enumerate(classes):
        E_c, I, K_gu, K_dn = _expert_stacks(experts, H, x.device)
        if I0 is not None and I != I0:
            raise ValueError("every class shares the intermediate width")
        I0 = I
        if emap.numel() != num_experts:
            raise ValueError(f"class {c}: expert map holds {emap.numel()} entries for {num_experts} experts")
        maps.append(_routing_ids(emap, x.device).reshape(-1))
        arr[c] = _lib.Exl3MoeClass(_lib.Exl3MoeWeights(*[experts[n].data_ptr() for n in MOE_TENSORS]),
                                   maps[-1].data_ptr(), E_c, K_gu, K_dn)
    ids, w = _routing(x, topk_ids, topk_weights)
    top_k = ids.shape[1]
    if out is None:
        out = torch.empty((T, H), dtype=x.dtype, device=x.device)
    _check_out(out, (T, H), x)
    lib = _lib.load()
    ws = workspace(x.device, lib.exl3_moe_classes_workspace_bytes(T, top_k, num_experts, H, I0, len(classes), arr),
                   "moe")
    _lib.check(lib.exl3_moe_forward_classes(x.contiguous().data_ptr(), int(x.dtype == torch.bfloat16), T, H,
                                            ids.data_ptr(), w.data_ptr(), top_k, num_experts, I0, arr, len(classes),
                                            int(codebook), out.data_ptr(), int(out.dtype == torch.bfloat16),
                                            ws.data_ptr(), ws.numel(), _stream(x.device)),
               "moe_forward_classes")
    return out


# ---- MoE per-launch stages: the launches the reference's unfused path runs after moe_align_block_size
# (cuda/src/sglang_exl3/kernels/marlin_moe.py:272-294: moe_had_in, moe_gemm for gate|up, moe_glu_had_in, moe_gemm for
# down, moe_combine), on the stored trellis stacks

def _routing_ids(topk_ids: torch.Tensor, device: torch.device) -> torch.Tensor:
    if topk_ids.dtype not in (torch.int32, torch.int64) or topk_ids.device != device:
        raise ValueError(f"topk_ids must be int32/int64 on {device}, got {topk_ids.dtype} on {topk_ids.device}")
    return topk_ids.to(torch.int32).contiguous()


def _ptr_array(tensors: list[torch.Tensor]):
    return (ctypes.c_void_p * len(tensors))(*[t.data_ptr() for t in tensors])


def moe_align(topk_ids: torch.Tensor, num_experts: int, block: int, expert_map: torch.Tensor | None = None):
    """(sorted_ids, expert_ids, num_post_padded) in the layout of vLLM's moe_align_block_size for one block size
    (the reference's moe_align_decode, cuda/csrc/exl3_marlin_moe.cu:546-618): each expert's slots padded to a multiple
    of `block` with the sentinel topk_ids.numel(), the expert (or expert_map[e]) of every block, -1 past the end."""
    ids = _routing_ids(topk_ids, topk_ids.device).reshape(-1)
    slots = ids.numel()
    cap, max_blocks = moe_align_capacity(slots, num_experts, block)
    dev = ids.device
    sorted_ids = torch.empty(cap, dtype=torch.int32, device=dev)
    expert_ids = torch.empty(max_blocks, dtype=torch.int32, device=dev)
    post = torch.empty(1, dtype=torch.int32, device=dev)
    emap = None
    if expert_map is not None:
        if expert_map.numel() != num_experts:
            raise ValueError(f"expert_map holds {expert_map.numel()} entries for {num_experts} experts")
        emap = _routing_ids(expert_map, dev)
    _lib.check(_lib.load().exl3_moe_align(ids.data_ptr(), slots, int(num_experts), _ptr(emap), int(block),
                                          sorted_ids.data_ptr(), cap, expert_ids.data_ptr(), max_blocks,
                                          post.data_ptr(), _stream(dev)), "moe_align")
    return sorted_ids, expert_ids, post


def moe_align_classes(topk_ids: torch.Tensor, num_experts: int, expert_maps: list[torch.Tensor],
                      blocks: list[int]) -> list[tuple[torch.Tensor, torch.Tensor, torch.Tensor]]:
    """moe_align for every K class of a mixed layer in one launch (the reference's moe_align_decode,
    cuda/csrc/exl3_marlin_moe.cu:532-618): per class (sorted_ids, expert_ids, num_post_padded) as moe_align gives with
    that class's expert map and block size (local expert ids)."""
    n = len(expert_maps)
    if not 1 <= n <= _lib.MAX_MOE_CLASSES or len(blocks) != n:
        raise ValueError(f"1..{_lib.MAX_MOE_CLASSES} classes, one block size each")
    ids = _routing_ids(topk_ids, topk_ids.device).reshape(-1)
    slots, dev = ids.numel(), ids.device
    maps = []
    for emap in expert_maps:
        if emap.numel() != num_experts:
            raise ValueError(f"an expert map holds {emap.numel()} entries for {num_experts} experts")
        maps.append(_routing_ids(emap, dev).reshape(-1))
    out = []
    for b in blocks:
        cap, mb = moe_align_capacity(slots, num_experts, b)
        out.append((torch.empty(cap, dtype=torch.int32, device=dev), torch.empty(mb, dtype=torch.int32, device=dev),
                    torch.empty(1, dtype=torch.int32, device=dev)))
    P, I = ctypes.c_void_p, ctypes.c_int
    _lib.check(_lib.load().exl3_moe_align_classes(
        ids.data_ptr(), slots, int(num_experts), n, (P * n)(*[m.data_ptr() for m in maps]), (I * n)(*blocks),
        (P * n)(*[o[0].data_ptr() for o in out]), (I * n)(*[o[0].numel() for o in out]),
        (P * n)(*[o[1].data_ptr() for o in out]), (I * n)(*[o[1].numel() for o in out]),
        (P * n)(*[o[2].data_ptr() for o in out]), _stream(dev)), "moe_align_classes")
    return out


def moe_had_in(x: torch.Tensor, suh: list[torch.Tensor], topk_ids: torch.Tensor,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """xh [shards * slots, k] fp16: fp16(Had(fp16(x[token]) * suh_s[e])) per (shard, slot) (the reference's
    moe_had_in, cuda/csrc/exl3_marlin_moe.cu:416-448); suh: one [E, k] fp16 stack per shard (gate, up)."""
    if x.dtype not in (torch.float16, torch.bfloat16) or x.dim() != 2:
        raise ValueError("x must be a 2-D fp16/bf16 tensor")
    T, k = x.shape
    ids = _routing_ids(topk_ids, x.device)
    if ids.dim() != 2 or ids.shape[0] != T:
        raise ValueError(f"topk_ids {tuple(topk_ids.shape)} must be [{T}, top_k]")
    if not 1 <= len(suh) <= 2:
        raise ValueError("one or two suh stacks")
    E = suh[0].shape[0]
    for t in suh:
        if t.dtype != torch.float16 or tuple(t.shape) != (E, k) or not t.is_contiguous() or t.device != x.device:
            raise ValueError(f"suh stacks must be contiguous fp16 [{E}, {k}] on {x.device}")
    slots = ids.numel()
    if out is None:
        out = torch.empty((len(suh) * slots, k), dtype=torch.float16, device=x.device)
    _check_out(out, (len(suh) * slots, k), x, (torch.float16,))
    _lib.check(_lib.load().exl3_moe_had_in(x.contiguous().data_ptr(), int(x.dtype == torch.bfloat16), T, k,
                                           ids.data_ptr(), ids.shape[1], E, _ptr_array(suh), len(suh),
                                           out.data_ptr(), _stream(x.device)), "moe_had_in")
    return out


def moe_gemm(a: torch.Tensor, trellis: list[torch.Tensor], svh: list[torch.Tensor] | None, sorted_ids: torch.Tensor,
             expert_ids: torch.Tensor, num_post_padded: torch.Tensor, block: int, codebook: int,
             out: torch.Tensor | None = None) -> torch.Tensor:
    """The grouped expert GEMM over align blocks (the reference's moe_gemm, cuda/csrc/exl3_marlin_moe.cu:376-412):
    a fp16 [shards * rows, k] (rotated inputs), trellis one [E, k/16, n/16, 16K] stack per shard; returns c fp16
    [rows, shards * n], with the output transform fp16(Had(fp16(acc)) * svh) when svh stacks ([E, n]) are given."""
    if a.dtype != torch.float16 or a.dim() != 2 or not a.is_contiguous():
        raise ValueError("a must be a contiguous fp16 [shards * rows, k] tensor")
    shards = len(trellis)
    if shards not in (1, 2) or a.shape[0] % shards:
        raise ValueError(f"one or two trellis stacks; a has {a.shape[0]} rows")
    rows, k = a.shape[0] // shards, a.shape[1]
    t0 = trellis[0]
    if any(t.dtype != torch.int16 or t.dim() != 4 or t.shape != t0.shape or not t.is_contiguous()
           or t.device != a.device for t in trellis):
        raise ValueError("trellis stacks must be contiguous int16 [E, k/16, n/16, 16K] of one shape on a's device")
    E, n, K = t0.shape[0], t0.shape[2] * 16, bits_of(t0)
    if t0.shape[1] * 16 != k:
        raise ValueError(f"trellis input width {t0.shape[1] * 16} != {k}")
    if svh is not None:
        if len(svh) != shards or any(v.dtype != torch.float16 or tuple(v.shape) != (E, n) or not v.is_contiguous()
                                     or v.device != a.device for v in svh):
            raise ValueError(f"svh must be {shards} contiguous fp16 [{E}, {n}] stacks")
    for name, t in (("sorted_ids", sorted_ids), ("expert_ids", expert_ids), ("num_post_padded", num_post_padded)):
        if t.dtype != torch.int32 or not t.is_contiguous() or t.device != a.device:
            raise ValueError(f"{name} must be a contiguous int32 tensor on {a.device}")
    max_blocks = expert_ids.numel()
    if max_blocks * block < sorted_ids.numel():
        raise ValueError(f"expert_ids ({max_blocks}) too short for {sorted_ids.numel()} sorted ids in blocks of {block}")
    if out is None:
        out = torch.empty((rows, shards * n), dtype=torch.float16, device=a.device)
    _check_out(out, (rows, shards * n), a, (torch.float16,))
    if rows == 0:
        return out
    lib = _lib.load()
    ws = workspace(a.device, lib.exl3_moe_gemm_workspace_bytes(rows, k, n, shards, max_blocks), "moe_stage")
    _lib.check(lib.exl3_moe_gemm(a.data_ptr(), rows, k, _ptr_array(trellis), None if svh is None else _ptr_array(svh),
                                 shards, n, sorted_ids.data_ptr(), expert_ids.data_ptr(), num_post_padded.data_ptr(),
                                 max_blocks, int(block), E, K, int(codebook), out.data_ptr(), ws.data_ptr(), ws.numel(),
                                 _stream(a.device)), "moe_gemm")
    return out


def moe_glu_had_in(gu: torch.Tensor, suh_down: torch.Tensor, topk_ids: torch.Tensor, act: torch.Tensor | None = None,
                   out: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """(act, xd): act = fp16(silu(g) * u) and the rotated down inputs xd = fp16(Had(fp16(act * suh_down[e]))) per slot
    from gu fp16 [slots, 2 inter] (the reference's moe_glu_had_in, cuda/csrc/exl3_marlin_moe.cu:450-477)."""
    if gu.dtype != torch.float16 or gu.dim() != 2 or not gu.is_contiguous() or gu.shape[1] % 256:
        raise ValueError("gu must be a contiguous fp16 [slots, 2 inter] tensor")
    slots, inter = gu.shape[0], gu.shape[1] // 2
    ids = _routing_ids(topk_ids, gu.device).reshape(-1)
    if ids.numel() != slots:
        raise ValueError(f"topk_ids holds {ids.numel()} slots, gu {slots}")
    if suh_down.dtype != torch.float16 or suh_down.dim() != 2 or suh_down.shape[1] != inter \
            or not suh_down.is_contiguous() or suh_down.device != gu.device:
        raise ValueError(f"suh_down must be a contiguous fp16 [E, {inter}] stack")
    if act is None:
        act = torch.empty((slots, inter), dtype=torch.float16, device=gu.device)
    if out is None:
        out = torch.empty((slots, inter), dtype=torch.float16, device=gu.device)
    _check_out(act, (slots, inter), gu, (torch.float16,))
    _check_out(out, (slots, inter), gu, (torch.float16,))
    _lib.check(_lib.load().exl3_moe_glu_had_in(gu.data_ptr(), slots, inter, ids.data_ptr(), suh_down.shape[0],
                                               suh_down.data_ptr(), act.data_ptr(), out.data_ptr(),
                                               _stream(gu.device)), "moe_glu_had_in")
    return act, out


def moe_combine(yd: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor, num_experts: int,
                out: torch.Tensor | None = None, out_dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """y [tokens, hidden] = sum_j w[t, j] * yd[t * top_k + j] in fp32, slot order, one rounding; slots with ids outside
    [0, num_experts) skipped (the reference's moe_combine, cuda/csrc/exl3_marlin_moe.cu:479-500)."""
    if yd.dtype != torch.float16 or yd.dim() != 2 or not yd.is_contiguous():
        raise ValueError("yd must be a contiguous fp16 [slots, hidden] tensor")
    ids = _routing_ids(topk_ids, yd.device)
    if ids.dim() != 2 or tuple(topk_weights.shape) != tuple(ids.shape) or ids.numel() != yd.shape[0]:
        raise ValueError(f"topk_ids {tuple(ids.shape)} / topk_weights {tuple(topk_weights.shape)} do not match "
                         f"{yd.shape[0]} rows")
    if topk_weights.device != yd.device:
        raise ValueError("topk_weights must be on yd's device")
    w = topk_weights.to(torch.float32).contiguous()
    T, top_k = ids.shape
    if out is None:
        out = torch.empty((T, yd.shape[1]), dtype=out_dtype, device=yd.device)
    _check_out(out, (T, yd.shape[1]), yd)
    _lib.check(_lib.load().exl3_moe_combine(yd.data_ptr(), w.data_ptr(), ids.data_ptr(), T, top_k, yd.shape[1],
                                            int(num_experts), out.data_ptr(), int(out.dtype == torch.bfloat16),
                                            _stream(yd.device)), "moe_combine")
    return out


def kv_decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, k_scale: torch.Tensor,
                        v_scale: torch.Tensor, page_table: torch.Tensor, seq_lens: torch.Tensor, bits: int,
                        sm_scale: float | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Single-token decode attention over a quantized paged KV cache (split-KV + log-sum-exp merge; the merge follows
    xpu/exl3xpu/fp8kv_prefill.py:85-117).  q fp16 [B, Hq, 128]; k_cache / v_cache int8 [P, Hkv, 16, 128] (bits=8)
    or uint8 [P, Hkv, 16, 64] (bits=4, packed nibbles); k_scale / v_scale fp16 [P, Hkv]; page_table int32
    [B, max_pages]; seq_lens int32 [B].  Returns fp16 [B, Hq, 128]."""
    if bits not in (4, 8):
        raise ValueError(f"bits must be 4 or 8, got {bits}")
    if q.dtype != torch.float16 or q.dim() != 3:
        raise ValueError("q must be fp16 [B, Hq, D]")
    B, Hq, D = q.shape
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise ValueError("k_cache / v_cache must have the same [P, Hkv, page, row] shape")
    P, Hkv, page, row = k_cache.shape
    if row != (D if bits == 8 else D // 2):
        raise ValueError(f"cache row of {row} bytes does not hold {D} {bits}-bit codes")
    if k_cache.element_size() != 1 or v_cache.element_size() != 1:
        raise ValueError("caches must hold 1-byte codes (int8 / uint8)")
    for name, t in (("k_scale", k_scale), ("v_scale", v_scale)):
        if t.dtype != torch.float16 or tuple(t.shape) != (P, Hkv):
            raise ValueError(f"{name} must be fp16 [{P}, {Hkv}]")
    if page_table.dtype != torch.int32 or page_table.dim() != 2 or page_table.shape[0] != B:
        raise ValueError("page_table must be int32 [B, max_pages]")
    if seq_lens.dtype != torch.int32 or tuple(seq_lens.shape) != (B,):
        raise ValueError("seq_lens must be int32 [B]")
    tensors = (q, k_cache, v_cache, k_scale, v_scale, page_table, seq_lens)
    if not all(t.is_cuda and t.is_contiguous() and t.device == q.device for t in tensors):
        raise ValueError("all inputs must be contiguous CUDA tensors on one device")
    if sm_scale is None:
        sm_scale = D ** -0.5
    if out is None:
        out = torch.empty((B, Hq, D), dtype=torch.float16, device=q.device)
    _check_out(out, (B, Hq, D), q, (torch.float16,))
    lib = _lib.load()
    max_pages = page_table.shape[1]
    ws = workspace(q.device, lib.exl3_kv_decode_workspace_bytes(B, Hq, Hkv, max_pages), "kv")
    _lib.check(lib.exl3_kv_decode_attention(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_scale.data_ptr(),
                                            v_scale.data_ptr(), P, page_table.data_ptr(), max_pages,
                                            seq_lens.data_ptr(), B, Hq, Hkv, D, page, int(bits), float(sm_scale),
                                            out.data_ptr(), ws.data_ptr(), ws.numel(), _stream(q.device)),
               "kv_decode_attention")
    return out
