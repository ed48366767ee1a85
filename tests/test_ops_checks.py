"""Argument checks of the torch-facing ops that stand between a caller and a raw device write: a caller-supplied
`out` must be exactly what the kernels write (shape, dtype, contiguity, device), and routing tensors must have the
shapes the C code reads.  The CPU tests exercise the shared check on host tensors; the `gpu` tests call the ops."""
import pytest
import torch

from trellis_serve_amd import ops


def test_check_out_rejects_what_the_kernels_cannot_write():
    like = torch.empty((3, 256), dtype=torch.float16)
    ops._check_out(torch.empty((3, 256), dtype=torch.float16), (3, 256), like)
    ops._check_out(torch.empty((3, 256), dtype=torch.bfloat16), (3, 256), like)
    with pytest.raises(ValueError, match="shape"):
        ops._check_out(torch.empty((3, 128), dtype=torch.float16), (3, 256), like)
    with pytest.raises(ValueError, match="must be one of"):
        ops._check_out(torch.empty((3, 256), dtype=torch.float32), (3, 256), like)
    with pytest.raises(ValueError, match="must be one of"):
        ops._check_out(torch.empty((3, 256), dtype=torch.bfloat16), (3, 256), like, (torch.float16,))
    with pytest.raises(ValueError, match="contiguous"):
        ops._check_out(torch.empty((256, 3), dtype=torch.float16).t(), (3, 256), like)
    with pytest.raises(ValueError, match="is on"):
        ops._check_out(torch.empty((3, 256), dtype=torch.float16, device="meta"), (3, 256), like)


def _group(k, ns, K=3, dev="cuda"):
    g = torch.Generator().manual_seed(1)
    trs = [torch.randint(-32768, 32768, (k // 16, n // 16, 16 * K), dtype=torch.int16, generator=g).to(dev) for n in ns]
    suhs = [torch.ones(k, dtype=torch.float16, device=dev) for _ in ns]
    svhs = [torch.ones(n, dtype=torch.float16, device=dev) for n in ns]
    return trs, suhs, svhs


@pytest.mark.gpu
def test_ops_reject_bad_out_and_routing_before_launching():
    trs, suhs, svhs = _group(256, [128, 256])
    x = torch.randn((2, 256), dtype=torch.float16, device="cuda")
    for bad in (torch.empty((2, 256), dtype=torch.float16, device="cuda"),          # too narrow
                torch.empty((2, 384), dtype=torch.float32, device="cuda"),          # fp32
                torch.empty((384, 2), dtype=torch.float16, device="cuda").t()):     # not contiguous
        with pytest.raises(ValueError):
            ops.linear(x, trs, suhs, svhs, 1, out=bad)
        with pytest.raises(ValueError):
            ops.linear_prefill(x, trs, suhs, svhs, 1, out=bad)
    E, H, I = 4, 256, 128
    g = torch.Generator().manual_seed(2)
    experts = {}
    for proj, (k, n) in {"gate": (H, I), "up": (H, I), "down": (I, H)}.items():
        experts[f"{proj}_trellis"] = torch.randint(-32768, 32768, (E, k // 16, n // 16, 48), dtype=torch.int16,
                                                   generator=g).cuda()
        experts[f"{proj}_suh"] = torch.ones((E, k), dtype=torch.float16, device="cuda")
        experts[f"{proj}_svh"] = torch.ones((E, n), dtype=torch.float16, device="cuda")
    xm = torch.randn((3, H), dtype=torch.float16, device="cuda")
    ids = torch.zeros((3, 2), dtype=torch.int32, device="cuda")
    w = torch.full((3, 2), 0.5, device="cuda")
    with pytest.raises(ValueError, match="top_k"):
        ops.moe_forward(xm, ids, w[:, :1].contiguous(), experts, 1)      # weights of another shape
    with pytest.raises(ValueError, match="top_k"):
        ops.moe_forward(xm, ids[:2], w[:2], experts, 1)                  # fewer routing rows than tokens
    with pytest.raises(ValueError):
        ops.moe_forward(xm, ids, w, experts, 1, out=torch.empty((3, H), dtype=torch.float32, device="cuda"))
