"""SwiGLU between the gate/up and down projections, on the HIP kernels swiglu_fwd/bwd_kernel.

Same computation as the reference's example kernels (solution/swiglu.py:15-37): fp32 math,
fp16 results; `swiglu(gate, up)` is the autograd entry point (solution/swiglu.py:40-61,226)."""

import torch

from ._lib import check, lib, ptr, stream_of


def swiglu_fwd(gate, up, out=None):
    gate = gate.contiguous()
    up = up.to(gate.dtype).contiguous()
    assert gate.dtype == torch.float16 and gate.shape == up.shape
    if out is None:
        out = torch.empty_like(gate)
    check(lib().dk_swiglu_fwd(ptr(gate), ptr(up), ptr(out), gate.numel(), stream_of(gate.device)))
    return out


def swiglu_bwd(grad, gate, up, out=None):
    """(dgate, dup); out=(gate, up) computes them in place."""
    grad = grad.to(torch.float16).contiguous()
    dgate, dup = out if out is not None else (torch.empty_like(gate), torch.empty_like(up))
    check(lib().dk_swiglu_bwd(ptr(grad), ptr(gate), ptr(up), ptr(dgate), ptr(dup), gate.numel(),
                              stream_of(gate.device)))
    return dgate, dup


class SwiGLU(torch.autograd.Function):
    """silu(gate) * up in one launch each way."""

    @staticmethod
    def forward(ctx, gate, up):
        gate = gate.contiguous()
        up = up.to(gate.dtype).contiguous()
        ctx.save_for_backward(gate, up)
        return swiglu_fwd(gate, up)

    @staticmethod
    def backward(ctx, grad):
        gate, up = ctx.saved_tensors
        return swiglu_bwd(grad, gate, up)


def swiglu(gate, up):
    return SwiGLU.apply(gate, up)
