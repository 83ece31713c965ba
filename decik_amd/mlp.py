"""Qwen2 MLP on NF4 weights: down(silu(gate(x)) * up(x)) with fused dequant-GEMMs.

Mirrors the reference's RecomputedMLP (solution/mlp.py:62-110) and its patch of Qwen2MLP
(solution/mlp.py:113-162):
- forward: gate and up share x, so they are ONE fused launch (two weights, one X tile stream)
  whose epilogue also applies SwiGLU; down is a second fused launch. Output fp16, as the
  reference returns.
- backward: gate and up are recomputed (recompute=True, the reference's default) or kept from
  the forward; dH = dY . W_down and the SwiGLU backward are one fused launch; then
  dX = dgate . W_gate + dup . W_up as ONE fused launch that accumulates both products in fp32
  and rounds once (the reference sums two fp16 matmul results in fp32, solution/mlp.py:106-109).
No fp16 weight is ever materialised.
"""

import torch

from . import nf4
from ._state import on_gpu


def _w(module):
    return module.weight.data, module.weight.quant_state


def _bias16(module):
    b = getattr(module, "bias", None)
    return None if b is None else b.to(torch.float16)


def mlp_forward(x16, gate, up, down, bias=(None, None, None), keep_gate_up=True):
    """(out, gate_out, up_out) for (packed, quant_state) pairs gate/up/down; x16 [M, K] fp16.
    keep_gate_up=False: gate_out and up_out are not stored (None)."""
    g, u, h = nf4.glu_forward(x16, dict(packed=gate[0], qs=gate[1], bias=bias[0]),
                              dict(packed=up[0], qs=up[1], bias=bias[1]), keep_gate_up=keep_gate_up)
    (out,) = nf4.linear_forward(h, [dict(packed=down[0], qs=down[1], bias=bias[2])])
    return out, g, u


def mlp_backward(grad16, x16, gate, up, down, saved=None, bias=(None, None, None), dx_fp32=False):
    """dX of the MLP; `saved` = (gate_out, up_out) from the forward, else they are recomputed."""
    m, k = x16.shape
    if saved is None:
        # the forward's own launch again (same kernel and plan, so the same bits); h is unused
        g, u, _ = nf4.glu_forward(x16, dict(packed=gate[0], qs=gate[1], bias=bias[0]),
                                  dict(packed=up[0], qs=up[1], bias=bias[1]))
    else:
        g, u = saved
    dgate, dup = nf4.linear_backward_swiglu(dict(packed=down[0], qs=down[1], dy=grad16), g, u,
                                            out=(g, u) if saved is None else None)
    return nf4.linear_backward([dict(packed=gate[0], qs=gate[1], dy=dgate),
                                dict(packed=up[0], qs=up[1], dy=dup)], m, k, dx_fp32=dx_fp32)


class FusedMLP(torch.autograd.Function):
    """down(silu(gate(x)) * up(x)) for the (packed, quant_state) weights; returns fp16 like the
    reference; the input gradient comes back in x's dtype."""

    @staticmethod
    def forward(ctx, x, gate_p, gate_qs, up_p, up_qs, down_p, down_qs, recompute=True,
                biases=(None, None, None)):
        shape = x.shape
        x16 = x.to(torch.float16).reshape(-1, shape[-1]).contiguous()
        gate, up, down = (gate_p, gate_qs), (up_p, up_qs), (down_p, down_qs)
        out, g, u = mlp_forward(x16, gate, up, down, biases, keep_gate_up=not recompute)
        ctx.weights, ctx.biases, ctx.recompute = (gate, up, down), biases, recompute
        ctx.shape, ctx.in_dtype = shape, x.dtype
        if recompute:
            ctx.save_for_backward(x16)
        else:
            ctx.save_for_backward(x16, g, u)
        return out.reshape(*shape[:-1], out.shape[-1])

    @staticmethod
    def backward(ctx, grad_out):
        saved = ctx.saved_tensors
        x16 = saved[0]
        g16 = grad_out.to(torch.float16).reshape(-1, grad_out.shape[-1]).contiguous()
        gate, up, down = ctx.weights
        dx = mlp_backward(g16, x16, gate, up, down, saved=None if ctx.recompute else saved[1:],
                          bias=ctx.biases, dx_fp32=ctx.in_dtype == torch.float32)
        dx = dx.to(ctx.in_dtype).reshape(ctx.shape)
        return dx, None, None, None, None, None, None, None, None


# The reference's class name for the same computation (solution/mlp.py:62).
RecomputedMLP = FusedMLP


def patch(recompute=False):
    """Send Qwen2MLP.forward through FusedMLP for fp32 input on NF4 fp16-compute projections,
    with the reference's gates (solution/mlp.py:113-162); anything else keeps the original."""
    import bitsandbytes as bnb
    from transformers.models.qwen2 import modeling_qwen2

    cls = modeling_qwen2.Qwen2MLP
    if getattr(cls.forward, "_skc", False):
        return
    original = cls.forward
    linear4bit = bnb.nn.Linear4bit

    def fp16_projection(module):
        return isinstance(module, linear4bit) and getattr(module, "compute_dtype", None) == torch.float16

    def usable(module, n_in):
        weight = getattr(module, "weight", None)
        bias = getattr(module, "bias", None)
        qs = getattr(weight, "quant_state", None)
        return (weight is not None and on_gpu(weight) and weight.dtype == torch.uint8
                and not weight.requires_grad and (bias is None or not bias.requires_grad)
                and nf4.supported(qs, n_in) and nf4.fused_ok(qs, n_in))

    def forward(self, x):
        config = getattr(self, "config", None)
        projections = [getattr(self, name, None) for name in ("gate_proj", "up_proj", "down_proj")]
        if not (isinstance(x, torch.Tensor) and on_gpu(x) and x.dtype == torch.float32
                and x.numel() > 0 and getattr(config, "hidden_act", None) == "silu"
                and all(fp16_projection(p) for p in projections)):
            return original(self, x)
        gate_proj, up_proj, down_proj = projections
        if not (usable(gate_proj, x.shape[-1]) and usable(up_proj, x.shape[-1])
                and usable(down_proj, gate_proj.weight.quant_state.shape[0])):
            return original(self, x)
        biases = tuple(_bias16(p) for p in projections)
        return FusedMLP.apply(x, *_w(gate_proj), *_w(up_proj), *_w(down_proj), recompute, biases)

    forward._skc = True
    cls.forward = forward
