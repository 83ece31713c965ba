"""Qwen2 MLP on NF4 weights: down(silu(gate(x)) * up(x)) with fused dequant-GEMMs.

Module API of the reference's solution/mlp.py: `_weight16`, `_linear16_with`, `_linear16`
(:28-39), `RecomputedMLP` (:62-110, same `apply` signature) and `patch` (:113-162). Underneath:
- forward: gate and up share x, so they are ONE fused launch (two weights, one X tile stream)
  whose epilogue also applies SwiGLU; down is a second fused launch. Output fp16, as the
  reference returns.
- backward: gate and up are recomputed (the reference's RecomputedMLP) or kept from the forward;
  dH = dY . W_down and the SwiGLU backward are one fused launch; then
  dX = dgate . W_gate + dup . W_up is ONE fused launch that accumulates both products in fp32 and
  rounds once (the reference rounds each fp16 matmul result and sums the two in fp32,
  solution/mlp.py:106-109; the difference is one fp16 rounding per product, within the bar).
No fp16 weight is ever materialised on the fused path. Weights the fused kernels do not take
run the reference's own algorithm on the GPU (dequantize, fp16 matmul, the SwiGLU kernels).
"""

import torch

from . import _state, nf4
from .swiglu import swiglu_bwd, swiglu_fwd


def _weight16(module):
    """The fp16 weight of an NF4 Linear4bit (solution/mlp.py:28-29)."""
    return nf4.dequantize_nf4(module.weight.data, module.weight.quant_state)


def _bias16(module):
    b = getattr(module, "bias", None)
    return None if b is None else b.to(torch.float16)


def _linear16_with(x16, weight16, module):
    """F.linear in fp16 with an already dequantized weight (solution/mlp.py:32-34)."""
    return torch.nn.functional.linear(x16, weight16, _bias16(module))


def _linear16(x16, module):
    """What bitsandbytes' Linear4bit computes for an fp16 input (solution/mlp.py:37-39), as one
    fused dequant-GEMM launch when the kernels take the weight."""
    qs = module.weight.quant_state
    packed = module.weight.data
    if nf4.fused_ok(qs, x16.shape[-1]) and x16.is_contiguous() and x16.numel() > 0:
        (y,) = nf4.linear_forward(x16, [dict(packed=packed, qs=qs, bias=_bias16(module))])
        return y.reshape(*x16.shape[:-1], y.shape[-1])
    return _linear16_with(x16, _weight16(module), module)


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


def _all_fused(x16, weights):
    k = x16.shape[-1]
    (_, gq), (_, uq), (_, dq) = weights
    return (nf4.fused_ok(gq, k) and nf4.fused_ok(uq, k) and nf4.fused_ok(dq, int(gq.shape[0]))
            and tuple(gq.shape) == tuple(uq.shape))


def _mlp_forward_any(x16, weights, biases, keep_gate_up):
    """(out, gate, up): the fused launches, or the reference's dequantize + fp16 matmul chain."""
    if _all_fused(x16, weights):
        return mlp_forward(x16, *weights, biases, keep_gate_up=keep_gate_up)
    (gp, gq), (up_, uq), (dp, dq) = weights
    gate = torch.nn.functional.linear(x16, nf4.dequantize_nf4(gp, gq), biases[0])
    up = torch.nn.functional.linear(x16, nf4.dequantize_nf4(up_, uq), biases[1])
    out = torch.nn.functional.linear(swiglu_fwd(gate, up), nf4.dequantize_nf4(dp, dq), biases[2])
    return out, (gate if keep_gate_up else None), (up if keep_gate_up else None)


def _mlp_backward_any(g16, x16, weights, biases, saved, in_dtype):
    """dX in in_dtype: the fused launches, or the reference's chain (solution/mlp.py:93-109)."""
    if _all_fused(x16, weights):
        dx = mlp_backward(g16, x16, *weights, saved=saved, bias=biases,
                          dx_fp32=in_dtype == torch.float32)
        return dx.to(in_dtype)
    (gp, gq), (up_, uq), (dp, dq) = weights
    grad_hidden = torch.matmul(g16, nf4.dequantize_nf4(dp, dq))
    w_gate, w_up = nf4.dequantize_nf4(gp, gq), nf4.dequantize_nf4(up_, uq)
    if saved is None:
        gate = torch.nn.functional.linear(x16, w_gate, biases[0])
        up = torch.nn.functional.linear(x16, w_up, biases[1])
        dgate, dup = swiglu_bwd(grad_hidden, gate, up, out=(gate, up))
    else:
        dgate, dup = swiglu_bwd(grad_hidden, *saved)
    return torch.matmul(dgate, w_gate).to(in_dtype) + torch.matmul(dup, w_up).to(in_dtype)


def _forward(ctx, x, weights, biases, recompute):
    shape = x.shape
    x16 = x.to(torch.float16).reshape(-1, shape[-1]).contiguous()
    out, g, u = _mlp_forward_any(x16, weights, biases, keep_gate_up=not recompute)
    ctx.weights, ctx.biases, ctx.recompute = weights, biases, recompute
    ctx.shape, ctx.in_dtype = shape, x.dtype
    if recompute:
        ctx.save_for_backward(x16)
    else:
        ctx.save_for_backward(x16, g, u)
    return out.reshape(*shape[:-1], out.shape[-1])


def _backward(ctx, grad_out):
    saved = ctx.saved_tensors
    x16 = saved[0]
    g16 = grad_out.to(torch.float16).reshape(-1, grad_out.shape[-1]).contiguous()
    dx = _mlp_backward_any(g16, x16, ctx.weights, ctx.biases,
                           None if ctx.recompute else tuple(saved[1:]), ctx.in_dtype)
    return dx.reshape(ctx.shape)


class FusedMLP(torch.autograd.Function):
    """down(silu(gate(x)) * up(x)) for (packed, quant_state) weights; returns fp16 like the
    reference; the input gradient comes back in x's dtype. recompute=False keeps gate and up
    from the forward instead of recomputing them (same bits either way)."""

    @staticmethod
    def forward(ctx, x, gate_p, gate_qs, up_p, up_qs, down_p, down_qs, recompute=True,
                biases=(None, None, None)):
        return _forward(ctx, x, ((gate_p, gate_qs), (up_p, up_qs), (down_p, down_qs)), biases,
                        recompute)

    @staticmethod
    def backward(ctx, grad_out):
        return (_backward(ctx, grad_out),) + (None,) * 8


def _module_weight(module):
    return module.weight.data, module.weight.quant_state


class RecomputedMLP(torch.autograd.Function):
    """The reference's RecomputedMLP.apply(x, gate_proj, up_proj, down_proj[, norm_input,
    norm_weight, eps, norm_delta]) on Linear4bit modules (solution/mlp.py:62-110): only the fp16
    input is saved and gate/up are recomputed in backward. The reference can rebuild that input
    from the RMSNorm's (bit-identically, :86-89); the RMSNorm kernel is outside this package, so
    the norm arguments are accepted and the fp16 input is kept instead -- the same numbers."""

    @staticmethod
    def forward(ctx, x, gate_proj, up_proj, down_proj, norm_input=None, norm_weight=None, eps=None,
                norm_delta=None):
        mods = (gate_proj, up_proj, down_proj)
        weights = tuple(_module_weight(m) for m in mods)
        biases = tuple(_bias16(m) for m in mods)
        return _forward(ctx, x, weights, biases, recompute=True)

    @staticmethod
    def backward(ctx, grad_out):
        return (_backward(ctx, grad_out),) + (None,) * 7


# ---- transformers' Qwen2MLP.forward, patched (solution/mlp.py:113-162) ---------------------------
# Same conditions as the reference, one predicate each; anything else keeps the original forward.

def _fp32_gpu_input(x):
    return isinstance(x, torch.Tensor) and _state.on_gpu(x) and x.dtype == torch.float32


def _silu_mlp(module):
    return getattr(getattr(module, "config", None), "hidden_act", None) == "silu"


def _frozen_nf4_projection(module, n_in):
    """A Linear4bit whose frozen NF4 weight the path takes (the reference's `recomputable`,
    :128-133, plus the fused kernels' shape conditions)."""
    weight = getattr(module, "weight", None)
    if weight is None or not nf4._frozen_nf4_bytes(weight):
        return False
    if not nf4._frozen_or_absent(getattr(module, "bias", None)):
        return False
    qs = getattr(weight, "quant_state", None)
    return nf4.supported(qs, n_in) and nf4.fused_ok(qs, n_in)


def patch(recompute=False):
    """Route Qwen2MLP.forward through the fused MLP for an fp32 GPU input on fp16-compute NF4
    projections (solution/mlp.py:113-162). recompute=True saves only the fp16 input and
    recomputes gate/up in backward (the reference's RecomputedMLP); False keeps them."""
    import bitsandbytes as bnb
    from transformers.models.qwen2 import modeling_qwen2

    cls = modeling_qwen2.Qwen2MLP
    if getattr(cls.forward, "_skc", False):
        return
    qwen_forward = cls.forward
    linear4bit = bnb.nn.Linear4bit

    def fp16_nf4(module):
        return isinstance(module, linear4bit) and nf4._fp16_compute(module)

    def forward(self, x):
        gate_proj, up_proj, down_proj = (getattr(self, n, None) for n in ("gate_proj", "up_proj", "down_proj"))
        if not (_fp32_gpu_input(x) and x.numel() > 0 and _silu_mlp(self)
                and all(fp16_nf4(p) for p in (gate_proj, up_proj, down_proj))):
            return qwen_forward(self, x)
        width = x.shape[-1]
        if not (_frozen_nf4_projection(gate_proj, width) and _frozen_nf4_projection(up_proj, width)
                and _frozen_nf4_projection(down_proj, int(gate_proj.weight.quant_state.shape[0]))):
            return qwen_forward(self, x)
        if recompute:
            return RecomputedMLP.apply(x, gate_proj, up_proj, down_proj)
        weights = [t for p in (gate_proj, up_proj, down_proj) for t in _module_weight(p)]
        return FusedMLP.apply(x, *weights, False, tuple(_bias16(p) for p in (gate_proj, up_proj, down_proj)))

    forward._skc = True
    cls.forward = forward
