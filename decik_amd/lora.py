"""LoRA on NF4 projections with the rank-r term fused into the GEMM epilogue.

peft's branch for a 4-bit layer under fp16 autocast is lora_B(lora_A(dropout(x))) * scaling
(solution/attn.py:344-346); LoRAPairFromNorm restates it for q and v (solution/attn.py:206-273):
  forward:  u = fp16(x . A^T)  [M, r];  out = fp16(u . B^T) * s, added to the projection output
  backward: g = dY * s; dB = g^T u; gu = g . B; dA = gu^T x; dX_lora = gu . A
Here the base projection and the LoRA term are one launch in each direction: the forward GEMM's
epilogue adds s * U.B^T (an extra rank-r MFMA per output tile) before the single fp16 rounding,
and the backward GEMM's epilogue adds GU.A to dX. U and GU come from small HIP kernels
(dk_lora_down, dk_lora_bwd), which also produce dA and dB in fp32. Dropout is not applied
(p = 0); its masks are a later addition.
"""

import torch

from . import nf4 as _nf4
from ._lib import check, lib, ptr, stream_of


def lora_down(x16, a16):
    """U = fp16(X . A^T): X fp16 [M, K], A fp16 [r, K] -> [M, r]."""
    x2 = x16.reshape(-1, x16.shape[-1])
    m, k = x2.shape
    r = a16.shape[0]
    u = torch.empty((m, r), dtype=torch.float16, device=x16.device)
    check(lib().dk_lora_down(ptr(x2), m, k, x2.stride(0), ptr(a16), r, ptr(u), stream_of(x16.device)))
    return u


def lora_grads(dy16, u16, x16, b16, scaling, want_da=True, want_db=True):
    """(GU fp16 [M, r], dA fp32 [r, K], dB fp32 [N, r]) for out = s * (U . B^T), U = X . A^T."""
    dy2 = dy16.reshape(-1, dy16.shape[-1])
    x2 = x16.reshape(-1, x16.shape[-1])
    m, n = dy2.shape
    k = x2.shape[1]
    r = u16.shape[1]
    dev = dy16.device
    gu = torch.empty((m, r), dtype=torch.float16, device=dev)
    da = torch.empty((r, k), dtype=torch.float32, device=dev) if want_da else None
    db = torch.empty((n, r), dtype=torch.float32, device=dev) if want_db else None
    check(lib().dk_lora_bwd(ptr(dy2), dy2.stride(0), ptr(u16), ptr(x2), x2.stride(0), ptr(b16), m, n, k,
                            r, float(scaling), ptr(gu), ptr(da), ptr(db), stream_of(dev)))
    return gu, da, db


class NF4LoRALinear(torch.autograd.Function):
    """Y = x16 . dequant(W)^T + bias + scaling * fp16(x16 . A^T) . B^T in one fused launch.

    x16 fp16 [.., K]; lora_a [r, K] and lora_b [N, r] are the adapter weights (any float dtype;
    used in fp16 as under autocast); gradients flow to x16, lora_a and lora_b."""

    @staticmethod
    def forward(ctx, x16, packed, bias16, quant_state, lora_a, lora_b, scaling):
        x2 = x16.reshape(-1, x16.shape[-1]).contiguous()
        a16 = lora_a.to(torch.float16).contiguous()
        b16 = lora_b.to(torch.float16).contiguous()
        u = lora_down(x2, a16)
        (y,) = _nf4.linear_forward(x2, [dict(packed=packed, qs=quant_state, bias=bias16, lora_u=u,
                                             lora_b=b16, lora_scale=scaling)],
                                   lora_rank=a16.shape[0])
        ctx.save_for_backward(x2, u, a16, b16)
        ctx.packed, ctx.quant_state, ctx.scaling = packed, quant_state, scaling
        ctx.x_shape, ctx.dtypes = x16.shape, (lora_a.dtype, lora_b.dtype)
        return y.reshape(*x16.shape[:-1], y.shape[-1])

    @staticmethod
    def backward(ctx, grad_out):
        x2, u, a16, b16 = ctx.saved_tensors
        g16 = grad_out.to(torch.float16).reshape(-1, grad_out.shape[-1]).contiguous()
        gu, da, db = lora_grads(g16, u, x2, b16, ctx.scaling, ctx.needs_input_grad[4],
                                ctx.needs_input_grad[5])
        grad_x = None
        if ctx.needs_input_grad[0]:
            m, k = x2.shape
            grad_x = _nf4.linear_backward([dict(packed=ctx.packed, qs=ctx.quant_state, dy=g16,
                                                lora_gu=gu, lora_a=a16)], m, k,
                                          lora_rank=a16.shape[0]).reshape(ctx.x_shape)
        da = None if da is None else da.to(ctx.dtypes[0])
        db = None if db is None else db.to(ctx.dtypes[1])
        return grad_x, None, None, None, da, db, None


class QKVProjection(torch.autograd.Function):
    """q, k, v = x16 . W_{q,k,v}^T + b_{q,k,v} (+ LoRA on any of them) in one fused forward launch
    and one fused backward launch for dX = sum of the three input gradients (+ LoRA terms), the
    call order of solution/attn.py:396-407 without the dropout draws.

    projections: tuple of 3 dicts {packed, qs, bias, lora_a, lora_b, scaling} (lora_* may be
    None); the adapter tensors are passed again as flat arguments so autograd sees them."""

    @staticmethod
    def forward(ctx, x16, projections, *adapters):
        x2 = x16.reshape(-1, x16.shape[-1]).contiguous()
        items, saved, rank = [], [], 0
        for p in projections:
            it = dict(packed=p["packed"], qs=p["qs"], bias=p.get("bias"))
            if p.get("lora_a") is not None:
                a16 = p["lora_a"].to(torch.float16).contiguous()
                b16 = p["lora_b"].to(torch.float16).contiguous()
                u = lora_down(x2, a16)
                it.update(lora_u=u, lora_b=b16, lora_scale=p["scaling"])
                rank = a16.shape[0]
                saved.append((u, a16, b16))
            else:
                saved.append(None)
            items.append(it)
        outs = _nf4.linear_forward(x2, items, lora_rank=rank)
        ctx.projections, ctx.saved_lora, ctx.rank = projections, saved, rank
        ctx.save_for_backward(x2)
        ctx.x_shape = x16.shape
        return tuple(o.reshape(*x16.shape[:-1], o.shape[-1]) for o in outs)

    @staticmethod
    def backward(ctx, *grads):
        (x2,) = ctx.saved_tensors
        m, k = x2.shape
        items, adapter_grads = [], []
        for p, sv, g in zip(ctx.projections, ctx.saved_lora, grads):
            if g is None:
                g = torch.zeros((m, int(p["qs"].shape[0])), dtype=torch.float16, device=x2.device)
            g16 = g.to(torch.float16).reshape(m, -1).contiguous()
            it = dict(packed=p["packed"], qs=p["qs"], dy=g16)
            if sv is not None:
                u, a16, b16 = sv
                gu, da, db = lora_grads(g16, u, x2, b16, p["scaling"])
                it.update(lora_gu=gu, lora_a=a16)
                adapter_grads += [da.to(p["lora_a"].dtype), db.to(p["lora_b"].dtype)]
            items.append(it)
        grad_x = _nf4.linear_backward(items, m, k, lora_rank=ctx.rank).reshape(ctx.x_shape)
        return (grad_x, None, *adapter_grads)


def qkv_projection(x16, projections):
    adapters = []
    for p in projections:
        if p.get("lora_a") is not None:
            adapters += [p["lora_a"], p["lora_b"]]
    return QKVProjection.apply(x16, projections, *adapters)
