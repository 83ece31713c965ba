"""LoRA on NF4 projections with the rank-r term fused into the GEMM epilogue.

peft's branch for a 4-bit layer under fp16 autocast is lora_B(lora_A(dropout(x))) * scaling
(solution/attn.py:344-346); LoRAPairFromNorm restates it for q and v (solution/attn.py:206-273):
  forward:  u = fp16(x . A^T)  [M, r];  out = fp16(u . B^T) * s, added to the projection output
  backward: g = dY * s; dB = g^T u; gu = g . B; dA = gu^T x; dX_lora = gu . A
Here the base projection and the LoRA term are one launch in each direction: the forward GEMM's
epilogue adds s * U.B^T (an extra rank-r MFMA per output tile) before the single fp16 rounding,
and the backward GEMM's epilogue adds GU.A to dX. U and GU come from small HIP kernels
(dk_lora_down, dk_lora_bwd), which also produce dA and dB in fp32. With dropout (p > 0) the
fused q/k/v launches (QKVProjection, QKVRopeProjection) take the packed keep-masks: U and dA
rebuild fp16(x * (keep * scale)) in registers (dk_lora_down_dropout, dk_lora_bwd_dropout) and the
backward GEMM masks each branch's input gradient in its epilogue, so no dropped-out input or
per-branch input gradient is ever stored. LoRAPair / LoRAPairFromNorm keep the reference's
separate branch (packed keep-masks, dropped-out fp16 inputs, the input gradient through the
masks: dk_lora_keep_pack, dk_lora_dropout_inputs, dk_lora_up, dk_lora_input_grad).
"""

import torch

from . import nf4 as _nf4
from ._lib import check, lib, ptr, stream_of


def _plain(x, keep_bits):
    return keep_bits is None and x.dtype == torch.float16


def _keep_args(x2, keep_bits, keep_scale):
    if keep_bits is None:
        return None, None
    m, k = x2.shape
    assert keep_bits.dtype == torch.uint8 and keep_bits.is_contiguous() and keep_bits.numel() == m * (k // 8)
    return keep_bits, keep_scale.to(torch.float32).reshape(1).contiguous()


def lora_down(x, a16, keep_bits=None, keep_scale=None):
    """U = fp16(X . A^T) [M, r] for A fp16 [r, K]. X = x for fp16 x [M, K]; for fp32 x, or with a
    dropout mask (keep_bits: packed keep bits [M, K / 8] from pack_keep, keep_scale: fp32 device
    scalar 1 / (1 - p)), X = fp16(x * (keep * scale)) is built inside the kernel
    (dk_lora_down_dropout), as skc_lora_inputs_kernel rounds it (solution/attn.py:153-165)."""
    x2 = x.reshape(-1, x.shape[-1])
    m, k = x2.shape
    r = a16.shape[0]
    u = torch.empty((m, r), dtype=torch.float16, device=x.device)
    if _plain(x, keep_bits):
        check(lib().dk_lora_down(ptr(x2), m, k, x2.stride(0), ptr(a16), r, ptr(u), stream_of(x.device)))
        return u
    bits, sc = _keep_args(x2, keep_bits, keep_scale)
    check(lib().dk_lora_down_dropout(ptr(x2), 1 if x2.dtype == torch.float32 else 0, m, k, x2.stride(0),
                                     ptr(bits), ptr(sc), ptr(a16), r, ptr(u), stream_of(x.device)))
    return u


def lora_grads(dy16, u16, x, b16, scaling, want_da=True, want_db=True, keep_bits=None, keep_scale=None):
    """(GU fp16 [M, r], dA fp32 [r, K], dB fp32 [N, r]) for out = s * (U . B^T), U = X . A^T, with X
    from x (and the dropout mask) as lora_down builds it."""
    dy2 = dy16.reshape(-1, dy16.shape[-1])
    x2 = x.reshape(-1, x.shape[-1])
    m, n = dy2.shape
    k = x2.shape[1]
    r = u16.shape[1]
    dev = dy16.device
    gu = torch.empty((m, r), dtype=torch.float16, device=dev)
    da = torch.empty((r, k), dtype=torch.float32, device=dev) if want_da else None
    db = torch.empty((n, r), dtype=torch.float32, device=dev) if want_db else None
    if _plain(x, keep_bits):
        check(lib().dk_lora_bwd(ptr(dy2), dy2.stride(0), ptr(u16), ptr(x2), x2.stride(0), ptr(b16), m, n, k,
                                r, float(scaling), ptr(gu), ptr(da), ptr(db), stream_of(dev)))
        return gu, da, db
    bits, sc = _keep_args(x2, keep_bits, keep_scale)
    check(lib().dk_lora_bwd_dropout(ptr(dy2), dy2.stride(0), ptr(u16), ptr(x2),
                                    1 if x2.dtype == torch.float32 else 0, x2.stride(0), ptr(bits), ptr(sc),
                                    ptr(b16), m, n, k, r, float(scaling), ptr(gu), ptr(da), ptr(db),
                                    stream_of(dev)))
    return gu, da, db


def pack_keep(keep_q, keep_v):
    """Two bool keep-masks [T, W] (W % 8 == 0) -> bit-packed uint8 [T, W / 8] each
    (pack_keep, solution/attn.py:195-203)."""
    rows, width = keep_q.shape
    bq = torch.empty((rows, width // 8), dtype=torch.uint8, device=keep_q.device)
    bv = torch.empty_like(bq)
    kq, kv = keep_q.contiguous().view(torch.uint8), keep_v.contiguous().view(torch.uint8)
    check(lib().dk_lora_keep_pack(ptr(kq), ptr(kv), ptr(bq), ptr(bv), rows, width, stream_of(kq.device)))
    return bq, bv


def lora_inputs(x, bits_q, bits_v, scale_q, scale_v):
    """fp16(x * dropout values) of the q and v branches, [T, W] each (_lora_inputs,
    solution/attn.py:183-192). x fp16 or fp32 [.., W]; scale_*: fp32 device scalars (1/(1-p))."""
    width = x.shape[-1]
    x2 = x.reshape(-1, width).contiguous()
    rows = x2.shape[0]
    xq = torch.empty((rows, width), dtype=torch.float16, device=x.device)
    xv = torch.empty_like(xq)
    sq = scale_q.to(torch.float32).reshape(1).contiguous()
    sv = scale_v.to(torch.float32).reshape(1).contiguous()
    check(lib().dk_lora_dropout_inputs(ptr(x2), 1 if x2.dtype == torch.float32 else 0, ptr(bits_q),
                                       ptr(bits_v), ptr(sq), ptr(sv), ptr(xq), ptr(xv), rows, width,
                                       stream_of(x.device)))
    return xq, xv


def lora_input_grad(gq, gv, bits_q, bits_v, scale_q, scale_v):
    """Input gradient of both branches through their dropout, fp32 [T, W]: (g * keep) * 1/(1-p)
    per branch, summed (skc_lora_input_grad_kernel, solution/attn.py:168-180, 259-266)."""
    rows, width = gq.shape
    out = torch.empty((rows, width), dtype=torch.float32, device=gq.device)
    check(lib().dk_lora_input_grad(ptr(gq.contiguous()), ptr(gv.contiguous()), ptr(bits_q), ptr(bits_v),
                                   float(scale_q), float(scale_v), ptr(out), rows, width,
                                   stream_of(gq.device)))
    return out


def lora_up(gu16, a16):
    """A branch's input gradient before dropout: fp16(GU . A) [M, K] (grad_u.mm(a16),
    solution/attn.py:257)."""
    m, r = gu16.shape
    k = a16.shape[1]
    out = torch.empty((m, k), dtype=torch.float16, device=gu16.device)
    check(lib().dk_lora_up(ptr(gu16.contiguous()), ptr(a16.contiguous()), r, ptr(out), m, k,
                           stream_of(gu16.device)))
    return out


class LoRAPair(torch.autograd.Function):
    """The q and v LoRA branches with dropout, lora_B(lora_A(dropout(x))) * scaling each, as
    LoRAPairFromNorm computes them on its packed-mask path (solution/attn.py:206-273): the masks
    are kept packed to bits and backward rebuilds the dropped-out inputs from x. (The reference
    rebuilds x itself from the RMSNorm input; here x is saved.) x: [.., W] fp16 or fp32;
    bits_*: packed keep-masks; scale_*: fp32 device scalars 1/(1-p); a_* [r, W], b_* [N, r]
    adapter weights (used in fp16); returns (out_q, out_v) fp16."""

    @staticmethod
    def forward(ctx, x, bits_q, scale_q, bits_v, scale_v, a_q, b_q, a_v, b_v, scaling_q, scaling_v,
                p_q, p_v):
        inputs = lora_inputs(x, bits_q, bits_v, scale_q, scale_v)
        outs, us = [], []
        for x16, a, b, s in zip(inputs, (a_q, a_v), (b_q, b_v), (scaling_q, scaling_v)):
            a16 = a.to(torch.float16).contiguous()
            u = lora_down(x16, a16)
            # fp16(u . B^T) (the rank-r up product), then * scaling in fp16 as torch scales
            up = lora_up(u, b.to(torch.float16).t().contiguous())
            outs.append(up * s)
            us.append(u)
        ctx.save_for_backward(x, bits_q, scale_q, bits_v, scale_v, us[0], us[1], a_q, b_q, a_v, b_v)
        ctx.scalings, ctx.ps = (scaling_q, scaling_v), (p_q, p_v)
        shape = x.shape[:-1]
        return outs[0].reshape(*shape, -1), outs[1].reshape(*shape, -1)

    @staticmethod
    def backward(ctx, grad_q, grad_v):
        x, bits_q, scale_q, bits_v, scale_v, u_q, u_v, a_q, b_q, a_v, b_v = ctx.saved_tensors
        inputs = lora_inputs(x, bits_q, bits_v, scale_q, scale_v)
        grads, input_grads = [], []
        branches = ((grad_q, u_q, a_q, b_q, ctx.scalings[0]), (grad_v, u_v, a_v, b_v, ctx.scalings[1]))
        for (grad, u, a, b, s), x16 in zip(branches, inputs):
            if grad is None:
                grad = torch.zeros(u.shape[:-1] + (b.shape[0],), dtype=torch.float16, device=u.device)
            g16 = grad.to(torch.float16).reshape(-1, grad.shape[-1]).contiguous()
            a16 = a.to(torch.float16).contiguous()
            gu, da, db = lora_grads(g16, u, x16, b.to(torch.float16).contiguous(), s)
            grads += [da.to(a.dtype), db.to(b.dtype)]
            input_grads.append(lora_up(gu, a16))
        grad_x = lora_input_grad(input_grads[0], input_grads[1], bits_q, bits_v,
                                 1.0 / (1.0 - ctx.ps[0]), 1.0 / (1.0 - ctx.ps[1]))
        return (grad_x.view(x.shape), None, None, None, None, grads[0], grads[1], grads[2], grads[3],
                None, None, None, None)


def _branch_input(x, scaled=None, mask=None, scale=None):
    """fp16(x * dropout) of one branch on the reference's unpacked path (solution/attn.py:219-223,
    240-243): the forward multiplies by `scaled` (the dropout output of ones, x-shaped), the
    backward rebuilds it from the mask and its kept value; no dropout: fp16(x)."""
    width = x.shape[-1]
    if scaled is not None:
        return (x * scaled).to(torch.float16).reshape(-1, width).contiguous()
    if mask is not None:
        return (x * (mask * scale)).to(torch.float16).reshape(-1, width).contiguous()
    return x.to(torch.float16).reshape(-1, width).contiguous()


class LoRAPairFromNorm(torch.autograd.Function):
    """The reference's LoRAPairFromNorm.apply(x, h, norm_weight, eps, scaled_q, mask_q, scale_q,
    scaled_v, mask_v, scale_v, a_q, b_q, a_v, b_v, scaling_q, scaling_v, p_q, p_v, packed)
    (solution/attn.py:206-273): peft's q and v LoRA branches, lora_B(lora_A(dropout(x))) *
    scaling, on this package's kernels.

    packed=True: mask_q / mask_v are bit-packed keep-masks (pack_keep) and scale_q / scale_v fp32
    device scalars; the dropped-out inputs and the input gradient through both masks are the HIP
    kernels of LoRAPair (bit-exact restatements). packed=False: the reference's elementwise
    torch ops on the GPU (`scaled_*` in the forward, mask * scale in the backward; a branch with
    no dropout passes None). The reference rebuilds x in backward from the RMSNorm input h
    (bit-identically, :240); the RMSNorm kernel is outside this package, so x is saved instead and
    h, norm_weight and eps are accepted unused. Returns (out_q, out_v) fp16; gradients flow to x
    (fp32) and the four adapter weights (their dtype)."""

    @staticmethod
    def forward(ctx, x, h, norm_weight, eps, scaled_q, mask_q, scale_q, scaled_v, mask_v, scale_v,
                a_q, b_q, a_v, b_v, scaling_q, scaling_v, p_q, p_v, packed):
        if packed:
            inputs = lora_inputs(x, mask_q, mask_v, scale_q, scale_v)
        else:
            inputs = (_branch_input(x, scaled_q), _branch_input(x, scaled_v))
        outs, us = [], []
        for x16, a, b, s in zip(inputs, (a_q, a_v), (b_q, b_v), (scaling_q, scaling_v)):
            u = lora_down(x16, a.to(torch.float16).contiguous())
            outs.append(lora_up(u, b.to(torch.float16).t().contiguous()) * s)
            us.append(u)
        ctx.save_for_backward(x, mask_q, scale_q, mask_v, scale_v, us[0], us[1], a_q, b_q, a_v, b_v)
        ctx.scalings, ctx.ps, ctx.packed = (scaling_q, scaling_v), (p_q, p_v), packed
        lead = x.shape[:-1]
        return outs[0].reshape(*lead, -1), outs[1].reshape(*lead, -1)

    @staticmethod
    def backward(ctx, grad_q, grad_v):
        x, mask_q, scale_q, mask_v, scale_v, u_q, u_v, a_q, b_q, a_v, b_v = ctx.saved_tensors
        width = x.shape[-1]
        if ctx.packed:
            inputs = lora_inputs(x, mask_q, mask_v, scale_q, scale_v)
        else:
            inputs = (_branch_input(x, None, mask_q, scale_q), _branch_input(x, None, mask_v, scale_v))
        grads, input_grads = [], []
        branches = ((grad_q, u_q, a_q, b_q, ctx.scalings[0]), (grad_v, u_v, a_v, b_v, ctx.scalings[1]))
        for (grad, u, a, b, s), x16 in zip(branches, inputs):
            if grad is None:
                grad = torch.zeros(u.shape[:-1] + (b.shape[0],), dtype=torch.float16, device=u.device)
            g16 = grad.to(torch.float16).reshape(-1, grad.shape[-1]).contiguous()
            gu, da, db = lora_grads(g16, u, x16, b.to(torch.float16).contiguous(), s)
            grads += [da.to(a.dtype), db.to(b.dtype)]
            input_grads.append(lora_up(gu, a.to(torch.float16).contiguous()))
        if ctx.packed:
            grad_x = lora_input_grad(input_grads[0], input_grads[1], mask_q, mask_v,
                                     1.0 / (1.0 - ctx.ps[0]), 1.0 / (1.0 - ctx.ps[1]))
        else:
            grad_x = None
            for gx16, m, p in zip(input_grads, (mask_q, mask_v), ctx.ps):
                gx = gx16.to(torch.float32)
                if m is not None:
                    gx = gx * m.reshape(-1, width) * (1.0 / (1.0 - p))
                grad_x = gx if grad_x is None else grad_x + gx
        return ((grad_x.view(x.shape),) + (None,) * 9 + tuple(grads) + (None,) * 5)


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


def _qkv_inputs(x):
    """(x rows [T, W] as given, fp16 rows for the base GEMM)."""
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    return x2, (x2 if x2.dtype == torch.float16 else x2.to(torch.float16))


def _qkv_forward_items(x2, x16, projections):
    """Forward launch items of q, k, v: U of each LoRA term from the branch input (x16, or x with
    its dropout mask), all of one rank. Returns (items, saved LoRA state per projection, rank)."""
    ranks = {int(p["lora_a"].shape[0]) for p in projections if p.get("lora_a") is not None}
    if len(ranks) > 1:
        # one launch runs one rank (its LoRA slices and the U / B row strides)
        raise ValueError(f"QKV projection: LoRA ranks differ within one launch: {sorted(ranks)}")
    items, saved, rank = [], [], 0
    for p in projections:
        it = dict(packed=p["packed"], qs=p["qs"], bias=p.get("bias"))
        if p.get("lora_a") is not None:
            a16 = p["lora_a"].to(torch.float16).contiguous()
            b16 = p["lora_b"].to(torch.float16).contiguous()
            if p.get("keep_bits") is not None:
                u = lora_down(x2, a16, p["keep_bits"], p["keep_scale"])
            else:
                u = lora_down(x16, a16)
            it.update(lora_u=u, lora_b=b16, lora_scale=p["scaling"])
            rank = a16.shape[0]
            saved.append((u, a16, b16))
        else:
            saved.append(None)
        items.append(it)
    return items, saved, rank


def _qkv_backward(x2, x16, projections, saved, grads, rank):
    """dX of the three projections and their LoRA terms in one launch (dX in x's dtype), and the
    adapter gradients. A branch with dropout: dA from the rebuilt dropped-out input, its input
    gradient masked in the GEMM's epilogue with 1 / (1 - p) (skc_lora_input_grad_kernel's
    scale, solution/attn.py:262-266)."""
    m, k = x2.shape
    items, adapter_grads = [], []
    for p, sv, g in zip(projections, saved, grads):
        if g is None:
            g = torch.zeros((m, int(p["qs"].shape[0])), dtype=torch.float16, device=x2.device)
        g16 = g.to(torch.float16).reshape(m, -1).contiguous()
        it = dict(packed=p["packed"], qs=p["qs"], dy=g16)
        if sv is not None:
            u, a16, b16 = sv
            if p.get("keep_bits") is not None:
                gu, da, db = lora_grads(g16, u, x2, b16, p["scaling"], keep_bits=p["keep_bits"],
                                        keep_scale=p["keep_scale"])
                it.update(lora_keep=p["keep_bits"], lora_keep_scale=1.0 / (1.0 - float(p["p"])))
            else:
                gu, da, db = lora_grads(g16, u, x16, b16, p["scaling"])
            it.update(lora_gu=gu, lora_a=a16)
            adapter_grads += [da.to(p["lora_a"].dtype), db.to(p["lora_b"].dtype)]
        items.append(it)
    grad_x = _nf4.linear_backward(items, m, k, dx_fp32=x2.dtype == torch.float32, lora_rank=rank)
    return grad_x, adapter_grads


class QKVProjection(torch.autograd.Function):
    """q, k, v = x . W_{q,k,v}^T + b_{q,k,v} (+ LoRA on any of them) in one fused forward launch
    and one fused backward launch for dX = sum of the three input gradients (+ LoRA terms), the
    call order of solution/attn.py:396-407.

    x: fp16, or fp32 (the norm output the reference's attention receives; the base projections
    take fp16(x), :398-401, and dX comes back fp32). projections: tuple of 3 dicts {packed, qs,
    bias, lora_a, lora_b, scaling} (lora_* may be None), and for a LoRA branch with dropout
    keep_bits (pack_keep's packed mask [T, W / 8]), keep_scale (fp32 device scalar 1 / (1 - p))
    and p: the branch input is fp16(x * (keep * scale)), built inside the U kernel and again
    for dA, and its input gradient is masked in the backward GEMM's epilogue (LoRAPairFromNorm's
    packed path, solution/attn.py:153-180, 206-273, without the dropped-out inputs in memory).
    The adapter tensors are passed again as flat arguments so autograd sees them."""

    @staticmethod
    def forward(ctx, x, projections, *adapters):
        x2, x16 = _qkv_inputs(x)
        items, saved, rank = _qkv_forward_items(x2, x16, projections)
        outs = _nf4.linear_forward(x16, items, lora_rank=rank)
        ctx.projections, ctx.saved_lora, ctx.rank = projections, saved, rank
        ctx.save_for_backward(x2, x16)
        ctx.x_shape = x.shape
        return tuple(o.reshape(*x.shape[:-1], o.shape[-1]) for o in outs)

    @staticmethod
    def backward(ctx, *grads):
        x2, x16 = ctx.saved_tensors
        grad_x, adapter_grads = _qkv_backward(x2, x16, ctx.projections, ctx.saved_lora, grads, ctx.rank)
        return (grad_x.reshape(ctx.x_shape), None, *adapter_grads)


class QKVRopeProjection(torch.autograd.Function):
    """The attention inputs of a Qwen2 layer in one fused launch each way: q, k, v = x . W^T + b
    (+ LoRA terms, with or without dropout, like QKVProjection), with q and k rotated (RoPE) and
    stored head-major in the launch's epilogue -- the projections and FusedQKRope's forward
    (solution/attn.py:27-66, 396-418) without a token-major q or k in memory. Returns (q [1, H, T,
    D], k [1, HK, T, D], v [T, HK*D]). Backward: the RoPE transpose (the same kernel as
    FusedQKRope's backward, solution/attn.py:69-86), then one fused launch for dX with the LoRA
    terms.

    projections: (q, k, v) dicts as for QKVProjection; cos, sin fp32 [T, D]."""

    @staticmethod
    def forward(ctx, x, projections, cos, sin, n_heads, n_kv_heads, *adapters):
        x2, x16 = _qkv_inputs(x)
        items, saved, rank = _qkv_forward_items(x2, x16, projections)
        q, k, v = _nf4.linear_rope_forward(x16, items, cos, sin, cos.shape[-1], 3, lora_rank=rank)
        ctx.projections, ctx.saved_lora, ctx.rank = projections, saved, rank
        ctx.save_for_backward(x2, x16, cos, sin)
        ctx.x_shape = x.shape
        return q.unsqueeze(0), k.unsqueeze(0), v

    @staticmethod
    def backward(ctx, grad_q, grad_k, grad_v):
        from .rope import rope_qk_backward

        x2, x16, cos, sin = ctx.saved_tensors
        m = x2.shape[0]
        n_q, n_k = (int(p["qs"].shape[0]) for p in ctx.projections[:2])
        head_dim = cos.shape[-1]
        if grad_q is None:
            grad_q = torch.zeros((n_q // head_dim, m, head_dim), dtype=torch.float16, device=x2.device)
        if grad_k is None:
            grad_k = torch.zeros((n_k // head_dim, m, head_dim), dtype=torch.float16, device=x2.device)
        dq, dk = rope_qk_backward(grad_q, grad_k, cos, sin)
        grad_x, adapter_grads = _qkv_backward(x2, x16, ctx.projections, ctx.saved_lora, (dq, dk, grad_v),
                                              ctx.rank)
        return (grad_x.reshape(ctx.x_shape), None, None, None, None, None, *adapter_grads)


def qkv_rope_projection(x, projections, cos, sin, n_heads, n_kv_heads):
    """q [1, H, T, D], k [1, HK, T, D] (rotated, head-major) and v [T, HK*D] of x (fp16 or fp32)
    in one fused launch each way (QKVRopeProjection). LoRA terms of one rank the kernels take (16
    or 32), with or without dropout masks."""
    adapters = []
    for p in projections:
        if p.get("lora_a") is not None:
            adapters += [p["lora_a"], p["lora_b"]]
    return QKVRopeProjection.apply(x, projections, cos, sin, n_heads, n_kv_heads, *adapters)


FUSED_RANKS = (16, 32)  # LoRA ranks the GEMM kernels' rank-16 MFMA slices take


def _project_one(x16, p):
    """One projection on its own: NF4Linear, NF4LoRALinear, or (a rank the kernels do not take)
    NF4Linear plus peft's fp16 LoRA products, summed in fp32 as the base sums them."""
    if p.get("lora_a") is None:
        return _nf4.NF4Linear.apply(x16, p["packed"], p.get("bias"), p["qs"])
    if int(p["lora_a"].shape[0]) in FUSED_RANKS:
        return NF4LoRALinear.apply(x16, p["packed"], p.get("bias"), p["qs"], p["lora_a"], p["lora_b"],
                                   p["scaling"])
    base = _nf4.NF4Linear.apply(x16, p["packed"], p.get("bias"), p["qs"])
    u = torch.nn.functional.linear(x16, p["lora_a"].to(torch.float16))
    lora = torch.nn.functional.linear(u, p["lora_b"].to(torch.float16)) * p["scaling"]
    return (base.float() + lora.float()).to(torch.float16)


def qkv_projection(x, projections):
    """q, k, v (+ LoRA, with or without dropout masks) of x (fp16 or fp32) in one fused launch each
    way when every LoRA term has one rank the kernels take (16 or 32); otherwise each projection
    runs on its own (no dropout masks there)."""
    ranks = {int(p["lora_a"].shape[0]) for p in projections if p.get("lora_a") is not None}
    if len(ranks) > 1 or not ranks <= set(FUSED_RANKS):
        if any(p.get("keep_bits") is not None for p in projections):
            raise ValueError("qkv_projection: dropout masks need one LoRA rank of 16 or 32")
        x16 = x if x.dtype == torch.float16 else x.to(torch.float16)
        return tuple(_project_one(x16, p) for p in projections)
    adapters = []
    for p in projections:
        if p.get("lora_a") is not None:
            adapters += [p["lora_a"], p["lora_b"]]
    return QKVProjection.apply(x, projections, *adapters)
