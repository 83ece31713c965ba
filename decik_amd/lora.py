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
from . import _lib
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


def lora_down_group(branches):
    """U of every branch, [M, r] fp16 each, for branches that share the token count, the input width
    and the rank (the q and v adapters of a layer): one launch (one per kind of input where the
    kinds differ) instead of one per branch, with the same bits as lora_down branch by branch
    (dk_lora_down_group). branches: list of (x, a16, keep_bits, keep_scale), as lora_down takes
    them."""
    n = len(branches)
    arr = (_lib.LoraBranch * n)()
    keep, us = [], []
    m = k = r = None
    for i, (x, a16, keep_bits, keep_scale) in enumerate(branches):
        x2 = x.reshape(-1, x.shape[-1])
        m, k = x2.shape
        r = a16.shape[0]
        bits, sc = _keep_args(x2, keep_bits, keep_scale)
        u = torch.empty((m, r), dtype=torch.float16, device=x.device)
        arr[i].x, arr[i].ldx, arr[i].x_fp32 = x2.data_ptr(), x2.stride(0), int(x2.dtype == torch.float32)
        arr[i].keep_bits, arr[i].keep_scale = ptr(bits), ptr(sc)
        arr[i].a, arr[i].u = a16.data_ptr(), u.data_ptr()
        keep += [x2, bits, sc, a16]
        us.append(u)
    check(lib().dk_lora_down_group(arr, n, m, k, r, stream_of(branches[0][0].device)))
    return us


def lora_grads_group(branches):
    """lora_grads of every branch, [(GU, dA, dB), ...], for branches that share the token count,
    the input width and the rank: GU and dB of all branches in one launch, dA in another (one per
    kind of input where the kinds differ), the same bits as lora_grads branch by branch
    (dk_lora_bwd_group). branches: list of dicts with dy16, u16, x, b16, scaling and optional
    want_da, want_db (default True), keep_bits, keep_scale."""
    n = len(branches)
    arr = (_lib.LoraBranch * n)()
    keep, outs = [], []
    m = k = r = None
    for i, br in enumerate(branches):
        dy2 = br["dy16"].reshape(-1, br["dy16"].shape[-1])
        x2 = br["x"].reshape(-1, br["x"].shape[-1])
        u16, b16 = br["u16"], br["b16"]
        m, nn = dy2.shape
        k = x2.shape[1]
        r = u16.shape[1]
        dev = dy2.device
        bits, sc = _keep_args(x2, br.get("keep_bits"), br.get("keep_scale"))
        gu = torch.empty((m, r), dtype=torch.float16, device=dev)
        da = torch.empty((r, k), dtype=torch.float32, device=dev) if br.get("want_da", True) else None
        db = torch.empty((nn, r), dtype=torch.float32, device=dev) if br.get("want_db", True) else None
        e = arr[i]
        e.x, e.ldx, e.x_fp32 = x2.data_ptr(), x2.stride(0), int(x2.dtype == torch.float32)
        e.keep_bits, e.keep_scale = ptr(bits), ptr(sc)
        e.u, e.dy, e.lddy, e.n, e.b = u16.data_ptr(), dy2.data_ptr(), dy2.stride(0), nn, b16.data_ptr()
        e.gu, e.da, e.db, e.scale = gu.data_ptr(), ptr(da), ptr(db), float(br["scaling"])
        keep += [dy2, x2, bits, sc, u16, b16]
        outs.append((gu, da, db))
    check(lib().dk_lora_bwd_group(arr, n, m, k, r, stream_of(branches[0]["dy16"].device)))
    return outs


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


class _QVDropout:
    """Dropout of the q and v LoRA branch inputs, in either form the reference accepts
    (solution/attn.py:206-273), as data for one implementation of the pair:

    packed: keep bits [T, W / 8] per branch (pack_keep) with fp32 device scalars 1 / (1 - p);
        one HIP pass forms fp16(x * (keep * scale)) of both branches (dk_lora_dropout_inputs, the
        same kernel forward and backward) and one the fp32 input gradient through both masks
        (dk_lora_input_grad, (g * keep) * 1/(1 - p) per branch, q's plus v's).
    elementwise: per branch an x-shaped fp32 tensor for the forward (the dropout output of ones)
        and a mask with its kept value for the backward, or None for a branch without dropout;
        plain torch ops on the GPU with the reference's operation order."""

    def __init__(self, packed, fwd, bwd, p):
        # fwd: (scaled_q, scaled_v); bwd: ((mask_q, scale_q), (mask_v, scale_v)); p: (p_q, p_v)
        self.packed, self.fwd, self.bwd, self.p = packed, fwd, bwd, p

    def inputs(self, x, forward):
        """fp16 rows [T, W] of both branch inputs."""
        if self.packed:
            (bq, sq), (bv, sv) = self.bwd
            return lora_inputs(x, bq, bv, sq, sv)
        width = x.shape[-1]
        out = []
        for i in range(2):
            if forward:
                f = self.fwd[i]
                v = x if f is None else x * f
            else:
                mask, kept = self.bwd[i]
                v = x if mask is None else x * (mask * kept)
            out.append(v.to(torch.float16).reshape(-1, width).contiguous())
        return tuple(out)

    def input_grad(self, gx16):
        """fp32 [T, W] input gradient of x through both branches' dropout (gx16: the fp16 input
        gradients of the q and v products)."""
        if self.packed:
            (bq, _), (bv, _) = self.bwd
            return lora_input_grad(gx16[0], gx16[1], bq, bv, 1.0 / (1.0 - self.p[0]), 1.0 / (1.0 - self.p[1]))
        total = None
        for gx, (mask, _), p in zip(gx16, self.bwd, self.p):
            term = gx.to(torch.float32)
            if mask is not None:
                term = term * mask.reshape(gx.shape) * (1.0 / (1.0 - p))
            total = term if total is None else total + term
        return total


def _qv_lora_forward(x, drop, adapters, scalings):
    """(out_q, out_v, u_q, u_v): out = fp16(fp16(U . B^T) * s), U = fp16(X . A^T) per branch, with
    X the branch's dropped-out fp16 input (solution/attn.py:224-228)."""
    xs = drop.inputs(x, True)
    us = lora_down_group([(x16, a.to(torch.float16).contiguous(), None, None) for x16, (a, _) in zip(xs, adapters)])
    outs = [lora_up(u, b.to(torch.float16).t().contiguous()) * s for u, (_, b), s in zip(us, adapters, scalings)]
    lead = x.shape[:-1]
    return outs[0].reshape(*lead, -1), outs[1].reshape(*lead, -1), us[0], us[1]


def _qv_lora_backward(x, drop, adapters, scalings, us, grads):
    """(dX fp32 in x's shape, [dA_q, dB_q, dA_v, dB_v] in the adapters' dtypes). For both branches
    at once dk_lora_bwd_group gives GU = fp16(s * dY . B), dB = s * dY^T . U and dA = GU^T . X in
    fp32 (the products autograd forms, solution/attn.py:251-257); GU . A is the branch's input
    gradient before its dropout. A branch that received no gradient contributes zeros, formed as the
    reference forms them."""
    xs = drop.inputs(x, False)
    rows = xs[0].shape[0]
    branches = []
    for x16, (a, b), s, u, g in zip(xs, adapters, scalings, us, grads):
        b16 = b.to(torch.float16).contiguous()
        if g is None:
            g16 = torch.zeros((rows, b16.shape[0]), dtype=torch.float16, device=x.device)
        else:
            g16 = g.to(torch.float16).reshape(rows, -1).contiguous()
        branches.append(dict(dy16=g16, u16=u, x=x16, b16=b16, scaling=s))
    adapter_grads, input_grads = [], []
    for (gu, da, db), (a, b) in zip(lora_grads_group(branches), adapters):
        adapter_grads += [da.to(a.dtype), db.to(b.dtype)]
        input_grads.append(lora_up(gu, a.to(torch.float16).contiguous()))
    return drop.input_grad(input_grads).view(x.shape), adapter_grads


class LoRAPairFromNorm(torch.autograd.Function):
    """The q and v LoRA branches of a Qwen2 attention layer, lora_B(lora_A(dropout(x))) * scaling
    each (peft under fp16 autocast, solution/attn.py:344-346), with the reference's argument list
    apply(x, h, norm_weight, eps, scaled_q, mask_q, scale_q, scaled_v, mask_v, scale_v, a_q, b_q,
    a_v, b_v, scaling_q, scaling_v, p_q, p_v, packed) (solution/attn.py:206-273).

    packed=True: mask_* are pack_keep bits and scale_* fp32 device scalars 1 / (1 - p);
    packed=False: scaled_* (forward) and mask_* * scale_* (backward) are x-shaped tensors, None
    for a branch without dropout (see _QVDropout). x is saved and the dropped-out inputs formed
    again in the backward; the reference rebuilds x from the RMSNorm input instead (:240), and the
    norm is outside this package, so h, norm_weight and eps are accepted unused. Returns (out_q,
    out_v) fp16; gradients reach x (fp32) and the four adapter weights (their dtype)."""

    @staticmethod
    def forward(ctx, x, h, norm_weight, eps, scaled_q, mask_q, scale_q, scaled_v, mask_v, scale_v,
                a_q, b_q, a_v, b_v, scaling_q, scaling_v, p_q, p_v, packed):
        drop = _QVDropout(bool(packed), (scaled_q, scaled_v), ((mask_q, scale_q), (mask_v, scale_v)),
                          (p_q, p_v))
        scalings = (scaling_q, scaling_v)
        out_q, out_v, u_q, u_v = _qv_lora_forward(x, drop, ((a_q, b_q), (a_v, b_v)), scalings)
        ctx.save_for_backward(x, u_q, u_v, a_q, b_q, a_v, b_v)
        ctx.drop, ctx.scalings = drop, scalings
        return out_q, out_v

    @staticmethod
    def backward(ctx, grad_q, grad_v):
        x, u_q, u_v, a_q, b_q, a_v, b_v = ctx.saved_tensors
        grad_x, adapter_grads = _qv_lora_backward(x, ctx.drop, ((a_q, b_q), (a_v, b_v)), ctx.scalings,
                                                  (u_q, u_v), (grad_q, grad_v))
        # gradients of x and the four adapters; the other 14 arguments take none
        return (grad_x, *(None,) * 9, *adapter_grads, *(None,) * 5)


class LoRAPair:
    """Both LoRA branches with packed dropout masks: apply(x, bits_q, scale_q, bits_v, scale_v,
    a_q, b_q, a_v, b_v, scaling_q, scaling_v, p_q, p_v) -> (out_q, out_v) fp16, i.e.
    LoRAPairFromNorm on its packed path. x: [.., W] fp16 or fp32; bits_*: pack_keep masks;
    scale_*: fp32 device scalars 1 / (1 - p); a_* [r, W], b_* [N, r] adapter weights (used in
    fp16); gradients reach x (fp32) and the adapters."""

    @staticmethod
    def apply(x, bits_q, scale_q, bits_v, scale_v, a_q, b_q, a_v, b_v, scaling_q, scaling_v, p_q, p_v):
        return LoRAPairFromNorm.apply(x, None, None, None, None, bits_q, scale_q, None, bits_v, scale_v,
                                      a_q, b_q, a_v, b_v, scaling_q, scaling_v, p_q, p_v, True)


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
    downs, adapters = [], {}
    for i, p in enumerate(projections):
        if p.get("lora_a") is not None:
            a16 = p["lora_a"].to(torch.float16).contiguous()
            adapters[i] = (a16, p["lora_b"].to(torch.float16).contiguous())
            if p.get("keep_bits") is not None:
                downs.append((x2, a16, p["keep_bits"], p["keep_scale"]))
            else:
                downs.append((x16, a16, None, None))
    us = iter(lora_down_group(downs) if downs else [])  # every branch's U in one launch
    for i, p in enumerate(projections):
        it = dict(packed=p["packed"], qs=p["qs"], bias=p.get("bias"))
        if i in adapters:
            a16, b16 = adapters[i]
            u = next(us)
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
    items, branches = [], []
    for p, sv, g in zip(projections, saved, grads):
        if g is None:
            g = torch.zeros((m, int(p["qs"].shape[0])), dtype=torch.float16, device=x2.device)
        g16 = g.to(torch.float16).reshape(m, -1).contiguous()
        it = dict(packed=p["packed"], qs=p["qs"], dy=g16)
        if sv is not None:
            u, a16, b16 = sv
            if p.get("keep_bits") is not None:
                branches.append(dict(dy16=g16, u16=u, x=x2, b16=b16, scaling=p["scaling"],
                                     keep_bits=p["keep_bits"], keep_scale=p["keep_scale"]))
                it.update(lora_keep=p["keep_bits"], lora_keep_scale=1.0 / (1.0 - float(p["p"])))
            else:
                branches.append(dict(dy16=g16, u16=u, x=x16, b16=b16, scaling=p["scaling"]))
            it.update(lora_a=a16)
        items.append(it)
    # GU, dB and dA of every branch: one launch per product
    grads_of = iter(lora_grads_group(branches) if branches else [])
    adapter_grads = []
    for p, sv, it in zip(projections, saved, items):
        if sv is not None:
            gu, da, db = next(grads_of)
            it["lora_gu"] = gu
            adapter_grads += [da.to(p["lora_a"].dtype), db.to(p["lora_b"].dtype)]
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
