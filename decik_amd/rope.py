"""RoPE of the attention inputs: (q_base + q_lora, k) -> rotated fp16 q, k, head-major.

Mirrors FusedQKRope (solution/attn.py:89-126) and its kernels (solution/attn.py:27-86) with one
HIP launch each way (dk_rope_qk_fwd / dk_rope_qk_bwd):
  forward:  q = fp32(q_base) + fp32(q_lora); q * cos + rotate_half(q) * sin in fp32, stored fp16
            as [1, H, T, D] for SDPA; k the same without LoRA
  backward: dq = g * cos + rotate_half^T(g * sin) in fp32, rounded to fp16 once; the projection
            and the LoRA branch both receive it (as in the base)
"""

import torch

from ._lib import check, lib, ptr, stream_of


def _rows(t):
    t2 = t.reshape(-1, t.shape[-1])
    return t2 if t2.stride(-1) == 1 else t2.contiguous()


def rope_qk_forward(q_base, q_lora, k, cos, sin, n_heads, n_kv_heads):
    """(q_out [H, T, D], k_out [HK, T, D]) fp16; q_base/q_lora [T, H*D], k [T, HK*D] fp16;
    cos/sin fp32 [T, D]. q_lora may be None (no addition)."""
    qb, kk = _rows(q_base), _rows(k)
    ql = None if q_lora is None else _rows(q_lora)
    n_tok = qb.shape[0]
    d = cos.shape[-1]
    c = cos.reshape(n_tok, d).to(torch.float32).contiguous()
    s = sin.reshape(n_tok, d).to(torch.float32).contiguous()
    q_out = torch.empty((n_heads, n_tok, d), dtype=torch.float16, device=qb.device)
    k_out = torch.empty((n_kv_heads, n_tok, d), dtype=torch.float16, device=qb.device)
    check(lib().dk_rope_qk_fwd(ptr(qb), ptr(ql), qb.stride(0), 0 if ql is None else ql.stride(0), ptr(kk),
                               kk.stride(0), ptr(c), ptr(s), ptr(q_out), ptr(k_out), n_tok, n_heads,
                               n_kv_heads, d, stream_of(qb.device)))
    return q_out, k_out


def rope_qk_backward(grad_q, grad_k, cos, sin):
    """(dq [T, H*D], dk [T, HK*D]) fp16 from head-major fp16 gradients [H, T, D], [HK, T, D]."""
    gq = grad_q.reshape(-1, grad_q.shape[-2], grad_q.shape[-1]).to(torch.float16).contiguous()
    gk = grad_k.reshape(-1, grad_k.shape[-2], grad_k.shape[-1]).to(torch.float16).contiguous()
    n_heads, n_tok, d = gq.shape
    n_kv = gk.shape[0]
    c = cos.reshape(n_tok, d).to(torch.float32).contiguous()
    s = sin.reshape(n_tok, d).to(torch.float32).contiguous()
    dq = torch.empty((n_tok, n_heads * d), dtype=torch.float16, device=gq.device)
    dk = torch.empty((n_tok, n_kv * d), dtype=torch.float16, device=gq.device)
    check(lib().dk_rope_qk_bwd(ptr(gq), ptr(gk), ptr(c), ptr(s), ptr(dq), dq.stride(0), ptr(dk), dk.stride(0),
                               n_tok, n_heads, n_kv, d, stream_of(gq.device)))
    return dq, dk


class FusedQKRope(torch.autograd.Function):
    """(q_base + q_lora, k) -> RoPE'd fp16 q [1, HQ, T, D] and k [1, HK, T, D]
    (solution/attn.py:89-126)."""

    @staticmethod
    def forward(ctx, q_base, q_lora, k, cos, sin, n_heads, n_kv_heads):
        q_out, k_out = rope_qk_forward(q_base, q_lora, k, cos, sin, n_heads, n_kv_heads)
        ctx.save_for_backward(cos, sin)
        return q_out.unsqueeze(0), k_out.unsqueeze(0)

    @staticmethod
    def backward(ctx, grad_q, grad_k):
        cos, sin = ctx.saved_tensors
        dq, dk = rope_qk_backward(grad_q, grad_k, cos, sin)
        # q_lora may be absent (None) when the LoRA term is already in q_base
        return dq, dq.clone() if ctx.needs_input_grad[1] else None, dk, None, None, None, None
