"""RoPE of q and k (solution/attn.py:27-126) on the GPU against the oracle, bit for bit (fp32
elementwise in the reference's order): Qwen2.5-1.5B heads (12 q heads, 2 kv heads, D = 128) at
830 packed tokens, positions restarting per sequence, with and without the q LoRA term."""

import numpy as np
import pytest
import torch

from helpers import randn16
from oracle import nf4 as O

pytestmark = pytest.mark.gpu


def rope_tables(lengths, d, base=1000000.0):
    """cos/sin [T, D] fp32 for packed sequences (positions restart at each sequence), as
    transformers' Qwen2 rotary embedding builds them (inv_freq = base^(-2i/D), emb = [f, f])."""
    pos = np.concatenate([np.arange(n) for n in lengths]).astype(np.float32)
    inv = (1.0 / (base ** (np.arange(0, d, 2, dtype=np.float32) / d))).astype(np.float32)
    f = pos[:, None] * inv[None, :]
    emb = np.concatenate([f, f], axis=1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


@pytest.mark.parametrize("with_lora", [True, False])
def test_rope_forward_backward_bit_exact(with_lora, device):
    from decik_amd.rope import FusedQKRope

    lengths = [100, 200, 130, 32, 150, 60, 90, 68]
    t, h, hk, d = sum(lengths), 12, 2, 128
    c, s = rope_tables(lengths, d)
    qb = randn16((t, h * d), seed=1, device=device)
    ql = randn16((t, h * d), seed=2, device=device, std=0.05) if with_lora else None
    k = randn16((t, hk * d), seed=3, device=device)
    ct, st = torch.from_numpy(c).to(device), torch.from_numpy(s).to(device)
    q_out, k_out = FusedQKRope.apply(qb, ql, k, ct, st, h, hk)
    assert q_out.shape == (1, h, t, d) and k_out.shape == (1, hk, t, d) and q_out.dtype == torch.float16
    rq, rk = O.rope_fwd_ref(qb.cpu().numpy(), None if ql is None else ql.cpu().numpy(), k.cpu().numpy(), c, s, h, hk)
    assert np.array_equal(q_out[0].cpu().numpy().view(np.uint16), rq.view(np.uint16))
    assert np.array_equal(k_out[0].cpu().numpy().view(np.uint16), rk.view(np.uint16))
    from decik_amd.rope import rope_qk_backward

    gq = randn16((h, t, d), seed=4, device=device, std=1e-2)
    gk = randn16((hk, t, d), seed=5, device=device, std=1e-2)
    dq, dk = rope_qk_backward(gq, gk, ct, st)
    rdq, rdk = O.rope_bwd_ref(gq.cpu().numpy(), gk.cpu().numpy(), c, s)
    assert np.array_equal(dq.cpu().numpy().view(np.uint16), rdq.view(np.uint16))
    assert np.array_equal(dk.cpu().numpy().view(np.uint16), rdk.view(np.uint16))


def test_rope_autograd_gives_both_branches_the_same_gradient(device):
    from decik_amd.rope import FusedQKRope

    t, h, hk, d = 64, 4, 2, 64
    c, s = rope_tables([64], d)
    ct, st = torch.from_numpy(c).to(device), torch.from_numpy(s).to(device)
    qb = randn16((t, h * d), seed=6, device=device).requires_grad_(True)
    ql = randn16((t, h * d), seed=7, device=device).requires_grad_(True)
    k = randn16((t, hk * d), seed=8, device=device).requires_grad_(True)
    q_out, k_out = FusedQKRope.apply(qb, ql, k, ct, st, h, hk)
    (q_out.float().sum() + 2 * k_out.float().sum()).backward()
    assert torch.equal(qb.grad, ql.grad) and k.grad.shape == k.shape
