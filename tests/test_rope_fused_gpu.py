"""RoPE fused into the q/k/v projection's epilogue (dk_nf4_linear_rope_fwd, QKVRopeProjection):
the projections of solution/attn.py:396-418 followed by FusedQKRope (solution/attn.py:27-126),
with q and k never stored token-major. Qwen2.5-1.5B attention inputs: q [1536, 1536], k / v
[256, 1536] with biases, LoRA r=16 on q and v, 12 q heads and 2 kv heads of 128, 830 packed
tokens from 8 sequences (positions restart per sequence).

- Same bits as the unfused launches: the projection (same plan) then the RoPE kernel on its fp16
  output, forward and backward.
- Against the oracle: the reference's order (projection rounded to fp16, then RoPE in fp32) on
  the oracle's linear and LoRA references, within the parity bar."""

import numpy as np
import pytest
import torch

from helpers import assert_close, make_weight, randn16
from oracle import nf4 as O
from test_rope_gpu import rope_tables

pytestmark = pytest.mark.gpu

LENGTHS = [100, 200, 130, 32, 150, 60, 90, 68]
H, HK, D = 12, 2, 128


def _projections(device, seed=800):
    projs, w16s = [], []
    g = torch.Generator().manual_seed(seed)
    for i, n in enumerate((H * D, HK * D, HK * D)):
        packed, qs, w16 = make_weight((n, 1536), seed=seed + i, device=device)
        p = dict(packed=packed, qs=qs, bias=randn16((n,), seed=seed + 10 + i, device=device, std=0.1),
                 lora_a=None, lora_b=None, scaling=2.0)
        if i != 1:
            a = ((torch.rand((16, 1536), generator=g) * 2 - 1) / np.sqrt(1536)).half().float().to(device)
            b = (torch.randn((n, 16), generator=g) * 3e-2).half().float().to(device)
            p["lora_a"], p["lora_b"] = a.requires_grad_(True), b.requires_grad_(True)
        projs.append(p)
        w16s.append(w16)
    return projs, w16s


@pytest.mark.parametrize("m,plan", [(830, None), (830, "7,3,8"), (300, "2,2,4"), (2048, "8,2,8")])
def test_fused_rope_matches_projection_then_rope(m, plan, device, monkeypatch):
    """The fused launch equals linear_forward (the same plan) followed by dk_rope_qk_fwd, bit for
    bit, for q and k; v is the plain projection output."""
    from decik_amd import lora, nf4
    from decik_amd.rope import rope_qk_forward

    if plan is not None:
        monkeypatch.setenv("DECIK_FWD_PLAN", plan)
    lengths = LENGTHS if m == 830 else [m]
    c, s = rope_tables(lengths, D)
    ct, st = torch.from_numpy(c).to(device), torch.from_numpy(s).to(device)
    projs, _ = _projections(device)
    x = randn16((m, 1536), seed=820, device=device)
    items = []
    for p in projs:
        it = dict(packed=p["packed"], qs=p["qs"], bias=p["bias"])
        if p["lora_a"] is not None:
            a16 = p["lora_a"].detach().half().contiguous()
            it.update(lora_u=lora.lora_down(x, a16), lora_b=p["lora_b"].detach().half().contiguous(),
                      lora_scale=p["scaling"])
        items.append(it)
    if plan is None:
        assert nf4.launch_plan(False, m, 1536, [H * D, HK * D, HK * D], lora=True)["splits"] >= 2
    q_rot, k_rot, v = nf4.linear_rope_forward(x, items, ct, st, D, 3, lora_rank=16)
    q, k, v_ref = nf4.linear_forward(x, items, lora_rank=16)
    rq, rk = rope_qk_forward(q, None, k, ct, st, H, HK)
    assert q_rot.shape == (H, m, D) and k_rot.shape == (HK, m, D) and v.shape == (m, HK * D)
    assert torch.equal(q_rot, rq) and torch.equal(k_rot, rk) and torch.equal(v, v_ref)


def test_qkv_rope_projection_against_oracle_and_unfused_autograd(device):
    """QKVRopeProjection (one fused launch each way) against QKVProjection + FusedQKRope: the same
    bits for outputs, dX, dA and dB; and the outputs against the oracle (projection outputs
    rounded to fp16, then RoPE)."""
    from decik_amd.lora import qkv_projection, qkv_rope_projection
    from decik_amd.rope import FusedQKRope

    c, s = rope_tables(LENGTHS, D)
    ct, st = torch.from_numpy(c).to(device), torch.from_numpy(s).to(device)
    m = sum(LENGTHS)
    projs, w16s = _projections(device, seed=830)
    x = randn16((m, 1536), seed=840, device=device)
    gq = randn16((1, H, m, D), seed=841, device=device, std=1e-2)
    gk = randn16((1, HK, m, D), seed=842, device=device, std=1e-2)
    gv = randn16((m, HK * D), seed=843, device=device, std=1e-2)

    def run(fused):
        xi = x.clone().requires_grad_(True)
        for p in projs:
            for key in ("lora_a", "lora_b"):
                if p[key] is not None:
                    p[key].grad = None
        if fused:
            q, k, v = qkv_rope_projection(xi, projs, ct, st, H, HK)
        else:
            qb, kb, v = qkv_projection(xi, projs)
            q, k = FusedQKRope.apply(qb, None, kb, ct, st, H, HK)
        torch.autograd.backward([q, k, v], [gq, gk, gv])
        grads = [xi.grad] + [p[key].grad.clone() for p in projs for key in ("lora_a", "lora_b") if p[key] is not None]
        return (q.detach(), k.detach(), v.detach()), grads

    outs_f, grads_f = run(True)
    outs_u, grads_u = run(False)
    for a, b in zip(outs_f, outs_u):
        assert torch.equal(a, b)
    for a, b in zip(grads_f, grads_u):
        assert torch.equal(a, b)
    # oracle: each projection rounded to fp16 (base + bias + LoRA), then RoPE in fp32
    xn = x.cpu().numpy()
    refs = []
    for p, w16 in zip(projs, w16s):
        y = O.linear_ref(xn, w16, p["bias"].cpu().numpy()).astype(np.float64)
        if p["lora_a"] is not None:
            _, lo = O.lora_fwd_ref(xn, p["lora_a"].detach().half().cpu().numpy(),
                                   p["lora_b"].detach().half().cpu().numpy(), p["scaling"])
            y = y + lo
        refs.append(y.astype(np.float32))
    rq, rk = O.rope_fwd_ref(refs[0].astype(np.float16), None, refs[1].astype(np.float16), c, s, H, HK)
    assert_close(outs_f[0][0], rq.astype(np.float32), what="q rotated")
    assert_close(outs_f[1][0], rk.astype(np.float32), what="k rotated")
    assert_close(outs_f[2], refs[2], what="v")


def test_rope_entry_rejects_bad_shapes(device):
    """head_dim not a multiple of 16, or a contraction too short to split, are errors."""
    from decik_amd import _lib, nf4

    projs, _ = _projections(device, seed=850)
    items = [dict(packed=p["packed"], qs=p["qs"]) for p in projs]
    x = randn16((64, 1536), seed=851, device=device)
    c = torch.ones((64, 24), dtype=torch.float32, device=device)
    with pytest.raises(_lib.DecikError, match="head_dim"):
        nf4.linear_rope_forward(x, items, c, c, 24, 3)


@pytest.mark.parametrize("plan", [None, "2,2,8"])
def test_fused_rope_shortest_contraction(plan, device, monkeypatch):
    """k = 128 is two 64-wide steps, the shortest contraction the RoPE epilogue (which lives in the
    split-K reduction) takes: with no forced plan the planner must still give it two splits. The
    output meets the bar against the oracle (projection rounded to fp16, then RoPE), and under one
    forced plan equals the projection followed by the RoPE kernel, bit for bit."""
    from decik_amd import nf4
    from decik_amd.rope import rope_qk_forward

    if plan is None:
        monkeypatch.delenv("DECIK_FWD_PLAN", raising=False)
    else:
        monkeypatch.setenv("DECIK_FWD_PLAN", plan)
    m, k, h, hk, d = 64, 128, 2, 1, 64
    lengths = [40, 24]
    c, s = rope_tables(lengths, d)
    ct, st = torch.from_numpy(c).to(device), torch.from_numpy(s).to(device)
    items, w16s = [], []
    for i, n in enumerate((h * d, hk * d, hk * d)):
        packed, qs, w16 = make_weight((n, k), seed=860 + i, device=device)
        items.append(dict(packed=packed, qs=qs, bias=randn16((n,), seed=870 + i, device=device, std=0.1)))
        w16s.append(w16)
    x = randn16((m, k), seed=880, device=device)
    q_rot, k_rot, v = nf4.linear_rope_forward(x, items, ct, st, d, 3)
    torch.cuda.synchronize()
    xn = x.cpu().numpy()
    refs = [O.linear_ref(xn, w, it["bias"].cpu().numpy()) for w, it in zip(w16s, items)]
    rq, rk = O.rope_fwd_ref(refs[0].astype(np.float16), None, refs[1].astype(np.float16), c, s, h, hk)
    assert_close(q_rot, rq.astype(np.float32), what="q rotated, k = 128")
    assert_close(k_rot, rk.astype(np.float32), what="k rotated, k = 128")
    assert_close(v, refs[2], what="v, k = 128")
    if plan is not None:
        q, kk, v2 = nf4.linear_forward(x, items)
        rq2, rk2 = rope_qk_forward(q, None, kk, ct, st, h, hk)
        assert torch.equal(q_rot, rq2) and torch.equal(k_rot, rk2) and torch.equal(v, v2)
