"""LoRA r=16 fused into the NF4 GEMM epilogues (config: Qwen2.5-1.5B attention projections,
830 packed tokens from 8 sequences). Reference semantics: solution/attn.py:225-228 (forward),
:251-257 (backward); bar: max|err| <= 1e-2 max|ref|, sum|err|/sum|ref| <= 1e-3."""

import numpy as np
import pytest
import torch

from helpers import assert_close, make_weight, randn16
from oracle import nf4 as O

pytestmark = pytest.mark.gpu


def packed_lengths(total=830, n_seq=8, lo=32, hi=200, seed=0):
    """8 sequence lengths drawn uniform in [32, 200] that sum to 830 (seeded rejection sampler);
    the projections are per token, so only the total matters to them."""
    rng = np.random.default_rng(seed)
    while True:
        lens = rng.integers(lo, hi + 1, n_seq)
        if lens.sum() == total:
            return lens


def adapters(n, k, seed, device, r=16):
    g = torch.Generator(device="cpu").manual_seed(seed)
    bound = 1.0 / np.sqrt(k)  # Kaiming-uniform bound of peft's default init for lora_A
    a = ((torch.rand((r, k), generator=g) * 2 - 1) * bound).to(torch.float16).to(device)
    b = (torch.randn((n, r), generator=g) * 1e-3).to(torch.float16).to(device)
    return a, b


def test_lengths_sum():
    lens = packed_lengths()
    assert lens.sum() == 830 and lens.min() >= 32 and lens.max() <= 200


@pytest.mark.parametrize("n", [1536, 256])
def test_nf4_lora_linear(n, device):
    from decik_amd.lora import NF4LoRALinear

    m, k, s = int(packed_lengths().sum()), 1536, 2.0
    packed, qs, w16 = make_weight((n, k), seed=n, device=device)
    bias = randn16((n,), seed=1, device=device, std=0.1)
    a, b = adapters(n, k, seed=2, device=device)
    a32, b32 = a.float().requires_grad_(True), b.float().requires_grad_(True)
    x = randn16((m, k), seed=3, device=device).requires_grad_(True)
    y = NF4LoRALinear.apply(x, packed, bias, qs, a32, b32, s)
    dy = randn16((m, n), seed=4, device=device, std=1e-2)
    y.backward(dy)

    xn, an, bn, dyn = (t.detach().cpu().numpy() for t in (x, a, b, dy))
    u16, lora = O.lora_fwd_ref(xn, an, bn, s)
    y_ref = O.linear_ref(xn, w16, bias.cpu().numpy()) + lora
    assert_close(y, y_ref, what="Y")
    gu16, da, db, dx_lora = O.lora_bwd_ref(dyn, xn, u16, an, bn, s)
    assert_close(x.grad, O.linear_dx_ref(dyn, w16) + dx_lora, what="dX")
    assert_close(a32.grad, da, what="dA")
    assert_close(b32.grad, db, what="dB")
    assert a32.grad.dtype == torch.float32 and b32.grad.dtype == torch.float32


def test_qkv_projection_with_lora_on_q_and_v(device):
    """q/k/v in one fused launch each way; LoRA on q and v only (the reference run)."""
    from decik_amd.lora import qkv_projection

    m, k, s = 830, 1536, 2.0
    x = randn16((m, k), seed=10, device=device).requires_grad_(True)
    projs, refs = [], []
    for i, (name, n) in enumerate([("q", 1536), ("k", 256), ("v", 256)]):
        packed, qs, w16 = make_weight((n, k), seed=50 + i, device=device)
        bias = randn16((n,), seed=60 + i, device=device, std=0.1)
        p = dict(packed=packed, qs=qs, bias=bias, lora_a=None, lora_b=None, scaling=s)
        if name in ("q", "v"):
            a, b = adapters(n, k, seed=70 + i, device=device)
            p["lora_a"], p["lora_b"] = a.float().requires_grad_(True), b.float().requires_grad_(True)
        projs.append(p)
        refs.append(w16)
    outs = qkv_projection(x, projs)
    grads = [randn16(o.shape, seed=80 + i, device=device, std=1e-2) for i, o in enumerate(outs)]
    torch.autograd.backward(outs, grads)

    xn = x.detach().cpu().numpy()
    dx_ref = np.zeros((m, k), np.float64)
    for p, w16, o, g in zip(projs, refs, outs, grads):
        gn = g.cpu().numpy()
        y_ref = O.linear_ref(xn, w16, p["bias"].cpu().numpy())
        dx_ref += O.linear_dx_ref(gn, w16)
        if p["lora_a"] is not None:
            an = p["lora_a"].detach().half().cpu().numpy()
            bn = p["lora_b"].detach().half().cpu().numpy()
            u16, lora = O.lora_fwd_ref(xn, an, bn, s)
            y_ref = y_ref + lora
            _, da, db, dxl = O.lora_bwd_ref(gn, xn, u16, an, bn, s)
            dx_ref += dxl
            assert_close(p["lora_a"].grad, da, what="dA")
            assert_close(p["lora_b"].grad, db, what="dB")
        assert_close(o, y_ref, what="qkv Y")
    assert_close(x.grad, dx_ref, what="qkv dX")
