"""Qwen2.5-1.5B MLP block forward + backward on NF4 weights (gate/up [8960, 1536], down
[1536, 8960], X [830, 1536] ~ N(0, 1), dY ~ N(0, 1e-2)), against the oracle's restatement of
RecomputedMLP (solution/mlp.py:62-110). Bar: max|err| <= 1e-2 max|ref|, mean rel <= 1e-3."""

import pytest
import torch

from helpers import assert_close, make_weight, randn16
from oracle import nf4 as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def block(device):
    gate = make_weight((8960, 1536), seed=1, device=device)
    up = make_weight((8960, 1536), seed=2, device=device)
    down = make_weight((1536, 8960), seed=3, device=device)
    x = randn16((830, 1536), seed=4, device=device)
    dy = randn16((830, 1536), seed=5, device=device, std=1e-2)
    ref = O.mlp_ref(x.cpu().numpy(), gate[2], up[2], down[2], dy.cpu().numpy())
    return gate, up, down, x, dy, ref


@pytest.mark.parametrize("recompute", [True, False])
def test_mlp_forward_backward(block, recompute):
    from decik_amd.mlp import FusedMLP

    gate, up, down, x, dy, ref = block
    xin = x.float().requires_grad_(True)  # the residual stream is fp32 in the reference
    out = FusedMLP.apply(xin, gate[0], gate[1], up[0], up[1], down[0], down[1], recompute)
    assert out.dtype == torch.float16
    out.backward(dy)
    assert xin.grad.dtype == torch.float32
    assert_close(out, ref["out"], what="out")
    # against the reference's sum of two fp16 products, and against the unrounded sum the
    # fused launch accumulates (its own accuracy)
    assert_close(xin.grad, ref["dx"], what="dX")
    assert_close(xin.grad, ref["dx_exact"], what="dX (unrounded products)")


def test_recompute_is_bit_identical(block):
    from decik_amd.mlp import FusedMLP

    gate, up, down, x, dy, _ = block
    res = []
    for recompute in (True, False):
        xin = x.float().requires_grad_(True)
        out = FusedMLP.apply(xin, gate[0], gate[1], up[0], up[1], down[0], down[1], recompute)
        out.backward(dy)
        res.append((out.detach(), xin.grad))
    assert torch.equal(res[0][0], res[1][0]) and torch.equal(res[0][1], res[1][1])


def test_intermediates(block):
    """gate/up from one two-weight launch, SwiGLU, and dH = dY . W_down."""
    from decik_amd.mlp import mlp_forward
    from decik_amd.nf4 import linear_backward
    from decik_amd.swiglu import swiglu_bwd

    gate, up, down, x, dy, ref = block
    out, g, u = mlp_forward(x, gate[:2], up[:2], down[:2])
    assert_close(g, ref["gate"], what="gate")
    assert_close(u, ref["up"], what="up")
    gh = linear_backward([dict(packed=down[0], qs=down[1], dy=dy)], 830, 8960)
    assert_close(gh, ref["gh"], what="dH")
    # SwiGLU backward on the oracle's own fp16 inputs
    gh16 = torch.from_numpy(ref["gh"]).half().to(g.device)
    g16 = torch.from_numpy(ref["gate"]).half().to(g.device)
    u16 = torch.from_numpy(ref["up"]).half().to(g.device)
    dg, du = swiglu_bwd(gh16, g16, u16)
    assert_close(dg, ref["dgate"], what="dgate")
    assert_close(du, ref["dup"], what="dup")
