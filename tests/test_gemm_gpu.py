"""Fused NF4 dequant x fp16 GEMM on the GPU against the oracle's fp32-accumulated products of
the bit-exact dequantized weight (solution/nf4.py:93-104).

Bar (written here, from the parity contract): max|y - ref| <= 1e-2 * max|ref| and
sum|y - ref| / sum|ref| <= 1e-3."""

import numpy as np
import pytest
import torch

from helpers import assert_close, make_weight, randn16
from oracle import nf4 as O

pytestmark = pytest.mark.gpu

# (M, N, K): Qwen2.5-1.5B projections at 830 packed tokens, the 7B sweep's small-M regime, and
# ragged shapes that leave partial tiles in every dimension.
FWD_SHAPES = [
    (830, 1536, 1536), (830, 256, 1536), (830, 8960, 1536), (830, 1536, 8960),
    (1, 3584, 3584), (8, 512, 3584), (64, 18944, 3584), (17, 96, 128), (300, 264, 160),
    (2048, 1536, 1536),
]


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("m,n,k", FWD_SHAPES)
def test_forward(m, n, k, bias, device):
    from decik_amd.nf4 import linear_forward

    packed, qs, w16 = make_weight((n, k), seed=n + k, device=device)
    x = randn16((m, k), seed=m, device=device)
    b = randn16((n,), seed=5, device=device, std=0.1) if bias else None
    (y,) = linear_forward(x, [dict(packed=packed, qs=qs, bias=b)])
    ref = O.linear_ref(x.cpu().numpy(), w16, None if b is None else b.cpu().numpy())
    assert y.shape == (m, n) and y.dtype == torch.float16
    assert_close(y, ref, what=f"fwd {m}x{n}x{k}")


@pytest.mark.parametrize("plan", ["9,1,8", "8,2,8"])
@pytest.mark.parametrize("m,n,k", [(830, 1536, 1536), (830, 8960, 1536), (300, 264, 192), (17, 96, 128),
                                   (2048, 1536, 1536)])
def test_forward_eight_wave_kernel(m, n, k, plan, device, monkeypatch):
    """The 8-wave forward kernel (288- or 256-token tiles, one work-group per CU), with bias, on
    its own and with a two-way split of the contraction (it takes k % 64 == 0)."""
    from decik_amd.nf4 import linear_forward

    monkeypatch.setenv("DECIK_FWD_PLAN", plan)
    packed, qs, w16 = make_weight((n, k), seed=n + k + 1, device=device)
    x = randn16((m, k), seed=m + 2, device=device)
    b = randn16((n,), seed=6, device=device, std=0.1)
    (y,) = linear_forward(x, [dict(packed=packed, qs=qs, bias=b)])
    ref = O.linear_ref(x.cpu().numpy(), w16, b.cpu().numpy())
    assert_close(y, ref, what=f"fwd8 {plan} {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(830, 1536, 1536), (830, 256, 1536), (830, 8960, 1536),
                                   (830, 1536, 8960), (1, 3584, 3584), (64, 512, 3584),
                                   (17, 96, 128), (300, 264, 160)])
def test_backward(m, n, k, device):
    from decik_amd.nf4 import linear_backward

    packed, qs, w16 = make_weight((n, k), seed=3 * n + k, device=device)
    dy = randn16((m, n), seed=m + 1, device=device, std=1e-2)
    dx = linear_backward([dict(packed=packed, qs=qs, dy=dy)], m, k)
    ref = O.linear_dx_ref(dy.cpu().numpy(), w16)
    assert dx.shape == (m, k) and dx.dtype == torch.float16
    assert_close(dx, ref, what=f"bwd {m}x{n}x{k}")


def test_backward_fp32_output(device):
    from decik_amd.nf4 import linear_backward

    packed, qs, w16 = make_weight((1536, 1536), seed=11, device=device)
    dy = randn16((830, 1536), seed=2, device=device, std=1e-2)
    dx32 = linear_backward([dict(packed=packed, qs=qs, dy=dy)], 830, 1536, dx_fp32=True)
    dx16 = linear_backward([dict(packed=packed, qs=qs, dy=dy)], 830, 1536)
    assert dx32.dtype == torch.float32
    ref = O.linear_dx_ref(dy.cpu().numpy(), w16)
    assert_close(dx32, ref, max_rel=1e-4, mean_rel=1e-5, what="bwd fp32")
    assert torch.equal(dx32.to(torch.float16), dx16)


@pytest.mark.parametrize("plan", ["2,1", "4,1", "1,3", "2,2,8", "4,1,8"])
def test_grouped_forward_equals_separate(plan, device, monkeypatch):
    """q, k, v sharing X in one launch = three launches with the same plan (bit for bit: the
    same tile shape and contraction splits give the same fp32 summation order), and each output
    meets the bar against the oracle with the planner's own choice."""
    from decik_amd.nf4 import linear_forward

    x = randn16((830, 1536), seed=1, device=device)
    ws = [make_weight(s, seed=20 + i, device=device) for i, s in
          enumerate([(1536, 1536), (256, 1536), (256, 1536)])]
    bs = [randn16((s[2].shape[0],), seed=30 + i, device=device, std=0.1) for i, s in enumerate(ws)]
    items = [dict(packed=p, qs=q, bias=b) for (p, q, _), b in zip(ws, bs)]
    planned = linear_forward(x, items)
    monkeypatch.setenv("DECIK_FWD_PLAN", plan)
    outs = linear_forward(x, items)
    for (p, q, w16), b, o, o2 in zip(ws, bs, outs, planned):
        (single,) = linear_forward(x, [dict(packed=p, qs=q, bias=b)])
        assert torch.equal(o, single)
        ref = O.linear_ref(x.cpu().numpy(), w16, b.cpu().numpy())
        assert_close(o, ref, what="grouped")
        assert_close(o2, ref, what="grouped, planned")


def test_grouped_backward_sums(device):
    """dX = dgate . Wg + dup . Wu in one launch (solution/mlp.py:106-109)."""
    from decik_amd.nf4 import linear_backward

    (pg, qg, wg), (pu, qu, wu) = (make_weight((8960, 1536), seed=40 + i, device=device) for i in range(2))
    dg = randn16((830, 8960), seed=1, device=device, std=1e-2)
    du = randn16((830, 8960), seed=2, device=device, std=1e-2)
    dx = linear_backward([dict(packed=pg, qs=qg, dy=dg), dict(packed=pu, qs=qu, dy=du)], 830, 1536,
                         dx_fp32=True)
    ref = O.linear_dx_ref(dg.cpu().numpy(), wg) + O.linear_dx_ref(du.cpu().numpy(), wu)
    assert_close(dx, ref, max_rel=1e-4, mean_rel=1e-5, what="grouped bwd")


@pytest.mark.parametrize("nested,blocksize", [(False, 64), (True, 128), (True, 256), (False, 32)])
def test_plain_and_other_blocksizes(nested, blocksize, device):
    from decik_amd.nf4 import linear_backward, linear_forward

    packed, qs, w16 = make_weight((512, 1024), seed=blocksize, device=device, nested=nested,
                                  blocksize=blocksize)
    x = randn16((100, 1024), seed=4, device=device)
    (y,) = linear_forward(x, [dict(packed=packed, qs=qs)])
    assert_close(y, O.linear_ref(x.cpu().numpy(), w16), what="fwd plain")
    dy = randn16((100, 512), seed=6, device=device)
    dx = linear_backward([dict(packed=packed, qs=qs, dy=dy)], 100, 1024)
    assert_close(dx, O.linear_dx_ref(dy.cpu().numpy(), w16), what="bwd plain")


def test_split_k_is_deterministic(device):
    """Shapes that take the split-K path give bitwise-identical results run to run, and the
    workspace counters are back at zero afterwards (the next call is still right)."""
    from decik_amd.nf4 import linear_backward, linear_forward

    packed, qs, w16 = make_weight((1536, 8960), seed=77, device=device)
    x = randn16((830, 8960), seed=8, device=device)
    (y1,) = linear_forward(x, [dict(packed=packed, qs=qs)])
    (y2,) = linear_forward(x, [dict(packed=packed, qs=qs)])
    assert torch.equal(y1, y2)
    dy = randn16((830, 1536), seed=9, device=device, std=1e-2)
    d1 = linear_backward([dict(packed=packed, qs=qs, dy=dy)], 830, 8960)
    d2 = linear_backward([dict(packed=packed, qs=qs, dy=dy)], 830, 8960)
    assert torch.equal(d1, d2)
    # a third call after a different shape reused the workspace: still identical
    linear_forward(x[:100], [dict(packed=packed, qs=qs)])
    (y3,) = linear_forward(x, [dict(packed=packed, qs=qs)])
    assert torch.equal(y1, y3)
    assert_close(y1, O.linear_ref(x.cpu().numpy(), w16), what="split-k fwd")
    assert_close(d1, O.linear_dx_ref(dy.cpu().numpy(), w16), what="split-k bwd")


def test_nf4linear_autograd(device):
    """NF4Linear (the reference's autograd Function) forward + backward through the fused path,
    with bias and a 3-D input."""
    from decik_amd.nf4 import NF4Linear

    packed, qs, w16 = make_weight((1536, 1536), seed=12, device=device)
    b = randn16((1536,), seed=13, device=device, std=0.1)
    x = randn16((2, 415, 1536), seed=14, device=device).requires_grad_(True)
    y = NF4Linear.apply(x, packed, b, qs)
    gy = randn16((2, 415, 1536), seed=15, device=device, std=1e-2)
    y.backward(gy)
    xn = x.detach().reshape(-1, 1536).cpu().numpy()
    assert_close(y.reshape(-1, 1536), O.linear_ref(xn, w16, b.cpu().numpy()), what="NF4Linear y")
    assert_close(x.grad.reshape(-1, 1536), O.linear_dx_ref(gy.reshape(-1, 1536).cpu().numpy(), w16),
                 what="NF4Linear dx")


def test_unsupported_k_takes_reference_algorithm(device):
    """k % 32 != 0: NF4Linear takes dequantize + F.linear on the GPU (the reference's own
    algorithm) and still meets the bar."""
    from decik_amd.nf4 import NF4Linear

    packed, qs, w16 = make_weight((64, 40), seed=16, device=device)
    x = randn16((10, 40), seed=17, device=device).requires_grad_(True)
    y = NF4Linear.apply(x, packed, None, qs)
    y.sum().backward()
    assert_close(y, O.linear_ref(x.detach().cpu().numpy(), w16), what="odd k")
    ref_dx = O.linear_dx_ref(np.ones((10, 64), np.float16), w16)
    assert_close(x.grad, ref_dx, what="odd k dx")


def test_scale_cache_follows_in_place_updates(device, monkeypatch):
    """Fused GEMMs switched to the derived fp32 block scales reuse the cached scales of a nested
    weight; changing a statistics tensor in place (its version counter moves) makes the next call
    recompute them."""
    from decik_amd import _lib, nf4
    from decik_amd.nf4 import linear_forward
    from helpers import oracle_state

    monkeypatch.setattr(nf4, "_launch_scales", nf4._scales)

    packed, qs, w16 = make_weight((512, 1024), seed=91, device=device)
    x = randn16((64, 1024), seed=92, device=device)
    (y1,) = linear_forward(x, [dict(packed=packed, qs=qs)])
    s1 = _lib.SCALES.get(packed, qs, device)
    assert _lib.SCALES.get(packed, qs, device) is s1  # a hit
    qs.state2.absmax.mul_(2.0)
    (y2,) = linear_forward(x, [dict(packed=packed, qs=qs)])
    s2 = _lib.SCALES.get(packed, qs, device)
    assert s2 is not s1 and not torch.equal(y1, y2)
    w16b = O.dequant_nf4(oracle_state(packed, qs), nthreads=0)
    assert_close(y2, O.linear_ref(x.cpu().numpy(), w16b), what="after in-place update")


def test_large_m_planned_launches(device):
    """M = 4096 tokens with the planner's own choices (eight-wave kernels, splits as planned):
    gate/up forward with the SwiGLU epilogue and the summed gate/up input gradient, against fp32
    GEMMs on the GPU of the oracle's bit-exact dequantized weights (fp32 reference of the same
    fp16 operands; the float64 CPU reference is too slow at this size)."""
    from decik_amd.nf4 import glu_forward, launch_plan, linear_backward

    m, n, k = 4096, 1024, 1536
    (pg, qg, wg), (pu, qu, wu) = (make_weight((n, k), seed=110 + i, device=device, nested=False) for i in range(2))
    x = randn16((m, k), seed=111, device=device)
    gate, up, h = glu_forward(x, dict(packed=pg, qs=qg), dict(packed=pu, qs=qu))
    wg32 = torch.from_numpy(wg.astype(np.float32)).to(device)
    wu32 = torch.from_numpy(wu.astype(np.float32)).to(device)
    g_ref = x.float() @ wg32.t()
    u_ref = x.float() @ wu32.t()
    assert_close(gate, g_ref.cpu().numpy(), what="large-M gate")
    assert_close(up, u_ref.cpu().numpy(), what="large-M up")
    dg = randn16((m, n), seed=112, device=device, std=1e-2)
    du = randn16((m, n), seed=113, device=device, std=1e-2)
    assert launch_plan(True, m, k, [n, n])["kernel"] == "nf4_bwd8_kernel"
    dx = linear_backward([dict(packed=pg, qs=qg, dy=dg), dict(packed=pu, qs=qu, dy=du)], m, k, dx_fp32=True)
    ref = dg.float() @ wg32 + du.float() @ wu32
    assert_close(dx, ref.cpu().numpy(), max_rel=1e-4, mean_rel=1e-5, what="large-M grouped bwd")


def test_empty_token_batches(device):
    """Zero token rows: NF4Linear (forward and backward, with and without leading dims), the
    fused linear entries and the GLU forward return empty outputs and launch nothing; the C
    entries accept m = 0 with valid shapes and return 0."""
    from decik_amd._lib import LinearBwdGroup, LinearFwdGroup, lib, ptr, stream_of, weight_desc
    from decik_amd.nf4 import NF4Linear, glu_forward, linear_backward, linear_forward

    n, k = 256, 512
    packed, qs, _ = make_weight((n, k), seed=5, device=device)
    for shape in ((0, k), (3, 0, k)):
        x = torch.zeros(shape, dtype=torch.float16, device=device, requires_grad=True)
        y = NF4Linear.apply(x, packed, None, qs)
        assert y.shape == shape[:-1] + (n,)
        y.sum().backward()
        assert x.grad.shape == shape
    x0 = torch.zeros((0, k), dtype=torch.float16, device=device)
    (y0,) = linear_forward(x0, [dict(packed=packed, qs=qs)])
    assert y0.shape == (0, n)
    dx0 = linear_backward([dict(packed=packed, qs=qs, dy=torch.zeros((0, n), dtype=torch.float16, device=device))], 0, k)
    assert dx0.shape == (0, k)
    g, u, h = glu_forward(x0, dict(packed=packed, qs=qs), dict(packed=packed, qs=qs))
    assert g.shape == u.shape == h.shape == (0, n)
    w, keep = weight_desc(packed, qs, device)
    fg = (LinearFwdGroup * 1)()
    fg[0].w = w
    out = torch.empty((1, n), dtype=torch.float16, device=device)
    fg[0].y, fg[0].ldy = out.data_ptr(), n
    xs = torch.zeros((1, k), dtype=torch.float16, device=device)
    assert lib().dk_nf4_linear_fwd(ptr(xs), 0, k, k, fg, 1, 0, None, 0, stream_of(device)) == 0
    bg = (LinearBwdGroup * 1)()
    bg[0].w = w
    dys = torch.zeros((1, n), dtype=torch.float16, device=device)
    bg[0].dy, bg[0].lddy = dys.data_ptr(), n
    dxs = torch.empty((1, k), dtype=torch.float16, device=device)
    assert lib().dk_nf4_linear_bwd(bg, 1, 0, k, ptr(dxs), k, 0, 0, None, 0, stream_of(device)) == 0
    torch.cuda.synchronize()
    del keep
