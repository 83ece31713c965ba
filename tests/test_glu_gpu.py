"""SwiGLU fused into the gate/up forward launch and into the down-projection input-gradient
launch (the Qwen2 MLP of solution/mlp.py:69-71, 95-104). Each fused entry must give the same
bits as the two-launch path it replaces -- the grouped GEMM (or dH = dY . W) followed by the
SwiGLU kernel -- when both run the same tile plan (pinned here: the same tile shape and no
contraction split give the same fp32 summation order), and the outputs meet the GEMM bar
against the oracle (max|err| <= 1e-2 max|ref|, mean rel <= 1e-3)."""

import pytest
import torch

from helpers import assert_close, make_weight, oracle_state, randn16
from oracle import nf4 as O

pytestmark = pytest.mark.gpu

# (M, N, K): the Qwen2.5-1.5B gate/up at 830 tokens, a ragged N (not a multiple of the 128-row
# GLU tile), N smaller than one tile, and a single token.
GLU_SHAPES = [(830, 8960, 1536), (64, 264, 256), (17, 96, 128), (1, 512, 512)]


def _separate_glu(x, gate_it, up_it):
    from decik_amd.nf4 import linear_forward
    from decik_amd.swiglu import swiglu_fwd

    g, u = linear_forward(x, [gate_it, up_it])
    return g, u, swiglu_fwd(g, u)


@pytest.mark.parametrize("plan", ["4,1", "2,1", "1,1", "2,1,8", "4,1,8", "9,1,8"])
@pytest.mark.parametrize("m,n,k", GLU_SHAPES)
def test_glu_forward_equals_separate(m, n, k, plan, device, monkeypatch):
    from decik_amd.nf4 import glu_forward

    monkeypatch.setenv("DECIK_FWD_PLAN", plan)
    pg, qg, wg = make_weight((n, k), seed=n + 1, device=device)
    pu, qu, wu = make_weight((n, k), seed=n + 2, device=device)
    x = randn16((m, k), seed=m + 3, device=device)
    bg = randn16((n,), seed=4, device=device, std=0.1)
    bu = randn16((n,), seed=5, device=device, std=0.1)
    gi, ui = dict(packed=pg, qs=qg, bias=bg), dict(packed=pu, qs=qu, bias=bu)
    g, u, h = glu_forward(x, gi, ui)
    g2, u2, h2 = _separate_glu(x, gi, ui)
    assert torch.equal(g, g2) and torch.equal(u, u2) and torch.equal(h, h2)
    _, _, h3 = glu_forward(x, gi, ui, keep_gate_up=False)
    assert torch.equal(h3, h)
    xn = x.cpu().numpy()
    assert_close(g, O.linear_ref(xn, wg, bg.cpu().numpy()), what=f"gate {m}x{n}x{k}")
    assert_close(u, O.linear_ref(xn, wu, bu.cpu().numpy()), what=f"up {m}x{n}x{k}")


def test_glu_forward_with_lora(device, monkeypatch):
    from decik_amd.lora import lora_down
    from decik_amd.nf4 import glu_forward

    monkeypatch.setenv("DECIK_FWD_PLAN", "4,1")
    m, n, k, r = 300, 384, 512, 16
    pg, qg, _ = make_weight((n, k), seed=41, device=device)
    pu, qu, _ = make_weight((n, k), seed=42, device=device)
    x = randn16((m, k), seed=43, device=device)
    items = []
    for i, (p, q) in enumerate([(pg, qg), (pu, qu)]):
        a = randn16((r, k), seed=50 + i, device=device, std=0.05)
        b = randn16((n, r), seed=60 + i, device=device, std=0.05)
        items.append(dict(packed=p, qs=q, lora_u=lora_down(x, a), lora_b=b, lora_scale=2.0))
    items[1]["lora_u"], items[1]["lora_b"] = None, None  # LoRA on gate only
    g, u, h = glu_forward(x, items[0], items[1], lora_rank=r)
    from decik_amd.nf4 import linear_forward
    from decik_amd.swiglu import swiglu_fwd

    g2, u2 = linear_forward(x, items, lora_rank=r)
    assert torch.equal(g, g2) and torch.equal(u, u2) and torch.equal(h, swiglu_fwd(g2, u2))


def _glu_groups(items, outs, n, device):
    from decik_amd._lib import LinearFwdGroup, weight_desc

    groups = (LinearFwdGroup * 2)()
    keep = []
    for i, ((p, q), y) in enumerate(zip(items, outs)):
        w, kp = weight_desc(p, q, device)  # the statistics as stored: no cached scales
        keep += kp
        groups[i].w = w
        groups[i].y = None if y is None else y.data_ptr()
        groups[i].ldy = n
    return groups, keep


@pytest.mark.parametrize("m,n,k,plan", [(64, 256, 256, "2,1,8"), (830, 8960, 1536, None), (300, 384, 512, "4,1,8")])
def test_glu_forward_nested_statistics_one_launch(m, n, k, plan, device, monkeypatch):
    """Raw double-quant statistics (bitsandbytes' nested absmax, decoded in the kernel with each
    weight's own code2 table) take the one-launch GLU forward: the same bits as the grouped launch
    on the derived fp32 block scales followed by the SwiGLU kernel, with or without the gate/up
    outputs."""
    from decik_amd._lib import lib, ptr, stream_of
    from decik_amd.nf4 import launch_plan

    if plan is not None:
        monkeypatch.setenv("DECIK_FWD_PLAN", plan)
    pg, qg, wg = make_weight((n, k), seed=71 + n, device=device)
    pu, qu, wu = make_weight((n, k), seed=72 + n, device=device)
    # different code2 tables for the two weights, so a wave reading the other weight's table fails
    qu.state2.code = qu.state2.code.flip(0).contiguous()
    wu = O.dequant_nf4(oracle_state(pu, qu), nthreads=0)
    x = randn16((m, k), seed=m + 73, device=device)
    g = torch.empty((m, n), dtype=torch.float16, device=device)
    u = torch.empty_like(g)
    h = torch.empty_like(g)
    groups, keep = _glu_groups([(pg, qg), (pu, qu)], [g, u], n, device)
    assert groups[0].w.nested == 1 and groups[1].w.nested == 1
    assert launch_plan(False, m, k, [n, n], glu=True, nested=True)["waves"] == 8
    rc = lib().dk_nf4_glu_fwd(ptr(x), m, k, k, groups, 0, ptr(h), n, stream_of(device))
    assert rc == 0, lib().dk_last_error()
    g2, u2, h2 = _separate_glu(x, dict(packed=pg, qs=qg), dict(packed=pu, qs=qu))
    torch.cuda.synchronize()
    assert torch.equal(g, g2) and torch.equal(u, u2) and torch.equal(h, h2)
    xn = x.cpu().numpy()
    assert_close(g, O.linear_ref(xn, wg, None), what="nested gate")
    assert_close(u, O.linear_ref(xn, wu, None), what="nested up")
    groups2, keep2 = _glu_groups([(pg, qg), (pu, qu)], [None, None], n, device)
    h3 = torch.empty_like(h)
    rc = lib().dk_nf4_glu_fwd(ptr(x), m, k, k, groups2, 0, ptr(h3), n, stream_of(device))
    assert rc == 0, lib().dk_last_error()
    torch.cuda.synchronize()
    assert torch.equal(h3, h)
    del keep, keep2


def test_glu_forward_narrow_blocks_take_two_launches(device):
    """Weights of 32-element blocks run the grouped launch and the SwiGLU kernel; without gate/up
    outputs the entry refuses."""
    from decik_amd._lib import lib, ptr, stream_of

    m, n, k = 64, 256, 256
    pg, qg, wg = make_weight((n, k), seed=81, device=device, blocksize=32)
    pu, qu, wu = make_weight((n, k), seed=82, device=device, blocksize=32)
    x = randn16((m, k), seed=83, device=device)
    g = torch.empty((m, n), dtype=torch.float16, device=device)
    u = torch.empty_like(g)
    h = torch.empty_like(g)
    groups, keep = _glu_groups([(pg, qg), (pu, qu)], [g, u], n, device)
    rc = lib().dk_nf4_glu_fwd(ptr(x), m, k, k, groups, 0, ptr(h), n, stream_of(device))
    assert rc == 0, lib().dk_last_error()
    torch.cuda.synchronize()
    from decik_amd.swiglu import swiglu_fwd

    assert_close(g, O.linear_ref(x.cpu().numpy(), wg, None), what="narrow-block gate")
    assert torch.equal(h, swiglu_fwd(g, u))
    groups[0].y = None
    rc = lib().dk_nf4_glu_fwd(ptr(x), m, k, k, groups, 0, ptr(h), n, stream_of(device))
    assert rc != 0 and b"gate and up outputs" in lib().dk_last_error()
    del keep


@pytest.mark.parametrize("blocksize", [32, 64])
@pytest.mark.parametrize("m,n,k", [(8, 256, 1024), (24, 1536, 1536)])
def test_glu_forward_few_rows_without_workspace(m, n, k, blocksize, device, monkeypatch):
    """The GLU entry takes no workspace. At 8 and 24 token rows with no forced plan, raw nested
    statistics take the one-launch GLU kernel (blocksize 64) and 32-element blocks the grouped
    launch plus the SwiGLU kernel, whose small-M forward would split these shapes when a workspace
    is allowed: it must run them in a single pass. Gate and up meet the bar against the oracle and
    h is the SwiGLU of the returned gate and up, bit for bit."""
    from decik_amd._lib import lib, ptr, stream_of
    from decik_amd.swiglu import swiglu_fwd

    monkeypatch.delenv("DECIK_FWD_PLAN", raising=False)
    monkeypatch.delenv("DECIK_SMALL_M", raising=False)
    pg, qg, wg = make_weight((n, k), seed=91 + m, device=device, blocksize=blocksize)
    pu, qu, wu = make_weight((n, k), seed=92 + m, device=device, blocksize=blocksize)
    x = randn16((m, k), seed=93 + m, device=device)
    g = torch.empty((m, n), dtype=torch.float16, device=device)
    u = torch.empty_like(g)
    h = torch.empty_like(g)
    groups, keep = _glu_groups([(pg, qg), (pu, qu)], [g, u], n, device)
    assert groups[0].w.nested == 1 and groups[1].w.nested == 1
    rc = lib().dk_nf4_glu_fwd(ptr(x), m, k, k, groups, 0, ptr(h), n, stream_of(device))
    assert rc == 0, lib().dk_last_error()
    g2, u2, h2 = _separate_glu(x, dict(packed=pg, qs=qg), dict(packed=pu, qs=qu))
    torch.cuda.synchronize()
    xn = x.cpu().numpy()
    assert_close(g, O.linear_ref(xn, wg, None), what=f"gate {m}x{n}x{k} bs {blocksize}")
    assert_close(u, O.linear_ref(xn, wu, None), what=f"up {m}x{n}x{k} bs {blocksize}")
    assert torch.equal(h, swiglu_fwd(g, u))
    if blocksize == 32:
        # the fallback is the separate path itself (the same small-M kernel, unsplit here)
        assert_close(g2, O.linear_ref(xn, wg, None), what="separate gate")
        assert torch.equal(h2, swiglu_fwd(g2, u2))
    del keep


BWD_SHAPES = [(830, 1536, 8960), (64, 264, 256), (17, 96, 128)]  # (M, N, K): W [N, K], dY [M, N]


@pytest.mark.parametrize("plan", ["2,1,8", "4,1,8"])
@pytest.mark.parametrize("m,n,k", BWD_SHAPES)
def test_bwd_swiglu_equals_separate(m, n, k, plan, device, monkeypatch):
    from decik_amd.nf4 import linear_backward, linear_backward_swiglu
    from decik_amd.swiglu import swiglu_bwd

    monkeypatch.setenv("DECIK_BWD_PLAN", plan)
    packed, qs, w16 = make_weight((n, k), seed=3 * n + k, device=device)
    dy = randn16((m, n), seed=m + 7, device=device, std=1e-2)
    gate = randn16((m, k), seed=8, device=device)
    up = randn16((m, k), seed=9, device=device)
    item = dict(packed=packed, qs=qs, dy=dy)
    dg, du = linear_backward_swiglu(item, gate, up)
    gh = linear_backward([item], m, k)
    dg2, du2 = swiglu_bwd(gh, gate, up)
    assert torch.equal(dg, dg2) and torch.equal(du, du2)
    # in place over gate / up (the MLP backward's buffers)
    g_, u_ = gate.clone(), up.clone()
    dg3, du3 = linear_backward_swiglu(item, g_, u_, out=(g_, u_))
    assert dg3.data_ptr() == g_.data_ptr() and torch.equal(dg3, dg) and torch.equal(du3, du)
    assert_close(gh, O.linear_dx_ref(dy.cpu().numpy(), w16), what=f"dH {m}x{n}x{k}")
