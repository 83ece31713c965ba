"""Weights with different NF4 code books in one launch. Each weight's descriptor carries its own
book (QuantState.code, solution/nf4.py:70-79); bitsandbytes always writes the same 16 values,
but the boundary takes any, and the kernels keep one book per weight: per column tile in the
grouped forward, per wave half in the GLU forward, and per contraction segment in the input
gradient (the eight-wave kernel rewrites its byte-pair book between weights). Here the second
weight's book is the first one reversed and scaled, so a lookup in the wrong book changes
every product; every kernel family is forced in turn and checked against the oracle's
dequantization of the same bytes with each weight's own book."""

import pytest

from helpers import O, assert_close, make_weight, oracle_state, randn16

pytestmark = pytest.mark.gpu


def _two_books(device, n1, n2, k, nested=True):
    p1, q1, w1 = make_weight((n1, k), seed=301 + n1, device=device, nested=nested)
    p2, q2, w2_first_book = make_weight((n2, k), seed=302 + n2, device=device, nested=nested)
    q2.code = (q2.code.flip(0) * 0.75).contiguous()
    w2 = O.dequant_nf4(oracle_state(p2, q2), nthreads=0)
    # a kernel that read the first book for the second weight would be far outside the bar
    assert O.tolerance(w2_first_book, w2)[0] > 0.5
    return (p1, q1, w1), (p2, q2, w2)


@pytest.mark.parametrize("plan", ["1,1,4", "2,2,4", "2,2,8", "4,1,8", "7,1,8", "8,2,8"])
def test_grouped_forward(plan, device, monkeypatch):
    from decik_amd.nf4 import linear_forward

    monkeypatch.setenv("DECIK_FWD_PLAN", plan)
    (p1, q1, w1), (p2, q2, w2) = _two_books(device, 256, 264, 512)
    x = randn16((300, 512), seed=310, device=device)
    y1, y2 = linear_forward(x, [dict(packed=p1, qs=q1), dict(packed=p2, qs=q2)])
    xn = x.cpu().numpy()
    assert_close(y1, O.linear_ref(xn, w1), what=f"first book, plan {plan}")
    assert_close(y2, O.linear_ref(xn, w2), what=f"second book, plan {plan}")


@pytest.mark.parametrize("plan", ["9,1,8", "2,1,8", "2,1"])
def test_glu_forward(plan, device, monkeypatch):
    from decik_amd.nf4 import glu_forward

    monkeypatch.setenv("DECIK_FWD_PLAN", plan)
    (pg, qg, wg), (pu, qu, wu) = _two_books(device, 384, 384, 512)
    x = randn16((300, 512), seed=311, device=device)
    g, u, h = glu_forward(x, dict(packed=pg, qs=qg), dict(packed=pu, qs=qu))
    xn = x.cpu().numpy()
    gr, ur = O.linear_ref(xn, wg), O.linear_ref(xn, wu)
    assert_close(g, gr, what=f"gate, plan {plan}")
    assert_close(u, ur, what=f"up, plan {plan}")
    assert_close(h, O.swiglu_fwd_ref(g.cpu().numpy(), u.cpu().numpy()), what=f"h, plan {plan}")


@pytest.mark.parametrize("plan", ["2,1,8", "2,2,8", "4,1,8", "4,2,8", "7,2,8"])
@pytest.mark.parametrize("nested,raw", [(True, False), (True, True), (False, False)])
def test_grouped_input_gradient(plan, nested, raw, device, monkeypatch):
    """raw: nested weights described by their double-quant statistics (the default); otherwise by
    the derived fp32 block scales."""
    from decik_amd import nf4
    from decik_amd.nf4 import linear_backward

    monkeypatch.setenv("DECIK_BWD_PLAN", plan)
    if not raw:
        monkeypatch.setattr(nf4, "_launch_scales", nf4._scales)
    (p1, q1, w1), (p2, q2, w2) = _two_books(device, 256, 200, 512, nested=nested)
    d1 = randn16((130, 256), seed=312, device=device, std=1e-2)
    d2 = randn16((130, 200), seed=313, device=device, std=1e-2)
    dx = linear_backward([dict(packed=p1, qs=q1, dy=d1), dict(packed=p2, qs=q2, dy=d2)], 130, 512, dx_fp32=True)
    ref = O.linear_dx_ref(d1.cpu().numpy(), w1) + O.linear_dx_ref(d2.cpu().numpy(), w2)
    assert_close(dx, ref, max_rel=1e-4, mean_rel=1e-5, what=f"two books, plan {plan}, nested={nested} raw={raw}")


@pytest.mark.parametrize("m,small", [(1, "gemv"), (2, "gemv"), (4, None), (8, "skinny")])
def test_small_m_forward(m, small, device, monkeypatch):
    """Two weights with different code books in one small-M launch: GEMV (forced, or the planner's
    choice for these small weights at 4 rows) and the small-M MFMA kernel."""
    from decik_amd.nf4 import launch_plan, linear_forward

    if small is not None:
        monkeypatch.setenv("DECIK_SMALL_M", small)
    (p1, q1, w1), (p2, q2, w2) = _two_books(device, 256, 264, 1024)
    plan = launch_plan(False, m, 1024, [256, 264])
    assert plan["kernel"] == ("nf4_skinny_kernel" if small == "skinny" else "nf4_gemv_kernel")
    x = randn16((m, 1024), seed=314 + m, device=device)
    y1, y2 = linear_forward(x, [dict(packed=p1, qs=q1), dict(packed=p2, qs=q2)])
    xn = x.cpu().numpy()
    assert_close(y1, O.linear_ref(xn, w1), what=f"first book, {plan['kernel']} m={m}")
    assert_close(y2, O.linear_ref(xn, w2), what=f"second book, {plan['kernel']} m={m}")
