"""Seeded random launch shapes through the fused forward and input-gradient entry points (the
products of solution/nf4.py:93-104), each with the planner's own plan and with one forced plan
per eight-wave tile size, against the oracle's products of the bit-exact weights. The shapes
are drawn so that token counts, weight rows and contraction lengths fall off every tile, step
and block boundary the kernels assume (token rows 1..700, weight rows multiples of 8 from 8 to
1000, contractions multiples of 64 (forward) or 32 (input gradient) from 64 to 2112), with
nested statistics of blocks 64..256 or plain statistics of block 32."""

import numpy as np
import pytest

from helpers import O, assert_close, make_weight, randn16

pytestmark = pytest.mark.gpu

_RNG = np.random.default_rng(20261202)
CASES = []
for _i in range(12):
    m = int(_RNG.integers(1, 701))
    n = 8 * int(_RNG.integers(1, 126))
    k = 64 * int(_RNG.integers(1, 34))
    nested, bs = [(True, 64), (True, 128), (True, 256), (False, 32)][int(_RNG.integers(0, 4))]
    if k % bs:
        k = bs * max(1, k // bs)
    CASES.append((m, n, k, nested, bs, 7000 + _i))


@pytest.mark.parametrize("m,n,k,nested,bs,seed", CASES)
@pytest.mark.parametrize("plan", [None, "2,{s},8", "4,{s},8", "7,{s},8"])
def test_random_forward(m, n, k, nested, bs, seed, plan, device, monkeypatch):
    from decik_amd.nf4 import linear_forward

    if plan is not None:
        s = 1 + seed % min(3, k // 64)
        monkeypatch.setenv("DECIK_FWD_PLAN", plan.format(s=s))
    packed, qs, w16 = make_weight((n, k), seed=seed, device=device, nested=nested, blocksize=bs)
    x = randn16((m, k), seed=seed + 1, device=device)
    b = randn16((n,), seed=seed + 2, device=device, std=0.1)
    (y,) = linear_forward(x, [dict(packed=packed, qs=qs, bias=b)])
    assert_close(y, O.linear_ref(x.cpu().numpy(), w16, b.cpu().numpy()),
                 what=f"fwd m={m} n={n} k={k} nested={nested} bs={bs} plan={plan}")


@pytest.mark.parametrize("m,n,k,nested,bs,seed", CASES)
@pytest.mark.parametrize("plan", [None, "2,{s},8", "4,{s},8", "8,{s},8"])
def test_random_input_gradient(m, n, k, nested, bs, seed, plan, device, monkeypatch):
    from decik_amd.nf4 import linear_backward

    if plan is not None:
        s = 1 + seed % min(3, (n + 63) // 64)
        monkeypatch.setenv("DECIK_BWD_PLAN", plan.format(s=s))
    k_in = k - 32 if k > 64 and seed % 2 else k  # the input gradient also takes k % 64 == 32
    if k_in % bs:
        k_in = k
    packed, qs, w16 = make_weight((n, k_in), seed=seed, device=device, nested=nested, blocksize=bs)
    dy = randn16((m, n), seed=seed + 3, device=device, std=1e-2)
    dx = linear_backward([dict(packed=packed, qs=qs, dy=dy)], m, k_in, dx_fp32=True)
    assert_close(dx, O.linear_dx_ref(dy.cpu().numpy(), w16), max_rel=1e-4, mean_rel=1e-5,
                 what=f"bwd m={m} n={n} k={k_in} nested={nested} bs={bs} plan={plan}")


# Few token rows (the decoding regime: GEMV at 1-2 rows and at 3-8 on small weights, the small-M
# kernel otherwise up to 32 rows, split along
# the contraction where the rows cannot fill the GPU), with contractions up to 20480 so that X of
# long rows takes the GEMV's eight-wave work-groups.
_RNG_S = np.random.default_rng(20261203)
SMALL = []
for _i in range(12):
    m = [1, 2, int(_RNG_S.integers(3, 33))][_i % 3]
    n = 8 * int(_RNG_S.integers(1, 400))
    k = 64 * int(_RNG_S.integers(1, 321))
    nested, bs = [(True, 64), (True, 128), (True, 256), (False, 32)][int(_RNG_S.integers(0, 4))]
    if k % bs:
        k = bs * max(1, k // bs)
    SMALL.append((m, n, k, nested, bs, 8000 + _i))
# shapes whose X fills the GEMV's LDS (eight-wave work-groups), the 7B down projection among them
SMALL += [(1, 3584, 18944, True, 64, 8100), (1, 200, 20480, False, 32, 8101), (2, 304, 8192, True, 64, 8102),
          (1, 136, 16384, True, 128, 8103)]


@pytest.mark.parametrize("m,n,k,nested,bs,seed", SMALL)
def test_random_small_m_forward(m, n, k, nested, bs, seed, device, monkeypatch):
    import torch

    from decik_amd.nf4 import launch_plan, linear_forward

    kernel = launch_plan(False, m, k, [n], blocksize=bs)["kernel"]
    monkeypatch.setenv("DECIK_SMALL_M", "gemv")  # whether the GEMV can take the launch at all
    fits = launch_plan(False, m, k, [n], blocksize=bs)["kernel"] == "nf4_gemv_kernel"
    monkeypatch.delenv("DECIK_SMALL_M")
    w = n * k
    if m == 1 or (m == 2 and fits and w < 2 ** 25 and (k <= 12288 or w <= 2 ** 24)):
        assert kernel == "nf4_gemv_kernel"
    elif 3 <= m <= 4 and fits and w <= 2 ** 24:
        assert kernel == "nf4_gemv_kernel"  # 3-4 rows: weights up to 2^24
    elif 5 <= m <= 8 and fits and w < 2 ** 23 and 4 * k * 2 <= 32768:
        assert kernel == "nf4_gemv_kernel"  # 5-8 rows on small weights
    else:
        assert kernel == ("nf4_fwd8_kernel" if m > 16 and (n + 63) // 64 > 256 else "nf4_skinny_kernel")
    packed, qs, w16 = make_weight((n, k), seed=seed, device=device, nested=nested, blocksize=bs)
    x = randn16((m, k), seed=seed + 1, device=device)
    b = randn16((n,), seed=seed + 2, device=device, std=0.1)
    (y,) = linear_forward(x, [dict(packed=packed, qs=qs, bias=b)])
    assert_close(y, O.linear_ref(x.cpu().numpy(), w16, b.cpu().numpy()),
                 what=f"small-m fwd m={m} n={n} k={k} nested={nested} bs={bs} kernel={kernel}")
    (y2,) = linear_forward(x, [dict(packed=packed, qs=qs, bias=b)])
    assert torch.equal(y, y2)


# The MLP's fused launches (solution/mlp.py:69-71, 95-104) at seeded random shapes with the
# planner's own plans: gate/up + SwiGLU forward, and the down-projection input gradient with the
# SwiGLU backward in its epilogue (contractions with k % 64 == 32 included).
_RNG_G = np.random.default_rng(20261204)
GLU = []
for _i in range(8):
    GLU.append((int(_RNG_G.integers(1, 701)), 8 * int(_RNG_G.integers(1, 200)),
                64 * int(_RNG_G.integers(1, 40)), 8200 + 10 * _i))


@pytest.mark.parametrize("m,n,k,seed", GLU)
def test_random_glu_forward(m, n, k, seed, device):
    import torch

    from decik_amd.nf4 import glu_forward
    from decik_amd.swiglu import swiglu_fwd

    pg, qg, wg = make_weight((n, k), seed=seed, device=device)
    pu, qu, wu = make_weight((n, k), seed=seed + 1, device=device)
    x = randn16((m, k), seed=seed + 2, device=device)
    bg = randn16((n,), seed=seed + 3, device=device, std=0.1)
    bu = randn16((n,), seed=seed + 4, device=device, std=0.1)
    g, u, h = glu_forward(x, dict(packed=pg, qs=qg, bias=bg), dict(packed=pu, qs=qu, bias=bu))
    xn = x.cpu().numpy()
    assert_close(g, O.linear_ref(xn, wg, bg.cpu().numpy()), what=f"gate m={m} n={n} k={k}")
    assert_close(u, O.linear_ref(xn, wu, bu.cpu().numpy()), what=f"up m={m} n={n} k={k}")
    assert torch.equal(h, swiglu_fwd(g, u))


@pytest.mark.parametrize("m,n,k,seed", GLU)
def test_random_bwd_swiglu(m, n, k, seed, device):
    import torch

    from decik_amd.nf4 import linear_backward_swiglu

    k_in = k - 32 if k > 64 and (seed // 10) % 2 else k  # W [n, k_in]: the down projection
    packed, qs, w16 = make_weight((n, k_in), seed=seed + 5, device=device)
    dy = randn16((m, n), seed=seed + 6, device=device, std=1e-2)
    gate = randn16((m, k_in), seed=seed + 7, device=device)
    up = randn16((m, k_in), seed=seed + 8, device=device)
    dg, du = linear_backward_swiglu(dict(packed=packed, qs=qs, dy=dy), gate, up)
    dh = torch.from_numpy(O.linear_dx_ref(dy.cpu().numpy(), w16)).half().numpy()
    dg_ref, du_ref = O.swiglu_bwd_ref(dh, gate.cpu().numpy(), up.cpu().numpy())
    assert_close(dg, dg_ref, what=f"dgate m={m} n={n} k={k_in}")
    assert_close(du, du_ref, what=f"dup m={m} n={n} k={k_in}")


@pytest.mark.parametrize("dx", [False, True])
def test_narrow_reduction_same_bits(dx, device, monkeypatch):
    """The split-K reduction of small launches (two columns a thread) sums every output's splits
    in the same order as the eight-column reduction of large ones: under one forced plan, the
    first 64 token rows of a 512-row launch (eight-column reduction) equal a 64-row launch of the
    same rows (two-column reduction) bit for bit, forward (fp16 out, bias) and input gradient
    (fp32 out)."""
    import torch

    from decik_amd.nf4 import linear_backward, linear_forward

    n, k = 2048, 1024
    packed, qs, _ = make_weight((n, k), seed=8300, device=device)
    if not dx:
        monkeypatch.setenv("DECIK_FWD_PLAN", "2,4,8")
        x = randn16((512, k), seed=8301, device=device)
        b = randn16((n,), seed=8302, device=device, std=0.1)
        (big,) = linear_forward(x, [dict(packed=packed, qs=qs, bias=b)])
        (small,) = linear_forward(x[:64].contiguous(), [dict(packed=packed, qs=qs, bias=b)])
    else:
        monkeypatch.setenv("DECIK_BWD_PLAN", "2,4,8")
        dy = randn16((512, n), seed=8303, device=device, std=1e-2)
        big = linear_backward([dict(packed=packed, qs=qs, dy=dy)], 512, k, dx_fp32=True)
        small = linear_backward([dict(packed=packed, qs=qs, dy=dy[:64].contiguous())], 64, k, dx_fp32=True)
    assert torch.equal(big[:64], small)
