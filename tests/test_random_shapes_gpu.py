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
