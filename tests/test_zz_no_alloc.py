"""dk_nf4_linear_bwd_noalloc (the input gradient with its split-K partials in a static device
array) through the C ABI, against dk_nf4_linear_bwd with a caller workspace, on consecutive
calls: the second with a smaller input, the third with a shape whose allocating plan needs more
than the scratch holds (the static entry then runs a plan with fewer splits). Same plan: the
same bits; capped plan: the parity bar, and every call against the oracle."""

import ctypes

import numpy as np
import pytest
import torch

from helpers import assert_close, make_weight, randn16
from oracle import nf4 as O

pytestmark = pytest.mark.gpu


def _groups(items, dev):
    from decik_amd import _lib
    from decik_amd.nf4 import _scales

    groups = (_lib.LinearBwdGroup * len(items))()
    keep = []
    for g, (packed, qs, dy) in enumerate(items):
        w, kp = _lib.weight_desc(packed, qs, dev, _scales(packed, qs, dev))
        keep += kp + [dy]
        groups[g].w = w
        groups[g].dy = dy.data_ptr()
        groups[g].lddy = dy.stride(0)
    return groups, keep


def _run(items, m, k, dx_fp32, noalloc):
    from decik_amd import _lib

    dev = items[0][2].device
    L = _lib.lib()
    groups, keep = _groups(items, dev)
    dx = torch.full((m, k), float("nan"), dtype=torch.float32 if dx_fp32 else torch.float16, device=dev)
    stream = _lib.stream_of(dev)
    if noalloc:
        rc = L.dk_nf4_linear_bwd_noalloc(groups, len(items), m, k, dx.data_ptr(), k, int(dx_fp32), 0, stream)
    else:
        ns = (ctypes.c_int64 * len(items))(*[int(it[1].shape[0]) for it in items])
        need = int(L.dk_nf4_linear_bwd_workspace(m, k, ns, len(items)))
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
        rc = L.dk_nf4_linear_bwd(groups, len(items), m, k, dx.data_ptr(), k, int(dx_fp32), 0,
                                 ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc)
    torch.cuda.synchronize()
    del keep
    return dx


def _workspace_need(m, k, ns):
    from decik_amd import _lib

    arr = (ctypes.c_int64 * len(ns))(*ns)
    return int(_lib.lib().dk_nf4_linear_bwd_workspace(m, k, arr, len(ns)))


def _oracle(items_np, m, cols):
    ref = np.zeros((m, len(cols)), np.float64)
    for w16, dy in items_np:
        ref += O._f64(dy) @ O._f64(w16[:, cols])
    return ref.astype(np.float32)


def test_noalloc_input_gradient_matches_allocating_entry(device):
    from decik_amd import _lib

    scratch = 64 << 20
    # Qwen2.5-1.5B gate/up input gradient (two weights summed), then a smaller call
    gate = make_weight((8960, 1536), seed=301, device=device)
    up = make_weight((8960, 1536), seed=302, device=device)
    for m, dx_fp32 in ((830, True), (300, False)):
        need = _workspace_need(m, 1536, [8960, 8960])
        assert 0 < need <= scratch  # a split plan that fits: both entries run it
        dg = randn16((m, 8960), seed=303 + m, device=device, std=1e-2)
        du = randn16((m, 8960), seed=304 + m, device=device, std=1e-2)
        items = [(gate[0], gate[1], dg), (up[0], up[1], du)]
        a = _run(items, m, 1536, dx_fp32, noalloc=False)
        b = _run(items, m, 1536, dx_fp32, noalloc=True)
        assert not torch.isnan(b).any()
        assert torch.equal(a, b), f"m={m}: the static-scratch entry differs from the allocating one"
        ref = _oracle([(gate[2], dg.cpu().numpy()), (up[2], du.cpu().numpy())], m, np.arange(1536))
        assert_close(b, ref, what=f"noalloc m={m}")
    # Qwen2.5-7B gate/up input gradient at the first token count whose allocating plan's
    # partials exceed the scratch (1660 with the present cost tables: five splits, 113 MiB)
    gate7 = make_weight((18944, 3584), seed=305, device=device)
    up7 = make_weight((18944, 3584), seed=306, device=device)
    m = next(t for t in (830, 1660, 3000, 8192) if _workspace_need(t, 3584, [18944, 18944]) > scratch)
    dg = randn16((m, 18944), seed=307, device=device, std=1e-2)
    du = randn16((m, 18944), seed=308, device=device, std=1e-2)
    items = [(gate7[0], gate7[1], dg), (up7[0], up7[1], du)]
    a = _run(items, m, 3584, False, noalloc=False)
    b = _run(items, m, 3584, False, noalloc=True)
    assert not torch.isnan(b.float()).any()
    assert_close(b, a.float().cpu().numpy(), what="noalloc capped plan vs allocating")
    cols = np.arange(0, 3584, 7)
    ref = _oracle([(gate7[2], dg.cpu().numpy()), (up7[2], du.cpu().numpy())], m, cols)
    assert_close(b[:, torch.as_tensor(cols, device=device)], ref, what="noalloc capped plan vs oracle")
    # and the first shape once more after the large call
    dg = randn16((300, 8960), seed=309, device=device, std=1e-2)
    items = [(gate[0], gate[1], dg)]
    assert torch.equal(_run(items, 300, 1536, False, noalloc=False), _run(items, 300, 1536, False, noalloc=True))
    assert _lib.lib().dk_last_error() == b""


def test_noalloc_two_launch_input_gradient(device):
    """The 7B down-projection input gradient at 830 tokens runs as two launches (the left-over
    columns split): its partials fit the scratch, so the static entry runs the same two launches
    and gives the same bits, fp16 and fp32."""
    from decik_amd.nf4 import launch_plan

    assert launch_plan(True, 830, 18944, [3584])["launches"] == 2
    assert 0 < _workspace_need(830, 18944, [3584]) <= 64 << 20
    down = make_weight((3584, 18944), seed=311, device=device)
    dy = randn16((830, 3584), seed=312, device=device, std=1e-2)
    items = [(down[0], down[1], dy)]
    for dx_fp32 in (False, True):
        a = _run(items, 830, 18944, dx_fp32, noalloc=False)
        b = _run(items, 830, 18944, dx_fp32, noalloc=True)
        assert not torch.isnan(b.float()).any()
        assert torch.equal(a, b)
    rows = np.arange(0, 830, 37)
    ref = O._f64(dy[torch.as_tensor(rows, device=device)].cpu().numpy()) @ O._f64(down[2])
    assert_close(b[torch.as_tensor(rows, device=device)], ref.astype(np.float32), what="noalloc two launches")
