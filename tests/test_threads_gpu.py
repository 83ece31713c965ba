"""Calls from several host threads at once, as a training step makes them: the forward on the
caller's thread while autograd's device thread runs a backward, or a second stream driven from
another thread. Each thread's results must equal the same calls made alone (the kernels are
deterministic, so bit for bit): the per-stream workspaces, the descriptor and block-scale caches
and the planner's memo are shared state, and the library entry points must be reentrant
(the reference's entry points are called from the main thread and from autograd's thread)."""

import threading

import pytest
import torch

from helpers import make_weight, randn16

pytestmark = pytest.mark.gpu


def _work(device, seed):
    """One iteration of this thread's work as a function: for three weights, the fused forward and
    input gradient (split-K shapes among them, which take the per-stream workspace) and
    NF4Linear's autograd round trip; returns the outputs."""
    from decik_amd.nf4 import NF4Linear, linear_backward, linear_forward

    shapes = [((1536, 1536), 830), ((256, 1536), 64), ((8960, 1536), 300)]
    items = []
    for i, ((n, k), m) in enumerate(shapes):
        packed, qs, _ = make_weight((n, k), seed=seed + i, device=device)
        x = randn16((m, k), seed=seed + 10 + i, device=device)
        dy = randn16((m, n), seed=seed + 20 + i, device=device, std=1e-2)
        items.append((packed, qs, x, dy))

    def one():
        outs = []
        for packed, qs, x, dy in items:
            (y,) = linear_forward(x, [dict(packed=packed, qs=qs)])
            dx = linear_backward([dict(packed=packed, qs=qs, dy=dy)], x.shape[0], x.shape[1])
            xa = x.clone().requires_grad_(True)
            ya = NF4Linear.apply(xa, packed, None, qs)
            ya.backward(dy)
            outs += [y, dx, ya.detach(), xa.grad]
        return outs

    return one


def test_two_threads_two_streams(device):
    """Two threads, each on its own stream, each repeating its own forward / input-gradient calls:
    every result equals what the same thread computes alone."""
    work = [_work(device, 500), _work(device, 600)]
    expected = []
    for w in work:
        out = w()
        torch.cuda.synchronize()
        expected.append([t.clone() for t in out])
    errors, results = [], [None, None]

    def run(i):
        try:
            s = torch.cuda.Stream(device=device)
            with torch.cuda.stream(s):
                got = []
                for _ in range(6):
                    got.append(work[i]())
                s.synchronize()
            results[i] = got
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(repr(e))

    threads = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors
    for i in range(2):
        for it in results[i]:
            for a, b in zip(it, expected[i]):
                assert torch.equal(a, b)


def test_forward_while_autograd_thread_runs_backward(device):
    """The training pattern: the caller's thread keeps launching forwards while autograd's own
    device thread runs the backward of an earlier graph (torch's default for CUDA tensors), on one
    stream: the gradients and the forwards equal the same calls made one after another."""
    from decik_amd.nf4 import NF4Linear, linear_forward

    packed, qs, _ = make_weight((1536, 8960), seed=700, device=device)
    p2, q2, _ = make_weight((8960, 1536), seed=701, device=device)
    x = randn16((830, 8960), seed=702, device=device)
    x2 = randn16((830, 1536), seed=703, device=device)
    dy = randn16((830, 1536), seed=704, device=device, std=1e-2)

    def backward_once():
        xa = x.clone().requires_grad_(True)
        NF4Linear.apply(xa, packed, None, qs).backward(dy)
        return xa.grad

    ref_grad = backward_once()
    (ref_y,) = linear_forward(x2, [dict(packed=p2, qs=q2)])
    torch.cuda.synchronize()
    ref_grad, ref_y = ref_grad.clone(), ref_y.clone()
    grads, ys, errors = [], [], []

    def backwards():
        try:
            for _ in range(8):
                grads.append(backward_once())
        except Exception as e:  # noqa: BLE001
            errors.append(repr(e))

    t = threading.Thread(target=backwards)
    t.start()
    for _ in range(16):
        ys.append(linear_forward(x2, [dict(packed=p2, qs=q2)])[0])
    t.join(timeout=120)
    torch.cuda.synchronize()
    assert not errors, errors
    assert all(torch.equal(g, ref_grad) for g in grads) and len(grads) == 8
    assert all(torch.equal(y, ref_y) for y in ys)
