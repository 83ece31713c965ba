"""The fused paths captured in a HIP graph (torch.cuda.graph) and replayed: one layer's attention
projections with LoRA, dropout masks and RoPE (solution/attn.py:396-418, 206-273, 27-126), and
the MLP block (solution/mlp.py:62-110), forward and backward (torch.autograd.grad), over two
weight sets in one graph. Every kernel and library call on these paths must be capturable and
replay to the same bits: each of several replays, with eager work and synchronisations between
them, is compared with the eager results, and the replays' outputs with each other (a fill
recorded as a memset node, or any state a first replay leaves behind, shows up as a difference
on a later replay)."""

import numpy as np
import pytest
import torch

from helpers import make_weight, randn16
from test_rope_gpu import rope_tables

pytestmark = pytest.mark.gpu

H, HK, D = 12, 2, 128
LENGTHS = [100, 200, 130, 32, 150, 60, 90, 68]


def _replay_and_check(step, sets, eager_work, replays=3):
    """Capture step(s) for every set in one graph; replay `replays` times, each time checking every
    set's outputs against the eager results of the same step."""
    ref = [[t.clone() for t in step(s)] for s in sets]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(sets[0])  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        outs = [step(s) for s in sets]
    for r in range(replays):
        g.replay()
        torch.cuda.synchronize()
        for si, (o, e) in enumerate(zip(outs, ref)):
            for ti, (a, b) in enumerate(zip(o, e)):
                assert torch.equal(a, b), f"replay {r}, set {si}, output {ti} differs from the eager step"
        eager_work()  # the program's own work between replays
        torch.cuda.synchronize()


def test_attention_step_in_graph(device):
    from decik_amd import lora, nf4

    m = sum(LENGTHS)
    c, s = rope_tables(LENGTHS, D)
    cos, sin = torch.from_numpy(c).to(device), torch.from_numpy(s).to(device)
    g = torch.Generator().manual_seed(900)
    x = torch.randn((m, 1536), generator=g).to(device).requires_grad_(True)  # fp32 norm output
    attn = randn16((m, 1536), seed=901, device=device).requires_grad_(True)
    keep_q = (torch.rand((m, 1536), generator=g) >= 0.05).to(device)
    keep_v = (torch.rand((m, 1536), generator=g) >= 0.05).to(device)
    scale = torch.tensor(1.0 / 0.95, dtype=torch.float32, device=device)
    gq = randn16((1, H, m, D), seed=902, device=device, std=1e-2)
    gk = randn16((1, HK, m, D), seed=903, device=device, std=1e-2)
    gv = randn16((m, HK * D), seed=904, device=device, std=1e-2)
    go = randn16((m, 1536), seed=905, device=device, std=1e-2)
    sets = []
    for li in range(2):
        L = {}
        for j, (name, n) in enumerate((("q", H * D), ("k", HK * D), ("v", HK * D), ("o", 1536))):
            packed, qs, _ = make_weight((n, 1536), seed=910 + 10 * li + j, device=device)
            L[name] = (packed, qs, randn16((n,), seed=950 + 10 * li + j, device=device, std=0.1))
        for name, n in (("q", H * D), ("v", HK * D)):
            a = ((torch.rand((16, 1536), generator=g) * 2 - 1) / np.sqrt(1536)).to(device).requires_grad_(True)
            b = (torch.randn((n, 16), generator=g) * 1e-2).to(device).requires_grad_(True)
            L[name + "_lora"] = (a, b)
        sets.append(L)

    def step(L):
        bq, bv = lora.pack_keep(keep_q, keep_v)
        (aq, bqw), (av, bvw) = L["q_lora"], L["v_lora"]
        projs = (dict(packed=L["q"][0], qs=L["q"][1], bias=L["q"][2], lora_a=aq, lora_b=bqw, scaling=2.0,
                      keep_bits=bq, keep_scale=scale, p=0.05),
                 dict(packed=L["k"][0], qs=L["k"][1], bias=L["k"][2]),
                 dict(packed=L["v"][0], qs=L["v"][1], bias=L["v"][2], lora_a=av, lora_b=bvw, scaling=2.0,
                      keep_bits=bv, keep_scale=scale, p=0.05))
        q, k, v = lora.qkv_rope_projection(x, projs, cos, sin, H, HK)
        o = nf4.NF4Linear.apply(attn, L["o"][0], None, L["o"][1])
        grads = torch.autograd.grad([q, k, v, o], [x, attn, aq, bqw, av, bvw], [gq, gk, gv, go])
        return [q.detach(), k.detach(), v.detach(), o.detach(), *grads]

    other = randn16((m, 1536), seed=906, device=device)
    _replay_and_check(step, sets, lambda: nf4.linear_forward(other, [dict(packed=sets[0]["o"][0], qs=sets[0]["o"][1])]))


def test_mlp_step_in_graph(device):
    from decik_amd import nf4
    from decik_amd.mlp import FusedMLP

    m = 830
    x = randn16((m, 1536), seed=960, device=device).requires_grad_(True)
    dy = randn16((m, 1536), seed=961, device=device, std=1e-2)
    sets = []
    for li in range(2):
        ws = [make_weight(shape, seed=970 + 10 * li + j, device=device)[:2]
              for j, shape in enumerate(((8960, 1536), (8960, 1536), (1536, 8960)))]
        sets.append(ws)

    def step(ws):
        (gp, gq), (upp, upq), (dp, dq) = ws
        y = FusedMLP.apply(x, gp, gq, upp, upq, dp, dq, False)
        (dx,) = torch.autograd.grad([y], [x], [dy])
        return [y.detach(), dx]

    other = randn16((64, 1536), seed=962, device=device)
    _replay_and_check(step, sets, lambda: nf4.linear_forward(other, [dict(packed=sets[1][0][0], qs=sets[1][0][1])]))
