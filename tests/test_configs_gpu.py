"""Full-size configurations on the GPU:

- C4, one Qwen2.5-1.5B layer: q/k/v (biases, LoRA r=16 on q and v) in one fused launch each way,
  o, and the MLP (gate+up+SwiGLU, down), forward and backward through the drop-in autograd API,
  against the oracle (float64 references of the same fp16 operands).
- C4, the 28-layer chain: all 196 NF4 weights (seeded, N(0, 0.02), bs 64, double quant), each
  layer fed by the previous layer's output (forward) or input gradient (backward), RMS-rescaled
  to fp16 between layers; every launch checked against fp32 GEMMs on the GPU of the oracle's
  bit-exact dequantized weights, on that launch's own inputs.
- C5, Qwen2.5-7B shapes at M in {1, 8, 64, 830, 8192}: forward and input gradient against the
  oracle on a subset of token rows (each output row depends on its own input row only).

Bar: max|err| <= 1e-2 max|ref|, sum|err| / sum|ref| <= 1e-3."""

import numpy as np
import pytest
import torch

from helpers import assert_close, make_weight, randn16
from oracle import nf4 as O

pytestmark = pytest.mark.gpu

M, HIDDEN, INTER = 830, 1536, 8960
SHAPES = [("q", 1536, 1536), ("k", 256, 1536), ("v", 256, 1536), ("o", 1536, 1536),
          ("gate", 8960, 1536), ("up", 8960, 1536), ("down", 1536, 8960)]


def _adapter(n, seed, device, r=16, b_std=3e-2):
    g = torch.Generator().manual_seed(seed)
    a = ((torch.rand((r, HIDDEN), generator=g) * 2 - 1) / np.sqrt(HIDDEN)).half().float().to(device)
    b = (torch.randn((n, r), generator=g) * b_std).half().float().to(device)
    return a.requires_grad_(True), b.requires_grad_(True)


def test_c4_one_layer_through_autograd(device):
    """One layer of the stack as a training step sees it: q/k/v with LoRA on q and v (one
    launch each way), o on the attention output, and the MLP on its own input, with gradients
    to the inputs and the adapters."""
    from decik_amd.lora import qkv_projection
    from decik_amd.mlp import FusedMLP
    from decik_amd.nf4 import NF4Linear

    s = 2.0
    w = {name: make_weight((n, k), seed=400 + j, device=device) for j, (name, n, k) in enumerate(SHAPES)}
    bias = {name: randn16((w[name][1].shape[0],), seed=410 + j, device=device, std=0.1)
            for j, name in enumerate(("q", "k", "v"))}
    (aq, bq), (av, bv) = _adapter(1536, 420, device), _adapter(256, 421, device)
    x = randn16((M, HIDDEN), seed=422, device=device).requires_grad_(True)
    attn = randn16((M, HIDDEN), seed=423, device=device).requires_grad_(True)
    x2 = randn16((M, HIDDEN), seed=424, device=device).float().requires_grad_(True)
    projs = [dict(packed=w["q"][0], qs=w["q"][1], bias=bias["q"], lora_a=aq, lora_b=bq, scaling=s),
             dict(packed=w["k"][0], qs=w["k"][1], bias=bias["k"], lora_a=None, lora_b=None, scaling=s),
             dict(packed=w["v"][0], qs=w["v"][1], bias=bias["v"], lora_a=av, lora_b=bv, scaling=s)]
    q, k, v = qkv_projection(x, projs)
    o = NF4Linear.apply(attn, w["o"][0], None, w["o"][1])
    mlp = FusedMLP.apply(x2, w["gate"][0], w["gate"][1], w["up"][0], w["up"][1], w["down"][0], w["down"][1], True)
    grads = [randn16(t.shape, seed=430 + i, device=device, std=1e-2) for i, t in enumerate((q, k, v, o, mlp))]
    torch.autograd.backward([q, k, v, o, mlp], grads)

    xn, an = x.detach().cpu().numpy(), attn.detach().cpu().numpy()
    gn = [g.cpu().numpy() for g in grads]
    dx_ref = np.zeros((M, HIDDEN), np.float64)
    for (name, out, ad), gr in zip((("q", q, (aq, bq)), ("k", k, None), ("v", v, (av, bv))), gn[:3]):
        w16 = w[name][2]
        y_ref = O.linear_ref(xn, w16, bias[name].cpu().numpy())
        dx_ref += O.linear_dx_ref(gr, w16)
        if ad is not None:
            a16, b16 = (t.detach().half().cpu().numpy() for t in ad)
            u16, lora = O.lora_fwd_ref(xn, a16, b16, s)
            y_ref = y_ref + lora
            _, da, db, dxl = O.lora_bwd_ref(gr, xn, u16, a16, b16, s)
            dx_ref += dxl
            assert_close(ad[0].grad, da, what=f"{name} dA")
            assert_close(ad[1].grad, db, what=f"{name} dB")
        assert_close(out, y_ref, what=f"{name} Y")
    assert_close(x.grad, dx_ref, what="q/k/v dX")
    assert_close(o, O.linear_ref(an, w["o"][2]), what="o Y")
    assert_close(attn.grad, O.linear_dx_ref(gn[3], w["o"][2]), what="o dX")
    ref = O.mlp_ref(x2.detach().half().cpu().numpy(), w["gate"][2], w["up"][2], w["down"][2], gn[4])
    assert_close(mlp, ref["out"], what="MLP out")
    assert_close(x2.grad, ref["dx"], what="MLP dX")


def _rms16(t):
    """RMS-rescaled fp16 copy (keeps the chain's activations at unit scale, as the RMSNorm
    between the reference's layers does)."""
    t = t.float()
    return (t / t.pow(2).mean(-1, keepdim=True).add(1e-6).sqrt()).half().contiguous()


def _check(got, ref, what):
    assert_close(got, ref.detach().cpu().numpy(), what=what)


def test_c4_28_layer_chain(device):
    """All 196 NF4 GEMMs of one training step of the 28-layer stack (plus the LoRA terms on q/v),
    in the order the step runs them, each launch checked on its own inputs against fp32 GEMMs of
    the oracle's dequantized weights."""
    from decik_amd import lora, nf4

    n_layers, s = 28, 2.0
    x = randn16((M, HIDDEN), seed=500, device=device)
    dy_top = randn16((M, HIDDEN), seed=501, device=device, std=1e-2)
    stack = []
    for layer in range(n_layers):
        ws = {}
        for j, (name, n, k) in enumerate(SHAPES):
            packed, qs, w16 = make_weight((n, k), seed=1000 + 7 * layer + j, device=device)
            ws[name] = (packed, qs, torch.from_numpy(w16).to(device))  # oracle's fp16 weights on the GPU
        ws["bias"] = {nm: randn16((ws[nm][1].shape[0],), seed=2000 + 3 * layer + j, device=device, std=0.1)
                      for j, nm in enumerate(("q", "k", "v"))}
        ws["lora"] = {nm: tuple(t.detach().half() for t in _adapter(n, 3000 + 2 * layer + j, device))
                      for j, (nm, n) in enumerate((("q", 1536), ("v", 256)))}
        stack.append(ws)

    def ref_lin(inp, name, ws, bias=None):
        y = inp.float() @ ws[name][2].float().t()
        return y if bias is None else y + bias.float()

    saved = []
    for layer, ws in enumerate(stack):
        lq, lv = ws["lora"]["q"], ws["lora"]["v"]
        uq, uv = lora.lora_down(x, lq[0]), lora.lora_down(x, lv[0])
        items = [dict(packed=ws["q"][0], qs=ws["q"][1], bias=ws["bias"]["q"], lora_u=uq, lora_b=lq[1], lora_scale=s),
                 dict(packed=ws["k"][0], qs=ws["k"][1], bias=ws["bias"]["k"]),
                 dict(packed=ws["v"][0], qs=ws["v"][1], bias=ws["bias"]["v"], lora_u=uv, lora_b=lv[1], lora_scale=s)]
        q, k, v = nf4.linear_forward(x, items, lora_rank=16)
        for out, nm, u, ad in ((q, "q", uq, lq), (k, "k", None, None), (v, "v", uv, lv)):
            ref = ref_lin(x, nm, ws, ws["bias"][nm])
            if u is not None:
                ref = ref + (u.float() @ ad[1].float().t()).half().float() * s
            _check(out, ref, f"layer {layer} {nm}")
        attn = _rms16(q)  # stands in for the attention output (attention is outside this path)
        (o,) = nf4.linear_forward(attn, [dict(packed=ws["o"][0], qs=ws["o"][1])])
        _check(o, ref_lin(attn, "o", ws), f"layer {layer} o")
        x2 = _rms16(x.float() + o.float())
        gate, up, h = nf4.glu_forward(x2, dict(packed=ws["gate"][0], qs=ws["gate"][1]),
                                      dict(packed=ws["up"][0], qs=ws["up"][1]))
        _check(gate, ref_lin(x2, "gate", ws), f"layer {layer} gate")
        _check(up, ref_lin(x2, "up", ws), f"layer {layer} up")
        (down,) = nf4.linear_forward(h, [dict(packed=ws["down"][0], qs=ws["down"][1])])
        _check(down, ref_lin(h, "down", ws), f"layer {layer} down")
        saved.append((x, uq, uv, attn, x2, gate, up))
        x = _rms16(x2.float() + down.float())

    dy = dy_top
    for layer in reversed(range(n_layers)):
        ws = stack[layer]
        xin, uq, uv, attn, x2, gate, up = saved[layer]
        g16, u16 = gate.clone(), up.clone()
        dgate, dup = nf4.linear_backward_swiglu(dict(packed=ws["down"][0], qs=ws["down"][1], dy=dy), gate, up)
        gh = (dy.float() @ ws["down"][2].float()).half().float()
        sg = torch.sigmoid(g16.float())
        _check(dgate, gh * u16.float() * sg * (1 + g16.float() * (1 - sg)), f"layer {layer} dgate")
        _check(dup, gh * g16.float() * sg, f"layer {layer} dup")
        dx2 = nf4.linear_backward([dict(packed=ws["gate"][0], qs=ws["gate"][1], dy=dgate),
                                   dict(packed=ws["up"][0], qs=ws["up"][1], dy=dup)], M, HIDDEN)
        _check(dx2, dgate.float() @ ws["gate"][2].float() + dup.float() @ ws["up"][2].float(), f"layer {layer} dX mlp")
        do = _rms16(dx2) * 1e-2
        dattn = nf4.linear_backward([dict(packed=ws["o"][0], qs=ws["o"][1], dy=do)], M, HIDDEN)
        _check(dattn, do.float() @ ws["o"][2].float(), f"layer {layer} dX o")
        dq = _rms16(dattn) * 1e-2
        dkv = (dq[:, :256] * 0.5).contiguous()
        lq, lv = ws["lora"]["q"], ws["lora"]["v"]
        guq, daq, dbq = lora.lora_grads(dq, uq, xin, lq[1], s)
        guv, dav, dbv = lora.lora_grads(dkv, uv, xin, lv[1], s)
        for gu, da, db, g_, u_, ad, nm in ((guq, daq, dbq, dq, uq, lq, "q"), (guv, dav, dbv, dkv, uv, lv, "v")):
            _check(da, gu.float().t() @ xin.float(), f"layer {layer} {nm} dA")
            _check(db, (g_.float() * s).t() @ u_.float(), f"layer {layer} {nm} dB")
        dx = nf4.linear_backward([dict(packed=ws["q"][0], qs=ws["q"][1], dy=dq, lora_gu=guq, lora_a=lq[0]),
                                  dict(packed=ws["k"][0], qs=ws["k"][1], dy=dkv),
                                  dict(packed=ws["v"][0], qs=ws["v"][1], dy=dkv, lora_gu=guv, lora_a=lv[0])],
                                 M, HIDDEN, lora_rank=16)
        ref = (dq.float() @ ws["q"][2].float() + dkv.float() @ ws["k"][2].float() + dkv.float() @ ws["v"][2].float()
               + guq.float() @ lq[0].float() + guv.float() @ lv[0].float())
        _check(dx, ref, f"layer {layer} dX qkv")
        dy = _rms16(dx.float() + dx2.float()) * 1e-2


C5_SHAPES = [("q/o", 3584, 3584), ("k/v", 512, 3584), ("gate/up", 18944, 3584), ("down", 3584, 18944)]


@pytest.fixture(scope="module")
def qwen7b_weights(device):
    return {name: make_weight((n, k), seed=600 + j, device=device) for j, (name, n, k) in enumerate(C5_SHAPES)}


@pytest.mark.parametrize("m", [1, 8, 64, 830, 8192])
@pytest.mark.parametrize("shape", [s[0] for s in C5_SHAPES])
def test_c5_qwen7b_shapes(shape, m, qwen7b_weights, device):
    """Forward at every M (the GEMV kernel at M = 1, MFMA kernels above, split-K where the
    planner splits) and the input gradient, each against the oracle on up to 48 token rows."""
    from decik_amd.nf4 import linear_backward, linear_forward

    packed, qs, w16 = qwen7b_weights[shape]
    n, k = (int(v) for v in qs.shape)
    x = randn16((m, k), seed=700 + m, device=device)
    dy = randn16((m, n), seed=701 + m, device=device, std=1e-2)
    rows = np.unique(np.linspace(0, m - 1, min(m, 48)).astype(np.int64))
    (y,) = linear_forward(x, [dict(packed=packed, qs=qs)])
    assert_close(y[rows], O.linear_ref(x[rows].cpu().numpy(), w16), what=f"7B {shape} fwd m={m}")
    dx = linear_backward([dict(packed=packed, qs=qs, dy=dy)], m, k)
    assert_close(dx[rows], O.linear_dx_ref(dy[rows].cpu().numpy(), w16), what=f"7B {shape} dX m={m}")


@pytest.mark.parametrize("dx_fp32", [False, True])
def test_c5_down_input_gradient_two_launches(dx_fp32, qwen7b_weights, device, monkeypatch):
    """The 7B down-projection input gradient at 830 tokens (296 tiles of 224 x 256 for 256 CUs)
    runs as two launches: the 64 column tiles of the full round unsplit, then the last 2560
    columns split over every CU and reduced. The first part gives the same bits as the one-launch
    unsplit plan; every column meets the bar against the oracle."""
    from decik_amd.nf4 import linear_backward

    packed, qs, w16 = qwen7b_weights["down"]
    n, k = (int(v) for v in qs.shape)
    m = 830
    dy = randn16((m, n), seed=731, device=device, std=1e-2)
    item = [dict(packed=packed, qs=qs, dy=dy)]
    dx = linear_backward(item, m, k, dx_fp32=dx_fp32)
    monkeypatch.setenv("DECIK_BWD_PLAN", "7,1")
    dx1 = linear_backward(item, m, k, dx_fp32=dx_fp32)
    monkeypatch.delenv("DECIK_BWD_PLAN")
    torch.cuda.synchronize()
    assert torch.equal(dx[:, :16384], dx1[:, :16384])
    rows = np.arange(0, m, 7)
    ref = O.linear_dx_ref(dy[rows].cpu().numpy(), w16)
    assert_close(dx[rows], ref, what="7B down dX, two launches")
    assert_close(dx[rows][:, 16384:], ref[:, 16384:], what="7B down dX, remainder columns")


def test_c5_down_input_gradient_two_launches_lora(qwen7b_weights, device):
    """The two-launch input gradient with a rank-16 LoRA term: each launch adds GU . A for its own
    columns (split 0 of the second launch), against the oracle."""
    from decik_amd.nf4 import linear_backward

    packed, qs, w16 = qwen7b_weights["down"]
    n, k = (int(v) for v in qs.shape)
    m, r = 830, 16
    dy = randn16((m, n), seed=741, device=device, std=1e-2)
    gu = randn16((m, r), seed=742, device=device, std=0.05)
    a = randn16((r, k), seed=743, device=device, std=0.05)
    dx = linear_backward([dict(packed=packed, qs=qs, dy=dy, lora_gu=gu, lora_a=a)], m, k, lora_rank=r)
    torch.cuda.synchronize()
    rows = np.arange(0, m, 11)
    ref = O.linear_dx_ref(dy[rows].cpu().numpy(), w16) + gu[rows].float().cpu().numpy() @ a.float().cpu().numpy()
    assert_close(dx[rows], ref, what="7B down dX + LoRA, two launches")
    assert_close(dx[rows][:, 16384:], ref[:, 16384:], what="7B down dX + LoRA, remainder columns")
