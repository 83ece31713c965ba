"""LoRA r=16 fused into the NF4 GEMM epilogues (config: Qwen2.5-1.5B attention projections,
830 packed tokens from 8 sequences). Reference semantics: solution/attn.py:225-228 (forward),
:251-257 (backward); bar: max|err| <= 1e-2 max|ref|, sum|err|/sum|ref| <= 1e-3."""

import numpy as np
import pytest
import torch

from helpers import assert_close, make_weight, randn16
from oracle import nf4 as O

pytestmark = pytest.mark.gpu


def packed_lengths(total=830, n_seq=8, lo=32, hi=200, seed=0):
    """8 sequence lengths drawn uniform in [32, 200] that sum to 830 (seeded rejection sampler);
    the projections are per token, so only the total matters to them."""
    rng = np.random.default_rng(seed)
    while True:
        lens = rng.integers(lo, hi + 1, n_seq)
        if lens.sum() == total:
            return lens


def adapters(n, k, seed, device, r=16):
    g = torch.Generator(device="cpu").manual_seed(seed)
    bound = 1.0 / np.sqrt(k)  # Kaiming-uniform bound of peft's default init for lora_A
    a = ((torch.rand((r, k), generator=g) * 2 - 1) * bound).to(torch.float16).to(device)
    b = (torch.randn((n, r), generator=g) * 1e-3).to(torch.float16).to(device)
    return a, b


def test_lengths_sum():
    lens = packed_lengths()
    assert lens.sum() == 830 and lens.min() >= 32 and lens.max() <= 200


@pytest.mark.parametrize("m,n,k", [(8, 8960, 1536), (24, 3584, 3584)])
def test_nf4_lora_linear_few_rows(m, n, k, device):
    """Few token rows with LoRA terms: such launches stay off the small-M kernel and run split
    MFMA plans, whose workspace the size query must cover (it cannot see the LoRA terms)."""
    from decik_amd.lora import NF4LoRALinear
    from decik_amd.nf4 import launch_plan

    assert launch_plan(False, m, k, [n], lora=True)["splits"] > 1
    packed, qs, w16 = make_weight((n, k), seed=n + m, device=device)
    bias = randn16((n,), seed=5, device=device, std=0.1)
    a, b = adapters(n, k, seed=6, device=device)
    x = randn16((m, k), seed=7, device=device)
    y = NF4LoRALinear.apply(x, packed, bias, qs, a.float(), b.float(), 2.0)
    xn = x.cpu().numpy()
    _, lora = O.lora_fwd_ref(xn, a.cpu().numpy(), b.cpu().numpy(), 2.0)
    assert_close(y, O.linear_ref(xn, w16, bias.cpu().numpy()) + lora, what=f"Y m={m} n={n}")


@pytest.mark.parametrize("n", [1536, 256])
def test_nf4_lora_linear(n, device):
    from decik_amd.lora import NF4LoRALinear

    m, k, s = int(packed_lengths().sum()), 1536, 2.0
    packed, qs, w16 = make_weight((n, k), seed=n, device=device)
    bias = randn16((n,), seed=1, device=device, std=0.1)
    a, b = adapters(n, k, seed=2, device=device)
    a32, b32 = a.float().requires_grad_(True), b.float().requires_grad_(True)
    x = randn16((m, k), seed=3, device=device).requires_grad_(True)
    y = NF4LoRALinear.apply(x, packed, bias, qs, a32, b32, s)
    dy = randn16((m, n), seed=4, device=device, std=1e-2)
    y.backward(dy)

    xn, an, bn, dyn = (t.detach().cpu().numpy() for t in (x, a, b, dy))
    u16, lora = O.lora_fwd_ref(xn, an, bn, s)
    y_ref = O.linear_ref(xn, w16, bias.cpu().numpy()) + lora
    assert_close(y, y_ref, what="Y")
    gu16, da, db, dx_lora = O.lora_bwd_ref(dyn, xn, u16, an, bn, s)
    assert_close(x.grad, O.linear_dx_ref(dyn, w16) + dx_lora, what="dX")
    assert_close(a32.grad, da, what="dA")
    assert_close(b32.grad, db, what="dB")
    assert a32.grad.dtype == torch.float32 and b32.grad.dtype == torch.float32


def test_qkv_projection_with_lora_on_q_and_v(device):
    """q/k/v in one fused launch each way; LoRA on q and v only (the reference run)."""
    from decik_amd.lora import qkv_projection

    m, k, s = 830, 1536, 2.0
    x = randn16((m, k), seed=10, device=device).requires_grad_(True)
    projs, refs = [], []
    for i, (name, n) in enumerate([("q", 1536), ("k", 256), ("v", 256)]):
        packed, qs, w16 = make_weight((n, k), seed=50 + i, device=device)
        bias = randn16((n,), seed=60 + i, device=device, std=0.1)
        p = dict(packed=packed, qs=qs, bias=bias, lora_a=None, lora_b=None, scaling=s)
        if name in ("q", "v"):
            a, b = adapters(n, k, seed=70 + i, device=device)
            p["lora_a"], p["lora_b"] = a.float().requires_grad_(True), b.float().requires_grad_(True)
        projs.append(p)
        refs.append(w16)
    outs = qkv_projection(x, projs)
    grads = [randn16(o.shape, seed=80 + i, device=device, std=1e-2) for i, o in enumerate(outs)]
    torch.autograd.backward(outs, grads)

    xn = x.detach().cpu().numpy()
    dx_ref = np.zeros((m, k), np.float64)
    for p, w16, o, g in zip(projs, refs, outs, grads):
        gn = g.cpu().numpy()
        y_ref = O.linear_ref(xn, w16, p["bias"].cpu().numpy())
        dx_ref += O.linear_dx_ref(gn, w16)
        if p["lora_a"] is not None:
            an = p["lora_a"].detach().half().cpu().numpy()
            bn = p["lora_b"].detach().half().cpu().numpy()
            u16, lora = O.lora_fwd_ref(xn, an, bn, s)
            y_ref = y_ref + lora
            _, da, db, dxl = O.lora_bwd_ref(gn, xn, u16, an, bn, s)
            dx_ref += dxl
            assert_close(p["lora_a"].grad, da, what="dA")
            assert_close(p["lora_b"].grad, db, what="dB")
        assert_close(o, y_ref, what="qkv Y")
    assert_close(x.grad, dx_ref, what="qkv dX")


def _masks(rows, width, p, seed, device):
    g = torch.Generator(device="cpu").manual_seed(seed)
    kq = torch.rand((rows, width), generator=g) >= p
    kv = torch.rand((rows, width), generator=g) >= p
    return kq.to(device), kv.to(device)


@pytest.mark.parametrize("xdtype", [torch.float32, torch.float16])
def test_dropout_steps_bit_exact(xdtype, device):
    """Mask packing, the dropped-out fp16 inputs and the input gradient through both masks match
    the oracle bit for bit (elementwise fp32 in the reference's order, solution/attn.py:129-180),
    on 830 tokens x 1536 with p = 0.05 (the real run's lora_dropout)."""
    from decik_amd.lora import lora_input_grad, lora_inputs, pack_keep

    rows, width, p = 830, 1536, 0.05
    kq, kv = _masks(rows, width, p, 11, device)
    bq, bv = pack_keep(kq, kv)
    assert np.array_equal(bq.cpu().numpy(), O.keep_pack(kq.cpu().numpy()))
    assert np.array_equal(bv.cpu().numpy(), O.keep_pack(kv.cpu().numpy()))
    x = (torch.randn((rows, width), generator=torch.Generator().manual_seed(12)) * 2).to(xdtype).to(device)
    s = torch.tensor(1.0 / (1.0 - p), dtype=torch.float32, device=device)
    xq, xv = lora_inputs(x, bq, bv, s, s)
    rq, rv = O.lora_dropout_inputs_ref(x.cpu().numpy(), bq.cpu().numpy(), bv.cpu().numpy(),
                                       1.0 / (1.0 - p), 1.0 / (1.0 - p))
    assert np.array_equal(xq.cpu().numpy().view(np.uint16), rq.view(np.uint16))
    assert np.array_equal(xv.cpu().numpy().view(np.uint16), rv.view(np.uint16))
    gq = randn16((rows, width), seed=13, device=device, std=1e-2)
    gv = randn16((rows, width), seed=14, device=device, std=1e-2)
    out = lora_input_grad(gq, gv, bq, bv, 1.0 / (1.0 - p), 1.0 / (1.0 - p))
    ref = O.lora_input_grad_ref(gq.cpu().numpy(), gv.cpu().numpy(), bq.cpu().numpy(), bv.cpu().numpy(),
                                1.0 / (1.0 - p), 1.0 / (1.0 - p))
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("r", [16, 32])
def test_lora_up(r, device):
    from decik_amd.lora import lora_up

    gu = randn16((830, r), seed=15, device=device, std=1e-2)
    a = randn16((r, 1536), seed=16, device=device, std=0.03)
    out = lora_up(gu, a)
    ref = (O._f64(gu.cpu().numpy()) @ O._f64(a.cpu().numpy())).astype(np.float32)
    assert out.dtype == torch.float16
    assert_close(out, ref, what=f"lora_up r={r}")


def test_lora_pair_with_dropout(device):
    """LoRAPair (q and v branches with p = 0.05 dropout) against the oracle restatement of
    LoRAPairFromNorm's packed path (solution/attn.py:206-273): outputs, dA/dB of both branches
    and the fp32 input gradient through both masks."""
    from decik_amd.lora import LoRAPair, pack_keep

    rows, width, p, s = 830, 1536, 0.05, 2.0
    kq, kv = _masks(rows, width, p, 21, device)
    bq, bv = pack_keep(kq, kv)
    x = torch.randn((rows, width), generator=torch.Generator().manual_seed(22)).to(device)  # fp32
    a_q, b_q = adapters(1536, width, 23, device)
    a_v, b_v = adapters(256, width, 24, device)
    b_q = (b_q.float() * 30).half()  # larger B so the outputs are not all rounding noise
    b_v = (b_v.float() * 30).half()
    ws = [t.float().requires_grad_(True) for t in (a_q, b_q, a_v, b_v)]
    sc = torch.tensor(1.0 / (1.0 - p), dtype=torch.float32, device=device)
    xin = x.clone().requires_grad_(True)
    out_q, out_v = LoRAPair.apply(xin, bq, sc, bv, sc, *ws, s, s, p, p)
    gq = randn16((rows, 1536), seed=25, device=device, std=1e-2)
    gv = randn16((rows, 256), seed=26, device=device, std=1e-2)
    torch.autograd.backward([out_q, out_v], [gq, gv])
    # oracle
    xn = x.cpu().numpy()
    bqn, bvn = bq.cpu().numpy(), bv.cpu().numpy()
    xq, xv = O.lora_dropout_inputs_ref(xn, bqn, bvn, 1.0 / (1.0 - p), 1.0 / (1.0 - p))
    gin = []
    for x16, a, b, g, out, (wa, wb) in ((xq, a_q, b_q, gq, out_q, ws[:2]), (xv, a_v, b_v, gv, out_v, ws[2:])):
        an, bn = a.cpu().numpy(), b.cpu().numpy()
        u16, lo = O.lora_fwd_ref(x16, an, bn, s)
        assert_close(out, lo, what="lora out")
        gu16, da, db, _ = O.lora_bwd_ref(g.cpu().numpy(), x16, u16, an, bn, s)
        assert_close(wa.grad, da, what="dA")
        assert_close(wb.grad, db, what="dB")
        gin.append((O._f64(gu16) @ O._f64(an)).astype(np.float16))
    ref_dx = O.lora_input_grad_ref(gin[0], gin[1], bqn, bvn, 1.0 / (1.0 - p), 1.0 / (1.0 - p))
    assert xin.grad.dtype == torch.float32
    assert_close(xin.grad, ref_dx, what="dX through dropout")


@pytest.mark.parametrize("ranks", [(16, 32), (16, 8)])
def test_qkv_projection_mixed_ranks(ranks, device):
    """LoRA ranks that differ between q and v (or one the kernels do not take) run each
    projection on its own; outputs and gradients still match the oracle."""
    from decik_amd.lora import qkv_projection

    m, k, s = 256, 1536, 2.0
    x = randn16((m, k), seed=90, device=device).requires_grad_(True)
    projs, refs = [], []
    for i, (n, r) in enumerate([(1536, ranks[0]), (256, None), (256, ranks[1])]):
        packed, qs, w16 = make_weight((n, k), seed=91 + i, device=device)
        p = dict(packed=packed, qs=qs, bias=None, lora_a=None, lora_b=None, scaling=s)
        if r is not None:
            a, b = adapters(n, k, seed=95 + i, device=device, r=r)
            p["lora_a"], p["lora_b"] = a.float().requires_grad_(True), (b.float() * 20).requires_grad_(True)
        projs.append(p)
        refs.append(w16)
    outs = qkv_projection(x, projs)
    grads = [randn16(o.shape, seed=99 + i, device=device, std=1e-2) for i, o in enumerate(outs)]
    torch.autograd.backward(outs, grads)
    xn = x.detach().cpu().numpy()
    dx_ref = np.zeros((m, k), np.float64)
    for p, w16, o, g in zip(projs, refs, outs, grads):
        gn = g.cpu().numpy()
        y_ref = O.linear_ref(xn, w16)
        dx_ref += O.linear_dx_ref(gn, w16)
        if p["lora_a"] is not None:
            an = p["lora_a"].detach().half().cpu().numpy()
            bn = p["lora_b"].detach().half().cpu().numpy()
            u16, lora = O.lora_fwd_ref(xn, an, bn, s)
            y_ref = y_ref + lora
            _, da, db, dxl = O.lora_bwd_ref(gn, xn, u16, an, bn, s)
            dx_ref += dxl
            assert_close(p["lora_a"].grad, da, what=f"dA r={an.shape[0]}")
            assert_close(p["lora_b"].grad, db, what=f"dB r={an.shape[0]}")
        assert_close(o, y_ref, what="Y")
    assert_close(x.grad, dx_ref, what="dX")


@pytest.mark.parametrize("r", [16, 32])
@pytest.mark.parametrize("m,k,n", [(1, 40, 8), (17, 1536, 256), (830, 104, 1536)])
def test_lora_kernels_edge_shapes(r, m, k, n, device):
    """dk_lora_down / dk_lora_bwd on shapes that leave partial tiles everywhere: token counts
    below and past one 16-row tile, widths that are not multiples of 32; dA / dB may be omitted.
    Against the oracle (exact variant: the kernels keep dA and dB in fp32)."""
    from decik_amd.lora import lora_down, lora_grads

    s = 2.0
    x = randn16((m, k), seed=150 + m, device=device)
    a = randn16((r, k), seed=151, device=device, std=0.05)
    b = randn16((n, r), seed=152, device=device, std=0.05)
    dy = randn16((m, n), seed=153, device=device, std=1e-2)
    u = lora_down(x, a)
    xn, an, bn, dyn = (t.cpu().numpy() for t in (x, a, b, dy))
    u_ref, _ = O.lora_fwd_ref(xn, an, bn, s)
    assert_close(u, u_ref.astype(np.float32), what="U")
    gu, da, db = lora_grads(dy, u, x, b, s)
    gu_ref, da_ref, db_ref, _ = O.lora_bwd_ref(dyn, xn, u.cpu().numpy(), an, bn, s, exact=True)
    assert_close(gu, gu_ref.astype(np.float32), what="GU")
    assert_close(da, da_ref, what="dA")
    assert_close(db, db_ref, what="dB")
    gu2, da2, db2 = lora_grads(dy, u, x, b, s, want_da=False, want_db=False)
    assert da2 is None and db2 is None and torch.equal(gu2, gu)
    # the same bits on a second call (fixed summation order)
    gu3, da3, db3 = lora_grads(dy, u, x, b, s)
    assert torch.equal(gu3, gu) and torch.equal(da3, da) and torch.equal(db3, db)
