"""LoRA dropout fused into the LoRA products and the input-gradient GEMM (LoRAPairFromNorm's
packed path, solution/attn.py:153-180, 206-273): the dropped-out input fp16(x * (keep * scale))
is rebuilt inside dk_lora_down_dropout / dk_lora_bwd_dropout and never stored, and the branch's
input gradient is masked in the epilogue of the backward GEMM (dk_linear_bwd_group.lora_keep).

- The fused U, GU, dA and dB equal the two-step path (dk_lora_dropout_inputs, then the plain
  products on the stored inputs) bit for bit.
- The masked epilogue: with dY = 0, dX is zero exactly where both masks drop and equals the
  reference's (fp32(fp16(GU . A)) * keep) * scale elsewhere (within an fp16 rounding of the
  product); with dY it meets the parity bar against the oracle for every backward variant.
- QKVProjection / QKVRopeProjection with x fp32 (the norm output) and p = 0.05 on q and v against
  the oracle's restatement of the reference's chain, outputs and every gradient."""

import numpy as np
import pytest
import torch

from helpers import assert_close, make_weight, randn16
from oracle import nf4 as O
from test_lora_gpu import _masks, adapters

pytestmark = pytest.mark.gpu

P = 0.05


def _x(rows, width, dtype, device, seed):
    x = torch.randn((rows, width), generator=torch.Generator().manual_seed(seed)) * 2
    return x.to(dtype).to(device)


@pytest.mark.parametrize("r", [16, 32])
@pytest.mark.parametrize("xdtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("m,k", [(830, 1536), (37, 96)])
def test_fused_dropout_products_match_two_step(r, xdtype, m, k, device):
    from decik_amd.lora import lora_down, lora_grads, lora_inputs, pack_keep

    kq, kv = _masks(m, k, 0.3, 31, device)
    bq, bv = pack_keep(kq, kv)
    x = _x(m, k, xdtype, device, 32)
    sc = torch.tensor(1.0 / (1.0 - 0.3), dtype=torch.float32, device=device)
    xq, _ = lora_inputs(x, bq, bv, sc, sc)
    a, b = adapters(256, k, 33, device, r=r)
    b = (b.float() * 30).half()
    u = lora_down(x, a, bq, sc)
    assert torch.equal(u, lora_down(xq, a)), "U from the fused dropout input"
    dy = randn16((m, 256), seed=34, device=device, std=1e-2)
    fused = lora_grads(dy, u, x, b, 2.0, keep_bits=bq, keep_scale=sc)
    plain = lora_grads(dy, u, xq, b, 2.0)
    for f, p_, what in zip(fused, plain, ("GU", "dA", "dB")):
        assert torch.equal(f, p_), what
    if xdtype == torch.float32:  # fp32 input without dropout: fp16(x)
        assert torch.equal(lora_down(x, a), lora_down(x.half(), a))
        assert torch.equal(lora_grads(dy, u, x, b, 2.0)[1], lora_grads(dy, u, x.half(), b, 2.0)[1])


def _bwd_items(w, dys, gus, as_, bits, scale):
    return [dict(packed=w[i][0], qs=w[i][1], dy=dys[i], lora_gu=gus[i], lora_a=as_[i],
                 lora_keep=bits[i], lora_keep_scale=scale) for i in range(len(dys))]


@pytest.mark.parametrize("plan", [None, "2,2,8", "2,1,8", "4,1,8", "4,3,8", "7,2,8", "8,1,8"])
def test_masked_lora_epilogue(plan, device, monkeypatch):
    """q (1536 rows) and v (256 rows) input gradients with both branches' dropout masks, over
    every input-gradient tile size (64, 128, 224 and 256 tokens), with and without split-K."""
    from decik_amd import nf4
    from decik_amd.lora import pack_keep

    if plan is not None:
        monkeypatch.setenv("DECIK_BWD_PLAN", plan)
    m, k, r, p = 830, 1536, 16, 0.5  # p = 0.5: half the entries dropped, easy to see misplaced bits
    kq, kv = _masks(m, k, p, 41, device)
    bq, bv = pack_keep(kq, kv)
    wq, wv = make_weight((1536, k), seed=42, device=device), make_weight((256, k), seed=43, device=device)
    gq = randn16((m, r), seed=44, device=device, std=0.3)
    gv = randn16((m, r), seed=45, device=device, std=0.3)
    aq = randn16((r, k), seed=46, device=device, std=0.05)
    av = randn16((r, k), seed=47, device=device, std=0.05)
    scale = 1.0 / (1.0 - p)
    # P of each branch as the reference forms it: fp16(GU . A), then the masked sum
    pq = (O._f64(gq.cpu().numpy()) @ O._f64(aq.cpu().numpy())).astype(np.float32).astype(np.float16)
    pv = (O._f64(gv.cpu().numpy()) @ O._f64(av.cpu().numpy())).astype(np.float32).astype(np.float16)
    lora_ref = O.lora_input_grad_ref(pq, pv, bq.cpu().numpy(), bv.cpu().numpy(), scale, scale)
    # dY = 0: dX is the masked LoRA part alone
    zq = torch.zeros((m, 1536), dtype=torch.float16, device=device)
    zv = torch.zeros((m, 256), dtype=torch.float16, device=device)
    dx = nf4.linear_backward(_bwd_items((wq, wv), (zq, zv), (gq, gv), (aq, av), (bq, bv), scale), m, k,
                             dx_fp32=True, lora_rank=r).cpu().numpy()
    dropped = ~(kq | kv).cpu().numpy()
    assert dropped.any() and np.all(dx[dropped] == 0.0), "a dropped entry got a LoRA term"
    # elsewhere the same up to one fp16 rounding of each branch's product
    err = np.abs(dx - lora_ref)
    tol = 2.0 * scale * ((np.abs(pq.astype(np.float32)) + np.abs(pv.astype(np.float32))) * 2.0 ** -10 + 2.0 ** -24)
    assert np.all(err <= tol), f"masked LoRA term off by {float((err / tol).max()):.2f} of an fp16 ulp"
    # with the base products: the parity bar against the oracle
    dyq = randn16((m, 1536), seed=48, device=device, std=1e-2)
    dyv = randn16((m, 256), seed=49, device=device, std=1e-2)
    dx = nf4.linear_backward(_bwd_items((wq, wv), (dyq, dyv), (gq, gv), (aq, av), (bq, bv), scale), m, k,
                             dx_fp32=True, lora_rank=r)
    base = O.linear_dx_ref(dyq.cpu().numpy(), wq[2]).astype(np.float64) + O.linear_dx_ref(dyv.cpu().numpy(), wv[2])
    assert_close(dx, (base + lora_ref).astype(np.float32), what=f"dX with masked LoRA terms, plan {plan}")


def test_masked_lora_rejected_with_swiglu(device):
    from decik_amd import _lib, nf4

    w = make_weight((1536, 256), seed=50, device=device)
    gate = randn16((64, 256), seed=51, device=device)
    up = randn16((64, 256), seed=52, device=device)
    dy = randn16((64, 1536), seed=53, device=device)
    gu = randn16((64, 16), seed=54, device=device)
    a = randn16((16, 256), seed=55, device=device)
    bits = torch.zeros((64, 32), dtype=torch.uint8, device=device)
    item = dict(packed=w[0], qs=w[1], dy=dy, lora_gu=gu, lora_a=a, lora_keep=bits, lora_keep_scale=1.0)
    with pytest.raises(_lib.DecikError, match="SwiGLU"):
        nf4.linear_backward_swiglu(item, gate, up, lora_rank=16)


def _qkv_case(device, seed):
    m, k = 830, 1536
    projs, w16 = [], []
    kq, kv = _masks(m, k, P, seed, device)
    from decik_amd.lora import pack_keep

    bq, bv = pack_keep(kq, kv)
    sc = torch.tensor(1.0 / (1.0 - P), dtype=torch.float32, device=device)
    for i, n in enumerate((1536, 256, 256)):
        packed, qs, w = make_weight((n, k), seed=seed + 1 + i, device=device)
        p = dict(packed=packed, qs=qs, bias=randn16((n,), seed=seed + 5 + i, device=device, std=0.1),
                 lora_a=None, lora_b=None, scaling=2.0)
        if i != 1:
            a, b = adapters(n, k, seed + 9 + i, device)
            p.update(lora_a=a.float().requires_grad_(True), lora_b=(b.float() * 30).requires_grad_(True),
                     keep_bits=bq if i == 0 else bv, keep_scale=sc, p=P)
        projs.append(p)
        w16.append(w)
    x = _x(m, k, torch.float32, device, seed + 20)  # the fp32 norm output
    return projs, w16, x, (bq, bv)


def test_qkv_projection_with_dropout_against_oracle(device):
    """x fp32, q/k/v with biases, LoRA r=16 with p = 0.05 on q and v (the real run), through
    QKVProjection: outputs, dX (fp32), dA and dB against the oracle."""
    from decik_amd.lora import qkv_projection

    projs, w16, x, (bq, bv) = _qkv_case(device, 600)
    m = x.shape[0]
    xi = x.clone().requires_grad_(True)
    outs = qkv_projection(xi, projs)
    grads = [randn16((m, int(p["qs"].shape[0])), seed=610 + i, device=device, std=1e-2) for i, p in enumerate(projs)]
    torch.autograd.backward(list(outs), grads)
    assert xi.grad.dtype == torch.float32
    xn = x.cpu().numpy()
    x16 = xn.astype(np.float16)
    xdrop = O.lora_dropout_inputs_ref(xn, bq.cpu().numpy(), bv.cpu().numpy(), 1.0 / (1.0 - P), 1.0 / (1.0 - P))
    dx_ref = np.zeros(xn.shape, np.float64)
    gin = []
    for i, (p, w, out, g) in enumerate(zip(projs, w16, outs, grads)):
        y = O.linear_ref(x16, w, p["bias"].cpu().numpy()).astype(np.float64)
        gn = g.cpu().numpy()
        dx_ref += O.linear_dx_ref(gn, w)
        if p["lora_a"] is not None:
            xb = xdrop[0 if i == 0 else 1]
            an = p["lora_a"].detach().half().cpu().numpy()
            bn = p["lora_b"].detach().half().cpu().numpy()
            u16, lo = O.lora_fwd_ref(xb, an, bn, 2.0)
            y += lo
            gu16, da, db, _ = O.lora_bwd_ref(gn, xb, u16, an, bn, 2.0)
            assert_close(p["lora_a"].grad, da, what=f"dA {i}")
            assert_close(p["lora_b"].grad, db, what=f"dB {i}")
            gin.append((O._f64(gu16) @ O._f64(an)).astype(np.float32).astype(np.float16))
        assert_close(out, y.astype(np.float32), what=f"projection {i}")
    dx_ref += O.lora_input_grad_ref(gin[0], gin[1], bq.cpu().numpy(), bv.cpu().numpy(), 1.0 / (1.0 - P),
                                    1.0 / (1.0 - P))
    assert_close(xi.grad, dx_ref.astype(np.float32), what="dX fp32 through both masks")


def test_qkv_rope_projection_with_dropout_matches_unfused(device):
    """QKVRopeProjection with the dropout masks equals QKVProjection + FusedQKRope bit for bit:
    outputs, dX, dA, dB."""
    from decik_amd.lora import qkv_projection, qkv_rope_projection
    from decik_amd.rope import FusedQKRope
    from test_rope_gpu import rope_tables

    projs, _, x, _ = _qkv_case(device, 700)
    c, s = rope_tables([100, 200, 130, 32, 150, 60, 90, 68], 128)
    ct, st = torch.from_numpy(c).to(device), torch.from_numpy(s).to(device)
    m = x.shape[0]
    gq = randn16((1, 12, m, 128), seed=710, device=device, std=1e-2)
    gk = randn16((1, 2, m, 128), seed=711, device=device, std=1e-2)
    gv = randn16((m, 256), seed=712, device=device, std=1e-2)

    def run(fused):
        xi = x.clone().requires_grad_(True)
        for p in projs:
            for key in ("lora_a", "lora_b"):
                if p[key] is not None:
                    p[key].grad = None
        if fused:
            q, k, v = qkv_rope_projection(xi, projs, ct, st, 12, 2)
        else:
            qb, kb, v = qkv_projection(xi, projs)
            q, k = FusedQKRope.apply(qb, None, kb, ct, st, 12, 2)
        torch.autograd.backward([q, k, v], [gq, gk, gv])
        return [q.detach(), k.detach(), v.detach(), xi.grad] + [
            p[key].grad.clone() for p in projs for key in ("lora_a", "lora_b") if p[key] is not None]

    for a, b in zip(run(True), run(False)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("r", [16, 32])
@pytest.mark.parametrize("m,k", [(830, 1536), (37, 96)])
def test_grouped_lora_launches_equal_per_branch(r, m, k, device):
    """dk_lora_down_group / dk_lora_bwd_group (every branch's product in one launch, one per kind of
    input): the same bits as the per-branch calls, for four branches of every input kind (fp16 or
    fp32, with or without dropout), different output widths n, and dA / dB left out of some."""
    from decik_amd.lora import lora_down, lora_down_group, lora_grads, lora_grads_group, pack_keep

    kq, kv = _masks(m, k, 0.3, 41, device)
    bq, bv = pack_keep(kq, kv)
    sq = torch.tensor(1.0 / 0.7, dtype=torch.float32, device=device)
    x16 = _x(m, k, torch.float16, device, 42)
    x32 = _x(m, k, torch.float32, device, 43)
    spec = [(x16, None, None, 1536, True, True), (x32, bq, sq, 256, True, True),
            (x16, bv, sq, 512, False, True), (x32, None, None, 264, True, False)]
    downs, ref_u, branches, ref_g = [], [], [], []
    for i, (x, bits, sc, n, want_da, want_db) in enumerate(spec):
        a, b = adapters(n, k, 44 + i, device, r=r)
        downs.append((x, a, bits, sc))
        ref_u.append(lora_down(x, a, bits, sc))
        dy = randn16((m, n), seed=50 + i, device=device, std=1e-2)
        branches.append(dict(dy16=dy, u16=ref_u[-1], x=x, b16=b, scaling=2.0, want_da=want_da, want_db=want_db,
                             keep_bits=bits, keep_scale=sc))
        ref_g.append(lora_grads(dy, ref_u[-1], x, b, 2.0, want_da, want_db, keep_bits=bits, keep_scale=sc))
    us = lora_down_group(downs)
    got = lora_grads_group(branches)
    torch.cuda.synchronize()
    for u, ru in zip(us, ref_u):
        assert torch.equal(u, ru)
    for g, rg in zip(got, ref_g):
        for t, rt in zip(g, rg):
            assert (t is None and rt is None) or torch.equal(t, rt)
