"""Every fused GEMM kernel variant on weights the Python layer would otherwise route through cached
fp32 block scales: nested double-quant statistics read by the kernels themselves (blocks of 64,
128 and 256 weights, so a block spans one to four 64-wide steps), plain blocksize-32 statistics
(two scales per lane), and weights whose row count leaves a partial last step in the backward
kernel. Plans are forced so that each kernel and its split-K path run (solution/nf4.py:93-104;
the summed input gradient of solution/mlp.py:106-109)."""
import pytest
import torch

from helpers import O, assert_close, make_weight, randn16

pytestmark = pytest.mark.gpu

CASES = [(True, 64), (True, 128), (True, 256), (False, 32)]


@pytest.fixture
def raw_statistics(monkeypatch):
    """Describe nested weights to every kernel as they are (no derived block scales: the default,
    made explicit here)."""
    from decik_amd import nf4

    monkeypatch.setattr(nf4, "_launch_scales", lambda packed, qs, device: None)


@pytest.mark.parametrize("plan", ["4,1,4", "2,3,4", "2,3,8", "4,1,8", "7,2,8", "8,1,8", "9,2,8"])
@pytest.mark.parametrize("nested,blocksize", CASES)
def test_forward_variants(nested, blocksize, plan, device, monkeypatch, raw_statistics):
    from decik_amd.nf4 import linear_forward

    monkeypatch.setenv("DECIK_FWD_PLAN", plan)
    packed, qs, w16 = make_weight((320, 1024), seed=blocksize + 7, device=device, nested=nested,
                                  blocksize=blocksize)
    x = randn16((300, 1024), seed=9, device=device)
    b = randn16((320,), seed=10, device=device, std=0.1)
    (y,) = linear_forward(x, [dict(packed=packed, qs=qs, bias=b)])
    assert_close(y, O.linear_ref(x.cpu().numpy(), w16, b.cpu().numpy()),
                 what=f"fwd {plan} nested={nested} bs={blocksize}")


@pytest.mark.parametrize("plan", ["2,1,8", "2,3,8", "4,1,8", "4,3,8", "8,1,8", "7,2,8"])
@pytest.mark.parametrize("nested,blocksize", CASES)
def test_backward_variants_partial_last_step(nested, blocksize, plan, device, monkeypatch, raw_statistics):
    """264 weight rows: the last 64-row step has 8 rows; dY columns and weight rows past them read
    zeros."""
    from decik_amd.nf4 import linear_backward

    monkeypatch.setenv("DECIK_BWD_PLAN", plan)
    packed, qs, w16 = make_weight((264, 1024), seed=blocksize + 11, device=device, nested=nested,
                                  blocksize=blocksize)
    dy = randn16((300, 264), seed=12, device=device, std=1e-2)
    dx = linear_backward([dict(packed=packed, qs=qs, dy=dy)], 300, 1024)
    assert_close(dx, O.linear_dx_ref(dy.cpu().numpy(), w16), what=f"bwd {plan} nested={nested} bs={blocksize}")


@pytest.mark.parametrize("plan", ["2,1,8", "2,3,8", "4,2,8", "8,2,8", "7,1,8", "7,3,8"])
def test_grouped_backward_partial_steps(plan, device, monkeypatch, raw_statistics):
    """Two weights of 264 and 200 rows in one launch: both groups end in a partial step, and the
    split boundaries fall inside and between groups."""
    from decik_amd.nf4 import linear_backward

    monkeypatch.setenv("DECIK_BWD_PLAN", plan)
    (p1, q1, w1), (p2, q2, w2) = (make_weight((n, 512), seed=60 + n, device=device, nested=True, blocksize=128)
                                  for n in (264, 200))
    d1 = randn16((130, 264), seed=13, device=device, std=1e-2)
    d2 = randn16((130, 200), seed=14, device=device, std=1e-2)
    dx = linear_backward([dict(packed=p1, qs=q1, dy=d1), dict(packed=p2, qs=q2, dy=d2)], 130, 512, dx_fp32=True)
    ref = O.linear_dx_ref(d1.cpu().numpy(), w1) + O.linear_dx_ref(d2.cpu().numpy(), w2)
    assert_close(dx, ref, max_rel=1e-4, mean_rel=1e-5, what=f"grouped bwd {plan}")


@pytest.mark.parametrize("plan", ["2,2,8", "4,1,8", "7,3,8", "8,2,8", "7,1,8"])
@pytest.mark.parametrize("nested,blocksize", CASES)
@pytest.mark.parametrize("dx_fp32", [False, True])
def test_eight_wave_backward_edges(nested, blocksize, plan, dx_fp32, device, monkeypatch, raw_statistics):
    """The eight-wave input-gradient kernel (256-column tiles of 32 columns per wave) at
    k = 1056: the last column tile holds one wave's 32 columns and seven waves past k; 200 weight
    rows (a partial last step); 300 tokens (a partial last token tile)."""
    from decik_amd.nf4 import linear_backward

    monkeypatch.setenv("DECIK_BWD_PLAN", plan)
    packed, qs, w16 = make_weight((200, 1056), seed=blocksize + 21, device=device, nested=nested,
                                  blocksize=blocksize)
    dy = randn16((300, 200), seed=22, device=device, std=1e-2)
    dx = linear_backward([dict(packed=packed, qs=qs, dy=dy)], 300, 1056, dx_fp32=dx_fp32)
    ref = O.linear_dx_ref(dy.cpu().numpy(), w16)
    if dx_fp32:
        assert_close(dx, ref, max_rel=1e-4, mean_rel=1e-5, what=f"bwd8 {plan} fp32 nested={nested} bs={blocksize}")
    else:
        assert_close(dx, ref, what=f"bwd8 {plan} nested={nested} bs={blocksize}")


@pytest.mark.parametrize("plan", ["2,1,8", "4,1,8", "8,2,8", "7,3,8"])
def test_eight_wave_backward_lora(plan, device, monkeypatch):
    """LoRA input-gradient terms GU . A (rank 16) in the eight-wave kernel, split 0 only."""
    from decik_amd.nf4 import linear_backward

    monkeypatch.setenv("DECIK_BWD_PLAN", plan)
    packed, qs, w16 = make_weight((256, 512), seed=31, device=device, nested=True, blocksize=64)
    dy = randn16((200, 256), seed=32, device=device, std=1e-2)
    gu = randn16((200, 16), seed=33, device=device, std=1e-2)
    la = randn16((16, 512), seed=34, device=device, std=1e-1)
    dx = linear_backward([dict(packed=packed, qs=qs, dy=dy, lora_gu=gu, lora_a=la)], 200, 512, dx_fp32=True,
                         lora_rank=16)
    ref = O.linear_dx_ref(dy.cpu().numpy(), w16) + gu.cpu().double().numpy() @ la.cpu().double().numpy()
    assert_close(dx, ref, max_rel=1e-4, mean_rel=1e-5, what=f"bwd8 lora {plan}")


@pytest.mark.parametrize("plan", ["2,3,8", "4,2,8", "8,3,8", "7,4,8"])
def test_eight_wave_backward_three_groups_lora(plan, device, monkeypatch):
    """Three weights of 1536, 256 and 264 rows (the last ends in a partial step) in one launch,
    LoRA terms on the first and last: every split adds its share of the contraction, split 0 the
    LoRA terms (the q/k/v input gradient of solution/attn.py:396-418)."""
    from decik_amd.nf4 import linear_backward

    monkeypatch.setenv("DECIK_BWD_PLAN", plan)
    m, k = 300, 512
    items, ref = [], 0.0
    for i, n in enumerate((1536, 256, 264)):
        packed, qs, w16 = make_weight((n, k), seed=90 + i, device=device, nested=True, blocksize=64)
        dy = randn16((m, n), seed=95 + i, device=device, std=1e-2)
        it = dict(packed=packed, qs=qs, dy=dy)
        ref = ref + O.linear_dx_ref(dy.cpu().numpy(), w16)
        if i != 1:
            gu = randn16((m, 16), seed=97 + i, device=device, std=1e-2)
            la = randn16((16, k), seed=99 + i, device=device, std=1e-1)
            it.update(lora_gu=gu, lora_a=la)
            ref = ref + gu.cpu().double().numpy() @ la.cpu().double().numpy()
        items.append(it)
    dx = linear_backward(items, m, k, dx_fp32=True, lora_rank=16)
    assert_close(dx, ref, max_rel=1e-4, mean_rel=1e-5, what=f"bwd8 three groups {plan}")


@pytest.fixture
def gemv(monkeypatch):
    """Forward launches of 1-2 token rows (3-8 on small weights) take the GEMV kernel (the
    default; DECIK_SMALL_M unset)."""
    monkeypatch.delenv("DECIK_SMALL_M", raising=False)


@pytest.fixture
def skinny(monkeypatch):
    """Send every small-M forward launch, 1-8 token rows included, to the skinny kernel."""
    monkeypatch.setenv("DECIK_SMALL_M", "skinny")


@pytest.mark.parametrize("m", [1, 2, 5, 16, 17, 32])
@pytest.mark.parametrize("nested,blocksize", CASES)
def test_skinny_small_m(m, nested, blocksize, device, raw_statistics, skinny):
    """The small-M kernel (forward launches of at most 32 token rows without LoRA terms): three
    weights in one launch (320, 64 and 72 rows: the last row group of the third is partial),
    with bias, statistics read raw, k = 1056 (the last 128-wide super-step is a quarter full)."""
    from decik_amd.nf4 import launch_plan, linear_forward

    assert launch_plan(False, m, 1056, [320, 64, 72])["kernel"] == "nf4_skinny_kernel"
    items, refs = [], []
    x = randn16((m, 1056), seed=160 + m, device=device)
    for i, n in enumerate((320, 64, 72)):
        packed, qs, w16 = make_weight((n, 1056), seed=161 + i + blocksize, device=device, nested=nested,
                                      blocksize=blocksize)
        b = randn16((n,), seed=165 + i, device=device, std=0.1)
        items.append(dict(packed=packed, qs=qs, bias=b))
        refs.append(O.linear_ref(x.cpu().numpy(), w16, b.cpu().numpy()))
    ys = linear_forward(x, items)
    for y, ref in zip(ys, refs):
        assert_close(y, ref, what=f"skinny m={m} nested={nested} bs={blocksize}")


@pytest.mark.parametrize("m", [3, 8, 17, 32])
@pytest.mark.parametrize("ns", [(16408, 64), (20496,)])
@pytest.mark.parametrize("raw", [False, True])
def test_skinny_tall_weights(m, ns, raw, device, monkeypatch, skinny):
    """Weights of more 64-row groups than a 256-CU device has CUs: the small-M kernel takes row
    groups of 80 (16408 + 64 rows: 206 + 1 groups) or 96 rows (20496: 214 groups, 257 of 80) so
    that they run in one round; the last group of each weight is partial, and at 17-32 token rows
    the kernel is still chosen (one round)."""
    from decik_amd import nf4
    from decik_amd.nf4 import launch_plan, linear_forward

    if not raw:  # the derived fp32 block scales instead of the statistics as stored
        monkeypatch.setattr(nf4, "_launch_scales", nf4._scales)
    k = 256
    assert launch_plan(False, m, k, list(ns))["kernel"] == "nf4_skinny_kernel"
    x = randn16((m, k), seed=180 + m, device=device)
    items, refs = [], []
    for i, n in enumerate(ns):
        packed, qs, w16 = make_weight((n, k), seed=181 + i, device=device)
        b = randn16((n,), seed=183 + i, device=device, std=0.1)
        items.append(dict(packed=packed, qs=qs, bias=b))
        refs.append(O.linear_ref(x.cpu().numpy(), w16, b.cpu().numpy()))
    ys = linear_forward(x, items)
    for y, ref in zip(ys, refs):
        assert_close(y, ref, what=f"skinny tall m={m} ns={ns} raw={raw}")


@pytest.mark.parametrize("m", [3, 8, 24])
def test_small_m_statistics_forms_same_bits(m, device, monkeypatch):
    """Small-M launches read nested statistics as stored (the default for every launch) or, through
    the hook, the derived fp32 scales: both forms give the same dequantized weights and the same
    sums, so the outputs are equal bit for bit."""
    from decik_amd import nf4
    from decik_amd.nf4 import linear_forward

    k, n = 512, 16408
    packed, qs, w16 = make_weight((n, k), seed=190, device=device)
    assert qs.nested
    x = randn16((m, k), seed=191 + m, device=device)
    (y_raw,) = linear_forward(x, [dict(packed=packed, qs=qs)])
    monkeypatch.setattr(nf4, "_launch_scales", nf4._scales)
    (y_cached,) = linear_forward(x, [dict(packed=packed, qs=qs)])
    assert torch.equal(y_raw, y_cached)
    assert_close(y_raw, O.linear_ref(x.cpu().numpy(), w16), what=f"small-M raw m={m}")


@pytest.mark.parametrize("m", [1, 8, 32])
@pytest.mark.parametrize("raw", [False, True])
def test_skinny_split_k(m, raw, device, monkeypatch, skinny):
    """Few rows and a long contraction (two weights of 128 and 64 rows, k = 8192): the small-M
    kernel splits the contraction over work-groups (fp32 partial slabs, then the split-K
    reduction adds bias and rounds), with cached block scales or raw nested statistics; the same
    bits on a second call."""
    from decik_amd import nf4
    from decik_amd.nf4 import launch_plan, linear_forward

    if not raw:  # the derived fp32 block scales instead of the statistics as stored
        monkeypatch.setattr(nf4, "_launch_scales", nf4._scales)
    plan = launch_plan(False, m, 8192, [128, 64])
    assert plan["kernel"] == "nf4_skinny_kernel" and plan["splits"] > 1
    x = randn16((m, 8192), seed=170 + m, device=device)
    items, refs = [], []
    for i, n in enumerate((128, 64)):
        packed, qs, w16 = make_weight((n, 8192), seed=171 + i, device=device)
        b = randn16((n,), seed=173 + i, device=device, std=0.1)
        items.append(dict(packed=packed, qs=qs, bias=b))
        refs.append(O.linear_ref(x.cpu().numpy(), w16, b.cpu().numpy()))
    ys = linear_forward(x, items)
    for y, ref in zip(ys, refs):
        assert_close(y, ref, what=f"skinny split m={m} raw={raw}")
    ys2 = linear_forward(x, items)
    assert all(bool((a == b).all()) for a, b in zip(ys, ys2))


@pytest.mark.parametrize("m", [1, 2])
@pytest.mark.parametrize("nested,blocksize", CASES)
def test_gemv_small_m(m, nested, blocksize, device, raw_statistics, gemv):
    """The GEMV kernel (forward launches of 1-2 token rows without LoRA terms): three
    weights in one launch (q/k/v-like, with bias; each weight's last work-group holds fewer
    rows), statistics read raw, k = 1056 (rows of 33 16-byte chunks: a work-group's chunk range
    and its X pieces wrap across rows at odd positions)."""
    from decik_amd.nf4 import launch_plan, linear_forward

    assert launch_plan(False, m, 1056, [320, 64, 64])["kernel"] == "nf4_gemv_kernel"
    items, refs = [], []
    x = randn16((m, 1056), seed=120 + m, device=device)
    for i, n in enumerate((320, 64, 64)):
        packed, qs, w16 = make_weight((n, 1056), seed=121 + i + blocksize, device=device, nested=nested,
                                      blocksize=blocksize)
        b = randn16((n,), seed=125 + i, device=device, std=0.1)
        items.append(dict(packed=packed, qs=qs, bias=b))
        refs.append(O.linear_ref(x.cpu().numpy(), w16, b.cpu().numpy()))
    ys = linear_forward(x, items)
    for y, ref in zip(ys, refs):
        assert_close(y, ref, what=f"gemv m={m} nested={nested} bs={blocksize}")


@pytest.mark.parametrize("m", [3, 4, 5, 8])
@pytest.mark.parametrize("k", [1056, 3584])
def test_gemv_more_rows(m, k, device, raw_statistics, monkeypatch):
    """The GEMV computed for four or eight token rows (m = 3, 5: rows past m read as zeros and
    are not stored), sent there on purpose: three weights with bias in one launch against the
    oracle, and the same bits on a second call."""
    import torch

    from decik_amd.nf4 import launch_plan, linear_forward

    monkeypatch.setenv("DECIK_SMALL_M", "gemv")
    assert launch_plan(False, m, k, [320, 64, 64])["kernel"] == "nf4_gemv_kernel"
    items, refs = [], []
    x = randn16((m, k), seed=160 + m, device=device)
    for i, n in enumerate((320, 64, 64)):
        packed, qs, w16 = make_weight((n, k), seed=161 + i + k, device=device)
        b = randn16((n,), seed=165 + i, device=device, std=0.1)
        items.append(dict(packed=packed, qs=qs, bias=b))
        refs.append(O.linear_ref(x.cpu().numpy(), w16, b.cpu().numpy()))
    ys = linear_forward(x, items)
    for y, ref in zip(ys, refs):
        assert_close(y, ref, what=f"gemv m={m} k={k}")
    for y, y2 in zip(ys, linear_forward(x, items)):
        assert torch.equal(y, y2)


@pytest.mark.parametrize("m", [1, 2])
def test_gemv_short_k_no_bias(m, device, gemv):
    """GEMV edges: k = 64 (two 16-byte chunks per row: a work-group takes hundreds of rows), two
    weights of 72 and 8 rows, no bias. Weight rows must be a multiple of 8: a 67-row weight is
    rejected with that message before anything runs."""
    from decik_amd import _lib
    from decik_amd.nf4 import launch_plan, linear_forward

    assert launch_plan(False, m, 64, [72, 8])["kernel"] == "nf4_gemv_kernel"
    x = randn16((m, 64), seed=140 + m, device=device)
    packed, qs, _ = make_weight((67, 64), seed=141, device=device)
    with pytest.raises(_lib.DecikError, match="multiple of 8"):
        linear_forward(x, [dict(packed=packed, qs=qs)])
    items, refs = [], []
    for i, n in enumerate((72, 8)):
        packed, qs, w16 = make_weight((n, 64), seed=142 + i, device=device)
        items.append(dict(packed=packed, qs=qs))
        refs.append(O.linear_ref(x.cpu().numpy(), w16))
    for y, ref in zip(linear_forward(x, items), refs):
        assert_close(y, ref, what=f"gemv short k m={m}")


@pytest.mark.parametrize("m", [1, 2])
def test_gemv_long_k(m, device, monkeypatch):
    """A long contraction (k = 18944, the 7B down projection's: 592 chunks a row, three rows a
    work-group of eight waves, X staged whole in LDS; sent to the GEMV explicitly, which the
    planner also picks for a weight this small): 40 rows against the oracle, and the same bits
    on a second call (the row sums run in a fixed order)."""
    import torch

    from decik_amd.nf4 import launch_plan, linear_forward

    monkeypatch.setenv("DECIK_SMALL_M", "gemv")
    k = 18944
    plan = launch_plan(False, m, k, [40])
    assert plan["kernel"] == "nf4_gemv_kernel" and plan["waves"] == 8
    packed, qs, w16 = make_weight((40, k), seed=150, device=device)
    x = randn16((m, k), seed=151 + m, device=device)
    b = randn16((40,), seed=153, device=device, std=0.1)
    (y,) = linear_forward(x, [dict(packed=packed, qs=qs, bias=b)])
    assert_close(y, O.linear_ref(x.cpu().numpy(), w16, b.cpu().numpy()), what=f"gemv long k m={m}")
    (y2,) = linear_forward(x, [dict(packed=packed, qs=qs, bias=b)])
    assert torch.equal(y, y2)


def test_gemv_not_used_with_lora_or_forced_plan(device, monkeypatch):
    """LoRA terms or a forced plan keep small launches on the MFMA kernels (same results)."""
    from decik_amd.nf4 import launch_plan, linear_forward

    assert launch_plan(False, 2, 512, [256], lora=True)["kernel"] != "nf4_gemv_kernel"
    packed, qs, w16 = make_weight((256, 512), seed=130, device=device)
    x = randn16((2, 512), seed=131, device=device)
    (y0,) = linear_forward(x, [dict(packed=packed, qs=qs)])
    monkeypatch.setenv("DECIK_FWD_PLAN", "1,2,4")
    assert launch_plan(False, 2, 512, [256])["kernel"] == "nf4_fwd_kernel"
    (y1,) = linear_forward(x, [dict(packed=packed, qs=qs)])
    ref = O.linear_ref(x.cpu().numpy(), w16)
    assert_close(y0, ref, what="gemv")
    assert_close(y1, ref, what="mfma at m=2")


@pytest.mark.parametrize("fwd_plan,bwd_plan", [("8,1,8", "8,1,8,256"), ("8,2,8", "8,3,8,256")])
def test_column_tiles_first_order(fwd_plan, bwd_plan, device, monkeypatch):
    """2048 token rows on 256-token tiles (eight token tiles, activations heavier than the packed
    weights): the eight-wave kernels take their tiles column tiles first, also with split-K.
    Every output row and column against the oracle, forward and input gradient."""
    from decik_amd.nf4 import launch_plan, linear_backward, linear_forward

    m, n, k = 2048, 2048, 512
    monkeypatch.setenv("DECIK_FWD_PLAN", fwd_plan)
    monkeypatch.setenv("DECIK_BWD_PLAN", bwd_plan)
    assert launch_plan(False, m, k, [n])["kernel"] == "nf4_fwd8_kernel"
    assert launch_plan(True, m, k, [n])["kernel"] == "nf4_bwd8_kernel"
    packed, qs, w16 = make_weight((n, k), seed=180, device=device)
    x = randn16((m, k), seed=181, device=device)
    dy = randn16((m, n), seed=182, device=device, std=1e-2)
    (y,) = linear_forward(x, [dict(packed=packed, qs=qs)])
    assert_close(y, O.linear_ref(x.cpu().numpy(), w16), what=f"fwd columns first {fwd_plan}")
    dx = linear_backward([dict(packed=packed, qs=qs, dy=dy)], m, k)
    assert_close(dx, O.linear_dx_ref(dy.cpu().numpy(), w16), what=f"bwd columns first {bwd_plan}")


@pytest.mark.parametrize("plan", ["2,1,8", "2,3,8", "4,1,8", "4,2,8"])
@pytest.mark.parametrize("m", [33, 64, 130])
def test_small_tile_forward(plan, m, device, monkeypatch):
    """The eight-wave forward kernel on 64- and 128-token tiles (MB = 2, 4): partial token tiles
    (33, 130 rows), two weights with a partial column tile (320 and 200 rows), bias, LoRA terms
    on the first weight only, split-K; then its GLU mode at the same sizes against the separate
    launches of the same tiles, unsplit. The first part reads raw nested statistics (blocks of 128 and 64), the GLU part
    cached block scales."""
    from decik_amd import nf4
    from decik_amd.lora import lora_down
    from decik_amd.nf4 import glu_forward, launch_plan, linear_forward
    from decik_amd.swiglu import swiglu_fwd

    monkeypatch.setenv("DECIK_FWD_PLAN", plan)
    k, r = 1024, 16
    assert launch_plan(False, m, k, [320, 200])["kernel"] == "nf4_fwd8_kernel"
    p1, q1, w1 = make_weight((320, k), seed=190, device=device, nested=True, blocksize=128)
    p2, q2, w2 = make_weight((200, k), seed=191, device=device)
    x = randn16((m, k), seed=192 + m, device=device)
    b1 = randn16((320,), seed=193, device=device, std=0.1)
    b2 = randn16((200,), seed=194, device=device, std=0.1)
    a = randn16((r, k), seed=195, device=device, std=0.05)
    lb = randn16((320, r), seed=196, device=device, std=0.05)
    u = lora_down(x, a)
    items = [dict(packed=p1, qs=q1, bias=b1, lora_u=u, lora_b=lb, lora_scale=2.0), dict(packed=p2, qs=q2, bias=b2)]
    y1, y2 = linear_forward(x, items, lora_rank=r)  # statistics as stored
    xn = x.cpu().numpy()
    lora = O.lora_fwd_ref(xn, a.cpu().numpy(), lb.cpu().numpy(), 2.0)[1]
    assert_close(y1, O.linear_ref(xn, w1, b1.cpu().numpy()) + lora, what=f"first weight, plan {plan}, m={m}")
    assert_close(y2, O.linear_ref(xn, w2, b2.cpu().numpy()), what=f"second weight, plan {plan}, m={m}")
    # the GLU launch never splits: the separate launches it must equal run unsplit too
    monkeypatch.setenv("DECIK_FWD_PLAN", plan.split(",")[0] + ",1,8")
    p3, q3, _ = make_weight((200, k), seed=197, device=device)
    gi, ui = dict(packed=p2, qs=q2, bias=b2), dict(packed=p3, qs=q3)
    g, up, h = glu_forward(x, gi, ui)
    g2, u2 = linear_forward(x, [gi, ui])
    assert torch.equal(g, g2) and torch.equal(up, u2) and torch.equal(h, swiglu_fwd(g2, u2))


@pytest.mark.parametrize("m", [64, 830])
def test_mfma_launches_statistics_forms_same_bits(m, device, monkeypatch):
    """The MFMA launches read nested statistics as stored by default (_launch_scales); on the
    derived fp32 block scales instead they give the same bits: forward (several weights, bias,
    LoRA), input gradient (with a LoRA term), the GLU forward, the SwiGLU backward and the RoPE
    forward."""
    from decik_amd import nf4
    from decik_amd.lora import lora_down
    from test_rope_gpu import rope_tables

    k, r = 1536, 16
    pq, qq, _ = make_weight((1536, k), seed=210, device=device)
    pk, qk, _ = make_weight((256, k), seed=211, device=device)
    pg, qg, _ = make_weight((1024, k), seed=212, device=device)
    pu, qu, _ = make_weight((1024, k), seed=213, device=device)
    pd, qd, _ = make_weight((k, 1024), seed=214, device=device)
    assert qq.nested and qd.nested
    x = randn16((m, k), seed=215, device=device)
    bias = randn16((1536,), seed=216, device=device, std=0.1)
    a = randn16((r, k), seed=217, device=device, std=0.05)
    lb = randn16((1536, r), seed=218, device=device, std=0.05)
    dyq = randn16((m, 1536), seed=219, device=device, std=1e-2)
    dyk = randn16((m, 256), seed=220, device=device, std=1e-2)
    dyd = randn16((m, k), seed=221, device=device, std=1e-2)
    gu = randn16((m, r), seed=222, device=device, std=1e-2)
    c, s = rope_tables([m], 128)
    cos, sin = torch.from_numpy(c).to(device), torch.from_numpy(s).to(device)

    def run():
        u = lora_down(x, a)
        items = [dict(packed=pq, qs=qq, bias=bias, lora_u=u, lora_b=lb, lora_scale=2.0), dict(packed=pk, qs=qk)]
        out = list(nf4.linear_forward(x, items, lora_rank=r))
        out += nf4.linear_forward(x, [dict(packed=pq, qs=qq), dict(packed=pk, qs=qk)])
        out.append(nf4.linear_backward([dict(packed=pq, qs=qq, dy=dyq, lora_gu=gu, lora_a=a),
                                        dict(packed=pk, qs=qk, dy=dyk)], m, k, lora_rank=r))
        g, up, h = nf4.glu_forward(x, dict(packed=pg, qs=qg), dict(packed=pu, qs=qu))
        out += [g, up, h]
        out += list(nf4.linear_backward_swiglu(dict(packed=pd, qs=qd, dy=dyd), g.clone(), up.clone()))
        out += nf4.linear_rope_forward(x, [dict(packed=pq, qs=qq), dict(packed=pk, qs=qk)], cos, sin, 128, 3)
        return out

    as_stored = run()
    monkeypatch.setattr(nf4, "_launch_scales", nf4._scales)
    cached = run()
    torch.cuda.synchronize()
    assert len(as_stored) == len(cached) == 12
    for i, (t1, t2) in enumerate(zip(as_stored, cached)):
        assert torch.equal(t1, t2), i
