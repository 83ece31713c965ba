"""Pins the CPU oracle (oracle/nf4.py, oracle/nf4_oracle.c) without trusting its own formulas.

The reference ships no golden vectors for this path and its own oracle (bitsandbytes) is absent,
so the oracle is pinned by what the mathematics fixes:
- exact rational arithmetic with explicit correct rounding (an independent implementation of
  IEEE round-to-nearest-even, below) for every byte value and for FMA-sensitive scales;
- numpy's own fp32 <-> fp16 conversions;
- closed forms of the NF4 table (nibble 7 is +0, nibbles 0/15 are -/+1, plain absmax 1);
- the reference's layout facts: high nibble first (README.md:120), flat block index
  (solution/nf4.py:36,40).
"""

from fractions import Fraction

import numpy as np
import pytest

from oracle import nf4 as O


def round_binary(fr, mant_bits, emin, emax):
    """Correctly rounded (ties to even) value of the rational `fr` in a binary format with
    `mant_bits` significand bits, smallest normal exponent `emin`, largest exponent `emax`."""
    if fr == 0:
        return 0.0
    sign = -1 if fr < 0 else 1
    a = abs(Fraction(fr))
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    quantum = Fraction(2) ** (e - (mant_bits - 1))
    q = a / quantum
    n = q.numerator // q.denominator
    rem = q - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    val = n * quantum
    if val >= Fraction(2) ** (emax + 1):
        return sign * float("inf")
    return sign * float(val)


def rf32(fr):
    return round_binary(fr, 24, -126, 127)


def rf16(fr):
    return round_binary(fr, 11, -14, 15)


def test_round_helper_agrees_with_hardware_float32():
    # the helper itself, checked against numpy's float64 -> float32 on values exact in float64
    rng = np.random.default_rng(1)
    for v in rng.standard_normal(2000) * 10.0 ** rng.integers(-40, 38, 2000):
        assert rf32(Fraction(float(v))) == float(np.float32(v))


def test_f32_to_f16_matches_numpy():
    rng = np.random.default_rng(0)
    exps = np.arange(256, dtype=np.uint32)
    mans = np.concatenate([
        np.array([0, 1, 0xFFF, 0x1000, 0x1001, 0x1FFF, 0x2000, 0x3000, 0x400000, 0x7FE000,
                  0x7FF000, 0x7FFFFF], dtype=np.uint32),
        rng.integers(0, 1 << 23, 200, dtype=np.uint32)])
    bits = (exps[:, None] << 23) | mans[None, :]
    bits = np.concatenate([bits.ravel(), bits.ravel() | np.uint32(0x80000000)])
    x = bits.view(np.float32)
    ours = O.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all(np.isnan(ours[nan].view(np.float16)))


def test_f16_to_f32_all_halves():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ours = O.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert np.all(np.isnan(ours[nan]))


def _plain_state(packed, absmax, shape, blocksize=64):
    return O.QuantNF4(np.asarray(packed, np.uint8), np.asarray(absmax, np.float32),
                      np.zeros(0, np.float32), np.zeros(0, np.float32), np.float32(0),
                      O.NF4_CODE.copy(), shape, blocksize, 256, False)


def test_plain_unit_absmax_gives_fp16_of_code():
    # every byte value once; 256 bytes = 512 weights = 8 blocks of 64, all absmax 1.0
    packed = np.arange(256, dtype=np.uint8)
    out = O.dequant_nf4(_plain_state(packed, np.ones(8), (4, 128))).reshape(-1)
    hi = O.NF4_CODE[packed >> 4].astype(np.float16)
    lo = O.NF4_CODE[packed & 15].astype(np.float16)
    assert np.array_equal(out[0::2].view(np.uint16), hi.view(np.uint16))
    assert np.array_equal(out[1::2].view(np.uint16), lo.view(np.uint16))


@pytest.mark.parametrize("scale", [0.03125, 0.0625, 1.5, 3.0])
def test_special_nibbles_and_high_nibble_first(scale):
    # 0xF0: high nibble 15 -> +scale at the even index, low nibble 0 -> -scale at the odd one;
    # 0x77: nibble 7 is code 0.0 -> +0.0 exactly
    packed = np.array([0xF0, 0x77] * 16, dtype=np.uint8)
    out = O.dequant_nf4(_plain_state(packed, [scale], (1, 64))).reshape(-1)
    assert out[0] == np.float16(scale) and out[1] == np.float16(-scale)
    assert out[2].view(np.uint16) == 0 and out[3].view(np.uint16) == 0


def _random_nested(rng, shape, blocksize=64, blocksize2=256):
    n = shape[0] * shape[1]
    n_blocks = -(-n // blocksize)
    n2 = -(-n_blocks // blocksize2)
    return O.QuantNF4(
        packed=rng.integers(0, 256, n // 2, dtype=np.uint8),
        absmax=rng.integers(0, 256, n_blocks, dtype=np.uint8),
        absmax2=(rng.random(n2).astype(np.float32) * 0.05 + 0.001).astype(np.float32),
        code2=O.dynamic_map_signed(),
        offset=np.float32(0.0213),
        code=O.NF4_CODE.copy(), shape=shape, blocksize=blocksize, blocksize2=blocksize2,
        nested=True)


def test_all_bytes_match_exact_arithmetic():
    """Every byte value with several nested scales, against exact rationals rounded twice."""
    rng = np.random.default_rng(7)
    q = _random_nested(rng, (8, 512))
    q.packed = np.tile(np.arange(256, dtype=np.uint8), 8)
    out = O.dequant_nf4(q).reshape(-1).view(np.uint16)
    for i in range(q.packed.size):
        blk = (2 * i) // q.blocksize
        s = rf32(Fraction(float(q.code2[q.absmax[blk]])) * Fraction(float(q.absmax2[blk // 256])))
        s = rf32(Fraction(s) + Fraction(float(q.offset)))
        b = int(q.packed[i])
        hi = rf16(Fraction(rf32(Fraction(float(O.NF4_CODE[b >> 4])) * Fraction(s))))
        lo = rf16(Fraction(rf32(Fraction(float(O.NF4_CODE[b & 15])) * Fraction(s))))
        assert out[2 * i] == np.float16(hi).view(np.uint16), (i, b)
        assert out[2 * i + 1] == np.float16(lo).view(np.uint16), (i, b)


def test_scale_is_not_fused():
    """Find code2/absmax2/offset where fma(c2, a2, off) rounds differently from the two-step
    sum, and check the oracle takes the two-step value (solution/nf4.py:39-41,84)."""
    rng = np.random.default_rng(3)
    found = 0
    for _ in range(20000):
        c2 = np.float32(rng.uniform(-1, 1))
        a2 = np.float32(rng.uniform(0.001, 0.1))
        off = np.float32(rng.uniform(0.0, 0.05))
        prod = Fraction(float(c2)) * Fraction(float(a2))
        two_step = rf32(Fraction(rf32(prod)) + Fraction(float(off)))
        fused = rf32(prod + Fraction(float(off)))
        if two_step == fused:
            continue
        code2 = np.zeros(256, np.float32)
        code2[5] = c2
        q = O.QuantNF4(np.array([0xF0] * 32, np.uint8), np.array([5], np.uint8),
                       np.array([a2], np.float32), code2, off, O.NF4_CODE.copy(), (1, 64))
        out = O.dequant_nf4(q).reshape(-1)
        # nibble 15 is code 1.0, so out[0] = fp16(scale)
        assert out[0] == np.float16(two_step)
        found += 1
        if found == 20:
            break
    assert found == 20


@pytest.mark.parametrize("shape,blocksize,blocksize2", [((3, 40), 64, 256), ((10, 96), 64, 2),
                                                        ((5, 1536), 64, 256), ((7, 10), 32, 3)])
def test_flat_block_index_straddles_rows(shape, blocksize, blocksize2):
    """Blocks and absmax2 groups run over the flat element index, across row ends
    (solution/nf4.py:36,40): every element's scale is that of block flat_index // blocksize."""
    rng = np.random.default_rng(11)
    q = _random_nested(rng, shape, blocksize, blocksize2)
    q.packed = np.full(q.packed.size, 0xFF, np.uint8)        # every weight is code[15] = 1.0
    out = O.dequant_nf4(q).reshape(-1).astype(np.float32)
    n_blocks = q.absmax.size
    expect_scale = np.empty(n_blocks, np.float32)
    for b in range(n_blocks):
        s = rf32(Fraction(float(q.code2[q.absmax[b]])) * Fraction(float(q.absmax2[b // blocksize2])))
        expect_scale[b] = rf32(Fraction(s) + Fraction(float(q.offset)))
    flat = np.arange(out.size)
    assert np.array_equal(out, expect_scale[flat // blocksize].astype(np.float16).astype(np.float32))


def test_dynamic_map_shape():
    c = O.dynamic_map_signed()
    assert c.shape == (256,) and np.all(np.diff(c) >= 0)
    assert c[-1] == 1.0 and 0.0 in c
    neg = c[c < 0]
    pos = c[(c > 0) & (c < 1)]
    assert neg.size == 127 and pos.size == 127
    assert np.array_equal(np.sort(-neg), pos)
    # smallest magnitudes: 10**-6 * midpoint(0.1, 1) = 5.5e-7
    assert abs(pos[0] - 5.5e-7) < 1e-12


@pytest.mark.parametrize("nested", [True, False])
def test_quantizer_invariants(nested):
    """Round trip bound and nearest-code choice (the quantizer is parity-unpinned vs bnb)."""
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((64, 256)) * 0.05).astype(np.float16)
    q = O.quantize_nf4(w, nested=nested)
    assert q.packed.shape == (w.size // 2,)
    deq = O.dequant_nf4(q).astype(np.float64).reshape(-1)
    wf = w.astype(np.float64).reshape(-1)
    true_absmax = np.abs(wf.reshape(-1, 64)).max(axis=1)
    scales = O.block_scales(q).astype(np.float64)
    blk = np.arange(wf.size) // 64
    # the stored scale is within the double-quant error of the true absmax
    tol = 1e-6 if not nested else 0.02 * true_absmax.max()
    assert np.max(np.abs(scales - true_absmax)) <= tol
    # the chosen code is the nearest one to w / absmax
    idx = np.empty(wf.size, np.int64)
    idx[0::2] = q.packed >> 4
    idx[1::2] = q.packed & 15
    normed = wf / true_absmax[blk]
    dist = np.abs(normed[:, None] - O.NF4_CODE.astype(np.float64)[None, :])
    chosen = dist[np.arange(wf.size), idx]
    assert np.all(chosen <= dist.min(axis=1) + 1e-6)
    # reconstruction error: half the widest code gap times the scale, plus rounding
    assert np.max(np.abs(deq - wf)) <= 0.17 * np.max(scales) + 1e-3


def test_linear_refs_closed_forms():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 8)).astype(np.float16)
    eye = np.eye(8, dtype=np.float16)
    assert np.array_equal(O.linear_ref(x, eye), x.astype(np.float32))
    perm = eye[[3, 1, 0, 7, 2, 6, 5, 4]]
    assert np.array_equal(O.linear_ref(x, perm), x[:, [3, 1, 0, 7, 2, 6, 5, 4]].astype(np.float32))
    b = np.arange(8, dtype=np.float16)
    assert np.array_equal(O.linear_ref(x, eye, b), x.astype(np.float32) + b.astype(np.float32))
    # dX = dY . W: rank one
    dy = np.ones((2, 3), np.float16)
    w = np.arange(12, dtype=np.float16).reshape(3, 4)
    assert np.array_equal(O.linear_dx_ref(dy, w), np.tile(w.astype(np.float32).sum(0), (2, 1)))


def test_swiglu_refs_closed_forms():
    g = np.array([0.0, 0.0, 30.0, -30.0], np.float16)
    u = np.array([2.0, -3.0, 1.0, 1.0], np.float16)
    out = O.swiglu_fwd_ref(g, u)
    assert out[0] == 0 and out[1] == 0 and abs(out[2] - 30.0) < 1e-6 and abs(out[3]) < 1e-10
    G = np.ones(4, np.float16)
    dgate, dup = O.swiglu_bwd_ref(G, g, u)
    # at g = 0: sigmoid 1/2, dgate = G u / 2, dup = 0
    assert dgate[0] == 1.0 and dgate[1] == -1.5 and dup[0] == 0 and dup[1] == 0
    # for large g: silu'(g) -> 1 and dup -> G g
    assert abs(dgate[2] - 1.0) < 1e-6 and abs(dup[2] - 30.0) < 1e-6


def test_lora_refs_closed_forms():
    # A = [I_r | 0], B = [I_r ; 0]: u = x[:, :r], out = s * x[:, :r] padded
    r, k, n = 4, 8, 6
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, k)).astype(np.float16)
    a = np.zeros((r, k), np.float16)
    a[:, :r] = np.eye(r)
    b = np.zeros((n, r), np.float16)
    b[:r] = np.eye(r)
    u, out = O.lora_fwd_ref(x, a, b, 2.0)
    assert np.array_equal(u, x[:, :r])
    assert np.array_equal(out[:, :r], 2.0 * x[:, :r].astype(np.float32))
    assert np.all(out[:, r:] == 0)
    dy = rng.standard_normal((3, n)).astype(np.float16)
    gu, da, db, dx = O.lora_bwd_ref(dy, x, u, a, b, 2.0, exact=True)
    g = 2.0 * dy.astype(np.float64)
    assert np.allclose(db, g.T @ u.astype(np.float64))
    # B = [I; 0]: gu = g[:, :r] (exact: a power-of-two scale of fp16 values)
    assert np.array_equal(gu.astype(np.float32), (g[:, :r]).astype(np.float16).astype(np.float32))
    # A = [I | 0]: dA = gu^T x in its first r columns is gu^T x[:, :r]; dX_lora = [gu | 0]
    gu64 = gu.astype(np.float64)
    assert np.allclose(da, gu64.T @ x.astype(np.float64), rtol=1e-6, atol=0)
    assert np.array_equal(dx[:, :r], gu.astype(np.float32)) and np.all(dx[:, r:] == 0)
    # the reference's roundings (fp16 dA, dB, dX_lora) of the same products
    gu_r, da_r, db_r, dx_r = O.lora_bwd_ref(dy, x, u, a, b, 2.0)
    assert np.array_equal(gu_r, gu)
    assert np.array_equal(da_r, (gu64.T @ x.astype(np.float64)).astype(np.float32).astype(np.float16).astype(np.float32))
    assert np.array_equal(dx_r, dx) and np.array_equal(db_r, db.astype(np.float16).astype(np.float32))


def test_tolerance_metric():
    ref = np.array([1.0, -2.0, 4.0])
    y = np.array([1.0, -2.0, 4.04])
    mx, mean = O.tolerance(y, ref)
    assert abs(mx - 0.01) < 1e-12 and abs(mean - 0.04 / 7.0) < 1e-12


def test_keep_pack_matches_numpy_packbits():
    """The oracle's bit packer against numpy's independent one (little bit order: bit j of a
    byte is column 8 c + j, solution/attn.py:138-141); unpacking inverts it."""
    rng = np.random.default_rng(3)
    keep = rng.random((37, 128)) > 0.05
    bits = O.keep_pack(keep)
    assert bits.dtype == np.uint8 and bits.shape == (37, 16)
    assert np.array_equal(bits, np.packbits(keep, axis=1, bitorder="little"))
    assert np.array_equal(O.keep_unpack(bits, 128), keep.astype(np.float32))


def test_dropout_refs_closed_forms():
    """All-keep masks with scale 1 give fp16(x) and x itself back as the gradient; empty masks
    give zeros carrying x's sign; the scale multiplies after the mask, in fp32."""
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((8, 64)) * 3).astype(np.float32)
    ones = O.keep_pack(np.ones((8, 64), dtype=bool))
    zeros = O.keep_pack(np.zeros((8, 64), dtype=bool))
    xq, xv = O.lora_dropout_inputs_ref(x, ones, zeros, 1.0, 1.0)
    assert np.array_equal(xq, x.astype(np.float16))
    assert np.all(xv == 0) and np.array_equal(np.signbit(xv), np.signbit(x))
    xq2, _ = O.lora_dropout_inputs_ref(x, ones, ones, 1.0 / 0.95, 1.0)
    assert np.array_equal(xq2, (x * np.float32(1.0 / 0.95)).astype(np.float16))
    g16 = x.astype(np.float16)
    out = O.lora_input_grad_ref(g16, g16, ones, zeros, 1.0, 2.0)
    assert np.array_equal(out, g16.astype(np.float32))
    out2 = O.lora_input_grad_ref(g16, g16, ones, ones, 2.0, 2.0)
    assert np.array_equal(out2, g16.astype(np.float32) * 4)


def test_rope_refs_closed_forms_and_transpose():
    """cos 1 / sin 0 leaves q + lora (rounded to fp16) unchanged; cos 0 / sin 1 is rotate_half;
    the backward is the transpose of the forward's linear map: <R x, g> = <x, R^T g> in float64
    for the same cos/sin (checked on the fp32 values before rounding, through tiny exact inputs)."""
    rng = np.random.default_rng(5)
    t, h, hk, d = 5, 3, 1, 16
    qb = rng.standard_normal((t, h * d)).astype(np.float16)
    ql = (rng.standard_normal((t, h * d)) * 0.1).astype(np.float16)
    k = rng.standard_normal((t, hk * d)).astype(np.float16)
    one, zero = np.ones((t, d), np.float32), np.zeros((t, d), np.float32)
    q_out, k_out = O.rope_fwd_ref(qb, ql, k, one, zero, h, hk)
    want = (qb.astype(np.float32) + ql.astype(np.float32)).astype(np.float16).reshape(t, h, d).transpose(1, 0, 2)
    assert np.array_equal(q_out, want)
    assert np.array_equal(k_out, k.reshape(t, hk, d).transpose(1, 0, 2))
    _, k_rot = O.rope_fwd_ref(qb, None, k, zero, one, h, hk)
    assert np.array_equal(k_rot, O.rotate_half(k.astype(np.float32).reshape(t, hk, d).transpose(1, 0, 2)).astype(np.float16))
    # transpose identity with small-integer inputs (every product and sum exact in fp32)
    xi = rng.integers(-4, 5, (t, hk * d)).astype(np.float16)
    gi = rng.integers(-4, 5, (hk, t, d)).astype(np.float16)
    ci = rng.integers(-2, 3, (t, d)).astype(np.float32)
    si = rng.integers(-2, 3, (t, d)).astype(np.float32)
    _, rx = O.rope_fwd_ref(np.zeros((t, h * d), np.float16), None, xi, ci, si, h, hk)
    _, rtg = O.rope_bwd_ref(np.zeros((h, t, d), np.float16), gi, ci, si)
    lhs = float((rx.astype(np.float64) * gi.astype(np.float64)).sum())
    rhs = float((xi.astype(np.float64) * rtg.astype(np.float64)).sum())
    assert lhs == rhs


# ---- float64 autograd pins of the backward references ---------------------------------------
# torch's autograd differentiates the forward formulas mechanically (product rule, sigmoid',
# matmul transposes), so a dropped term, a wrong scale or a transposed operand in the oracle's
# hand-written backward shows up as a mismatch. The oracle's own fp16 roundings (where the
# reference rounds) keep it within a few 1e-4 of the unrounded float64 chain; the checks below
# allow 2e-3, while the planted mistakes of test_pins_catch_planted_mistakes move them by 0.1 or
# more.

def _t(a, grad=False):
    import torch

    return torch.tensor(np.asarray(a).astype(np.float64), requires_grad=grad)


def _check_swiglu_bwd(fn):
    """swiglu_bwd_ref(G, g, u) against autograd of g * sigmoid(g) * u (solution/swiglu.py:15-37),
    over g in [-8, 8] (every sigmoid regime, not only where 1 + g (1 - s) is 1)."""
    import torch

    rng = np.random.default_rng(8)
    g = rng.uniform(-8, 8, 4096).astype(np.float16)
    u = rng.standard_normal(4096).astype(np.float16)
    G = rng.standard_normal(4096).astype(np.float16)
    gt, ut = _t(g, True), _t(u, True)
    dgate, dup = torch.autograd.grad(gt * torch.sigmoid(gt) * ut, (gt, ut), _t(G))
    og, ou = fn(G, g, u)
    np.testing.assert_allclose(og, dgate.numpy(), rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(ou, dup.numpy(), rtol=1e-6, atol=1e-9)


def _lora_case(seed=31, m=64, k=256, n=192, r=16):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float16)
    a = ((rng.random((r, k)) * 2 - 1) / np.sqrt(k)).astype(np.float16)
    b = (rng.standard_normal((n, r)) * 0.05).astype(np.float16)
    dy = rng.standard_normal((m, n)).astype(np.float16)
    return x, a, b, dy


def _check_lora_bwd(fn, scaling):
    """lora_bwd_ref against autograd: out = (U . B^T) s with U the forward's fp16 u gives dU and
    dB; U = x . A^T, back-propagated from fp16(dU) (the reference's fp16 grad_u,
    solution/attn.py:255), gives dA and dX_lora. Both roundings of the oracle (reference) and its
    exact variant are checked: every output of both, each against its own bar."""
    import torch

    x, a, b, dy = _lora_case()
    u16, _ = O.lora_fwd_ref(x, a, b, scaling)
    U, B = _t(u16, True), _t(b, True)
    dU, dB = torch.autograd.grad((U @ B.T) * scaling, (U, B), _t(dy))
    gu = dU.numpy().astype(np.float32).astype(np.float16)
    X, A = _t(x, True), _t(a, True)
    dX, dA = torch.autograd.grad(X @ A.T, (X, A), _t(gu))
    for exact, bar in ((False, 2e-3), (True, 1e-6)):
        gu16, da, db, dxl = fn(dy, x, u16, a, b, scaling, exact=exact)
        for name, got, want in (("gu", gu16, dU.numpy()), ("dA", da, dA.numpy()), ("dB", db, dB.numpy()),
                                ("dX", dxl, dX.numpy())):
            mx, mean = O.tolerance(got, want)
            lim = 2e-3 if name == "gu" else bar  # gu is fp16 in both variants
            assert mx <= lim and mean <= lim, f"{name} exact={exact}: {mx:.2e} {mean:.2e}"


def _check_mlp(fn):
    """mlp_ref's out and dx against autograd of down(silu(gate(x)) * up(x)) in float64."""
    import torch

    rng = np.random.default_rng(31)
    m, k, n = 64, 128, 256
    x = rng.standard_normal((m, k)).astype(np.float16)
    wg, wu = ((rng.standard_normal((n, k)) * 0.1).astype(np.float16) for _ in range(2))
    wd = (rng.standard_normal((k, n)) * 0.1).astype(np.float16)
    dy = rng.standard_normal((m, k)).astype(np.float16)
    ref = fn(x, wg, wu, wd, dy)
    X = _t(x, True)
    gate, up = X @ _t(wg).T, X @ _t(wu).T
    out = (gate * torch.sigmoid(gate) * up) @ _t(wd).T
    (dx,) = torch.autograd.grad(out, (X,), _t(dy))
    for name, got, want in (("out", ref["out"], out.detach().numpy()), ("dx", ref["dx"], dx.numpy()),
                            ("dx_exact", ref["dx_exact"], dx.numpy())):
        mx, mean = O.tolerance(got, want)
        assert mx <= 2e-3 and mean <= 2e-3, f"{name}: {mx:.2e} {mean:.2e}"


def test_swiglu_bwd_ref_matches_autograd():
    _check_swiglu_bwd(O.swiglu_bwd_ref)


def test_swiglu_fwd_ref_matches_torch():
    import torch

    rng = np.random.default_rng(9)
    g = rng.uniform(-8, 8, 4096).astype(np.float16)
    u = rng.standard_normal(4096).astype(np.float16)
    want = (torch.nn.functional.silu(_t(g)) * _t(u)).numpy()
    np.testing.assert_allclose(O.swiglu_fwd_ref(g, u), want, rtol=1e-6, atol=1e-9)


@pytest.mark.parametrize("scaling", [2.0, 0.75])
def test_lora_bwd_ref_matches_autograd(scaling):
    _check_lora_bwd(O.lora_bwd_ref, scaling)


def test_lora_fwd_ref_matches_torch_fp16_matmul():
    """u = fp16(x . A^T) and out = fp16(u . B^T) * s, as torch's fp16 linear (fp32 accumulate,
    one rounding) computes them; the oracle's out stays fp32 before the scale's rounding."""
    import torch

    x, a, b, _ = _lora_case(seed=5)
    u16, out = O.lora_fwd_ref(x, a, b, 2.0)
    tu = (_t(x) @ _t(a).T).float().half()
    assert np.array_equal(u16.view(np.uint16), tu.numpy().view(np.uint16))
    tout = (tu.double() @ _t(b).T) * 2.0
    mx, mean = O.tolerance(out, tout.numpy())
    assert mx <= 1e-6 and mean <= 1e-6


def test_mlp_ref_matches_autograd():
    _check_mlp(O.mlp_ref)


def test_pins_catch_planted_mistakes(monkeypatch):
    """The checks above fail on plausible mistakes planted in the oracle (on the CPU): dgate
    without its (1 + g (1 - s)) factor, dup with u for g, dA doubled, dX_lora tripled, dB from the
    unscaled gradient, and the MLP built on the broken SwiGLU backward."""
    def dgate_no_factor(G, g, u):
        G, g, u = O._f64(G), O._f64(g), O._f64(u)
        s = 1.0 / (1.0 + np.exp(-g))
        return (G * u * s).astype(np.float32), (G * g * s).astype(np.float32)

    def dup_swapped(G, g, u):
        dg, _ = O.swiglu_bwd_ref(G, g, u)
        G, g, u = O._f64(G), O._f64(g), O._f64(u)
        return dg, (G * u / (1.0 + np.exp(-g))).astype(np.float32)

    good_lora = O.lora_bwd_ref

    def scaled(i, f):
        def fn(*args, **kw):
            out = list(good_lora(*args, **kw))
            out[i] = (out[i] * f).astype(out[i].dtype)
            return tuple(out)
        return fn

    def db_unscaled(dy, x, u, a, b, s, exact=False):
        gu, da, db, dx = good_lora(dy, x, u, a, b, s, exact=exact)
        return gu, da, (db / np.float32(s)).astype(np.float32), dx

    for bad in (dgate_no_factor, dup_swapped):
        with pytest.raises(AssertionError):
            _check_swiglu_bwd(bad)
    for bad in (scaled(1, 2.0), scaled(3, 3.0), db_unscaled):
        with pytest.raises(AssertionError):
            _check_lora_bwd(bad, 2.0)
    monkeypatch.setattr(O, "swiglu_bwd_ref", dgate_no_factor)
    with pytest.raises(AssertionError):
        _check_mlp(O.mlp_ref)
