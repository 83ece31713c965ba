"""CPU oracle: NF4 dequantization, the bitsandbytes NF4 quantizer, and fp32 references.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): imported by tests/, smoke() and bench.py's
cpu_baseline leg; never by the product path.

What each function restates, and what pins it (the tests live in tests/test_oracle.py):

- `dequant_nf4` -> C `oracle_nf4_dequant`, restating skc_nf4_dequant_kernel
  (solution/nf4.py:27-48) and its launch wrapper (solution/nf4.py:66-85). Pinned by:
  the fp32->fp16 conversion against numpy's independent conversion over every fp32 exponent
  and a spread of mantissas; closed forms (nibble 7 -> +0, nibbles 0/15 -> -/+scale exactly,
  plain absmax 1 -> fp16(code)); brute force over all 256 byte values checked against exact
  rational arithmetic with explicit two-step rounding; inputs where an FMA would change the
  scale; blocks and double-quant groups that straddle rows; high nibble first.
- `quantize_nf4` -> bitsandbytes 0.50.2 `functional.quantize_4bit(..., quant_type="nf4",
  compress_statistics=True)`, `quantize_blockwise` and `create_dynamic_map(signed=True)`
  (third party; pinned in the reference at README.md:210-211, called at solution/nf4.py:108-115
  and solution/test_solution.py:18). bitsandbytes is neither vendored nor installed, so the
  quantizer is PARITY UNPINNED against it; tests check its invariants instead (nearest code,
  reconstruction bound, layout). Dequant parity does not depend on it: the packed bytes and
  statistics are inputs.
- `keep_pack`, `lora_dropout_inputs_ref`, `lora_input_grad_ref`: the LoRA dropout steps of
  solution/attn.py:129-180, elementwise fp32 in the reference's order (exact). Pinned by
  numpy.packbits (an independent bit packer) and closed forms (all-keep / no-keep masks, scale 1).
- `rope_fwd_ref`, `rope_bwd_ref`: RoPE of q/k (solution/attn.py:27-86), elementwise fp32 in the
  reference's order (exact). Pinned by closed forms (cos 1 / sin 0 is the identity, cos 0 /
  sin 1 is rotate_half) and by the backward being the forward's transpose (float64 inner
  products).
- `linear_ref`, `lora_*_ref`, `swiglu_*_ref`, `mlp_ref`: float64 accumulation of the exact fp16
  operands, rounded where the reference rounds (solution/nf4.py:93-104, solution/mlp.py:62-110,
  solution/swiglu.py:15-37, solution/attn.py:206-273). Pinned by closed forms in the tests
  (identity and permutation weights, rank-one inputs, sigmoid identities) and, for every
  backward (swiglu_bwd_ref, lora_bwd_ref's gu/dA/dB/dX, mlp_ref's dx), by torch's float64
  autograd of the forward formulas, with planted mistakes (a dropped factor, a wrong scale, a
  swapped operand) shown to fail those checks.
"""

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle_nf4.so")
_lib = None

# bitsandbytes' NF4 code book (functional.get_4bit_type("nf4")), the NormalFloat4 values of the
# QLoRA paper (arXiv:2305.14314, appendix E), stored as fp32.
NF4_CODE = np.array([
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0], dtype=np.float32)


def build():
    """Compile the C oracle (oracle/Makefile) into oracle/_build/."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        i64, i32, vp, f32 = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_float
        L.oracle_nf4_dequant.argtypes = [vp, vp, vp, vp, vp, f32, vp, vp, i64, i32, i64, i64, i32]
        L.oracle_nf4_dequant.restype = None
        L.oracle_f32_to_f16_array.argtypes = [vp, vp, i64]
        L.oracle_f16_to_f32_array.argtypes = [vp, vp, i64]
        L.oracle_num_threads.restype = i32
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def f32_to_f16_bits(x):
    """The oracle's own fp32 -> fp16 RNE conversion (uint16 bit patterns)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_f16_array(_ptr(x), _ptr(out), x.size)
    return out


def f16_bits_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().oracle_f16_to_f32_array(_ptr(h), _ptr(out), h.size)
    return out


@dataclass
class QuantNF4:
    """The tensors of a bitsandbytes nf4 Params4bit + QuantState (solution/nf4.py:54-58,70-79)."""
    packed: np.ndarray          # uint8 [N*K/2], two weights per byte, high nibble first
    absmax: np.ndarray          # nested: uint8 codes [n_blocks]; plain: fp32 [n_blocks]
    absmax2: np.ndarray         # nested: fp32 [ceil(n_blocks / blocksize2)]; plain: empty
    code2: np.ndarray           # nested: fp32 [256] (signed dynamic map); plain: empty
    offset: np.float32          # nested: fp32 mean of the block absmax; plain: 0
    code: np.ndarray            # fp32 [16] NF4 code book
    shape: tuple                # (N, K)
    blocksize: int = 64
    blocksize2: int = 256
    nested: bool = True


def dequant_nf4(q: QuantNF4, nthreads=1):
    """fp16 [N, K] weights, bit-exact restatement of solution/nf4.py:27-48,66-85."""
    n_out, n_in = q.shape
    n_bytes = n_out * n_in // 2
    out = np.empty(2 * n_bytes, dtype=np.uint16)
    packed = np.ascontiguousarray(q.packed, dtype=np.uint8)
    code = np.ascontiguousarray(q.code, dtype=np.float32)
    if q.nested:
        a8 = np.ascontiguousarray(q.absmax, dtype=np.uint8)
        a2 = np.ascontiguousarray(q.absmax2, dtype=np.float32)
        c2 = np.ascontiguousarray(q.code2, dtype=np.float32)
        lib().oracle_nf4_dequant(_ptr(packed), _ptr(a8), None, _ptr(a2), _ptr(c2),
                                 float(q.offset), _ptr(code), _ptr(out), n_bytes, 1,
                                 q.blocksize, q.blocksize2, nthreads)
    else:
        af = np.ascontiguousarray(q.absmax, dtype=np.float32)
        lib().oracle_nf4_dequant(_ptr(packed), None, _ptr(af), None, None, 0.0, _ptr(code),
                                 _ptr(out), n_bytes, 0, q.blocksize, 256, nthreads)
    return out.view(np.float16).reshape(n_out, n_in)


def linspace_f32(start, end, steps):
    """torch.linspace for float32 as its CPU kernel computes it (which bitsandbytes calls):
    step = (end - start) / (steps - 1) in fp32; the first half counts up from start, the second
    half down from end."""
    start, end = np.float32(start), np.float32(end)
    step = np.float32((end - start) / np.float32(steps - 1))
    out = np.empty(steps, np.float32)
    half = steps // 2
    for i in range(steps):
        out[i] = start + step * np.float32(i) if i < half else end - step * np.float32(steps - i - 1)
    return out


def dynamic_map_signed(max_exponent_bits=7, total_bits=8):
    """bitsandbytes functional.create_dynamic_map(signed=True): 256 sorted fp32 values.

    For exponent i (0..6) the 2**i midpoints of linspace(0.1, 1, 2**i + 1) scaled by 10**(i-6),
    with both signs, plus 0 and 1.0."""
    data = []
    non_sign_bits = total_bits - 1
    for i in range(max_exponent_bits):
        fraction_items = 2 ** (i + non_sign_bits - max_exponent_bits) + 1
        boundaries = linspace_f32(0.1, 1, fraction_items)
        means = ((boundaries[:-1] + boundaries[1:]) / np.float32(2.0)).astype(np.float32)
        scale = np.float32(10 ** (-(max_exponent_bits - 1) + i))
        data += (scale * means).astype(np.float32).tolist()
        data += (-scale * means).astype(np.float32).tolist()
    data.append(0.0)
    data.append(1.0)
    assert len(data) == 2 ** total_bits
    data.sort()
    return np.array(data, dtype=np.float32)


def _blockwise_absmax(a, blocksize):
    n = a.size
    n_blocks = -(-n // blocksize)
    padded = np.zeros(n_blocks * blocksize, dtype=np.float32)
    padded[:n] = a
    blocks = padded.reshape(n_blocks, blocksize)
    absmax = np.abs(blocks).max(axis=1).astype(np.float32)
    inv = np.zeros_like(absmax)
    nz = absmax > 0
    inv[nz] = np.float32(1.0) / absmax[nz]
    normed = (blocks * inv[:, None]).astype(np.float32)
    return absmax, normed


def quantize_nf4(w16, blocksize=64, nested=True, blocksize2=256):
    """Restatement of bitsandbytes quantize_4bit(quant_type="nf4") (PARITY UNPINNED vs bnb).

    Block absmax over `blocksize` flat elements, x * (1/absmax), NF4 index = number of
    midpoints between adjacent code values that x exceeds (the CUDA decision tree), two indices
    per byte with the even element in the high nibble. Double quant: offset = mean(absmax),
    absmax - offset quantized blockwise (blocksize2) to the nearest signed dynamic-map code."""
    w = np.asarray(w16)
    assert w.ndim == 2 and w.size % 2 == 0
    a = w.astype(np.float32).reshape(-1)
    absmax, normed = _blockwise_absmax(a, blocksize)
    thresholds = ((NF4_CODE[:-1].astype(np.float64) + NF4_CODE[1:].astype(np.float64)) / 2.0)
    thresholds = thresholds.astype(np.float32)
    idx = np.searchsorted(thresholds, normed.reshape(-1), side="left").astype(np.uint8)[:a.size]
    packed = ((idx[0::2] << 4) | idx[1::2]).astype(np.uint8)
    if not nested:
        return QuantNF4(packed, absmax, np.zeros(0, np.float32), np.zeros(0, np.float32),
                        np.float32(0), NF4_CODE.copy(), tuple(w.shape), blocksize, blocksize2,
                        False)
    offset = np.float32(absmax.astype(np.float64).mean())
    centred = (absmax - offset).astype(np.float32)
    code2 = dynamic_map_signed()
    absmax2, normed2 = _blockwise_absmax(centred, blocksize2)
    flat2 = normed2.reshape(-1)[:centred.size]
    # nearest code value; code2 is sorted, so compare the two neighbours of the insertion point
    hi = np.clip(np.searchsorted(code2, flat2, side="left"), 1, 255)
    lo = hi - 1
    pick_hi = np.abs(code2[hi] - flat2) < np.abs(flat2 - code2[lo])
    q8 = np.where(pick_hi, hi, lo).astype(np.uint8)
    return QuantNF4(packed, q8, absmax2, code2, offset, NF4_CODE.copy(), tuple(w.shape),
                    blocksize, blocksize2, True)


def block_scales(q: QuantNF4):
    """The fp32 per-block scales dequant uses (solution/nf4.py:37-43), for the checks."""
    if not q.nested:
        return np.asarray(q.absmax, dtype=np.float32)
    blocks = np.arange(q.absmax.size)
    s = (q.code2[q.absmax.astype(np.int64)] * q.absmax2[blocks // q.blocksize2]).astype(np.float32)
    return (s + np.float32(q.offset)).astype(np.float32)


# ----------------------------------------------------------------------------------------------
# fp32-accumulated references (float64 sums of exact fp16 operands)

def _f64(a):
    return np.asarray(a).astype(np.float64)


def linear_ref(x16, w16, bias16=None):
    """Y = X . W^T (+ b) accumulated exactly, as fp32 (solution/nf4.py:94-96)."""
    y = _f64(x16) @ _f64(w16).T
    if bias16 is not None:
        y = y + _f64(bias16)[None, :]
    return y.astype(np.float32)


def linear_dx_ref(dy16, w16):
    """dX = dY . W accumulated exactly, as fp32 (solution/nf4.py:101-103)."""
    return (_f64(dy16) @ _f64(w16)).astype(np.float32)


def lora_fwd_ref(x16, a16, b16, scaling):
    """peft's lora_B(lora_A(x)) * scaling under fp16 autocast (solution/attn.py:225-228,344-346):
    u = fp16(x . A^T) [M, r]; out = fp16(u . B^T) * scaling. Returns (u16, out as fp32)."""
    u16 = (_f64(x16) @ _f64(a16).T).astype(np.float32).astype(np.float16)
    out = (_f64(u16) @ _f64(b16).T) * float(scaling)
    return u16, out.astype(np.float32)


def _f16(a):
    """Round to fp16 (through fp32, as a torch fp16 matmul stores its fp32 accumulator)."""
    return np.asarray(a).astype(np.float32).astype(np.float16)


def lora_bwd_ref(dy16, x16, u16, a16, b16, scaling, exact=False):
    """The products LoRAPairFromNorm.backward forms for out = (u . B^T) * s, u = x . A^T
    (solution/attn.py:251-257), with the reference's fp16 tensors rounded where it rounds them:
      g = fp16(dY * s)                  (:252, fp16 tensor times a Python float)
      dB = fp32(fp16(g^T . u))          (:254, fp16 mm, then .to(float32) at :256)
      gu = fp16(g . B16)                (:255)
      dA = fp32(fp16(gu^T . x16))       (:256)
      dX_lora = fp16(gu . A16)          (:257, before the dropout-mask step)
    Returns (gu16, dA, dB, dX_lora) as (fp16, fp32, fp32, fp32).

    exact=True: the same chain without the roundings of g, dA, dB and dX_lora (gu stays fp16: it
    is an fp16 operand of the next product in both implementations) -- what the fused kernels
    compute (fp32 accumulators stored once); the reference's roundings are within the bar of it."""
    s = float(scaling)
    if exact:
        g = _f64(dy16) * s
        gu16 = _f16(g @ _f64(b16))
        db = g.T @ _f64(u16)
        da = _f64(gu16).T @ _f64(x16)
        dx = _f64(gu16) @ _f64(a16)
        return gu16, da.astype(np.float32), db.astype(np.float32), dx.astype(np.float32)
    g16 = _f16(_f64(dy16).astype(np.float32) * np.float32(s))
    gu16 = _f16(_f64(g16) @ _f64(b16))
    db = _f16(_f64(g16).T @ _f64(u16))
    da = _f16(_f64(gu16).T @ _f64(x16))
    dx = _f16(_f64(gu16) @ _f64(a16))
    return gu16, da.astype(np.float32), db.astype(np.float32), dx.astype(np.float32)


# LoRA dropout with packed keep-masks (solution/attn.py:129-180): elementwise fp32 arithmetic in the
# reference's order, so these are exact restatements (numpy float32 ops round like the GPU's).

def keep_pack(keep):
    """bool [rows, width] -> uint8 [rows, width / 8], bit j of byte c = keep[r, 8 c + j]
    (skc_keep_pack_kernel, solution/attn.py:129-144)."""
    k = np.asarray(keep).astype(np.uint8).reshape(keep.shape[0], -1, 8)
    return np.bitwise_or.reduce(k << np.arange(8, dtype=np.uint8), axis=2).astype(np.uint8)


def keep_unpack(bits, width):
    """Inverse of keep_pack: float32 0/1 [rows, width] (the reference's _keep,
    solution/attn.py:147-150)."""
    b = np.asarray(bits).astype(np.uint32)
    cols = np.arange(width)
    return ((b[:, cols // 8] >> (cols % 8)) & 1).astype(np.float32)


def lora_dropout_inputs_ref(x, bits_q, bits_v, scale_q, scale_v):
    """fp16(x * (keep * scale)) in fp32 for the q and v branches (skc_lora_inputs_kernel,
    solution/attn.py:153-165)."""
    xf = np.asarray(x).astype(np.float32)
    w = xf.shape[1]
    mq = keep_unpack(bits_q, w) * np.float32(scale_q)
    mv = keep_unpack(bits_v, w) * np.float32(scale_v)
    return (xf * mq).astype(np.float16), (xf * mv).astype(np.float16)


def lora_input_grad_ref(gq16, gv16, bits_q, bits_v, scale_q, scale_v):
    """(fp32(gq) * keep_q) * sq + (fp32(gv) * keep_v) * sv (skc_lora_input_grad_kernel,
    solution/attn.py:168-180)."""
    w = np.asarray(gq16).shape[1]
    tq = (np.asarray(gq16).astype(np.float32) * keep_unpack(bits_q, w)) * np.float32(scale_q)
    tv = (np.asarray(gv16).astype(np.float32) * keep_unpack(bits_v, w)) * np.float32(scale_v)
    return (tq + tv).astype(np.float32)


def rotate_half(x):
    """[-x[D/2:], x[:D/2]] along the last axis (transformers' rotate_half)."""
    h = x.shape[-1] // 2
    return np.concatenate([-x[..., h:], x[..., :h]], axis=-1)


def rope_fwd_ref(q_base16, q_lora16, k16, cos, sin, n_heads, n_kv_heads):
    """skc_rope_fwd_kernel (solution/attn.py:27-66): q = fp32(base) + fp32(lora); q cos +
    rotate_half(q) sin in fp32 (no FMA); fp16 head-major [H, T, D]. q_lora16 None: no add."""
    t = q_base16.shape[0]
    d = cos.shape[-1]
    c, s = np.asarray(cos, np.float32), np.asarray(sin, np.float32)
    def one(x, heads):
        x = x.reshape(t, heads, d).transpose(1, 0, 2)  # [H, T, D] fp32
        return ((x * c[None]) + (rotate_half(x) * s[None])).astype(np.float16)
    q = np.asarray(q_base16).astype(np.float32)
    if q_lora16 is not None:
        q = q + np.asarray(q_lora16).astype(np.float32)
    return one(q, n_heads), one(np.asarray(k16).astype(np.float32), n_kv_heads)


def rope_bwd_ref(grad_q16, grad_k16, cos, sin):
    """skc_rope_bwd_kernel (solution/attn.py:69-86): d = g cos + rotate_half^T(g sin) in fp32,
    fp16 token-major [T, H*D]; rotate_half^T(y)[d] = y[d + D/2] for d < D/2, -y[d - D/2] after."""
    c, s = np.asarray(cos, np.float32), np.asarray(sin, np.float32)
    def one(g):
        g = np.asarray(g).astype(np.float32)  # [H, T, D]
        a = g * c[None]
        b = g * s[None]
        h = g.shape[-1] // 2
        bt = np.concatenate([b[..., h:], -b[..., :h]], axis=-1)
        out = (a + bt).astype(np.float16)
        return out.transpose(1, 0, 2).reshape(g.shape[1], -1)
    return one(grad_q16), one(grad_k16)


def _sigmoid64(x):
    return 1.0 / (1.0 + np.exp(-x))


def swiglu_fwd_ref(gate16, up16):
    """fp16(silu(g) * u) computed in fp32 (solution/swiglu.py:15-23)."""
    g = _f64(gate16)
    return (g * _sigmoid64(g) * _f64(up16)).astype(np.float32)


def swiglu_bwd_ref(grad16, gate16, up16):
    """dup = G g s, dgate = G u s (1 + g (1 - s)), s = sigmoid(g) (solution/swiglu.py:25-37)."""
    G, g, u = _f64(grad16), _f64(gate16), _f64(up16)
    s = _sigmoid64(g)
    dup = G * g * s
    dgate = G * u * s * (1.0 + g * (1.0 - s))
    return dgate.astype(np.float32), dup.astype(np.float32)


def mlp_ref(x16, wg16, wu16, wd16, dy16):
    """Qwen2 MLP forward and input gradient as RecomputedMLP computes it (solution/mlp.py:62-110):
    gate, up, h rounded to fp16 where the fp16 matmuls and the SwiGLU kernel round (:69-71);
    out = the fp32-accumulated down projection (:73; the reference stores it as fp16);
    gh = fp16(dY . Wd) (:95); dgate / dup from the SwiGLU backward, fp16 (:104); and
    dx = fp32(fp16(dgate . Wg)) + fp32(fp16(dup . Wu)) -- two fp16 matmul results, each cast to
    fp32, then summed (:106-109).
    dx_exact = fp32(dgate . Wg + dup . Wu) with no rounding of the two products: the fused kernel
    accumulates both in one fp32 tile and rounds once, so this measures its own accuracy; dx (the
    reference's two roundings) lies within the bar of it.
    Returns a dict of fp32 arrays (gate, up, h, out, gh, dgate, dup, dx, dx_exact)."""
    gate = linear_ref(x16, wg16).astype(np.float16)
    up = linear_ref(x16, wu16).astype(np.float16)
    h = swiglu_fwd_ref(gate, up).astype(np.float16)
    out = linear_ref(h, wd16)
    gh = linear_dx_ref(dy16, wd16).astype(np.float16)
    dgate, dup = swiglu_bwd_ref(gh, gate, up)
    dgate16, dup16 = dgate.astype(np.float16), dup.astype(np.float16)
    pg = _f64(dgate16) @ _f64(wg16)
    pu = _f64(dup16) @ _f64(wu16)
    dx = (_f64(_f16(pg)) + _f64(_f16(pu))).astype(np.float32)
    dx_exact = (pg + pu).astype(np.float32)
    return dict(gate=gate.astype(np.float32), up=up.astype(np.float32),
                h=h.astype(np.float32), out=out, gh=gh.astype(np.float32),
                dgate=dgate, dup=dup, dx=dx, dx_exact=dx_exact)


def tolerance(y, ref):
    """(max|y-ref| / max|ref|, sum|y-ref| / sum|ref|): the two numbers the parity bar bounds
    (<= 1e-2 and <= 1e-3); the first is the reference's own `rel` (dev/test_cpu_bnb.py:66)."""
    y = _f64(y)
    ref = _f64(ref)
    err = np.abs(y - ref)
    denom_max = max(np.abs(ref).max(), 1e-30)
    denom_sum = max(np.abs(ref).sum(), 1e-30)
    return float(err.max() / denom_max), float(err.sum() / denom_sum)
