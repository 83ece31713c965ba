"""NF4 dequantization on the GPU: bit-exact against the oracle and the golden fixtures.

Mirrors the reference's own checks: solution/test_solution.py:9-19 (4 Qwen2.5-1.5B shapes x
nested on/off, w = randn * 0.05) and dev/test_cpu_kernels.py:24-36 ((96, 128), (256, 2560)),
with the oracle in place of bitsandbytes (absent here)."""

import numpy as np
import pytest
import torch

from helpers import golden_cases, make_weight, oracle_state
from oracle import nf4 as O

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1)


@pytest.mark.parametrize("name", sorted(golden_cases()))
def test_golden_fixtures(name, device):
    from decik_amd.nf4 import dequantize_nf4
    from decik_amd.quant import from_arrays

    c = golden_cases()[name]
    packed, qs = from_arrays(c["packed"], c["absmax"], c["absmax2"], c["code2"], c["offset"],
                             c["code"], c["shape"], c["blocksize"], c["blocksize2"], c["nested"],
                             device=device)
    out = dequantize_nf4(packed, qs)
    assert out.shape == c["shape"] and out.dtype == torch.float16
    assert np.array_equal(_bits(out), c["expected"])


@pytest.mark.parametrize("nested", [True, False])
@pytest.mark.parametrize("shape", [(1536, 1536), (256, 1536), (8960, 1536), (1536, 8960),
                                   (96, 128), (256, 2560)])
def test_bit_exact_vs_oracle(shape, nested, device):
    from decik_amd.nf4 import dequantize_nf4

    packed, qs, ref = make_weight(shape, seed=shape[0] * 7 + shape[1], device=device,
                                  nested=nested, std=0.05)
    out = dequantize_nf4(packed, qs)
    assert np.array_equal(_bits(out), ref.reshape(-1).view(np.uint16))


def test_every_byte_and_random_statistics(device):
    """Random packed bytes (every value) and random nested statistics, incl. blocks and
    256-groups straddling rows (k = 40)."""
    from decik_amd.nf4 import dequantize_nf4
    from decik_amd.quant import from_arrays

    rng = np.random.default_rng(9)
    for shape in [(64, 1024), (33, 40), (5, 6)]:
        n = shape[0] * shape[1]
        nb = -(-n // 64)
        packed = rng.integers(0, 256, n // 2, dtype=np.uint8)
        absmax = rng.integers(0, 256, nb, dtype=np.uint8)
        absmax2 = (rng.random(-(-nb // 256)) * 0.1).astype(np.float32)
        q = O.QuantNF4(packed, absmax, absmax2, O.dynamic_map_signed(), np.float32(0.013),
                       O.NF4_CODE.copy(), shape)
        ref = O.dequant_nf4(q).reshape(-1).view(np.uint16)
        p_t, qs = from_arrays(packed, absmax, absmax2, q.code2, q.offset, q.code, shape,
                              device=device)
        assert np.array_equal(_bits(dequantize_nf4(p_t, qs)), ref), shape


@pytest.mark.parametrize("blocksize", [32, 128, 256, 1024])
def test_other_blocksizes(blocksize, device):
    from decik_amd.nf4 import dequantize_nf4

    packed, qs, ref = make_weight((192, 1024), seed=blocksize, device=device, blocksize=blocksize)
    assert np.array_equal(_bits(dequantize_nf4(packed, qs)), ref.reshape(-1).view(np.uint16))


def test_unaligned_packed_takes_generic_path(device):
    """A packed view that starts 1 byte into its buffer (no 16-byte loads) is still exact."""
    from decik_amd.nf4 import dequantize_nf4

    packed, qs, ref = make_weight((64, 256), seed=3, device=device)
    buf = torch.empty(packed.numel() + 1, dtype=torch.uint8, device=device)
    buf[1:] = packed.reshape(-1)
    out = dequantize_nf4(buf[1:], qs)
    assert np.array_equal(_bits(out), ref.reshape(-1).view(np.uint16))


def test_batched_equals_single(device):
    from decik_amd.nf4 import dequantize_nf4, dequantize_nf4_many

    pairs, refs = [], []
    for i, shape in enumerate([(1536, 1536), (256, 1536), (256, 1536), (1536, 1536),
                               (8960, 1536), (8960, 1536), (1536, 8960), (3, 40), (96, 128)]):
        packed, qs, ref = make_weight(shape, seed=100 + i, device=device, nested=(i % 3 != 2))
        pairs.append((packed, qs))
        refs.append(ref)
    outs = dequantize_nf4_many(pairs)
    for o, (p, q), r in zip(outs, pairs, refs):
        assert np.array_equal(_bits(o), r.reshape(-1).view(np.uint16))
        assert torch.equal(o, dequantize_nf4(p, q))


def test_empty_weight(device):
    from decik_amd.nf4 import dequantize_nf4
    from decik_amd.quant import QuantState

    qs = QuantState(absmax=torch.zeros(0, dtype=torch.float32, device=device), shape=(0, 64),
                    code=torch.tensor(O.NF4_CODE, device=device), blocksize=64)
    out = dequantize_nf4(torch.zeros(0, dtype=torch.uint8, device=device), qs)
    assert out.shape == (0, 64)


def test_oracle_state_roundtrip(device):
    """The GPU quantizer's bytes, read back, are the bytes the oracle dequantizes."""
    packed, qs, _ = make_weight((16, 128), seed=1, device=device)
    q = oracle_state(packed, qs)
    assert q.packed.size == 16 * 128 // 2 and q.absmax.size == 16 * 128 // 64


@pytest.mark.parametrize("shape,blocksize", [((1536, 1536), 64), ((256, 2560), 128), ((96, 128), 32),
                                             ((300, 264), 64)])
def test_block_scales_bit_exact(shape, blocksize, device):
    """dk_nf4_block_scales = the scale step of the reference kernel (solution/nf4.py:37-43), and a
    plain description with those scales dequantizes to the same bits as the nested weight."""
    import ctypes

    from decik_amd import _lib

    packed, qs, w16 = make_weight(shape, seed=sum(shape) + blocksize, device=device,
                                  blocksize=blocksize)
    scales = _lib.SCALES.get(packed, qs, device)
    ref = O.block_scales(oracle_state(packed, qs))
    got = scales[: ref.size].cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32))
    w, keep = _lib.weight_desc(packed, qs, device, scales)
    out = torch.empty(shape, dtype=torch.float16, device=device)
    _lib.check(_lib.lib().dk_nf4_dequant(ctypes.byref(w), out.data_ptr(), _lib.stream_of(device)))
    assert np.array_equal(_bits(out), w16.view(np.uint16).reshape(-1))
