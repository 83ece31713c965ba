"""Host-side logic without a GPU: the reference's gate `supported`, the QuantState stand-in,
the torch quantizer against the oracle's numpy quantizer, and the `solution` drop-in names."""

import numpy as np
import pytest
import torch

from oracle import nf4 as O


def test_torch_quantizer_matches_oracle_quantizer():
    from decik_amd.quant import quantize_nf4

    g = torch.Generator().manual_seed(0)
    for shape, nested in [((96, 128), True), ((256, 2560), True), ((64, 256), False), ((3, 40), True)]:
        w = (torch.randn(shape, generator=g) * 0.05).half()
        packed, qs = quantize_nf4(w, compress_statistics=nested)
        q = O.quantize_nf4(w.numpy(), nested=nested)
        assert np.array_equal(packed.numpy().reshape(-1), q.packed)
        if nested:
            # torch's vectorised linspace and the oracle's scalar restatement may round the map's
            # entries a few ulp apart (both restate bitsandbytes; neither is pinned to it)
            ulps = np.abs(qs.state2.code.numpy().view(np.int32) - q.code2.view(np.int32))
            assert ulps.max() <= 4
            assert np.float32(qs.offset.item()) == q.offset
            # the 8-bit codes may differ by one step where the nearest choice is a near-tie
            diff = np.abs(qs.absmax.numpy().astype(int) - q.absmax.astype(int))
            assert diff.max() <= 1 and (diff > 0).mean() < 0.01
            assert np.allclose(qs.state2.absmax.numpy(), q.absmax2)
        else:
            assert np.array_equal(qs.absmax.numpy(), q.absmax)


def test_supported_gate():
    from decik_amd.nf4 import fused_ok, supported
    from decik_amd.quant import quantize_nf4

    w = torch.randn(64, 128).half()
    _, qs = quantize_nf4(w)
    assert supported(qs) and supported(qs, 128) and not supported(qs, 64)
    assert fused_ok(qs, 128)
    assert not supported(None)
    _, qp = quantize_nf4(w, compress_statistics=False)
    assert supported(qp)
    qs.quant_type = "fp4"
    assert not supported(qs)

    class Broken:
        quant_type = "nf4"

    assert not supported(Broken())  # AttributeError -> False, as the reference
    _, q40 = quantize_nf4(torch.randn(64, 40).half())
    assert supported(q40) and not fused_ok(q40)


def test_solution_names_are_decik_modules():
    import decik_amd
    import solution
    import solution.nf4
    from solution.nf4 import BYTES_PER_PROGRAM, NUM_WARPS, NF4Linear, dequantize_nf4, patch, supported  # noqa: F401

    assert solution.nf4 is decik_amd.nf4
    assert BYTES_PER_PROGRAM == 4096 and NUM_WARPS == 4
    import solution._state as st

    t = torch.zeros(1)
    assert st.on_gpu(t) is False
    # the NF4-path names of solution/attn.py (RoPE, LoRA dropout helpers)
    import solution.attn
    from solution.attn import FusedQKRope, _lora_inputs, pack_keep  # noqa: F401

    assert solution.attn is decik_amd.attn


def test_apply_without_bitsandbytes_is_a_no_op(monkeypatch):
    import importlib.util

    import solution

    if importlib.util.find_spec("bitsandbytes") is not None:
        pytest.skip("bitsandbytes installed")
    monkeypatch.setenv("SKC_WARMUP", "0")
    solution.apply()


def test_product_path_has_no_cpu_fallback():
    """On a CPU tensor the fused path refuses rather than computing on the host."""
    from decik_amd import nf4
    from decik_amd.quant import quantize_nf4

    packed, qs = quantize_nf4(torch.randn(64, 128).half())
    with pytest.raises(Exception):
        nf4.dequantize_nf4(packed, qs)
