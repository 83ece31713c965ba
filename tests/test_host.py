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


def test_bnb_format_round_trip_through_safetensors(tmp_path):
    """An nf4 weight written in bitsandbytes' serialized layout (QuantState.as_dict(packed=True),
    keys under '<prefix>.weight.') survives a safetensors file and loads back to the same bytes
    and statistics; the dequantized weight is bit-identical (oracle). Agreement with
    bitsandbytes' own serializer is parity unpinned (not installed): the layout is checked."""
    import json

    from safetensors.torch import load_file, save_file

    from decik_amd import bnb_format
    from decik_amd.quant import quantize_nf4
    from oracle import nf4 as O

    from helpers import oracle_state

    w = (torch.randn(96, 128, generator=torch.Generator().manual_seed(9)) * 0.02).half()
    packed, qs = quantize_nf4(w, blocksize=64, compress_statistics=True)
    sd = {}
    bnb_format.save_nf4_weight(sd, "model.layers.0.mlp.gate_proj", packed, qs)
    assert set(sd) == {"model.layers.0.mlp.gate_proj.weight"} | {
        "model.layers.0.mlp.gate_proj.weight." + k for k in
        ("absmax", "quant_map", "nested_absmax", "nested_quant_map", "quant_state.bitsandbytes__nf4")}
    meta = json.loads(bytes(sd["model.layers.0.mlp.gate_proj.weight.quant_state.bitsandbytes__nf4"].tolist()))
    assert meta == {"quant_type": "nf4", "blocksize": 64, "dtype": "float16", "shape": [96, 128],
                    "nested_blocksize": 256, "nested_dtype": "float32", "nested_offset": float(qs.offset.item())}
    path = tmp_path / "w.safetensors"
    save_file({k: v.contiguous() for k, v in sd.items()}, str(path))
    back = load_file(str(path))
    assert bnb_format.nf4_prefixes(back) == ["model.layers.0.mlp.gate_proj"]
    p2, q2 = bnb_format.load_nf4_weight(back, "model.layers.0.mlp.gate_proj")
    assert torch.equal(p2, packed) and tuple(q2.shape) == (96, 128) and q2.nested and q2.blocksize == 64
    assert torch.equal(q2.absmax, qs.absmax) and torch.equal(q2.state2.absmax, qs.state2.absmax)
    assert torch.equal(q2.code, qs.code) and torch.equal(q2.state2.code, qs.state2.code)
    assert q2.offset.dtype == torch.float32 and float(q2.offset) == float(qs.offset)
    a = O.dequant_nf4(oracle_state(packed, qs))
    b = O.dequant_nf4(oracle_state(p2, q2))
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


def test_bnb_format_plain_and_errors():
    from decik_amd import bnb_format
    from decik_amd.quant import quantize_nf4

    w = (torch.randn(32, 64, generator=torch.Generator().manual_seed(10)) * 0.02).half()
    packed, qs = quantize_nf4(w, blocksize=64, compress_statistics=False)
    d = bnb_format.quant_state_as_dict(qs, packed=True)
    assert set(d) == {"absmax", "quant_map", "quant_state.bitsandbytes__nf4"}
    q2 = bnb_format.quant_state_from_dict(d)
    assert not q2.nested and torch.equal(q2.absmax, qs.absmax)
    unpacked = bnb_format.quant_state_as_dict(qs, packed=False)
    assert unpacked["shape"] == (32, 64) and unpacked["dtype"] == "float16"
    with pytest.raises(KeyError):
        bnb_format.load_nf4_weight({}, "x")
    with pytest.raises(ValueError):
        bnb_format.quant_state_from_dict({"absmax": qs.absmax})


def test_bnb_checkpoint_loader_sharded(tmp_path):
    """A checkpoint split over two safetensors shards, with a non-nf4 tensor beside the nf4
    weights, loads every nf4 weight by module prefix."""
    from safetensors.torch import save_file

    from decik_amd import bnb_format
    from decik_amd.quant import quantize_nf4

    g = torch.Generator().manual_seed(11)
    shards = [{}, {}]
    ref = {}
    for i, name in enumerate(["model.layers.0.mlp.up_proj", "model.layers.0.self_attn.q_proj"]):
        w = (torch.randn(64, 128, generator=g) * 0.02).half()
        packed, qs = quantize_nf4(w, blocksize=64, compress_statistics=bool(i))
        bnb_format.save_nf4_weight(shards[i], name, packed, qs)
        ref[name] = (packed, qs)
    shards[0]["model.norm.weight"] = torch.ones(128, dtype=torch.float16)
    for i, s in enumerate(shards):
        save_file({k: v.contiguous() for k, v in s.items()}, str(tmp_path / f"model-0000{i + 1}.safetensors"))
    got = bnb_format.load_nf4_checkpoint(str(tmp_path))
    assert sorted(got) == sorted(ref)
    for name, (packed, qs) in ref.items():
        p2, q2 = got[name]
        assert torch.equal(p2, packed) and torch.equal(q2.absmax, qs.absmax) and q2.nested == qs.nested
    with pytest.raises(FileNotFoundError):
        bnb_format.load_nf4_checkpoint(str(tmp_path / "none"))
