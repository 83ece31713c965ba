"""The patched entry points without a GPU: bitsandbytes' Linear4bit.forward (solution/nf4.py:107-138)
and transformers' Qwen2MLP.forward (solution/mlp.py:113-162), driven through a stand-in
bitsandbytes package (tests/standin_bnb.py). `on_gpu` is replaced, as the reference's own CPU
tests do (dev/test_cpu_kernels.py:12-13), and the fused autograd functions are replaced by
recorders, so each test sees which path a call takes and with which arguments; nothing runs on
a GPU. The GPU tests (test_patch_gpu.py) run the same patches for real."""

import pytest
import torch

import standin_bnb
from decik_amd import _state, mlp, nf4
from decik_amd.quant import quantize_nf4


def _linear(cls, n_out, n_in, bias=False, seed=0, **kw):
    g = torch.Generator().manual_seed(seed)
    packed, qs = quantize_nf4((torch.randn(n_out, n_in, generator=g) * 0.02).half())
    b = (torch.randn(n_out, generator=g) * 0.1).half() if bias else None
    return cls(packed, qs, bias=b, **kw)


class Recorder:
    def __init__(self, out_features=None):
        self.calls = []
        self.out_features = out_features

    def __call__(self, *args):
        self.calls.append(args)
        x = args[0]
        n = self.out_features if self.out_features is not None else args[3].shape[0]
        return torch.zeros(x.shape[:-1] + (int(n),), dtype=torch.float16)


@pytest.fixture
def bnb(monkeypatch):
    return standin_bnb.install(monkeypatch)


@pytest.fixture
def gpu_everywhere(monkeypatch):
    monkeypatch.setattr(_state, "on_gpu", lambda t: True)


def test_nf4_patch_fast_path_casts(bnb, gpu_everywhere, monkeypatch):
    """Every condition holds: NF4Linear gets fp16 x, the weight bytes, an fp16 bias and the
    QuantState; the result comes back in x's dtype (fp32 in, fp32 out)."""
    rec = Recorder()
    monkeypatch.setattr(nf4.NF4Linear, "apply", rec)
    nf4.patch()
    layer = _linear(bnb.nn.Linear4bit, 96, 64, bias=True)
    x = torch.randn(5, 64)
    y = layer(x)
    assert len(rec.calls) == 1 and bnb.nn.Linear4bit.original_calls == 0
    x16, packed, bias16, qs = rec.calls[0]
    assert x16.dtype == torch.float16 and torch.equal(x16, x.half())
    assert packed.data_ptr() == layer.weight.data_ptr()
    assert bias16.dtype == torch.float16 and qs is layer.weight.quant_state
    assert y.dtype == torch.float32 and y.shape == (5, 96)
    y16 = layer(x.half())
    assert y16.dtype == torch.float16 and rec.calls[-1][2] is not None


def test_nf4_patch_is_idempotent(bnb):
    nf4.patch()
    first = bnb.nn.Linear4bit.forward
    assert getattr(first, "_skc", False)
    nf4.patch()
    assert bnb.nn.Linear4bit.forward is first


@pytest.mark.parametrize("case", ["cpu_input", "empty", "fp32_compute", "grad_weight", "grad_bias",
                                  "width", "fp4", "not_tensor"])
def test_nf4_patch_falls_back(case, bnb, monkeypatch):
    """Each failed condition of the reference's gate (solution/nf4.py:125-131) runs bitsandbytes'
    own forward."""
    rec = Recorder()
    monkeypatch.setattr(nf4.NF4Linear, "apply", rec)
    nf4.patch()
    layer = _linear(bnb.nn.Linear4bit, 96, 64, bias=True,
                    compute_dtype=torch.float32 if case == "fp32_compute" else torch.float16)
    x = torch.randn(5, 64)
    if case != "cpu_input":
        monkeypatch.setattr(_state, "on_gpu", lambda t: True)
    if case == "empty":
        x = torch.randn(0, 64)
    if case == "grad_weight":
        class Grad:
            pass

        w = Grad()
        w.data, w.dtype, w.requires_grad = layer.weight.data, torch.uint8, True
        w.quant_state = layer.weight.quant_state
        layer.__dict__["weight"] = w
        del layer._parameters["weight"]
    if case == "grad_bias":
        layer.bias.requires_grad_(False)
        layer.bias = torch.nn.Parameter(layer.bias.detach().float(), requires_grad=True)
    if case == "width":
        x = torch.randn(5, 32)
    if case == "fp4":
        layer.weight.quant_state.quant_type = "fp4"
    if case == "not_tensor":
        x = [1.0] * 64
        monkeypatch.setattr(bnb.nn.Linear4bit, "__call__", lambda self, v: type(self).forward(self, v))
        with pytest.raises(Exception):
            layer(x)  # bitsandbytes' own forward gets the list (and fails on it)
        assert not rec.calls
        return
    out = layer(x)
    assert not rec.calls and bnb.nn.Linear4bit.original_calls == 1
    assert torch.all(out == -7.0)


def test_nf4_patch_repairs_lost_quant_state(bnb, gpu_everywhere, monkeypatch):
    """A weight that lost its quant_state gets it back through bitsandbytes' helper before the
    gate (solution/nf4.py:119-122), then takes the fast path."""
    rec = Recorder()
    monkeypatch.setattr(nf4.NF4Linear, "apply", rec)
    nf4.patch()
    layer = _linear(bnb.nn.Linear4bit, 96, 64)
    layer.weight.quant_state = None
    layer(torch.randn(3, 64))
    assert layer.weight.quant_state is layer.quant_state_backup and len(rec.calls) == 1


@pytest.fixture
def qwen_mlp_restored(monkeypatch):
    from transformers.models.qwen2 import modeling_qwen2

    monkeypatch.setattr(modeling_qwen2.Qwen2MLP, "forward", modeling_qwen2.Qwen2MLP.forward)
    return modeling_qwen2.Qwen2MLP


@pytest.mark.parametrize("recompute", [True, False])
def test_mlp_patch_routes_fp32_input(recompute, bnb, gpu_everywhere, qwen_mlp_restored, monkeypatch):
    """An fp32 input on fp16-compute NF4 projections with SiLU goes to the fused MLP: the
    reference's RecomputedMLP(x, gate_proj, up_proj, down_proj) with recompute, FusedMLP with the
    module weights otherwise."""
    rec_r, rec_f = Recorder(64), Recorder(64)
    monkeypatch.setattr(mlp.RecomputedMLP, "apply", rec_r)
    monkeypatch.setattr(mlp.FusedMLP, "apply", rec_f)
    mlp.patch(recompute=recompute)
    m = standin_bnb.qwen2_mlp(64, 128, lambda o, i: _linear(bnb.nn.Linear4bit, o, i, seed=o + i))
    x = torch.randn(2, 3, 64)
    m(x)
    if recompute:
        assert len(rec_r.calls) == 1 and not rec_f.calls
        args = rec_r.calls[0]
        assert args[0] is x and args[1] is m.gate_proj and args[2] is m.up_proj and args[3] is m.down_proj
    else:
        assert len(rec_f.calls) == 1 and not rec_r.calls
        args = rec_f.calls[0]
        assert args[1].data_ptr() == m.gate_proj.weight.data_ptr() and args[2] is m.gate_proj.weight.quant_state
        assert args[7] is False
    assert bnb.nn.Linear4bit.original_calls == 0


@pytest.mark.parametrize("case", ["fp16_input", "gelu", "fp32_compute", "cpu", "width", "empty"])
def test_mlp_patch_falls_back(case, bnb, qwen_mlp_restored, monkeypatch):
    """Anything outside the reference's conditions keeps transformers' own forward (whose
    projections are then bitsandbytes' own forwards here)."""
    rec_r, rec_f = Recorder(64), Recorder(64)
    monkeypatch.setattr(mlp.RecomputedMLP, "apply", rec_r)
    monkeypatch.setattr(mlp.FusedMLP, "apply", rec_f)
    if case != "cpu":
        monkeypatch.setattr(_state, "on_gpu", lambda t: True)
    mlp.patch(recompute=True)
    act = "gelu" if case == "gelu" else "silu"
    cdt = torch.float32 if case == "fp32_compute" else torch.float16
    m = standin_bnb.qwen2_mlp(64, 128, lambda o, i: _linear(bnb.nn.Linear4bit, o, i, compute_dtype=cdt),
                              hidden_act=act)
    x = torch.randn(4, 64)
    if case == "fp16_input":
        x = x.half()
    if case == "width":
        m.down_proj = _linear(bnb.nn.Linear4bit, 64, 96)  # down's input width is not gate's rows
    if case == "empty":
        x = torch.randn(0, 64)
    m(x)
    assert not rec_r.calls and not rec_f.calls
    assert bnb.nn.Linear4bit.original_calls >= 1


def test_mlp_patch_is_idempotent(bnb, qwen_mlp_restored):
    mlp.patch(recompute=True)
    first = qwen_mlp_restored.forward
    assert getattr(first, "_skc", False)
    mlp.patch(recompute=False)
    assert qwen_mlp_restored.forward is first


def test_solution_apply_installs_both_patches(bnb, qwen_mlp_restored, monkeypatch):
    """solution.apply() with bitsandbytes present installs the Linear4bit and Qwen2MLP patches
    (solution/__init__.py:30-51); SKC_NF4=0 / SKC_MLP=0 leave them out."""
    import importlib.util

    import solution

    real_find = importlib.util.find_spec
    monkeypatch.setattr(importlib.util, "find_spec",
                        lambda name, *a: object() if name == "bitsandbytes" else real_find(name, *a))
    monkeypatch.setenv("SKC_WARMUP", "0")
    monkeypatch.setenv("SKC_MLP", "0")
    solution.apply()
    assert getattr(bnb.nn.Linear4bit.forward, "_skc", False)
    assert not getattr(qwen_mlp_restored.forward, "_skc", False)
    monkeypatch.setenv("SKC_MLP", "1")
    solution.apply()
    assert getattr(qwen_mlp_restored.forward, "_skc", False)


def test_reference_mlp_names(bnb):
    """solution.mlp keeps the reference's helper names (solution/mlp.py:28-39, 62)."""
    import inspect

    import solution.mlp as smlp

    for name in ("_weight16", "_linear16_with", "_linear16", "RecomputedMLP", "patch"):
        assert hasattr(smlp, name), name
    params = list(inspect.signature(smlp.RecomputedMLP.forward).parameters)
    assert params == ["ctx", "x", "gate_proj", "up_proj", "down_proj", "norm_input", "norm_weight",
                      "eps", "norm_delta"]
    import solution.attn as sattn

    params = list(inspect.signature(sattn.LoRAPairFromNorm.forward).parameters)
    assert params[:5] == ["ctx", "x", "h", "norm_weight", "eps"] and params[-1] == "packed"
    assert len(params) == 20
