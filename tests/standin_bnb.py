"""A stand-in `bitsandbytes` package for the patch tests (bitsandbytes is not installed here).

It has what the patches touch (solution/nf4.py:107-138, solution/mlp.py:113-162):
`bitsandbytes.nn.Linear4bit` (a module with a uint8 `weight` carrying `quant_state`, `bias`,
`compute_dtype`) whose own forward only records that it ran, and
`bitsandbytes.nn.modules.fix_4bit_weight_quant_state_from_module`, which restores a weight's
quant_state from the module. `install(monkeypatch)` puts it into sys.modules for one test.
"""

import sys
import types

import torch


class Linear4bit(torch.nn.Module):
    """Linear4bit's fields as the patches read them. `forward` is bitsandbytes' own path: here it
    records the call and returns a marker tensor, so a test sees which path ran."""

    original_calls = 0

    def __init__(self, packed, quant_state, bias=None, compute_dtype=torch.float16):
        super().__init__()
        self.weight = torch.nn.Parameter(packed, requires_grad=False)
        self.weight.quant_state = quant_state
        self.quant_state_backup = quant_state
        self.bias = None if bias is None else torch.nn.Parameter(bias, requires_grad=False)
        self.compute_dtype = compute_dtype
        self.out_features = int(quant_state.shape[0])

    def forward(self, x):
        type(self).original_calls += 1
        return torch.full(x.shape[:-1] + (self.out_features,), -7.0, dtype=x.dtype, device=x.device)


def fix_4bit_weight_quant_state_from_module(module):
    module.weight.quant_state = module.quant_state_backup


def install(monkeypatch):
    """A fresh stand-in package (a new Linear4bit class, so patches do not leak between tests)."""
    cls = type("Linear4bit", (Linear4bit,), {"original_calls": 0, "forward": Linear4bit.forward})
    bnb = types.ModuleType("bitsandbytes")
    nn = types.ModuleType("bitsandbytes.nn")
    modules = types.ModuleType("bitsandbytes.nn.modules")
    nn.Linear4bit = cls
    nn.modules = modules
    modules.Linear4bit = cls
    modules.fix_4bit_weight_quant_state_from_module = fix_4bit_weight_quant_state_from_module
    bnb.nn = nn
    for name, mod in (("bitsandbytes", bnb), ("bitsandbytes.nn", nn), ("bitsandbytes.nn.modules", modules)):
        monkeypatch.setitem(sys.modules, name, mod)
    return bnb


def qwen2_mlp(hidden, intermediate, make_linear, hidden_act="silu"):
    """transformers' Qwen2MLP with its three projections replaced by make_linear(n_out, n_in)."""
    from transformers import Qwen2Config
    from transformers.models.qwen2 import modeling_qwen2

    cfg = Qwen2Config(hidden_size=hidden, intermediate_size=intermediate, hidden_act=hidden_act,
                      num_attention_heads=2, num_key_value_heads=1, num_hidden_layers=1,
                      vocab_size=32)
    mlp = modeling_qwen2.Qwen2MLP(cfg)
    mlp.gate_proj = make_linear(intermediate, hidden)
    mlp.up_proj = make_linear(intermediate, hidden)
    mlp.down_proj = make_linear(hidden, intermediate)
    return mlp
