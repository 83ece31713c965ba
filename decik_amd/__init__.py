"""decik_amd: the NF4 quantized-linear path of tokha-t/decik, rebuilt for MI355X (gfx950).

Hand-written HIP kernels (decik_amd/csrc, C ABI in include/decik_nf4.h) behind the reference's
Python API (the `solution` package name is kept as an alias, see solution/__init__.py):
- nf4.py     NF4 dequantization (bit-exact) and the fused dequant x fp16 GEMM linear
- mlp.py     Qwen2 MLP: gate+up in one fused launch, SwiGLU, down; fused backward
- lora.py    LoRA r=16 with the A.B term fused into the GEMM epilogues; q/k/v in one launch
- swiglu.py  SwiGLU forward/backward kernels
- quant.py   bitsandbytes-layout NF4 quantizer and QuantState stand-in (no bitsandbytes needed)

apply() installs the patches the reference installs for this path (solution/__init__.py:30-51):
bitsandbytes' Linear4bit.forward and transformers' Qwen2MLP.forward. The reference's other
patches (RMSNorm, fused head, padding-free attention, RoPE, embedding) are outside this path and
are not provided. SKC_<NAME>=0 turns a part off, as in the reference.
"""

import os


def _enabled(name):
    return os.environ.get(f"SKC_{name}", "1") != "0"


def apply():
    import importlib.util

    import torch

    from . import mlp, nf4, warmup

    if _enabled("WARMUP") and torch.cuda.is_available():
        warmup.start()
    have_bnb = importlib.util.find_spec("bitsandbytes") is not None
    if not have_bnb:
        # Nothing to patch: Linear4bit only exists with bitsandbytes installed.
        return
    if _enabled("NF4"):
        nf4.patch()
    if _enabled("MLP") and importlib.util.find_spec("transformers") is not None:
        mlp.patch(recompute=os.environ.get("SKC_RECOMPUTE", "1") == "1")
