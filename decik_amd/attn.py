"""The NF4-path pieces of the reference's attention module (solution/attn.py) under its names:
RoPE of q/k (FusedQKRope, solution/attn.py:89-126) and the LoRA dropout helpers (pack_keep,
_lora_inputs, solution/attn.py:183-203) and LoRAPairFromNorm (solution/attn.py:206-273, same
`apply` signature), backed by this package's HIP kernels."""

from .lora import LoRAPair, LoRAPairFromNorm, lora_input_grad, lora_inputs, pack_keep  # noqa: F401
from .rope import FusedQKRope, rope_qk_backward, rope_qk_forward  # noqa: F401


def _lora_inputs(x, bits_q, bits_v, scale_q, scale_v):
    """fp16(x * dropout values) of the q and v branches, [T, W] each (solution/attn.py:183-192)."""
    return lora_inputs(x, bits_q, bits_v, scale_q, scale_v)
