"""Drop-in name for the reference's package (tokha-t/decik `solution/`).

`import solution; solution.apply()` and `from solution.nf4 import dequantize_nf4` keep working:
the modules are decik_amd's, registered under the reference's names."""

import sys

import decik_amd as _impl
from decik_amd import _state, _enabled, apply, attn, lora, mlp, nf4, rope, swiglu, warmup  # noqa: F401

for _name in ("nf4", "mlp", "swiglu", "warmup", "_state", "lora", "attn", "rope"):
    sys.modules[f"{__name__}.{_name}"] = getattr(_impl, _name)
