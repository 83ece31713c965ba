"""CPU oracle for the NF4 quantized-linear path.

TEST INFRASTRUCTURE ONLY. Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py` may import this package, and only to produce expected results (bench.py also times
it as the CPU baseline). The product path (`decik_amd`, `solution`) never imports it and has no CPU fallback.

Contents (each function cites the reference file:line it restates):
- `nf4.py`   bit-exact NF4 dequantization (C library `nf4_oracle.c`, built by `Makefile`),
             a numpy restatement of the bitsandbytes NF4 / double-quant quantizer, and fp32
             references for the linear, LoRA and SwiGLU/MLP computations.

Parity status (what pins each function) is listed in the module docstring of `nf4.py`.
"""
