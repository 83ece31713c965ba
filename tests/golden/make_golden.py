"""Writes tests/golden/nf4_dequant.npz: NF4 dequant input/output vectors made by the oracle.

Inputs are seeded synthetic weights quantized by the oracle's quantizer; expected outputs are the
oracle's bit-exact dequantization (uint16 fp16 bit patterns). Shapes follow the reference's own
dequant tests (dev/test_cpu_kernels.py:28, weights randn * 0.05) plus cases whose 64-blocks and
256-groups straddle row ends. Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import nf4 as O  # noqa: E402

CASES = [
    ("cpu96x128_nested", (96, 128), True, 64, 256),
    ("cpu96x128_plain", (96, 128), False, 64, 256),
    ("cpu32x2560_nested", (32, 2560), True, 64, 256),
    ("straddle3x40_nested", (3, 40), True, 64, 256),
    ("straddle10x96_nested_bs2_2", (10, 96), True, 64, 2),
    ("odd7x10_plain_bs32", (7, 10), False, 32, 256),
]


def main():
    rng = np.random.default_rng(20240601)
    arrays = {}
    for name, shape, nested, bs, bs2 in CASES:
        w = (rng.standard_normal(shape) * 0.05).astype(np.float16)
        q = O.quantize_nf4(w, blocksize=bs, nested=nested, blocksize2=bs2)
        out = O.dequant_nf4(q).reshape(-1).view(np.uint16)
        arrays[f"{name}/packed"] = q.packed
        arrays[f"{name}/absmax"] = q.absmax
        arrays[f"{name}/absmax2"] = q.absmax2
        arrays[f"{name}/code2"] = q.code2
        arrays[f"{name}/offset"] = np.array([q.offset], np.float32)
        arrays[f"{name}/code"] = q.code
        arrays[f"{name}/meta"] = np.array([shape[0], shape[1], bs, bs2, int(nested)], np.int64)
        arrays[f"{name}/expected"] = out
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "nf4_dequant.npz")
    np.savez_compressed(path, **arrays)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
