"""Shared helpers for the tests: seeded NF4 weights on the GPU plus their oracle twins."""

import os

import numpy as np
import torch

from oracle import nf4 as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "nf4_dequant.npz")


def golden_cases():
    z = np.load(GOLDEN, allow_pickle=False)
    names = sorted({k.split("/")[0] for k in z.files})
    out = {}
    for n in names:
        meta = z[f"{n}/meta"]
        out[n] = dict(packed=z[f"{n}/packed"], absmax=z[f"{n}/absmax"], absmax2=z[f"{n}/absmax2"],
                      code2=z[f"{n}/code2"], offset=z[f"{n}/offset"][0], code=z[f"{n}/code"],
                      shape=(int(meta[0]), int(meta[1])), blocksize=int(meta[2]),
                      blocksize2=int(meta[3]), nested=bool(meta[4]), expected=z[f"{n}/expected"])
    return out


def oracle_state(packed, qs):
    """The oracle's QuantNF4 holding the same bytes and statistics as (packed, qs)."""
    cpu = lambda t: t.detach().cpu().numpy()  # noqa: E731
    if qs.nested:
        return O.QuantNF4(cpu(packed).reshape(-1), cpu(qs.absmax), cpu(qs.state2.absmax),
                          cpu(qs.state2.code), np.float32(cpu(qs.offset)), cpu(qs.code),
                          tuple(int(s) for s in qs.shape), int(qs.blocksize),
                          int(qs.state2.blocksize), True)
    return O.QuantNF4(cpu(packed).reshape(-1), cpu(qs.absmax), np.zeros(0, np.float32),
                      np.zeros(0, np.float32), np.float32(0), cpu(qs.code),
                      tuple(int(s) for s in qs.shape), int(qs.blocksize), 256, False)


def make_weight(shape, seed, device, nested=True, std=0.02, blocksize=64):
    """Seeded fp16 N(0, std) weight quantized on `device`; returns (packed, qs, w16_oracle) where
    w16_oracle is the oracle's bit-exact fp16 dequantization (numpy)."""
    from decik_amd.quant import quantize_nf4

    g = torch.Generator(device="cpu").manual_seed(seed)
    w = (torch.randn(shape, generator=g) * std).to(torch.float16).to(device)
    packed, qs = quantize_nf4(w, blocksize=blocksize, compress_statistics=nested)
    return packed, qs, O.dequant_nf4(oracle_state(packed, qs), nthreads=0)


def randn16(shape, seed, device, std=1.0):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(torch.float16).to(device)


def assert_close(y, ref, max_rel=1e-2, mean_rel=1e-3, what=""):
    """The parity bar: max|y-ref| <= 1e-2 max|ref| and sum|y-ref| / sum|ref| <= 1e-3."""
    y = y.detach().float().cpu().numpy() if torch.is_tensor(y) else y
    mx, mean = O.tolerance(y, ref)
    assert mx <= max_rel and mean <= mean_rel, f"{what}: max_rel={mx:.3e} mean_rel={mean:.3e}"
    return mx, mean
