"""bitsandbytes-layout NF4 weights without bitsandbytes: a QuantState stand-in and a quantizer.

The kernels read the fields that the reference reads from bitsandbytes' QuantState
(solution/nf4.py:54-58, 70-79): quant_type, dtype, shape, blocksize, code, nested, absmax,
offset, state2.{absmax, code, blocksize}. Real bitsandbytes QuantStates work unchanged; this
module builds equivalent ones so that tests and benchmarks need no bitsandbytes.

`quantize_nf4` follows bitsandbytes 0.50.2 `quantize_4bit(..., quant_type="nf4")` with
`compress_statistics=True` (double quant): block absmax over `blocksize` flat elements, x/absmax
mapped to the nearest NF4 code (midpoint thresholds), two codes per byte with the even element in
the high nibble; offset = mean(absmax), absmax - offset quantized blockwise (256) to the nearest
value of the signed 8-bit dynamic map. bitsandbytes is not installed here, so byte-for-byte
agreement with its quantizer is not verified (its dequantization is: the kernels take these bytes
as inputs).
"""

from dataclasses import dataclass
from typing import Optional

import torch

NF4_CODE = [
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0]


@dataclass
class State2:
    absmax: torch.Tensor      # fp32 [ceil(n_blocks / blocksize)]
    code: torch.Tensor        # fp32 [256]
    blocksize: int = 256


@dataclass
class QuantState:
    """Duck type of bitsandbytes.functional.QuantState (the fields the path reads)."""
    absmax: torch.Tensor                  # nested: uint8 [n_blocks]; plain: fp32 [n_blocks]
    shape: tuple
    code: torch.Tensor                    # fp32 [16]
    blocksize: int = 64
    quant_type: str = "nf4"
    dtype: torch.dtype = torch.float16
    offset: Optional[torch.Tensor] = None  # fp32 0-d (nested)
    state2: Optional[State2] = None

    @property
    def nested(self):
        return self.state2 is not None

    def to(self, device):
        s2 = None if self.state2 is None else State2(self.state2.absmax.to(device),
                                                      self.state2.code.to(device),
                                                      self.state2.blocksize)
        return QuantState(self.absmax.to(device), self.shape, self.code.to(device),
                          self.blocksize, self.quant_type, self.dtype,
                          None if self.offset is None else self.offset.to(device), s2)


def dynamic_map_signed(device=None):
    """bitsandbytes create_dynamic_map(signed=True): 256 sorted fp32 values."""
    data = []
    for i in range(7):
        items = 2 ** i + 1
        bounds = torch.linspace(0.1, 1, items, dtype=torch.float32)
        means = (bounds[:-1] + bounds[1:]) / 2.0
        data += ((10 ** (-6 + i)) * means).tolist()
        data += (-(10 ** (-6 + i)) * means).tolist()
    data += [0.0, 1.0]
    data.sort()
    return torch.tensor(data, dtype=torch.float32, device=device)


def _block_absmax(a, blocksize):
    n = a.numel()
    n_blocks = -(-n // blocksize)
    padded = torch.zeros(n_blocks * blocksize, dtype=torch.float32, device=a.device)
    padded[:n] = a
    blocks = padded.view(n_blocks, blocksize)
    absmax = blocks.abs().amax(dim=1)
    inv = torch.where(absmax > 0, 1.0 / absmax, torch.zeros_like(absmax))
    return absmax, blocks * inv[:, None]


@torch.no_grad()
def quantize_nf4(w, blocksize=64, compress_statistics=True, blocksize2=256):
    """(packed uint8 [n*k/2, 1], QuantState) of an fp16 [n, k] weight, on w's device."""
    assert w.dim() == 2 and w.numel() % 2 == 0
    dev = w.device
    a = w.detach().to(torch.float32).reshape(-1)
    absmax, normed = _block_absmax(a, blocksize)
    code = torch.tensor(NF4_CODE, dtype=torch.float32, device=dev)
    thresholds = ((code[:-1].double() + code[1:].double()) / 2).float()
    idx = torch.searchsorted(thresholds, normed.reshape(-1).contiguous(), right=False)
    idx = idx[: a.numel()].to(torch.uint8)
    packed = ((idx[0::2] << 4) | idx[1::2]).to(torch.uint8).reshape(-1, 1)
    if not compress_statistics:
        return packed, QuantState(absmax=absmax.contiguous(), shape=tuple(w.shape), code=code,
                                  blocksize=blocksize)
    offset = absmax.double().mean().float()
    centred = absmax - offset
    code2 = dynamic_map_signed(dev)
    absmax2, normed2 = _block_absmax(centred, blocksize2)
    flat = normed2.reshape(-1)[: centred.numel()].contiguous()
    hi = torch.searchsorted(code2, flat, right=False).clamp(1, 255)
    lo = hi - 1
    pick_hi = (code2[hi] - flat).abs() < (flat - code2[lo]).abs()
    q8 = torch.where(pick_hi, hi, lo).to(torch.uint8)
    state = QuantState(absmax=q8.contiguous(), shape=tuple(w.shape), code=code,
                       blocksize=blocksize, offset=offset.reshape(()),
                       state2=State2(absmax2.contiguous(), code2, blocksize2))
    return packed, state


def from_arrays(packed, absmax, absmax2, code2, offset, code, shape, blocksize=64, blocksize2=256,
                nested=True, device=None):
    """QuantState + packed tensor from raw arrays (e.g. the golden fixtures)."""
    t = lambda x, dt: torch.as_tensor(x).to(device=device, dtype=dt).contiguous()  # noqa: E731
    packed_t = t(packed, torch.uint8).reshape(-1, 1)
    if nested:
        st = QuantState(absmax=t(absmax, torch.uint8), shape=tuple(shape), code=t(code, torch.float32),
                        blocksize=blocksize, offset=t(offset, torch.float32).reshape(()),
                        state2=State2(t(absmax2, torch.float32), t(code2, torch.float32), blocksize2))
    else:
        st = QuantState(absmax=t(absmax, torch.float32), shape=tuple(shape),
                        code=t(code, torch.float32), blocksize=blocksize)
    return packed_t, st
