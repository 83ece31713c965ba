"""bitsandbytes' serialized form of NF4 weights, read and written without bitsandbytes.

A quantized Linear4bit saves (bitsandbytes 0.50.2, `Params4bit` / `QuantState.as_dict(packed=True)`
and `QuantState.from_dict`, the format transformers writes to safetensors):
    <prefix>.weight                                      uint8 [N*K/2, 1]  packed codes
    <prefix>.weight.absmax                               uint8 (nested) or fp32 block absmax
    <prefix>.weight.quant_map                            fp32 [16]          code book
    <prefix>.weight.nested_absmax                        fp32               absmax2 (nested)
    <prefix>.weight.nested_quant_map                     fp32 [256]         code2 (nested)
    <prefix>.weight.quant_state.bitsandbytes__nf4        uint8              JSON of the scalars:
        {"quant_type", "blocksize", "dtype", "shape", and when nested "nested_blocksize",
         "nested_dtype", "nested_offset"}
These are exactly the QuantState fields the reference reads (solution/nf4.py:54-58, 70-79), so a
checkpoint loaded here feeds the kernels as its bytes stand. bitsandbytes itself is not installed,
so agreement with its serializer is PARITY UNPINNED: the key names and the JSON payload follow
its published 0.50.2 source, and the tests check round trips and the layout.
"""

import json

import torch

from .quant import QuantState, State2

_PACKED_KEY = "quant_state.bitsandbytes__"


def _dtype_name(dt):
    return str(dt).replace("torch.", "")


def _dtype_of(name):
    return getattr(torch, name)


def pack_dict_to_tensor(d):
    """JSON of the non-tensor QuantState fields as a uint8 tensor (bitsandbytes
    utils.pack_dict_to_tensor)."""
    return torch.tensor(list(json.dumps(d).encode("utf-8")), dtype=torch.uint8)


def unpack_tensor_to_dict(t):
    """Inverse of pack_dict_to_tensor."""
    return json.loads(bytes(t.to("cpu").to(torch.uint8).tolist()).decode("utf-8"))


def quant_state_as_dict(qs, packed=True):
    """QuantState.as_dict: tensors plus scalars; packed=True folds the scalars into one uint8
    tensor under 'quant_state.bitsandbytes__<quant_type>' (safetensors holds tensors only)."""
    d = {"quant_type": qs.quant_type, "absmax": qs.absmax, "blocksize": int(qs.blocksize),
         "quant_map": qs.code, "dtype": _dtype_name(qs.dtype), "shape": tuple(int(s) for s in qs.shape)}
    if qs.nested:
        d.update({"nested_absmax": qs.state2.absmax, "nested_blocksize": int(qs.state2.blocksize),
                  "nested_quant_map": qs.state2.code.clone(), "nested_dtype": "float32",
                  "nested_offset": float(qs.offset.item())})
    if not packed:
        return d
    out = {k: v for k, v in d.items() if isinstance(v, torch.Tensor)}
    scalars = {k: (list(v) if isinstance(v, tuple) else v) for k, v in d.items() if not isinstance(v, torch.Tensor)}
    out[_PACKED_KEY + qs.quant_type] = pack_dict_to_tensor(scalars)
    return out


def quant_state_from_dict(d, device=None):
    """QuantState.from_dict: accepts the packed or unpacked form (keys without the module
    prefix)."""
    d = dict(d)
    packed = [k for k in d if k.startswith(_PACKED_KEY)]
    if len(packed) > 1:
        raise ValueError(f"more than one packed quant_state entry: {packed}")
    if packed:
        d.update(unpack_tensor_to_dict(d.pop(packed[0])))
    for k in ("quant_type", "absmax", "blocksize", "quant_map", "dtype", "shape"):
        if k not in d:
            raise ValueError(f"quant_state is missing '{k}'")
    dev = device if device is not None else d["absmax"].device
    state2 = offset = None
    if "nested_absmax" in d:
        offset = torch.tensor(float(d["nested_offset"]), dtype=torch.float32, device=dev)
        state2 = State2(d["nested_absmax"].to(dev), d["nested_quant_map"].to(dev), int(d["nested_blocksize"]))
    return QuantState(absmax=d["absmax"].to(dev), shape=torch.Size(d["shape"]), code=d["quant_map"].to(dev),
                      blocksize=int(d["blocksize"]), quant_type=d["quant_type"], dtype=_dtype_of(d["dtype"]),
                      offset=offset, state2=state2)


def save_nf4_weight(state_dict, prefix, packed, qs):
    """Write one Linear4bit weight into `state_dict` under `prefix` (e.g.
    'model.layers.0.mlp.gate_proj') as bitsandbytes lays it out."""
    state_dict[prefix + ".weight"] = packed
    for k, v in quant_state_as_dict(qs, packed=True).items():
        state_dict[prefix + ".weight." + k] = v


def load_nf4_weight(state_dict, prefix, device=None):
    """(packed uint8 [N*K/2, 1], QuantState) of the Linear4bit weight under `prefix`."""
    head = prefix + ".weight."
    parts = {k[len(head):]: v for k, v in state_dict.items() if k.startswith(head)}
    if prefix + ".weight" not in state_dict or not parts:
        raise KeyError(f"no bitsandbytes nf4 weight under '{prefix}'")
    qs = quant_state_from_dict(parts, device)
    packed = state_dict[prefix + ".weight"]
    packed = packed.to(device) if device is not None else packed
    if packed.dtype != torch.uint8 or packed.numel() * 2 != qs.shape[0] * qs.shape[1]:
        raise ValueError(f"'{prefix}.weight' is not the packed nf4 bytes of shape {tuple(qs.shape)}")
    return packed, qs


def nf4_prefixes(state_dict):
    """Module prefixes of every nf4 weight in a state dict."""
    tail = ".weight." + _PACKED_KEY + "nf4"
    return sorted(k[: -len(tail)] for k in state_dict if k.endswith(tail))


def load_nf4_checkpoint(path, device=None, prefixes=None):
    """{prefix: (packed, QuantState)} of the nf4 weights in a local checkpoint: one safetensors
    file, or a directory of them (sharded with 'model.safetensors.index.json' or not), as
    transformers saves a bitsandbytes-quantized model. Only the nf4 tensors are read."""
    import os

    from safetensors import safe_open

    if os.path.isdir(path):
        files = sorted(os.path.join(path, f) for f in os.listdir(path) if f.endswith(".safetensors"))
    else:
        files = [path]
    if not files:
        raise FileNotFoundError(f"no .safetensors files under '{path}'")
    where = {}
    for f in files:
        with safe_open(f, framework="pt") as h:
            for k in h.keys():
                where[k] = f
    want = nf4_prefixes(where) if prefixes is None else list(prefixes)
    sd = {}
    for f in files:
        with safe_open(f, framework="pt") as h:
            for k in h.keys():
                if any(k == p + ".weight" or k.startswith(p + ".weight.") for p in want):
                    sd[k] = h.get_tensor(k)
    return {p: load_nf4_weight(sd, p, device) for p in want}
