"""ctypes binding of libdecik_nf4.so (include/decik_nf4.h) and the tensor -> descriptor glue.

The library is built in-tree by `python -m decik_amd.build` (or __graft_entry__.build()). There
is no fallback: every entry point raises if the library is missing or returns an error.
"""

import ctypes
import os
import threading
import weakref

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libdecik_nf4.so")
MAX_GROUPS = 4
# dk_nf4_linear_plan flags and kernel ids (include/decik_nf4.h)
PLAN_GLU, PLAN_LORA, PLAN_NO_SPLIT, PLAN_NESTED, PLAN_PARTS = 1, 2, 4, 8, 16
# dk_nf4_linear_plan's kernel ids (2, an earlier input-gradient kernel, is no longer returned)
PLAN_KERNELS = ("nf4_fwd_kernel", "nf4_fwd8_kernel", "retired", "nf4_bwd8_kernel", "nf4_gemv_kernel",
                "nf4_skinny_kernel")

_lib = None
_lock = threading.Lock()

c_i64, c_i32, c_vp, c_f32 = ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p, ctypes.c_float


class NF4Weight(ctypes.Structure):
    _fields_ = [("packed", c_vp), ("absmax", c_vp), ("absmax2", c_vp), ("code2", c_vp),
                ("offset", c_vp), ("code", c_vp), ("n", c_i64), ("k", c_i64),
                ("blocksize", c_i32), ("blocksize2", c_i32), ("nested", c_i32),
                ("reserved", c_i32)]


class LinearFwdGroup(ctypes.Structure):
    _fields_ = [("w", NF4Weight), ("bias", c_vp), ("lora_u", c_vp), ("lora_b", c_vp),
                ("lora_scale", c_f32), ("reserved", c_i32), ("y", c_vp), ("ldy", c_i64)]


class LinearBwdGroup(ctypes.Structure):
    _fields_ = [("w", NF4Weight), ("dy", c_vp), ("lddy", c_i64), ("lora_gu", c_vp),
                ("lora_a", c_vp), ("lora_keep", c_vp), ("lora_keep_scale", ctypes.c_float),
                ("reserved", c_i32)]


class LoraBranch(ctypes.Structure):
    """dk_lora_branch: one adapter of a grouped LoRA call (dk_lora_down_group, dk_lora_bwd_group)."""
    _fields_ = [("x", c_vp), ("keep_bits", c_vp), ("keep_scale", c_vp), ("a", c_vp), ("u", c_vp),
                ("dy", c_vp), ("b", c_vp), ("gu", c_vp), ("da", c_vp), ("db", c_vp),
                ("ldx", c_i64), ("lddy", c_i64), ("n", c_i64), ("scale", c_f32), ("x_fp32", c_i32)]


EXPORTS = {
    "dk_nf4_dequant": ([ctypes.POINTER(NF4Weight), c_vp, c_vp], c_i32),
    "dk_nf4_dequant_batched": ([ctypes.POINTER(NF4Weight), ctypes.POINTER(c_vp), c_i32, c_vp], c_i32),
    "dk_probe_mfma_f16": ([ctypes.c_int64, ctypes.c_int32, c_vp, c_vp], c_i32),
    "dk_probe_hbm": ([c_vp, c_vp, c_i64, c_i32, c_vp, c_vp], c_i32),
    "dk_nf4_linear_plan": ([c_i32, c_i64, c_i64, ctypes.POINTER(c_i64), c_i32, c_i32, c_i32,
                            ctypes.POINTER(ctypes.c_int32)], c_i32),
    "dk_nf4_block_scales": ([ctypes.POINTER(NF4Weight), c_vp, c_vp], c_i32),
    "dk_nf4_linear_fwd_workspace": ([c_i64, c_i64, ctypes.POINTER(c_i64), c_i32], c_i64),
    "dk_nf4_linear_fwd": ([c_vp, c_i64, c_i64, c_i64, ctypes.POINTER(LinearFwdGroup), c_i32, c_i32,
                           c_vp, c_i64, c_vp], c_i32),
    "dk_nf4_linear_bwd_workspace": ([c_i64, c_i64, ctypes.POINTER(c_i64), c_i32], c_i64),
    "dk_nf4_linear_bwd": ([ctypes.POINTER(LinearBwdGroup), c_i32, c_i64, c_i64, c_vp, c_i64, c_i32,
                           c_i32, c_vp, c_i64, c_vp], c_i32),
    "dk_nf4_linear_rope_fwd_workspace": ([c_i64, c_i64, ctypes.POINTER(c_i64), c_i32], c_i64),
    "dk_nf4_linear_rope_fwd": ([c_vp, c_i64, c_i64, c_i64, ctypes.POINTER(LinearFwdGroup), c_i32, c_i32, c_vp,
                                c_vp, c_i32, c_i32, ctypes.POINTER(c_vp), c_vp, c_i64, c_vp], c_i32),
    "dk_nf4_linear_bwd_noalloc": ([ctypes.POINTER(LinearBwdGroup), c_i32, c_i64, c_i64, c_vp, c_i64, c_i32,
                                   c_i32, c_vp], c_i32),
    "dk_nf4_glu_fwd": ([c_vp, c_i64, c_i64, c_i64, ctypes.POINTER(LinearFwdGroup), c_i32, c_vp, c_i64,
                        c_vp], c_i32),
    "dk_nf4_linear_bwd_swiglu": ([ctypes.POINTER(LinearBwdGroup), c_i64, c_i64, c_i32, c_vp, c_vp, c_i64,
                                  c_vp, c_vp, c_i64, c_vp], c_i32),
    "dk_lora_down": ([c_vp, c_i64, c_i64, c_i64, c_vp, c_i32, c_vp, c_vp], c_i32),
    "dk_lora_down_dropout": ([c_vp, c_i32, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_i32, c_vp, c_vp], c_i32),
    "dk_lora_bwd_dropout": ([c_vp, c_i64, c_vp, c_vp, c_i32, c_i64, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i32,
                             c_f32, c_vp, c_vp, c_vp, c_vp], c_i32),
    "dk_lora_bwd": ([c_vp, c_i64, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_i64, c_i32, c_f32, c_vp,
                     c_vp, c_vp, c_vp], c_i32),
    "dk_lora_down_group": ([ctypes.POINTER(LoraBranch), c_i32, c_i64, c_i64, c_i32, c_vp], c_i32),
    "dk_lora_bwd_group": ([ctypes.POINTER(LoraBranch), c_i32, c_i64, c_i64, c_i32, c_vp], c_i32),
    "dk_lora_keep_pack": ([c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_vp], c_i32),
    "dk_lora_dropout_inputs": ([c_vp, c_i32, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_vp], c_i32),
    "dk_lora_input_grad": ([c_vp, c_vp, c_vp, c_vp, c_f32, c_f32, c_vp, c_i64, c_i64, c_vp], c_i32),
    "dk_lora_up": ([c_vp, c_vp, c_i32, c_vp, c_i64, c_i64, c_vp], c_i32),
    "dk_rope_qk_fwd": ([c_vp, c_vp, c_i64, c_i64, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_i64, c_i32, c_i32,
                        c_i32, c_vp], c_i32),
    "dk_rope_qk_bwd": ([c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_i64, c_i32, c_i32, c_i32, c_vp],
                       c_i32),
    "dk_swiglu_fwd": ([c_vp, c_vp, c_vp, c_i64, c_vp], c_i32),
    "dk_swiglu_bwd": ([c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_vp], c_i32),
    "dk_last_error": ([], ctypes.c_char_p),
    "dk_version": ([], c_i32),
}


class DecikError(RuntimeError):
    pass


def lib():
    """The loaded library (raises DecikError if it was not built)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise DecikError(f"{LIB_PATH} is missing: build it with `python -m decik_amd.build`")
                L = ctypes.CDLL(LIB_PATH)
                for name, (args, res) in EXPORTS.items():
                    fn = getattr(L, name)
                    fn.argtypes = args
                    fn.restype = res
                _lib = L
    return _lib


def check(rc):
    if rc != 0:
        raise DecikError(lib().dk_last_error().decode())


_raw_stream = torch._C._cuda_getCurrentRawStream


def raw_stream(device):
    """The current HIP stream of `device` as an integer handle (what torch.cuda.current_stream(
    device).cuda_stream returns, without building a Stream object on every call)."""
    idx = device.index
    return _raw_stream(torch.cuda.current_device() if idx is None else idx)


def stream_of(device):
    return ctypes.c_void_p(raw_stream(device))


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def weight_desc(packed, qs, device, scales=None):
    """NF4Weight of a packed uint8 tensor and its QuantState (fields of solution/nf4.py:70-79).
    With `scales` (fp32 block scales from dk_nf4_block_scales), a nested weight is described as
    plain with those scales: the same dequantized bits, a shorter path in the fused GEMMs."""
    n, k = (int(s) for s in qs.shape)
    code = qs.code if qs.code.device == device else qs.code.to(device)
    w = NF4Weight()
    w.packed = packed.data_ptr()
    w.code = code.data_ptr()
    w.n, w.k = n, k
    w.blocksize = int(qs.blocksize)
    w.nested = 1 if qs.nested else 0
    keep = [packed, code]
    if scales is not None:
        w.nested = 0
        w.absmax = scales.data_ptr()
        w.blocksize2 = 256
        keep.append(scales)
    elif qs.nested:
        w.absmax = qs.absmax.data_ptr()
        w.absmax2 = qs.state2.absmax.data_ptr()
        w.code2 = qs.state2.code.data_ptr()
        offset = qs.offset
        if not torch.is_tensor(offset):
            offset = torch.tensor(float(offset), dtype=torch.float32, device=device)
        w.offset = offset.data_ptr()
        w.blocksize2 = int(qs.state2.blocksize)
        keep += [qs.absmax, qs.state2.absmax, qs.state2.code, offset]
    else:
        w.absmax = qs.absmax.data_ptr()
        w.blocksize2 = 256
        keep.append(qs.absmax)
    return w, keep


def _stats(qs):
    """The statistics tensors (and scalars) a QuantState's block scales are computed from."""
    if qs.nested:
        s2 = qs.state2
        return (qs.absmax, s2.absmax, s2.code, qs.offset)
    return (qs.absmax,)


def _version_key(qs):
    """What the block scales of a nested QuantState depend on: identity and in-place version of
    each statistics tensor (the cache entry keeps the tensors alive, so an identity is never
    reused while it is compared), the offset and the block sizes."""
    key = [int(qs.blocksize), tuple(qs.shape)]
    for t in _stats(qs):
        if isinstance(t, torch.Tensor):
            key += (id(t), t._version)
        else:
            key.append(float(t))
    if qs.nested:
        key.append(int(qs.state2.blocksize))
    return tuple(key)


class ScaleCache:
    """fp32 block scales of nested weights (dk_nf4_block_scales), computed once per QuantState
    and reused while its statistics tensors are unchanged (a frozen QLoRA base weight). An
    in-place change of any statistics tensor bumps its version and forces a recomputation; the
    entry goes away with the QuantState."""

    def __init__(self):
        self._d = {}
        self._lock = threading.Lock()

    def get(self, packed, qs, device):
        key, ver = id(qs), _version_key(qs)
        with self._lock:
            ent = self._d.get(key)
        if ent is not None and ent[0] == ver and ent[2]() is qs:
            return ent[1]
        n, k = (int(s) for s in qs.shape)
        nblocks = (n * k + int(qs.blocksize) - 1) // int(qs.blocksize)
        scales = torch.empty(max(nblocks, 1), dtype=torch.float32, device=device)
        w, keep = weight_desc(packed, qs, device)
        check(lib().dk_nf4_block_scales(ctypes.byref(w), scales.data_ptr(), stream_of(device)))
        del keep

        def drop(_ref, key=key):
            with self._lock:
                self._d.pop(key, None)

        with self._lock:
            self._d[key] = (ver, scales, weakref.ref(qs, drop), _stats(qs))
        return scales


SCALES = ScaleCache()


class DescCache:
    """The NF4Weight descriptor the fused GEMMs take for a (packed, QuantState) pair -- with its
    statistics as stored or with the cached block scales of a nested weight -- built once and reused while it stays valid: the
    same packed tensor, statistics tensors and scales (compared by identity; the entry keeps them
    alive, so an identity is not reused meanwhile). An in-place change of the statistics leaves
    the descriptor's pointers valid; the scales cache notices it and hands out new scales, which
    rebuilds the descriptor. The check costs a few attribute reads, building the descriptor
    several times that."""

    def __init__(self):
        self._d = {}
        self._lock = threading.Lock()

    def get(self, packed, qs, device, scales_of=None):
        """(NF4Weight, tensors to keep alive). scales_of(packed, qs, device) gives the block
        scales to describe the weight with (None: its own statistics); default: the cached
        scales of a nested weight."""
        if scales_of is None:
            scales = SCALES.get(packed, qs, device) if qs.nested else None
        else:
            scales = scales_of(packed, qs, device)
        # one entry per weight and form (cached scales or its own statistics), so that calls
        # alternating between the two reuse both descriptors
        key = (id(qs), scales is None)
        ver = (id(packed), packed.data_ptr(), device.index, id(scales), id(qs.code), int(qs.blocksize),
               tuple(id(t) if isinstance(t, torch.Tensor) else float(t) for t in _stats(qs)))
        with self._lock:
            ent = self._d.get(key)
        if ent is not None and ent[0] == ver and ent[3]() is qs:
            return ent[1], ent[2]
        w, keep = weight_desc(packed, qs, device, scales)

        def drop(_ref, key=key):
            with self._lock:
                self._d.pop(key, None)

        with self._lock:
            self._d[key] = (ver, w, keep + [qs.code, scales, *_stats(qs)], weakref.ref(qs, drop))
        return w, keep


DESCS = DescCache()


class Workspace:
    """Split-K workspaces (fp32 partial slabs), one per (device, stream), grown on demand."""

    def __init__(self):
        self._bufs = {}
        self._lock = threading.Lock()

    def get(self, nbytes, device):
        if nbytes <= 0:
            return None, 0
        key = (device.index, raw_stream(device))
        with self._lock:
            buf = self._bufs.get(key)
            if buf is None or buf.numel() < nbytes:
                size = max(nbytes, 0 if buf is None else 2 * buf.numel())
                buf = torch.empty(size, dtype=torch.uint8, device=device)
                self._bufs[key] = buf
        return buf, buf.numel()


WORKSPACE = Workspace()
