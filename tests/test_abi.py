"""The C ABI (include/decik_nf4.h) without a GPU: the built library exports every declared
entry point, the ctypes mirrors have the C layout, and argument errors come back as codes with
a message (validation runs before any GPU call)."""

import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "decik_nf4.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(dk_\w+)\s*\(", text, re.M)))


def test_header_declares_the_path():
    names = declared()
    for n in ["dk_nf4_dequant", "dk_nf4_dequant_batched", "dk_nf4_linear_fwd", "dk_nf4_linear_bwd",
              "dk_nf4_linear_fwd_workspace", "dk_nf4_linear_bwd_workspace", "dk_lora_down",
              "dk_lora_bwd", "dk_swiglu_fwd", "dk_swiglu_bwd", "dk_last_error", "dk_version"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    from decik_amd import _lib

    L = _lib.lib()
    for n in declared():
        assert hasattr(L, n), n
    assert set(declared()) == set(_lib.EXPORTS)


def test_struct_layout_matches_c(tmp_path):
    """sizeof/offsetof from the C compiler vs the ctypes mirrors."""
    from decik_amd import _lib

    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "decik_nf4.h"\n'
                   "int main(void){printf(\"%zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu %zu\\n\","
                   "sizeof(dk_nf4_weight), offsetof(dk_nf4_weight, n), offsetof(dk_nf4_weight, nested),"
                   "sizeof(dk_linear_fwd_group), offsetof(dk_linear_fwd_group, lora_scale),"
                   "offsetof(dk_linear_fwd_group, y), sizeof(dk_linear_bwd_group),"
                   "offsetof(dk_linear_bwd_group, lora_a), sizeof(dk_lora_branch),"
                   "offsetof(dk_lora_branch, ldx), offsetof(dk_lora_branch, scale),"
                   "offsetof(dk_lora_branch, x_fp32));return 0;}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.dirname(HEADER), "-o", str(exe), str(src)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True,
                                          check=True).stdout.split()]
    W, F, B, R = _lib.NF4Weight, _lib.LinearFwdGroup, _lib.LinearBwdGroup, _lib.LoraBranch
    want = [ctypes.sizeof(W), W.n.offset, W.nested.offset, ctypes.sizeof(F), F.lora_scale.offset,
            F.y.offset, ctypes.sizeof(B), B.lora_a.offset, ctypes.sizeof(R), R.ldx.offset, R.scale.offset,
            R.x_fp32.offset]
    assert got == want


def test_argument_errors_are_reported():
    from decik_amd import _lib

    L = _lib.lib()
    g = (_lib.LinearFwdGroup * 1)()
    # k not a multiple of 32: rejected before anything touches the GPU
    rc = L.dk_nf4_linear_fwd(ctypes.c_void_p(16), 8, 40, 40, g, 1, 0, None, 0, None)
    assert rc != 0 and b"multiple of 32" in L.dk_last_error()
    rc = L.dk_nf4_linear_fwd(ctypes.c_void_p(16), 8, 64, 64, g, 5, 0, None, 0, None)
    assert rc != 0 and b"1..4 groups" in L.dk_last_error()
    rc = L.dk_lora_down(ctypes.c_void_p(16), 8, 64, 64, ctypes.c_void_p(16), 8, ctypes.c_void_p(16), None)
    assert rc != 0 and b"rank" in L.dk_last_error()
    rc = L.dk_probe_hbm(ctypes.c_void_p(16), ctypes.c_void_p(16), 1024, 2 + 64, ctypes.c_void_p(16), None)
    assert rc != 0 and b"bad arguments" in L.dk_last_error()  # no such probe variant
    rc = L.dk_probe_hbm(ctypes.c_void_p(16), ctypes.c_void_p(16), 1024, 2 + 48, ctypes.c_void_p(16), None)
    assert rc != 0 and b"bad arguments" in L.dk_last_error()
    w = _lib.NF4Weight()
    w.n, w.k, w.blocksize = 8, 64, 64
    rc = L.dk_nf4_dequant(ctypes.byref(w), None, None)
    assert rc != 0 and b"must be set" in L.dk_last_error()
    with pytest.raises(_lib.DecikError):
        _lib.check(1)


def _fake_weight(n, k):
    """A descriptor with aligned non-null fake device pointers: only argument checks run."""
    from decik_amd import _lib

    w = _lib.NF4Weight()
    w.packed = w.absmax = w.code = 256
    w.n, w.k, w.blocksize, w.blocksize2, w.nested = n, k, 64, 256, 0
    return w


@pytest.mark.parametrize("m", [1, 830])  # the GEMV path and the (split-K) MFMA path
def test_forward_rejects_rows_not_multiple_of_8(m):
    """n % 8 != 0 would move 8-column output chunks across a group's end (the caller's row
    padding, the next group's partial-slab columns, bias read past its end): every forward entry
    rejects it before any GPU call, whatever ldy leaves room for."""
    from decik_amd import _lib

    L = _lib.lib()
    g = (_lib.LinearFwdGroup * 2)()
    for i in range(2):
        g[i].w = _fake_weight(67, 1536)
        g[i].y, g[i].ldy = 4096, 72  # padded rows: room for the chunk, still rejected
    ws = ctypes.c_void_p(1 << 20)
    rc = L.dk_nf4_linear_fwd(ctypes.c_void_p(16), m, 1536, 1536, g, 1, 0, ws, 1 << 40, None)
    assert rc != 0 and b"multiple of 8" in L.dk_last_error()
    rc = L.dk_nf4_linear_fwd(ctypes.c_void_p(16), m, 1536, 1536, g, 2, 0, ws, 1 << 40, None)
    assert rc != 0 and b"multiple of 8" in L.dk_last_error()
    rc = L.dk_nf4_glu_fwd(ctypes.c_void_p(16), m, 1536, 1536, g, 0, ctypes.c_void_p(8192), 72, None)
    assert rc != 0 and b"multiple of 8" in L.dk_last_error()
    b = (_lib.LinearBwdGroup * 1)()
    b[0].w = _fake_weight(67, 1536)
    b[0].dy, b[0].lddy = 4096, 72
    rc = L.dk_nf4_linear_bwd(b, 1, m, 1536, ctypes.c_void_p(8192), 1536, 0, 0, ws, 1 << 40, None)
    assert rc != 0 and b"multiple of 8" in L.dk_last_error()


def test_zero_token_rows_are_a_no_op():
    """m = 0 (an empty batch, which the reference's dequantize + F.linear path accepts): every fused
    linear entry checks shapes and descriptors, launches nothing and returns 0, with NULL
    activation and output pointers and any row strides (an empty tensor's strides carry no
    meaning: the gradient of a sum is an expanded tensor of stride 0); a bad shape is still
    rejected."""
    from decik_amd import _lib

    L = _lib.lib()
    g = (_lib.LinearFwdGroup * 2)()
    for i in range(2):
        g[i].w = _fake_weight(64, 1536)
        g[i].y, g[i].ldy = None, 0
    assert L.dk_nf4_linear_fwd(None, 0, 1536, 0, g, 2, 0, None, 0, None) == 0
    assert L.dk_nf4_glu_fwd(None, 0, 1536, 0, g, 0, None, 0, None) == 0
    heads = (ctypes.c_void_p * 2)(None, None)
    tab = ctypes.c_void_p(256)
    assert L.dk_nf4_linear_rope_fwd(None, 0, 1536, 0, g, 2, 0, tab, tab, 64, 1, heads, None, 0, None) == 0
    b = (_lib.LinearBwdGroup * 2)()
    for i in range(2):
        b[i].w = _fake_weight(64, 1536)
        b[i].dy, b[i].lddy = None, 0
    assert L.dk_nf4_linear_bwd(b, 2, 0, 1536, None, 0, 0, 0, None, 0, None) == 0
    assert L.dk_nf4_linear_bwd_swiglu(b, 0, 1536, 0, None, None, 0, None, None, 0, None) == 0
    rc = L.dk_nf4_linear_fwd(None, 0, 1000, 1000, g, 1, 0, None, 0, None)
    assert rc != 0 and b"multiple of 32" in L.dk_last_error()
    # one row: the row checks apply again
    rc = L.dk_nf4_linear_fwd(ctypes.c_void_p(16), 1, 1536, 0, g, 1, 0, None, 0, None)
    assert rc != 0 and b"ldx >= k" in L.dk_last_error()
    rc = L.dk_nf4_linear_bwd(b, 1, 1, 1536, ctypes.c_void_p(16), 1536, 0, 0, None, 0, None)
    assert rc != 0 and b"dy must be" in L.dk_last_error()
    g[1].w = _fake_weight(60, 1536)
    rc = L.dk_nf4_glu_fwd(None, 0, 1536, 1536, g, 0, None, 64, None)
    assert rc != 0 and b"shapes differ" in L.dk_last_error()


def test_workspace_sizes():
    from decik_amd import _lib

    L = _lib.lib()
    ns = (ctypes.c_int64 * 1)(1536)
    # split-K plans need counters + partial tiles; plans without a split need nothing
    assert L.dk_nf4_linear_bwd_workspace(830, 8960, ns, 1) >= 0
    assert L.dk_nf4_linear_fwd_workspace(0, 1536, ns, 1) == 0


def test_launch_plans():
    """dk_nf4_linear_plan (host-only): the eight-wave input-gradient kernel serves the MLP's
    gate/up input gradient at M = 830; SwiGLU-epilogue launches never split and use at most 4
    token blocks; the fused GLU forward never splits; forced plans apply only where
    their kernel may run; bad arguments are reported."""
    from decik_amd import _lib
    from decik_amd.nf4 import launch_plan

    gu = launch_plan(True, 830, 1536, [8960, 8960])
    assert gu["kernel"] == "nf4_bwd8_kernel" and gu["splits"] > 1
    # the SwiGLU epilogue: never split, and only with at most 4 token blocks
    sw = launch_plan(True, 830, 8960, [1536], glu=True)
    assert sw["splits"] == 1
    assert sw["kernel"] == "nf4_bwd8_kernel" and sw["rows_blocks"] <= 4
    # at most 32 token rows, no LoRA, no GLU epilogue: the small-M kernel, split along the
    # contraction only where the rows cannot fill the GPU
    assert launch_plan(False, 1, 3584, [18944])["kernel"] == "nf4_gemv_kernel"
    # two rows: the GEMV below 2^25 weights (k <= 12288, any k up to 2^24 weights), the small-M
    # kernel above (7B gate: 67.9M)
    assert launch_plan(False, 2, 20480, [256])["kernel"] == "nf4_gemv_kernel"
    assert launch_plan(False, 2, 18944, [3584])["kernel"] == "nf4_skinny_kernel"
    assert launch_plan(False, 2, 3584, [18944])["kernel"] == "nf4_skinny_kernel"
    assert launch_plan(False, 2, 1536, [8960])["kernel"] == "nf4_gemv_kernel"
    assert launch_plan(False, 2, 3584, [3584])["kernel"] == "nf4_gemv_kernel"
    # forward split-K with few outputs: each split lengthens the reduction's chain of dependent
    # loads, so these split less than the slab bytes alone would have them (7B k/v, q/o at 64 tokens)
    assert launch_plan(False, 64, 3584, [512])["splits"] == 14
    assert launch_plan(False, 64, 3584, [3584])["splits"] == 8
    # the forward workspace query covers launches of few rows with LoRA terms (tiled, split plans)
    for m, k, ns in ((8, 3584, [18944]), (8, 1536, [8960]), (24, 3584, [3584])):
        plan = launch_plan(False, m, k, ns, lora=True)
        arr = (ctypes.c_int64 * len(ns))(*ns)
        assert _lib.lib().dk_nf4_linear_fwd_workspace(m, k, arr, len(ns)) >= plan["splits"] * m * sum(ns) * 4
    # GEMV work-groups: four waves, eight where X of long rows fills the LDS (7B down at one token)
    assert launch_plan(False, 1, 3584, [18944])["waves"] == 4
    assert launch_plan(False, 1, 18944, [3584])["waves"] == 8
    assert launch_plan(False, 1, 8960, [1536])["waves"] == 4
    for m in (3, 8, 16):
        assert launch_plan(False, m, 3584, [18944])["kernel"] == "nf4_skinny_kernel"
    # past 16 rows, the small-M kernel keeps weights whose row groups fit one work-group per CU
    # (7B gate: 296 groups of 64 rows, 237 of 80 on 256 CUs); taller ones (24592 rows: 257 groups
    # of 96) take the MFMA kernels
    assert launch_plan(False, 32, 3584, [18944])["kernel"] == "nf4_skinny_kernel"
    assert launch_plan(False, 32, 3584, [24592])["kernel"] == "nf4_fwd8_kernel"
    assert launch_plan(False, 16, 3584, [24592])["kernel"] == "nf4_skinny_kernel"
    assert launch_plan(False, 32, 18944, [3584])["kernel"] == "nf4_skinny_kernel"
    assert launch_plan(False, 8, 3584, [18944])["splits"] == 1
    assert launch_plan(False, 8, 18944, [3584])["splits"] > 1
    # every fused launch reads nested statistics as stored (no derived block scales)
    from decik_amd import nf4 as _nf4
    assert _nf4._launch_scales(None, None, None) is None
    # 3-8 rows: small weights take the GEMV (4 token rows a work-group) while X of 4 rows fits
    # 32 KB; larger weights and longer rows the small-M kernel
    assert launch_plan(False, 3, 3584, [512])["kernel"] == "nf4_gemv_kernel"  # 7B k/v
    assert launch_plan(False, 8, 1536, [1536, 256, 256])["kernel"] == "nf4_gemv_kernel"  # 1.5B q/k/v
    assert launch_plan(False, 6, 3584, [3584])["kernel"] == "nf4_skinny_kernel"  # 7B q/o
    assert launch_plan(False, 8, 3584, [512])["kernel"] == "nf4_gemv_kernel"  # 7B k/v, two token groups
    assert launch_plan(False, 5, 8960, [256])["kernel"] == "nf4_skinny_kernel"  # X of 4 rows: 70 KB
    # 3-4 rows: weights up to 2^24 (1.5B down, 7B q/o), not larger
    assert launch_plan(False, 4, 8960, [1536])["kernel"] == "nf4_gemv_kernel"
    assert launch_plan(False, 3, 3584, [3584])["kernel"] == "nf4_gemv_kernel"
    assert launch_plan(False, 3, 8192, [3584])["kernel"] == "nf4_skinny_kernel"
    assert launch_plan(False, 33, 3584, [18944])["kernel"] != "nf4_skinny_kernel"
    assert launch_plan(False, 1, 3584, [18944], lora=True)["kernel"] not in ("nf4_skinny_kernel", "nf4_gemv_kernel")
    old_sm = os.environ.get("DECIK_SMALL_M")
    try:
        os.environ["DECIK_SMALL_M"] = "skinny"
        # few row groups (7B k/v: 8 groups of 64 rows, 28 super-steps): split down to two super-steps
        assert launch_plan(False, 8, 3584, [512])["splits"] == 14
        assert launch_plan(False, 1, 3584, [18944])["kernel"] == "nf4_skinny_kernel"
        assert launch_plan(False, 3, 3584, [18944])["kernel"] == "nf4_skinny_kernel"
    finally:
        if old_sm is None:
            os.environ.pop("DECIK_SMALL_M", None)
        else:
            os.environ["DECIK_SMALL_M"] = old_sm
    glu = launch_plan(False, 830, 1536, [8960, 8960], glu=True)
    assert glu["splits"] == 1 and glu["kernel"] == "nf4_fwd8_kernel"
    # nested statistics in the fused GLU forward: eight-wave variants only (at every M)
    for m in (1, 8, 64, 830):
        assert launch_plan(False, m, 1536, [8960, 8960], glu=True, nested=True)["waves"] == 8
    # an input gradient whose tiles overrun a round of CUs by a partial round runs the left-over
    # columns as a second, split launch (7B down at 830 tokens: 296 tiles of 224 x 256); the MLP
    # launches, and launches that fill whole rounds, stay one launch
    down7 = launch_plan(True, 830, 18944, [3584])
    assert down7["launches"] == 2 and down7["splits"] == 1 and down7["splits_second"] > 1
    for m, k, ns in ((830, 1536, [8960, 8960]), (830, 8960, [1536]), (8192, 3584, [3584]), (830, 3584, [18944])):
        assert launch_plan(True, m, k, ns)["launches"] == 1
    arr = (ctypes.c_int64 * 1)(3584)
    need = _lib.lib().dk_nf4_linear_bwd_workspace(830, 18944, arr, 1)
    assert need == down7["splits_second"] * 830 * (18944 - 64 * 256) * 4
    # 64 and 128 token rows: the eight-wave forward kernel on 64- / 128-token tiles (two waves
    # per SIMD where the four-wave kernel's tiles left one)
    assert launch_plan(False, 64, 3584, [18944]) == dict(rows_blocks=2, waves=8, splits=3, kernel="nf4_fwd8_kernel", launches=1, splits_second=0)
    assert launch_plan(False, 128, 3584, [18944]) == dict(rows_blocks=4, waves=8, splits=3, kernel="nf4_fwd8_kernel", launches=1, splits_second=0)
    assert launch_plan(False, 64, 3584, [18944, 18944], glu=True)["rows_blocks"] == 2
    # k % blocksize != 0: the eight-wave forward kernel may not run
    assert launch_plan(False, 830, 1536, [8960], blocksize=1024)["kernel"] == "nf4_fwd_kernel"
    assert launch_plan(True, 830, 1536, [8960, 8960], no_split=True)["splits"] == 1
    # few token rows without a workspace (the GLU entry's two-launch fallback): the small-M kernel
    # runs unsplit, though it would split these launches when a workspace is allowed
    for m, k, ns in ((8, 8960, [256, 256]), (24, 1536, [1536, 1536])):
        assert launch_plan(False, m, k, ns)["splits"] > 1
        assert launch_plan(False, m, k, ns, no_split=True) == dict(
            rows_blocks=1 if m <= 16 else 2, waves=8, splits=1, kernel="nf4_skinny_kernel", launches=1, splits_second=0)
    # the RoPE epilogue lives in the split-K reduction: a contraction of exactly two 64-wide steps
    # still gets a two-split plan (a workspace of two fp32 slabs), never a single pass
    qkv = (ctypes.c_int64 * 3)(1536, 256, 256)
    assert _lib.lib().dk_nf4_linear_rope_fwd_workspace(64, 128, qkv, 3) == 2 * 64 * 2048 * 4
    old = os.environ.get("DECIK_BWD_PLAN")
    try:
        os.environ["DECIK_BWD_PLAN"] = "8,3,8"
        assert launch_plan(True, 830, 1536, [8960]) == dict(rows_blocks=8, waves=8, splits=3,
                                                             kernel="nf4_bwd8_kernel", launches=1, splits_second=0)
        # no SwiGLU epilogue with 8 token blocks: the forced plan does not apply
        assert launch_plan(True, 830, 1536, [8960], glu=True)["rows_blocks"] != 8
        # variants that spilled registers are not offered: a forced plan naming one is ignored
        os.environ["DECIK_BWD_PLAN"] = "9,3,8"
        assert launch_plan(True, 830, 1536, [8960])["rows_blocks"] != 9
        os.environ["DECIK_BWD_PLAN"] = "4,2,8,256"
        assert launch_plan(True, 830, 1536, [8960]) == dict(rows_blocks=4, waves=8, splits=2,
                                                             kernel="nf4_bwd8_kernel", launches=1, splits_second=0)
        # the retired four-wave input-gradient variants are not offered: a forced plan naming one
        # is ignored
        os.environ["DECIK_BWD_PLAN"] = "2,1,4"
        assert launch_plan(True, 830, 1536, [8960])["kernel"] == "nf4_bwd8_kernel"
    finally:
        if old is None:
            os.environ.pop("DECIK_BWD_PLAN", None)
        else:
            os.environ["DECIK_BWD_PLAN"] = old
    L = _lib.lib()
    out = (ctypes.c_int32 * 4)()
    ns = (ctypes.c_int64 * 1)(64)
    assert L.dk_nf4_linear_plan(1, 8, 64, ns, 1, 0, 48, out) != 0
    assert b"bad arguments" in L.dk_last_error()


def test_no_bit_cast_of_vector_elements():
    """hipcc compiles __builtin_bit_cast(T, v[i]) of an ext_vector_type element as element 0
    whatever i is (found twice in this library); the kernels copy elements to scalars first.
    Flags any bit_cast whose operand is a subscript of a variable declared as one of the
    library's vector types."""
    import glob

    csrc = os.path.join(ROOT, "decik_amd", "csrc")
    vec_types = r"(?:u32x4_t|u32x2_t|half2_t|half4_t|half8_t|float2_t|float4_t|float16_t)"
    bad = []
    for path in sorted(glob.glob(os.path.join(csrc, "*.hip")) + glob.glob(os.path.join(csrc, "*.h"))):
        text = open(path).read()
        vec_vars = set(re.findall(vec_types + r"\s+(\w+)(?:\s*\[[^\]]*\])*\s*[=;,{)]", text))
        vec_vars |= set(re.findall(vec_types + r"\s+\w+(?:\s*\[[^\]]*\])*\s*(?:=[^,;()]*)?,\s*(\w+)", text))
        for mt in re.finditer(r"__builtin_bit_cast\(\s*\w+\s*,\s*(\w+)((?:\s*\[[^\]]*\])+)\s*\)", text):
            if mt.group(1) in vec_vars:
                bad.append(f"{os.path.basename(path)}: {mt.group(0)}")
    assert not bad, bad


def test_descriptor_cache_follows_the_scales_hook():
    """DESCS keys a cached NF4Weight on the scales it was built with: describing a nested weight
    by its raw statistics (a hook returning None, as the MFMA launches' default does) and then by
    block scales (the GEMV's form, and the bench's cached-scales timing) gives two different
    descriptors, each reused
    while nothing changes; new scales (what the scales cache hands out after an in-place change
    of the statistics) or a replaced statistics tensor rebuild it."""
    import torch

    from decik_amd import _lib
    from decik_amd.quant import quantize_nf4

    w16 = (torch.randn(64, 128, generator=torch.Generator().manual_seed(5)) * 0.02).half()
    packed, qs = quantize_nf4(w16, blocksize=64, compress_statistics=True)
    cpu = torch.device("cpu")
    cache = _lib.DescCache()
    raw, _ = cache.get(packed, qs, cpu, lambda p, q, d: None)
    assert raw.nested == 1 and raw.absmax == qs.absmax.data_ptr()
    scales = torch.ones(128 * 64 // 64, dtype=torch.float32)
    cooked, keep = cache.get(packed, qs, cpu, lambda p, q, d: scales)
    assert cooked.nested == 0 and cooked.absmax == scales.data_ptr() and any(t is scales for t in keep)
    again, _ = cache.get(packed, qs, cpu, lambda p, q, d: scales)
    assert again is cooked  # reused
    qs.absmax.add_(0)  # in place: the descriptor's pointers stay valid
    assert cache.get(packed, qs, cpu, lambda p, q, d: scales)[0] is cooked
    scales2 = scales.clone()
    rebuilt, _ = cache.get(packed, qs, cpu, lambda p, q, d: scales2)
    assert rebuilt is not cooked and rebuilt.absmax == scales2.data_ptr()
    qs.absmax = qs.absmax.clone()  # a replaced statistics tensor
    raw2, _ = cache.get(packed, qs, cpu, lambda p, q, d: None)
    assert raw2.absmax == qs.absmax.data_ptr()


def test_scale_cache_version_key_tracks_statistics():
    """The block-scale cache's key changes with an in-place write to any statistics tensor and
    with a replaced tensor, and not otherwise."""
    import torch

    from decik_amd import _lib
    from decik_amd.quant import quantize_nf4

    w16 = (torch.randn(32, 256, generator=torch.Generator().manual_seed(6)) * 0.02).half()
    _, qs = quantize_nf4(w16, blocksize=64, compress_statistics=True)
    k0 = _lib._version_key(qs)
    assert _lib._version_key(qs) == k0
    qs.state2.absmax.mul_(1)
    k1 = _lib._version_key(qs)
    assert k1 != k0
    qs.absmax = qs.absmax.clone()
    assert _lib._version_key(qs) != k1


def test_plan_memo_follows_the_tuning_variables(monkeypatch):
    """Plans are memoized per argument list; a forced plan (DECIK_FWD_PLAN / DECIK_BWD_PLAN) set
    or cleared between calls is seen by the next call, and the memo gives the same plan again."""
    from decik_amd.nf4 import launch_plan

    monkeypatch.delenv("DECIK_FWD_PLAN", raising=False)
    monkeypatch.delenv("DECIK_BWD_PLAN", raising=False)
    base = launch_plan(False, 830, 1536, [1536])
    assert launch_plan(False, 830, 1536, [1536]) == base
    monkeypatch.setenv("DECIK_FWD_PLAN", "4,2")
    forced = launch_plan(False, 830, 1536, [1536])
    assert forced["rows_blocks"] == 4 and forced["splits"] == 2
    monkeypatch.setenv("DECIK_FWD_PLAN", "7,3")
    assert launch_plan(False, 830, 1536, [1536])["rows_blocks"] == 7
    monkeypatch.delenv("DECIK_FWD_PLAN")
    assert launch_plan(False, 830, 1536, [1536]) == base
    bwd = launch_plan(True, 830, 1536, [1536])
    monkeypatch.setenv("DECIK_BWD_PLAN", "4,1")
    assert launch_plan(True, 830, 1536, [1536])["splits"] == 1
    monkeypatch.delenv("DECIK_BWD_PLAN")
    assert launch_plan(True, 830, 1536, [1536]) == bwd


def test_workspace_queries_cover_every_plan():
    """Property test of the planner (host-only): for random launch shapes, every plan the forward
    and input-gradient entries may choose -- with or without LoRA terms, any block size, the GLU
    and SwiGLU forms -- fits the workspace the matching query reports (a plan needing more made
    a call fail with 'workspace too small'), no-split plans never split, and every split gets work."""
    from hypothesis import HealthCheck, given, settings
    from hypothesis import strategies as st

    from decik_amd import _lib
    from decik_amd.nf4 import launch_plan

    L = _lib.lib()

    @settings(max_examples=250, deadline=None, suppress_health_check=[HealthCheck.too_slow])
    @given(m=st.one_of(st.integers(1, 40), st.integers(41, 9000)),
           k=st.integers(1, 640).map(lambda v: 32 * v),
           ns=st.lists(st.integers(1, 3000).map(lambda v: 8 * v), min_size=1, max_size=4),
           blocksize=st.sampled_from([32, 64, 128, 256]))
    def check(m, k, ns, blocksize):
        arr = (ctypes.c_int64 * len(ns))(*ns)
        fwd_ws = L.dk_nf4_linear_fwd_workspace(m, k, arr, len(ns))
        bwd_ws = L.dk_nf4_linear_bwd_workspace(m, k, arr, len(ns))
        ncols = sum(ns)
        steps64 = -(-k // 64)
        for lora in (False, True):
            p = launch_plan(False, m, k, ns, lora=lora, blocksize=blocksize)
            assert 1 <= p["splits"] <= max(steps64, 1)
            if p["splits"] > 1:
                assert fwd_ws >= p["splits"] * m * ncols * 4, (m, k, ns, blocksize, lora, p, fwd_ws)
            assert launch_plan(False, m, k, ns, lora=lora, no_split=True, blocksize=blocksize)["splits"] == 1
        if len(ns) == 2 and ns[0] == ns[1]:
            assert launch_plan(False, m, k, ns, glu=True, blocksize=blocksize)["splits"] == 1
        b = launch_plan(True, m, k, ns, blocksize=blocksize)
        assert b["splits"] >= 1 and b["launches"] in (1, 2)
        if b["launches"] == 1 and b["splits"] > 1:
            assert bwd_ws >= b["splits"] * m * k * 4, (m, k, ns, blocksize, b, bwd_ws)
        if b["launches"] == 2 and b["splits_second"] > 1:
            # the left-over columns' own split launch: its slabs (fewer columns than k) need a workspace
            assert bwd_ws > 0, (m, k, ns, blocksize, b)
        assert launch_plan(True, m, k, ns, no_split=True, blocksize=blocksize)["splits"] == 1
        if len(ns) == 1:
            assert launch_plan(True, m, k, ns, glu=True, blocksize=blocksize)["splits"] == 1

    check()
