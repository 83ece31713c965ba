"""Benchmark of the NF4 quantized-linear path on one MI355X.

Workload (one "step"): the Qwen2.5-1.5B MLP block forward + backward on NF4 weights at 830 packed
tokens -- gate/up [8960, 1536] and down [1536, 8960] (fp16 N(0, 0.02), NF4 blocksize 64 with
double quant), X [830, 1536] ~ N(0, 1), dY ~ N(0, 1e-2), SwiGLU between the projections, dX
through the dequantized weights. Per step: 4 fused dequant-GEMM launches = 6 GEMMs of
2*830*8960*1536 flops: gate+up forward with SwiGLU in its epilogue, down forward, down backward
with the SwiGLU backward in its epilogue, gate+up backward. gate/up are kept from the forward (no
recompute). Weights rotate over enough layers' worth of seeded weights (seed = 7 * layer +
projection) to total more than 512 MB of NF4 data, so the 256 MB Infinity Cache cannot serve
repeats.

Also measured: the standalone NF4 dequantization of all seven Qwen2.5-1.5B projections (q, k, v,
o, gate, up, down) over 8 layers per iteration (942 MB of algorithmic traffic, more than the
256 MB Infinity Cache), in GB/s against the HBM peak.

Prints one JSON line. `value` = whole-step dequant-GEMM throughput in TFLOP/s (inputs resident in
HBM). `roofline` describes the kernel symbol with the largest share of the step time (launch
durations from HIP events on the launch stream). `measured_peaks` gives this device's ceilings as
measured here (a large device copy; a dense loop of the same MFMA instruction), and the roofline
objects also give their fractions of those. `cpu_baseline` times the CPU restatement of the
reference algorithm (dequantize the whole weight, then an fp32 GEMM) on this host.
"""

import argparse
import contextlib
import gc
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "NF4 dequant GB/s + dequant-GEMM fwd/bwd TFLOP/s, Qwen2.5-1.5B shapes, M=830"
HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
M, HIDDEN, INTER = 830, 1536, 8960
QWEN15_SHAPES = [("q", 1536, 1536), ("k", 256, 1536), ("v", 256, 1536), ("o", 1536, 1536),
                 ("gate", 8960, 1536), ("up", 8960, 1536), ("down", 1536, 8960)]


def dequant_bytes(n, k):
    """Algorithmic bytes of one dequantization: 0.5 B packed + 1/64 B absmax code + 2 B fp16 out
    per weight, 4 B per 16384 weights of absmax2, 1092 B of tables and offset."""
    w = n * k
    return w * 0.5 + w / 64 + 2 * w + 4 * -(-w // 16384) + 1092


def gemm_flops(n, k, m=M):
    return 2.0 * m * n * k


def seeded_fp16(shape, seed, std, device):
    import torch

    g = torch.Generator(device="cpu").manual_seed(seed)
    return (torch.randn(shape, generator=g) * std).to(torch.float16).to(device)


def make_layers(n_layers, names, device, base_seed=0):
    from decik_amd.quant import quantize_nf4

    shapes = {s[0]: (s[1], s[2]) for s in QWEN15_SHAPES}
    order = [s[0] for s in QWEN15_SHAPES]
    layers = []
    for layer in range(n_layers):
        d = {}
        for name in names:
            w = seeded_fp16(shapes[name], base_seed + 7 * layer + order.index(name), 0.02, device)
            d[name] = quantize_nf4(w, blocksize=64, compress_statistics=True)
            del w
        layers.append(d)
    return layers


def split_launch(kind):
    """Whether this launch kind takes the split-K path (then the call is the GEMM kernel plus
    splitk_reduce_kernel): the library asks for a workspace only then."""
    import ctypes

    from decik_amd import _lib

    if kind in ("fwd_gate_up", "bwd_down"):
        return False  # the SwiGLU-fused launches never split
    L = _lib.lib()
    shapes = {"fwd_gate_up": ("fwd", HIDDEN, [INTER, INTER]), "fwd_down": ("fwd", INTER, [HIDDEN]),
              "bwd_down": ("bwd", INTER, [HIDDEN]), "bwd_gate_up": ("bwd", HIDDEN, [INTER, INTER])}
    d, k, ns = shapes[kind]
    arr = (ctypes.c_int64 * len(ns))(*ns)
    fn = L.dk_nf4_linear_fwd_workspace if d == "fwd" else L.dk_nf4_linear_bwd_workspace
    return fn(M, k, arr, len(ns)) > 0


def nf4_bytes(n, k):
    """Bytes of one NF4 weight in HBM: packed codes, absmax codes, absmax2, tables."""
    w = n * k
    return w // 2 + w // 64 + 4 * -(-w // 16384) + 1092


def mlp_weight_sets(min_bytes=512 << 20):
    """Weight sets (gate, up, down) the MLP bench rotates through: more than `min_bytes` in all."""
    per_set = 2 * nf4_bytes(INTER, HIDDEN) + nf4_bytes(HIDDEN, INTER)
    return max(4, -(-min_bytes // per_set) + 1)


@contextlib.contextmanager
def no_gc():
    """Python's garbage collector off while timing (as the timeit module does): a collection
    pause in the host loop stalls the launch queue and would be charged to the GPU work."""
    gc.collect()
    gc.disable()
    try:
        yield
    finally:
        gc.enable()


def bench_mlp(steps, warmup, device, n_sets=None, only=None):
    import torch

    from decik_amd import nf4

    n_sets = n_sets or mlp_weight_sets()
    layers = make_layers(n_sets, ["gate", "up", "down"], device)
    x = seeded_fp16((M, HIDDEN), 1001, 1.0, device)
    dy = seeded_fp16((M, HIDDEN), 1002, 1e-2, device)
    launches = ["fwd_gate_up", "fwd_down", "bwd_down", "bwd_gate_up"]
    if only is not None:
        launches = [only]
    # the GEMM kernel each launch runs, as the library's planner chooses it for these shapes
    symbol = {"fwd_gate_up": nf4.launch_plan(False, M, HIDDEN, [INTER, INTER], glu=True)["kernel"],
              "fwd_down": nf4.launch_plan(False, M, INTER, [HIDDEN])["kernel"],
              "bwd_down": nf4.launch_plan(True, M, INTER, [HIDDEN], glu=True)["kernel"],
              "bwd_gate_up": nf4.launch_plan(True, M, HIDDEN, [INTER, INTER])["kernel"]}
    flops = {"fwd_gate_up": 2 * gemm_flops(INTER, HIDDEN), "fwd_down": gemm_flops(HIDDEN, INTER),
             "bwd_down": gemm_flops(INTER, HIDDEN), "bwd_gate_up": 2 * gemm_flops(INTER, HIDDEN)}

    def step(i):
        L = layers[i % n_sets]
        g, u = L["gate"], L["up"]
        dn = L["down"]
        gate, up, h = nf4.glu_forward(x, dict(packed=g[0], qs=g[1]), dict(packed=u[0], qs=u[1]))
        (out,) = nf4.linear_forward(h, [dict(packed=dn[0], qs=dn[1])])
        dgate, dup = nf4.linear_backward_swiglu(dict(packed=dn[0], qs=dn[1], dy=dy), gate, up,
                                                out=(gate, up))
        dx = nf4.linear_backward([dict(packed=g[0], qs=g[1], dy=dgate),
                                  dict(packed=u[0], qs=u[1], dy=dup)], M, HIDDEN)
        return out, dx

    # setup: one pass over every weight set fills the per-weight descriptor cache before the
    # warm-up steps
    for i in range(n_sets):
        step(i)
    torch.cuda.synchronize()
    ms_step = None
    if only is None:
        for i in range(warmup):
            step(i)
        torch.cuda.synchronize()
        # whole-step timing: K steps between two synchronisations
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        for i in range(steps):
            step(i)
        t1.record()
        torch.cuda.synchronize()
        ms_step = t0.elapsed_time(t1) / steps
    graph_ms = graph_mlp_steps(step, n_sets) if only is None else None
    # Per-launch timing: each launch kind back to back (same inputs as one step, weight sets
    # rotating), HIP events on the launch stream around the loop. Unlike events between the
    # launches of one step, this excludes host-side gaps, so the average matches the kernel's
    # duration in a rocprofv3 kernel trace of this same program.
    gate0, up0, h0 = nf4.glu_forward(x, dict(packed=layers[0]["gate"][0], qs=layers[0]["gate"][1]),
                                     dict(packed=layers[0]["up"][0], qs=layers[0]["up"][1]))
    dg0, du0 = nf4.linear_backward_swiglu(dict(packed=layers[0]["down"][0], qs=layers[0]["down"][1], dy=dy),
                                          gate0, up0)

    def one(kind, i):
        L = layers[i % n_sets]
        g, u, dn = L["gate"], L["up"], L["down"]
        if kind == "fwd_gate_up":
            nf4.glu_forward(x, dict(packed=g[0], qs=g[1]), dict(packed=u[0], qs=u[1]))
        elif kind == "fwd_down":
            nf4.linear_forward(h0, [dict(packed=dn[0], qs=dn[1])])
        elif kind == "bwd_down":
            nf4.linear_backward_swiglu(dict(packed=dn[0], qs=dn[1], dy=dy), gate0, up0)
        else:
            nf4.linear_backward([dict(packed=g[0], qs=g[1], dy=dg0), dict(packed=u[0], qs=u[1], dy=du0)],
                                M, HIDDEN)

    per = {}
    for kind in launches:
        for i in range(2):
            one(kind, i)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(steps):
            one(kind, i)
        b.record()
        torch.cuda.synchronize()
        per[kind] = a.elapsed_time(b) / steps
    launch_ms = per
    # The same launches on the derived fp32 block scales (dk_nf4_block_scales, computed once per
    # frozen weight before timing) instead of the statistics as stored: each kernel then loads one
    # fp32 scale per block instead of an absmax code and forming code2[q] * absmax2 + offset.
    cached = {}
    from decik_amd import _lib

    for L in layers:  # the derived scales exist before timing (computed once per frozen weight)
        for name in ("gate", "up", "down"):
            _lib.SCALES.get(L[name][0], L[name][1], device)
    torch.cuda.synchronize()
    saved_form = nf4._launch_scales
    nf4._launch_scales = nf4._scales
    try:
        if only is not None:
            launches = []  # counter runs (--only) time the cached launch alone
        gate0, up0, h0 = nf4.glu_forward(x, dict(packed=layers[0]["gate"][0], qs=layers[0]["gate"][1]),
                                         dict(packed=layers[0]["up"][0], qs=layers[0]["up"][1]))
        dg0, du0 = nf4.linear_backward_swiglu(dict(packed=layers[0]["down"][0], qs=layers[0]["down"][1], dy=dy),
                                              gate0, up0)
        for kind in launches:
            for i in range(2):
                one(kind, i)
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for i in range(steps):
                one(kind, i)
            b.record()
            torch.cuda.synchronize()
            cached[kind] = a.elapsed_time(b) / steps
    finally:
        nf4._launch_scales = saved_form
    step_flops = sum(flops.values())
    return dict(ms_step=ms_step, launch_ms=launch_ms, flops=flops, symbol=symbol,
                step_flops=step_flops, n_sets=n_sets, cached_ms=cached, graph_ms=graph_ms)


def bench_mlp_gpu_baselines(steps, warmup, device, our_ms):
    """The same MLP block on the same GPU without the fused kernels, for scale:

    reference_algorithm -- the reference's RecomputedMLP step as it computes it
        (solution/mlp.py:62-110): every weight dequantized to fp16 before each use (3 + 3 per
        step; this library's dequantization kernel stands in for skc_nf4_dequant_kernel, bit for
        bit), fp16 F.linear / matmul on torch (hipBLASLt), the SwiGLU kernels, gate/up recomputed
        in the backward (8 GEMMs), dX as two fp16 products summed in fp32.
    fp16_library_gemms -- the fused step's six products (gate/up forward, down forward, down
        input gradient, gate/up input gradient) as plain fp16 torch GEMMs on weights dequantized
        once before timing, plus the SwiGLU kernels: the vendor library's rate at these shapes
        with no dequantization in the step at all.
    Both rotate over weight sets larger than the 256 MB Infinity Cache, as the fused step does
    (fp16 weights: 27.5 MB a projection). Time per step = K eager steps between two events."""
    import torch
    import torch.nn.functional as F

    from decik_amd import nf4
    from decik_amd.swiglu import swiglu_bwd, swiglu_fwd

    x = seeded_fp16((M, HIDDEN), 1001, 1.0, device)
    dy = seeded_fp16((M, HIDDEN), 1002, 1e-2, device)
    n_sets = 4  # 4 x 82.6 MB of fp16 weights for the library GEMMs (330 MB > the Infinity Cache)
    layers = make_layers(max(n_sets, mlp_weight_sets()), ["gate", "up", "down"], device)
    n_ref = len(layers)

    def ref_step(i):
        L = layers[i % n_ref]
        wg = nf4.dequantize_nf4(*L["gate"])
        gate = F.linear(x, wg)
        wu = nf4.dequantize_nf4(*L["up"])
        up = F.linear(x, wu)
        h = swiglu_fwd(gate, up)
        del gate, up
        wd = nf4.dequantize_nf4(*L["down"])
        out = F.linear(h, wd)
        wd = nf4.dequantize_nf4(*L["down"])
        gh = torch.matmul(dy, wd)
        wg = nf4.dequantize_nf4(*L["gate"])
        gate = F.linear(x, wg)
        wu = nf4.dequantize_nf4(*L["up"])
        up = F.linear(x, wu)
        dgate, dup = swiglu_bwd(gh, gate, up, out=(gate, up))
        dx = torch.matmul(dgate, wg).float() + torch.matmul(dup, wu).float()
        return out, dx

    w16 = [{n: nf4.dequantize_nf4(*layers[s][n]) for n in ("gate", "up", "down")} for s in range(n_sets)]

    def lib_step(i):
        W = w16[i % n_sets]
        gate = F.linear(x, W["gate"])
        up = F.linear(x, W["up"])
        h = swiglu_fwd(gate, up)
        out = F.linear(h, W["down"])
        gh = torch.matmul(dy, W["down"])
        dgate, dup = swiglu_bwd(gh, gate, up, out=(gate, up))
        dx = torch.matmul(dgate, W["gate"]).float() + torch.matmul(dup, W["up"]).float()
        return out, dx

    def timed(step, sets):
        for i in range(max(warmup, sets)):
            step(i)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(steps):
            step(i)
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / steps

    flops = 3 * gemm_flops(INTER, HIDDEN) * 2  # the fused step's six products
    res = {}
    # launches per step: dequantizations + GEMMs + the two SwiGLU kernels + two fp32 casts and their sum
    for name, step, sets, launches, gemms in (("reference_algorithm", ref_step, n_ref, 6 + 8 + 2 + 3, 8),
                                              ("fp16_library_gemms", lib_step, n_sets, 6 + 2 + 3, 6)):
        ms = timed(step, sets)
        res[name] = dict(ms_per_step=round(ms, 4), tflops=round(flops / (ms * 1e-3) / 1e12, 1),
                         fused_speedup=round(ms / our_ms, 3), launches=launches, gemms=gemms)
    del w16, layers
    torch.cuda.empty_cache()
    res["note"] = ("tflops: the fused step's 137.1 GFLOP (6 products) over each step's time; the "
                   "reference's step does 8 products (gate/up recomputed) and 6 whole-weight "
                   "dequantizations; fused_speedup = that step's time / the fused step's")
    return res


def graph_mlp_steps(step, n_sets, reps=3):
    """The MLP step (its six kernels) over every weight set, captured once in a HIP graph and
    replayed: ms per step with the host's launch cost and the gaps between eager launches taken
    out. The replay's last outputs must equal the same step run eagerly; None if capture fails."""
    import torch

    try:
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step(0)  # warm-up on the capture stream
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        with torch.cuda.graph(g):
            outs = [step(i) for i in range(n_sets)]
        g.replay()
        torch.cuda.synchronize()
        ref = step(n_sets - 1)
        torch.cuda.synchronize()
        if not (torch.equal(outs[-1][0], ref[0]) and torch.equal(outs[-1][1], ref[1])):
            return None
        times = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            g.replay()
            b.record()
            torch.cuda.synchronize()
            times.append(a.elapsed_time(b) / n_sets)
        del g, outs
        return statistics.median(times)
    except Exception:  # noqa: BLE001 - reported as null
        return None


def bench_dequant(iters, warmup, device, n_layers=24):
    """The standalone dequantization of every projection of `n_layers` Qwen2.5-1.5B layers per
    iteration, back to back (the batched entry point, up to 24 weights per launch). With 24
    layers the packed weights (561 MB) exceed the 256 MB Infinity Cache, so every iteration
    reads them from HBM; with 8 (187 MB) they stay cached between iterations (the outputs are
    stored non-temporally and do not evict them) and only the writes reach HBM."""
    import torch

    from decik_amd import nf4

    names = [s[0] for s in QWEN15_SHAPES]
    layers = make_layers(n_layers, names, device, base_seed=10_000)
    pairs = [L[n] for L in layers for n in names]
    outs = nf4.dequantize_nf4_many(pairs)  # allocate the outputs once; reused below
    import ctypes

    from decik_amd import _lib

    descs, keep = [], []
    for (packed, qs) in pairs:
        w, kp = _lib.weight_desc(packed, qs, device)
        descs.append(w)
        keep += kp
    arr = (_lib.NF4Weight * len(descs))(*descs)
    optr = (ctypes.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
    L = _lib.lib()

    def run():
        _lib.check(L.dk_nf4_dequant_batched(arr, optr, len(descs), _lib.stream_of(device)))

    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    times = []
    for _ in range(iters):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        run()
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b))
    ms = statistics.median(times)
    total_bytes = n_layers * sum(dequant_bytes(n, k) for _, n, k in QWEN15_SHAPES)
    write_bytes = n_layers * sum(2 * n * k for _, n, k in QWEN15_SHAPES)
    launches = -(-len(descs) // 24)  # dk_nf4_dequant_batched: up to 24 weights per launch
    return dict(ms=ms, bytes=total_bytes, gbs=total_bytes / ms / 1e6, launches=launches,
                read=total_bytes - write_bytes, write=write_bytes)


def measured_peaks(device):
    """This device's ceilings as measured here: HBM read, write and copy rates of dk_probe_hbm (the
    dequantization kernel's access pattern: 16-byte lanes; the best of 4, 8 or 16 chunks in flight
    per thread, non-temporal or plain loads and stores) over 1 GiB buffers (past the 256 MB
    Infinity Cache), median of 7; and the
    dense fp16 MFMA rate of a register-only loop of v_mfma_f32_32x32x16_f16 (dk_probe_mfma_f16,
    1024 work-groups of 8 waves)."""
    import torch

    from decik_amd import _lib

    L = _lib.lib()
    stream = _lib.stream_of(device)
    nbytes = 1 << 30
    src = torch.ones(nbytes // 4, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    sums = torch.zeros(nbytes // 16384 + 1, dtype=torch.float32, device=device)
    rates = {}
    # the best of the probe's variants: chunks per thread (+ 16, + 32), plain loads (+ 8) and
    # plain stores (+ 4)
    var = [u + l for u in (0, 16, 32) for l in (0, 8)]
    for name, modes, moved in (("read", tuple(v for v in var), nbytes),
                               ("write", tuple(v + s + 1 for v in (0, 16, 32) for s in (0, 4)), nbytes),
                               ("copy", tuple(v + s + 2 for v in var for s in (0, 4)), 2 * nbytes)):
        best = 0.0
        for mode in modes:
            times = []
            for i in range(9):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                _lib.check(L.dk_probe_hbm(src.data_ptr(), dst.data_ptr(), nbytes, mode, sums.data_ptr(), stream))
                b.record()
                torch.cuda.synchronize()
                if i >= 2:
                    times.append(a.elapsed_time(b))
            best = max(best, moved / statistics.median(times) / 1e6)
        rates[name] = best
    del src, dst, sums
    wgs, iters = 1024, 4096
    out = torch.empty(wgs * 512, dtype=torch.float32, device=device)
    _lib.check(L.dk_probe_mfma_f16(wgs, 64, out.data_ptr(), stream))
    torch.cuda.synchronize()
    times = []
    for _ in range(3):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        _lib.check(L.dk_probe_mfma_f16(wgs, iters, out.data_ptr(), stream))
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b))
    flops = wgs * 8 * iters * 8 * 2 * 32 * 32 * 16
    mfma_tf = flops / statistics.median(times) / 1e9
    return dict(hbm_read_gbs=round(rates["read"], 1), hbm_write_gbs=round(rates["write"], 1),
                hbm_copy_gbs=round(rates["copy"], 1), mfma_f16_tflops=round(mfma_tf, 1),
                method="dk_probe_hbm over 1 GiB (read / write / copy, bytes moved per second); "
                       "register-only v_mfma_f32_32x32x16_f16 loop")


def mixed_ceiling(peaks, read_bytes, write_bytes):
    """The measured ceiling of a stream that reads and writes these amounts: each byte at its own
    measured rate, t = R / read + W / write."""
    t = read_bytes / peaks["hbm_read_gbs"] + write_bytes / peaks["hbm_write_gbs"]
    return (read_bytes + write_bytes) / t


def cpu_baseline(sample_steps=3):
    """The reference algorithm on this host: dequantize each whole weight to fp16 (the oracle's
    C restatement of the reference kernel, OpenMP on every core we may use), then fp32 GEMMs
    (torch CPU) for the same MLP step: gate, up, SwiGLU, down forward; down, gate, up backward.
    Sample: `sample_steps` full steps after one warm-up step; median."""
    import numpy as np
    import torch

    from oracle import nf4 as O

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cpu_model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    rng = np.random.default_rng(0)
    ws = {}
    for name, n, k in [("gate", INTER, HIDDEN), ("up", INTER, HIDDEN), ("down", HIDDEN, INTER)]:
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
        ws[name] = O.quantize_nf4(w)
    x = torch.from_numpy((rng.standard_normal((M, HIDDEN))).astype(np.float16)).float()
    dy = torch.from_numpy((rng.standard_normal((M, HIDDEN)) * 1e-2).astype(np.float16)).float()

    def step():
        w16 = {k: torch.from_numpy(O.dequant_nf4(q, nthreads=cores)) for k, q in ws.items()}
        wf = {k: v.float() for k, v in w16.items()}
        gate = x @ wf["gate"].T
        up = x @ wf["up"].T
        h = gate * torch.sigmoid(gate) * up
        _ = h @ wf["down"].T
        gh = dy @ wf["down"]
        s = torch.sigmoid(gate)
        dgate = gh * up * s * (1 + gate * (1 - s))
        dup = gh * gate * s
        return dgate @ wf["gate"] + dup @ wf["up"]

    step()
    times = []
    for _ in range(sample_steps):
        t = time.perf_counter()
        step()
        times.append(time.perf_counter() - t)
    sec = statistics.median(times)
    flops = 6 * gemm_flops(INTER, HIDDEN)
    return dict(value=round(flops / sec / 1e12, 4), unit="TFLOP/s", cores=cores, cpu=cpu_model, kind="port",
                sample=f"{sample_steps} full MLP fwd+bwd steps (M=830, 3 NF4 weights dequantized by "
                       f"the C oracle with {cores} OpenMP threads + torch fp32 CPU GEMMs), median "
                       f"{sec * 1e3:.0f} ms/step")


# ---- config C3: attention projections with LoRA on q and v, one layer fwd + bwd ------------------

C3_LENGTHS = (100, 200, 130, 32, 150, 60, 90, 68)  # 8 packed sequences, 830 tokens
N_HEADS, N_KV_HEADS, HEAD_DIM = 12, 2, 128
LORA_P = 0.05  # the real run's lora_dropout


def attn_weight_sets(min_bytes=512 << 20):
    """Layers of q/k/v/o weights the C3 bench rotates through: more than `min_bytes` in all."""
    per_set = 2 * nf4_bytes(HIDDEN, HIDDEN) + 2 * nf4_bytes(256, HIDDEN)
    return max(4, -(-min_bytes // per_set) + 1)


def rope_tables(lengths, d, base=1000000.0):
    """cos / sin [T, D] fp32 of packed sequences (positions restart per sequence), Qwen2's rotary
    embedding (inv_freq = base^(-2i/D), emb = [f, f])."""
    import numpy as np

    pos = np.concatenate([np.arange(n) for n in lengths]).astype(np.float32)
    inv = (1.0 / (base ** (np.arange(0, d, 2, dtype=np.float32) / d))).astype(np.float32)
    f = pos[:, None] * inv[None, :]
    emb = np.concatenate([f, f], axis=1)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def count_kernels(fn):
    """(kernels launched, their summed duration in us) for one call of fn, from torch.profiler's
    device events; (None, None) if the profiler is unavailable. The summed duration is the GPU
    time of the call without the gaps between launches (the host's share of an eager step)."""
    import torch

    try:
        from torch.profiler import ProfilerActivity, profile

        torch.cuda.synchronize()
        with profile(activities=[ProfilerActivity.CUDA]) as prof:
            fn()
            torch.cuda.synchronize()
        ev = [e for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA]
        busy = sum(float(getattr(e, "device_time", None) or e.cuda_time) for e in ev)
        return len(ev), busy
    except Exception:  # noqa: BLE001 - a missing profiler only drops the count
        return None, None


def graph_steps(step_grads, layers, reps=3):
    """Per-step GPU time of step_grads(L) (a forward and torch.autograd.grad of it, returning the
    gradients) over every layer in `layers`, captured once in a HIP graph and replayed `reps`
    times: the host's Python and launch cost, which bounds the eager step, drops out. After every
    replay the last step's gradients are compared with the same step run eagerly, bit for bit.
    Returns (ms per step, median of the replays) or (None, reason) when capture fails or a replay
    differs."""
    import torch

    ref = [t.clone() for t in step_grads(layers[-1])]
    torch.cuda.synchronize()
    try:
        g = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step_grads(layers[0])  # warm-up on the capture stream
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        outs = []
        with torch.cuda.graph(g):
            for L in layers:
                outs.append(step_grads(L))
        times = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            g.replay()
            b.record()
            torch.cuda.synchronize()
            if not all(torch.equal(o, r) for o, r in zip(outs[-1], ref)):
                return None, "a replay differs from the eager step"
            times.append(a.elapsed_time(b) / len(layers))
        del g, outs
        return statistics.median(times), None
    except Exception as e:  # noqa: BLE001 - reported instead of a graph time
        return None, f"capture failed: {type(e).__name__}: {str(e)[:100]}"


def bench_c3(steps, warmup, device):
    """Config C3: the attention projections of one Qwen2.5-1.5B layer at 830 packed tokens, forward
    and backward: q [1536, 1536], k / v [256, 1536] with biases, LoRA r=16 (alpha 32, dropout
    p = 0.05, fp32 adapters) on q and v, RoPE on q and k (12 and 2 heads of 128), o [1536, 1536];
    the fp32 norm output x and the attention output are fixed synthetic inputs, the gradients of
    q, k, v and o fixed synthetic tensors (solution/attn.py:396-418, 206-273, 27-126).

    fused: pack_keep, QKVRopeProjection (U of q and v from x and the keep bits; q/k/v + biases +
    LoRA + RoPE in one launch and its reduction; backward: the RoPE transpose, GU/dB and dA per
    branch, one dX launch with the masked LoRA terms), and o.
    reference_order: the reference's sequence of operations on this package's kernels: three
    base projections on their own fp16 casts of x, LoRAPairFromNorm's packed path (dropped-out
    inputs, U, up-projection, scaling, per branch), v = fp16(v_base + v_lora) in fp32, FusedQKRope,
    o, and autograd's backward of all that.
    Both rotate over enough layers' weights (more than 512 MB) that repeats miss the Infinity Cache."""
    import torch

    from decik_amd import lora, nf4
    from decik_amd.rope import FusedQKRope

    n_sets = attn_weight_sets()
    layers = make_layers(n_sets, ("q", "k", "v", "o"), device, base_seed=40_000)
    bound = 1.0 / (HIDDEN ** 0.5)
    for li, L in enumerate(layers):
        for j, name in enumerate(("q", "k", "v")):
            L[name + "_bias"] = seeded_fp16((L[name][1].shape[0],), 41_000 + 3 * li + j, 0.1, device)
        g = torch.Generator(device="cpu").manual_seed(42_000 + li)
        for name, n in (("q", 1536), ("v", 256)):
            a = ((torch.rand((LORA_R, HIDDEN), generator=g) * 2 - 1) * bound).to(device).requires_grad_(True)
            b = (torch.randn((n, LORA_R), generator=g) * 1e-3).to(device).requires_grad_(True)
            L[name + "_lora"] = (a, b)
    gen = torch.Generator(device="cpu").manual_seed(43_000)
    x = torch.randn((M, HIDDEN), generator=gen).to(device).requires_grad_(True)  # fp32 norm output
    attn = seeded_fp16((M, HIDDEN), 43_001, 1.0, device).requires_grad_(True)
    keep_q = (torch.rand((M, HIDDEN), generator=gen) >= LORA_P).to(device)
    keep_v = (torch.rand((M, HIDDEN), generator=gen) >= LORA_P).to(device)
    scale = torch.tensor(1.0 / (1.0 - LORA_P), dtype=torch.float32, device=device)
    c, s_ = rope_tables(C3_LENGTHS, HEAD_DIM)
    cos, sin = torch.from_numpy(c).to(device), torch.from_numpy(s_).to(device)
    gq = seeded_fp16((1, N_HEADS, M, HEAD_DIM), 43_002, 1e-2, device)
    gk = seeded_fp16((1, N_KV_HEADS, M, HEAD_DIM), 43_003, 1e-2, device)
    gv = seeded_fp16((M, N_KV_HEADS * HEAD_DIM), 43_004, 1e-2, device)
    go = seeded_fp16((M, HIDDEN), 43_005, 1e-2, device)
    sc = LORA_ALPHA / LORA_R

    def fused(L):
        bq, bv = lora.pack_keep(keep_q, keep_v)
        (aq, bq_w), (av, bv_w) = L["q_lora"], L["v_lora"]
        projs = (dict(packed=L["q"][0], qs=L["q"][1], bias=L["q_bias"], lora_a=aq, lora_b=bq_w, scaling=sc,
                      keep_bits=bq, keep_scale=scale, p=LORA_P),
                 dict(packed=L["k"][0], qs=L["k"][1], bias=L["k_bias"]),
                 dict(packed=L["v"][0], qs=L["v"][1], bias=L["v_bias"], lora_a=av, lora_b=bv_w, scaling=sc,
                      keep_bits=bv, keep_scale=scale, p=LORA_P))
        q, k, v = lora.qkv_rope_projection(x, projs, cos, sin, N_HEADS, N_KV_HEADS)
        o = nf4.NF4Linear.apply(attn, L["o"][0], None, L["o"][1])
        return [q, k, v, o]

    def reference_order(L):
        (aq, bq_w), (av, bv_w) = L["q_lora"], L["v_lora"]
        q_base = nf4.NF4Linear.apply(x.to(torch.float16), L["q"][0], L["q_bias"], L["q"][1])
        k = nf4.NF4Linear.apply(x.to(torch.float16), L["k"][0], L["k_bias"], L["k"][1])
        v_base = nf4.NF4Linear.apply(x.to(torch.float16), L["v"][0], L["v_bias"], L["v"][1])
        bq, bv = lora.pack_keep(keep_q, keep_v)
        q_lora, v_lora = lora.LoRAPairFromNorm.apply(x, None, None, None, None, bq, scale, None, bv, scale,
                                                     aq, bq_w, av, bv_w, sc, sc, LORA_P, LORA_P, True)
        v = (v_base.float() + v_lora.float()).to(torch.float16)
        q, k = FusedQKRope.apply(q_base, q_lora.to(torch.float16), k, cos, sin, N_HEADS, N_KV_HEADS)
        o = nf4.NF4Linear.apply(attn, L["o"][0], None, L["o"][1])
        return [q, k, v, o]

    def step(forward):
        """forward + backward with the gradients accumulated into .grad (the eager step)"""
        def run(L):
            torch.autograd.backward(forward(L), [gq, gk, gv, go])
        return run

    def step_grads(forward):
        """forward + backward returning the gradients of x, the attention output and the four
        adapters (graph capture: no accumulation into .grad)"""
        def run(L):
            (aq, bq_w), (av, bv_w) = L["q_lora"], L["v_lora"]
            return torch.autograd.grad(forward(L), [x, attn, aq, bq_w, av, bv_w], [gq, gk, gv, go])
        return run

    def clear():
        x.grad = attn.grad = None
        for L in layers:
            for a, b in (L["q_lora"], L["v_lora"]):
                a.grad = b.grad = None

    res = {}
    for name, forward in (("fused", fused), ("reference_order", reference_order)):
        fn = step(forward)
        for i in range(n_sets):  # fills every weight's descriptor cache
            fn(layers[i])
            clear()
        for i in range(warmup):
            fn(layers[i % n_sets])
            clear()
        # five timed blocks of `steps` steps: the eager step is bound by the host, whose speed
        # drifts between blocks; the median is reported, the spread beside it
        blocks = []
        for _ in range(5):
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for i in range(steps):
                fn(layers[i % n_sets])
                clear()
            b.record()
            torch.cuda.synchronize()
            blocks.append(a.elapsed_time(b) / steps)
        # the same eager steps with autograd's backward on the calling thread instead of its
        # per-device worker thread (torch.autograd.set_multithreading_enabled(False)): the
        # difference is the engine's thread hand-off, a host cost of torch, not of these kernels
        single = []
        with torch.autograd.set_multithreading_enabled(False):
            for _ in range(3):
                torch.cuda.synchronize()
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                for i in range(steps):
                    fn(layers[i % n_sets])
                    clear()
                b.record()
                torch.cuda.synchronize()
                single.append(a.elapsed_time(b) / steps)
        launches, busy = count_kernels(lambda fn=fn: (fn(layers[-1]), clear()))
        graph_ms, graph_note = graph_steps(step_grads(forward), layers)
        res[name] = dict(ms=statistics.median(blocks), spread=(min(blocks), max(blocks)), launches=launches,
                         busy_us=busy, graph_ms=graph_ms, graph_note=graph_note,
                         single_ms=statistics.median(single))
    gemm = 2 * sum(gemm_flops(n, k) for name, n, k in QWEN15_SHAPES if name in ("q", "k", "v", "o"))
    lora_f = sum(2 * M * LORA_R * (HIDDEN + n) + 2 * M * LORA_R * (2 * HIDDEN + 2 * n) for n in (1536, 256))
    out = dict(workload="Qwen2.5-1.5B attention projections, one layer fwd+bwd, M=830 (8 packed sequences): "
                        "q [1536,1536], k/v [256,1536] + biases, LoRA r=16 alpha 32 dropout 0.05 on q/v "
                        "(fp32 x and adapters), RoPE 12/2 heads x 128, o [1536,1536]; NF4 bs 64 double quant; "
                        f"{n_sets} layers of weights rotated",
               step_gflops=round((gemm + lora_f) / 1e9, 2))
    for name, r in res.items():
        out[name] = dict(ms=round(r["ms"], 4), ms_range=[round(v, 4) for v in r["spread"]],
                         tflops=round((gemm + lora_f) / (r["ms"] * 1e-3) / 1e12, 1),
                         backward_on_caller_ms=round(r["single_ms"], 4),
                         launches=r["launches"],
                         gpu_busy_ms=None if r["busy_us"] is None else round(r["busy_us"] / 1e3, 4),
                         graph_ms=None if r["graph_ms"] is None else round(r["graph_ms"], 4),
                         graph_tflops=None if r["graph_ms"] is None else
                         round((gemm + lora_f) / (r["graph_ms"] * 1e-3) / 1e12, 1))
        if r["graph_note"]:
            out[name]["graph_note"] = r["graph_note"]
    out["speedup"] = round(res["reference_order"]["ms"] / res["fused"]["ms"], 3)
    if res["fused"]["graph_ms"] and res["reference_order"]["graph_ms"]:
        out["graph_speedup"] = round(res["reference_order"]["graph_ms"] / res["fused"]["graph_ms"], 3)
    if res["fused"]["busy_us"] and res["reference_order"]["busy_us"]:
        out["gpu_busy_speedup"] = round(res["reference_order"]["busy_us"] / res["fused"]["busy_us"], 3)
    out["note"] = ("ms: eager steps back to back (HIP events), bound by the host's Python and launch "
                   "overhead at this size: median of five blocks of steps (ms_range: the fastest and "
                   "slowest block); backward_on_caller_ms: the same eager steps with autograd's backward "
                   "on the calling thread (torch.autograd.set_multithreading_enabled(False)), the "
                   "difference being torch's hand-off to its device thread; gpu_busy_ms: the kernels' "
                   "summed durations in one profiled step; "
                   "graph_ms: the same step over every layer's weights captured once in a HIP graph "
                   "(forward + torch.autograd.grad) and replayed, median of three replays, each "
                   "replay's last gradients equal to the eager step's bit for bit")
    return out


# ---- config C4: the full Qwen2.5-1.5B frozen-linear stack, one training step ------------------

LORA_R, LORA_ALPHA = 16, 32


def make_stack(n_layers, device, base_seed=20_000):
    """n_layers Qwen2.5-1.5B layers: the seven NF4 weights (seed = base + 7 * layer + projection),
    fp16 biases on q/k/v (Qwen2), LoRA r=16 on q and v (A Kaiming-uniform, B ~ N(0, 1e-3), fp16)."""
    import torch

    from decik_amd.quant import quantize_nf4

    bound = 1.0 / (HIDDEN ** 0.5)
    layers = []
    for layer in range(n_layers):
        d = {}
        for j, (name, n, k) in enumerate(QWEN15_SHAPES):
            w = seeded_fp16((n, k), base_seed + 7 * layer + j, 0.02, device)
            d[name] = quantize_nf4(w, blocksize=64, compress_statistics=True)
            del w
        for j, name in enumerate(("q", "k", "v")):
            d[name + "_bias"] = seeded_fp16((d[name][1].shape[0],), base_seed + 1000 + 3 * layer + j, 0.1, device)
        g = torch.Generator(device="cpu").manual_seed(base_seed + 5000 + layer)
        for name, n in (("q", 1536), ("v", 256)):
            a = ((torch.rand((LORA_R, HIDDEN), generator=g) * 2 - 1) * bound).half().to(device)
            b = (torch.randn((n, LORA_R), generator=g) * 1e-3).half().to(device)
            d[name + "_lora"] = (a, b)
        layers.append(d)
    return layers


def stack_flops(n_layers):
    """Base GEMM flops of one training step of the stack (forward + input gradient), and the
    LoRA products' flops (forward u, out; backward dB, gu, dA, dX)."""
    base = 2 * sum(gemm_flops(n, k) for _, n, k in QWEN15_SHAPES) * n_layers
    lora = sum(2 * M * LORA_R * (HIDDEN + n) + 2 * M * LORA_R * (2 * HIDDEN + 2 * n)
               for n in (1536, 256)) * n_layers
    return base, lora


def bench_c4(steps, warmup, device, n_layers=28):
    """One training step of the 28-layer stack (solution/varlen.py:254-257 -> attn.py:396-418,
    mlp.py:62-110): per layer forward q/k/v with LoRA q/v (one fused launch, U of both adapters
    from one dk_lora_down_group launch), o, gate+up+SwiGLU, down; backward down with the SwiGLU
    backward, gate+up, o, q/k/v with the LoRA input-gradient terms (GU, dB of both adapters in one
    launch and dA in another, dk_lora_bwd_group). Attention and the
    norms are outside this path: each layer's attention output and MLP input are fixed synthetic
    tensors; gate/up are kept from the forward (no recompute). Also timed: the same step with U
    and GU precomputed (the dequant-GEMM launches alone)."""
    import torch

    from decik_amd import lora, nf4

    layers = make_stack(n_layers, device)
    s = LORA_ALPHA / LORA_R
    x = seeded_fp16((M, HIDDEN), 2001, 1.0, device)
    attn = seeded_fp16((M, HIDDEN), 2002, 1.0, device)
    x2 = seeded_fp16((M, HIDDEN), 2003, 1.0, device)
    dy = seeded_fp16((M, HIDDEN), 2004, 1e-2, device)
    dq = seeded_fp16((M, 1536), 2005, 1e-2, device)
    dkv = seeded_fp16((M, 256), 2006, 1e-2, device)
    pre = {}  # U / GU per layer, for the GEMM-only step

    def layer_step(L, li, lora_kernels):
        (aq, bq), (av, bv) = L["q_lora"], L["v_lora"]
        if lora_kernels:
            uq, uv = lora.lora_down_group([(x, aq, None, None), (x, av, None, None)])
        else:
            uq, uv = pre[li][0], pre[li][1]
        items = [dict(packed=L["q"][0], qs=L["q"][1], bias=L["q_bias"], lora_u=uq, lora_b=bq, lora_scale=s),
                 dict(packed=L["k"][0], qs=L["k"][1], bias=L["k_bias"]),
                 dict(packed=L["v"][0], qs=L["v"][1], bias=L["v_bias"], lora_u=uv, lora_b=bv, lora_scale=s)]
        nf4.linear_forward(x, items, lora_rank=LORA_R)
        nf4.linear_forward(attn, [dict(packed=L["o"][0], qs=L["o"][1])])
        gate, up, h = nf4.glu_forward(x2, dict(packed=L["gate"][0], qs=L["gate"][1]),
                                      dict(packed=L["up"][0], qs=L["up"][1]))
        nf4.linear_forward(h, [dict(packed=L["down"][0], qs=L["down"][1])])
        return uq, uv, gate, up

    def layer_back(L, li, saved, lora_kernels):
        uq, uv, gate, up = saved
        (aq, bq), (av, bv) = L["q_lora"], L["v_lora"]
        dgate, dup = nf4.linear_backward_swiglu(dict(packed=L["down"][0], qs=L["down"][1], dy=dy), gate, up,
                                                out=(gate, up))
        nf4.linear_backward([dict(packed=L["gate"][0], qs=L["gate"][1], dy=dgate),
                             dict(packed=L["up"][0], qs=L["up"][1], dy=dup)], M, HIDDEN)
        nf4.linear_backward([dict(packed=L["o"][0], qs=L["o"][1], dy=dy)], M, HIDDEN)
        if lora_kernels:
            (guq, _, _), (guv, _, _) = lora.lora_grads_group([dict(dy16=dq, u16=uq, x=x, b16=bq, scaling=s),
                                                              dict(dy16=dkv, u16=uv, x=x, b16=bv, scaling=s)])
        else:
            guq, guv = pre[li][2], pre[li][3]
        nf4.linear_backward([dict(packed=L["q"][0], qs=L["q"][1], dy=dq, lora_gu=guq, lora_a=aq),
                             dict(packed=L["k"][0], qs=L["k"][1], dy=dkv),
                             dict(packed=L["v"][0], qs=L["v"][1], dy=dkv, lora_gu=guv, lora_a=av)],
                            M, HIDDEN, lora_rank=LORA_R)

    def step(lora_kernels=True):
        saved = [layer_step(L, li, lora_kernels) for li, L in enumerate(layers)]
        for li in reversed(range(n_layers)):
            layer_back(layers[li], li, saved[li], lora_kernels)

    for li, L in enumerate(layers):
        (aq, bq), (av, bv) = L["q_lora"], L["v_lora"]
        uq, uv = lora.lora_down(x, aq), lora.lora_down(x, av)
        pre[li] = (uq, uv, lora.lora_grads(dq, uq, x, bq, s)[0], lora.lora_grads(dkv, uv, x, bv, s)[0])
    step()  # fills the descriptor cache of every weight
    torch.cuda.synchronize()
    res = {}
    for name, lk in (("step", True), ("gemm_only", False)):
        for _ in range(warmup):
            step(lk)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            step(lk)
        b.record()
        torch.cuda.synchronize()
        res[name] = a.elapsed_time(b) / steps
    launches, busy = count_kernels(step)
    base, lora_f = stack_flops(n_layers)
    return dict(
        workload=f"Qwen2.5-1.5B {n_layers} layers x {{q,k,v,o,gate,up,down}} NF4 (bs 64, double quant) + "
                 f"LoRA r=16 on q/v, M={M}, one training step: 8 fused dequant-GEMM launches per layer "
                 f"({7 * n_layers} forward + {7 * n_layers} input-gradient GEMMs) + 3 LoRA side launches "
                 f"(U of q and v in one; GU with dB of q and v in one, then dA of q and v in one)",
        ms_per_step=round(res["step"], 4), dequant_gemm_ms=round(res["gemm_only"], 4),
        dequant_gemm_share=round(res["gemm_only"] / res["step"], 4),
        tflops=round((base + lora_f) / (res["step"] * 1e-3) / 1e12, 1),
        gemm_tflops=round(base / (res["gemm_only"] * 1e-3) / 1e12, 1),
        frac=round(base / (res["gemm_only"] * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4),
        step_gflops=round((base + lora_f) / 1e9, 1), launches_per_step=launches,
        gpu_busy_ms=None if busy is None else round(busy / 1e3, 4),
        note="ms_per_step: steps back to back (HIP events); gpu_busy_ms: the kernels' summed durations in "
             "one profiled step (the gap to ms_per_step is host launch overhead)")


# ---- config C5: the Qwen2.5-7B sweep -----------------------------------------------------------

QWEN7_SHAPES = [("q/o", 3584, 3584), ("k/v", 512, 3584), ("gate/up", 18944, 3584), ("down", 3584, 18944)]
C5_M = (1, 8, 64, 830, 8192)


def fused_bytes(n, k, m):
    """Algorithmic HBM bytes of one fused call: the NF4 weight once, X in and Y out (fp16)."""
    return nf4_bytes(n, k) + 2 * m * (n + k)


def bench_c5(device, reps=3, min_bytes=512 << 20, m_list=C5_M, shapes=tuple(s[0] for s in QWEN7_SHAPES)):
    """Each 7B projection shape at every M: forward Y = X.W^T (the GEMV kernel at M = 1, the
    small-M kernel at M = 8, the MFMA kernels above) and, for M >= 64, the input gradient
    dX = dY.W. Enough copies of the weight to total more than 512 MB of NF4 data are called back
    to back, so every call reads its weight from HBM (the 256 MB Infinity Cache cannot hold the
    set) while X / dY stay cached, as they would between consecutive layers. The calls are
    captured once in a HIP graph and the graph is replayed: what is timed is the GPU's work (the
    host's per-call Python and launch cost would otherwise bound the small shapes). Each replay's
    last output is checked against the same call run eagerly; a shape whose capture fails or
    differs is timed eagerly instead (`timing` says which). Per-call time = replay time / copies,
    median of `reps` replays."""
    import torch

    from decik_amd import nf4
    from decik_amd.quant import quantize_nf4

    rows = []
    for si, (name, n, k) in enumerate(QWEN7_SHAPES):
        if name not in shapes:
            continue
        copies = max(2, min(600, -(-min_bytes // nf4_bytes(n, k))))
        base = seeded_fp16((n, k), 30_000 + si, 0.02, device)
        ws = []
        for c in range(copies):
            # distinct weights (a sign flip of a seeded pattern per copy) so no two calls share lines
            ws.append(quantize_nf4(base if c % 2 == 0 else -base, blocksize=64, compress_statistics=True))
        del base
        for m in m_list:
            x = seeded_fp16((m, k), 31_000 + m, 1.0, device)
            dy = seeded_fp16((m, n), 32_000 + m, 1e-2, device)
            kinds = {"fwd": lambda p, q: nf4.linear_forward(x, [dict(packed=p, qs=q)])[0]}
            if m >= 64:
                kinds["bwd"] = lambda p, q: nf4.linear_backward([dict(packed=p, qs=q, dy=dy)], m, k)
            for d, call in kinds.items():
                for p, q in ws:  # fills the descriptor and block-scale caches and the workspace
                    call(p, q)
                torch.cuda.synchronize()
                ref = call(*ws[-1]).clone()
                timing = "graph"
                try:
                    g = torch.cuda.CUDAGraph()
                    side = torch.cuda.Stream()
                    side.wait_stream(torch.cuda.current_stream())
                    with torch.cuda.stream(side):
                        call(*ws[0])  # warm-up on the capture stream
                    torch.cuda.current_stream().wait_stream(side)
                    torch.cuda.synchronize()
                    outs = []
                    with torch.cuda.graph(g):
                        for p, q in ws:
                            outs.append(call(p, q))
                    g.replay()
                    torch.cuda.synchronize()
                    if not torch.equal(outs[-1], ref):
                        raise RuntimeError("graph replay differs from the eager call")
                    run = g.replay
                except Exception:  # noqa: BLE001 - timed eagerly instead
                    timing, g, outs = "eager", None, None
                    run = lambda: [call(p, q) for p, q in ws]  # noqa: E731
                times = []
                for _ in range(reps):
                    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    a.record()
                    run()
                    b.record()
                    torch.cuda.synchronize()
                    times.append(a.elapsed_time(b) / copies)
                if outs is not None and not torch.equal(outs[-1], ref):
                    raise RuntimeError(f"C5 {name} m={m} {d}: a graph replay differs from the eager call")
                del g, outs
                ms = statistics.median(times)
                fl = gemm_flops(n, k, m)
                by = fused_bytes(n, k, m)
                plan = nf4.launch_plan(d == "bwd", m, k, [n])
                rows.append([name, m, d, round(ms * 1e3, 2), round(by / (ms * 1e-3) / 1e9, 1),
                             round(by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), round(fl / (ms * 1e-3) / 1e12, 2),
                             round(fl / (ms * 1e-3) / 1e12 / FP16_PEAK_TFLOPS, 4), plan["kernel"], plan["splits"],
                             plan["launches"], copies, timing])
            torch.cuda.empty_cache()
        del ws
        torch.cuda.empty_cache()
    return dict(workload="Qwen2.5-7B projections (NF4 bs 64, double quant, statistics as stored), each shape "
                         "and M: back-to-back calls over weight copies totalling > 512 MB (weights from HBM), "
                         "replayed from a HIP graph",
                shapes={name: [n, k] for name, n, k in QWEN7_SHAPES},
                columns=["shape", "m", "dir", "us", "gbs", "hbm_frac", "tflops", "mfma_frac", "kernel", "splits",
                         "gemm_launches", "copies", "timing"],
                rows=rows)


def mlp_plan(kind):
    """The launch plan of MLP launch `kind` as the library's planner chooses it (host-only)."""
    from decik_amd import nf4

    args = {"fwd_gate_up": (False, HIDDEN, [INTER, INTER], True), "fwd_down": (False, INTER, [HIDDEN], False),
            "bwd_down": (True, INTER, [HIDDEN], True), "bwd_gate_up": (True, HIDDEN, [INTER, INTER], False)}[kind]
    plan = nf4.launch_plan(args[0], M, args[1], args[2], glu=args[3])
    # the form in which the kernels read nested statistics (the bytes a launch moves depend on it)
    plan["statistics"] = "fp32 block scales" if nf4._launch_scales is nf4._scales else "as stored"
    return plan


def load_traffic(kind):
    """(HBM bytes per call of launch `kind`, None) from the committed rocprofv3 --pmc FETCH_SIZE /
    WRITE_SIZE summary (profiles/traffic.json, made with `bench.py --only <kind>`), or (None, why)
    if that summary covers another launch or was measured on another launch plan than the
    planner's current one (a stale summary)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        if t["launch"] != kind:
            return None, f"profiles/traffic.json covers {t['launch']}"
        if t.get("plan") != mlp_plan(kind):
            return None, f"profiles/traffic.json was measured on plan {t.get('plan')}, the planner now picks {mlp_plan(kind)}"
        return t["bytes_per_call"], None
    except (OSError, ValueError, KeyError, TypeError) as e:
        return None, f"profiles/traffic.json unreadable ({type(e).__name__})"


def copy_probe(device):
    """The fp32 -> fp16 conversion of 128 Mi values three times: one elementwise kernel of known
    traffic (512 MiB read, 256 MiB written) that scales rocprofv3's FETCH_SIZE / WRITE_SIZE."""
    import torch

    src = torch.ones(128 << 20, dtype=torch.float32, device=device)
    dst = torch.empty(128 << 20, dtype=torch.float16, device=device)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--skip-dequant", action="store_true")
    ap.add_argument("--skip-configs", action="store_true",
                    help="skip the attention-projection step (C3), the 28-layer stack step (C4) and "
                         "the Qwen2.5-7B sweep (C5)")
    ap.add_argument("--configs", default="c3,c4,c5",
                    help="comma-separated subset of c3, c4, c5 to run besides the headline MLP step")
    ap.add_argument("--only", default=None,
                    choices=["fwd_gate_up", "fwd_down", "bwd_down", "bwd_gate_up", "dequant", "c5"],
                    help="time only this launch kind, or the standalone dequantization (for counter runs); "
                         "prints its roofline only")
    ap.add_argument("--c5-m", default=",".join(str(m) for m in C5_M),
                    help="token counts of the Qwen2.5-7B sweep (C5)")
    ap.add_argument("--c5-shapes", default=",".join(s[0] for s in QWEN7_SHAPES),
                    help="projections of the Qwen2.5-7B sweep (C5): q/o, k/v, gate/up, down")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also convert 128 Mi fp32 values to fp16 three times: one elementwise "
                         "kernel of known traffic (512 MiB read, 256 MiB written), to scale "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: measures one GPU only (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE={world}); the NF4 path needs no collectives and is not run on several GPUs.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from decik_amd import _lib

    _lib.lib()  # fails loudly if the HIP library was not built
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)

    c5_m = tuple(int(v) for v in args.c5_m.split(",") if v.strip())
    c5_shapes = tuple(v.strip() for v in args.c5_shapes.split(",") if v.strip())
    if args.only == "c5":
        # counter runs of the 7B sweep alone (the small-M kernels' traffic)
        if args.copy_probe:
            copy_probe(device)
        with no_gc():
            print(json.dumps(dict(only="c5", c5_qwen7b_sweep=bench_c5(device, m_list=c5_m, shapes=c5_shapes))))
        return
    if args.only == "dequant":
        if args.copy_probe:
            copy_probe(device)
        with no_gc():
            deq = bench_dequant(max(args.steps, 10), args.warmup, device)
        print(json.dumps(dict(only="dequant", gbs=round(deq["gbs"], 1), ms=round(deq["ms"], 4), bytes=deq["bytes"],
                              frac=round(deq["gbs"] / HBM_PEAK_GBS, 4))))
        return
    with no_gc():
        mlp = bench_mlp(args.steps, args.warmup, device, only=args.only)
    baselines = None
    if args.only is None and not args.skip_configs:
        torch.cuda.empty_cache()
        with no_gc():
            baselines = bench_mlp_gpu_baselines(args.steps, args.warmup, device, mlp["ms_step"])
    if args.copy_probe:
        copy_probe(device)
    with no_gc():
        deq = None if (args.skip_dequant or args.only) else bench_dequant(max(args.steps, 10), args.warmup, device)
        deq_cached = None if deq is None else bench_dequant(max(args.steps, 10), args.warmup, device, n_layers=8)
    torch.cuda.empty_cache()
    c3 = c4 = c5 = None
    configs = set() if (args.skip_configs or args.only) else {c.strip() for c in args.configs.split(",") if c.strip()}
    if "c3" in configs:
        with no_gc():
            c3 = bench_c3(max(args.steps, 10), args.warmup, device)
        torch.cuda.empty_cache()
    if "c4" in configs:
        with no_gc():
            c4 = bench_c4(max(2, min(args.steps, 5)), 1, device)
        torch.cuda.empty_cache()
    if "c5" in configs:
        with no_gc():
            c5 = bench_c5(device, m_list=c5_m, shapes=c5_shapes)
        torch.cuda.empty_cache()

    # Dominant launch: the fused GEMM call with the largest time. Its kernels: the GEMM kernel,
    # plus splitk_reduce_kernel when the call takes the split-K path. `achieved` = the call's
    # algorithmic flops / its average duration (HIP events on the launch stream around
    # back-to-back calls); rocprofv3 lists the same call as the sum of its kernels' durations.
    gemm = [k for k in mlp["launch_ms"] if mlp["flops"][k]]
    dom = max(gemm, key=lambda k: mlp["launch_ms"][k])
    ms = mlp["launch_ms"][dom]
    achieved = mlp["flops"][dom] / (ms * 1e-3) / 1e12
    kern = mlp["symbol"][dom] + (" + splitk_reduce_kernel" if split_launch(dom) else "")
    traffic, traffic_note = load_traffic(dom)
    roofline = dict(kernel=kern, launch=dom, bound="mfma", achieved=round(achieved, 2),
                    peak=FP16_PEAK_TFLOPS, unit="TFLOP/s", frac=round(achieved / FP16_PEAK_TFLOPS, 4),
                    flops_per_launch=mlp["flops"][dom], avg_launch_ms=round(ms, 5),
                    traffic=traffic, plan=mlp_plan(dom))
    if traffic_note is not None:
        roofline["traffic_note"] = traffic_note
    if args.only is not None:
        print(json.dumps(dict(only=args.only, roofline=roofline)))
        return
    value = mlp["step_flops"] / (mlp["ms_step"] * 1e-3) / 1e12
    peaks = measured_peaks(device)
    roofline["frac_of_measured"] = round(achieved / peaks["mfma_f16_tflops"], 4)
    line = dict(
        metric=METRIC, value=round(value, 2), unit="TFLOP/s", n_gpus=1, steps=args.steps,
        warmup=args.warmup, ms_per_step=round(mlp["ms_step"], 4), higher_is_better=True,
        scaling="weak", vs_baseline=None, dtype="fp16", data="synthetic",
        config=dict(workload="Qwen2.5-1.5B MLP block fwd+bwd on NF4 weights: gate/up [8960,1536], "
                             "down [1536,8960], blocksize 64, double quant; X [830,1536]; SwiGLU; "
                             "dX through W; gate/up kept from the forward",
                    m=M, hidden=HIDDEN, intermediate=INTER, weight_sets=mlp["n_sets"],
                    block_scales="bitsandbytes' double-quant statistics as stored (uint8 absmax codes, "
                                 "fp32 absmax2 and offset), each block's scale formed in the kernels; "
                                 "kernels_cached_scales times the same launches on fp32 block scales "
                                 "derived once per frozen weight (+12.5% of the packed bytes)"),
        roofline=roofline,
        measured_peaks=peaks,
        kernels={k: dict(ms=round(v, 4),
                         tflops=round(mlp["flops"][k] / (v * 1e-3) / 1e12, 1) if mlp["flops"][k] else None)
                 for k, v in mlp["launch_ms"].items()},
        kernels_cached_scales={k: dict(ms=round(v, 4), tflops=round(mlp["flops"][k] / (v * 1e-3) / 1e12, 1))
                               for k, v in mlp["cached_ms"].items()},
        graph_step=None if mlp["graph_ms"] is None else dict(
            ms_per_step=round(mlp["graph_ms"], 4),
            tflops=round(mlp["step_flops"] / (mlp["graph_ms"] * 1e-3) / 1e12, 2),
            note="the same step captured once in a HIP graph (one step per weight set) and replayed; "
                 "value stays the eager step"),
    )
    if baselines is not None:
        line["gpu_baselines"] = baselines
    if c3 is not None:
        line["c3_attention_step"] = c3
    if c4 is not None:
        line["c4_stack_step"] = c4
    if c5 is not None:
        line["c5_qwen7b_sweep"] = c5
    # the dequantization last but one: the end of the line is what a truncated log keeps
    if deq is not None:
        probe = mixed_ceiling(peaks, deq["read"], deq["write"])
        roof = dict(bound="hbm", achieved=round(deq["gbs"], 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(deq["gbs"] / HBM_PEAK_GBS, 4), probe_mix_gbs=round(probe, 1))
        if deq["gbs"] <= probe:
            roof["frac_of_measured"] = round(deq["gbs"] / probe, 4)
        else:
            # the streaming probes do not reach this kernel's own rate: no measured ceiling is claimed
            roof["note"] = ("the dequantization runs above dk_probe_hbm's rates for its read/write mix "
                            "(every probe variant, 64 MB to 1 GiB buffers): no measured ceiling is "
                            "claimed, frac is against the published peak")
        line["dequant"] = dict(value=round(deq["gbs"], 1), unit="GB/s", ms=round(deq["ms"], 4),
                               bytes=deq["bytes"], launches=deq["launches"],
                               workload="all 7 Qwen2.5-1.5B projections x 24 layers per iteration (561 MB "
                                        "packed: read from HBM, past the 256 MB Infinity Cache)",
                               roofline=roof,
                               cache_resident=dict(value=round(deq_cached["gbs"], 1), unit="GB/s",
                                                   workload="x 8 layers (187 MB packed, stays in the "
                                                            "Infinity Cache between iterations)"))
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline()
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line))


if __name__ == "__main__":
    main()
