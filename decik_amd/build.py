"""Build the HIP library libdecik_nf4.so in-tree (gfx950) with hipcc.

python -m decik_amd.build            # build
python -m decik_amd.build --asm DIR  # also keep the AMDGPU assembly of the kernels in DIR
"""

import argparse
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libdecik_nf4.so")
SOURCES = ["capi.hip", "nf4_dequant.hip", "nf4_fwd.hip", "nf4_fwd8.hip", "nf4_gemv.hip", "nf4_skinny.hip", "nf4_bwd8.hip", "splitk.hip", "lora.hip", "lora_dropout.hip", "rope.hip", "swiglu.hip", "probe.hip"]
ARCH = os.environ.get("DECIK_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
    # two roundings for the double-quant scale, as the reference (no contraction into FMA)
    "-ffp-contract=off",
    # keep fp32 subnormals (bit-exact dequant of tiny scales)
    "-fno-gpu-flush-denormals-to-zero",
    # no packed-fp32 instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", "hipcc"):
        if cand and (os.path.isabs(cand) and os.path.exists(cand) or not os.path.isabs(cand)):
            return cand
    return "hipcc"


OBJ_DIR = os.path.join(HERE, "_build")


def build(asm_dir=None, verbose=False, jobs=None):
    """Compile every source to an object file (in parallel), then link the shared library."""
    from concurrent.futures import ThreadPoolExecutor

    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    os.makedirs(OBJ_DIR, exist_ok=True)
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
    cflags = [f for f in FLAGS if f != "-shared"]

    def compile_one(src):
        obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
        cmd = [hipcc()] + cflags + inc + ["-c", "-o", obj, src]
        if verbose:
            print(" ".join(cmd))
        subprocess.run(cmd, check=True)
        return obj

    jobs = jobs or min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = LIB + ".tmp"
    subprocess.run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs, check=True)
    os.replace(tmp, LIB)
    if asm_dir:
        os.makedirs(asm_dir, exist_ok=True)
        for s in srcs:
            out = os.path.join(asm_dir, os.path.basename(s) + ".s")
            subprocess.run([hipcc()] + [f for f in FLAGS if f not in ("-shared", "-fPIC")] +
                           ["-I", os.path.join(ROOT, "include"), "-I", CSRC,
                            "--cuda-device-only", "-S", "-o", out, s], check=True)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--asm", default=None)
    ap.add_argument("-v", action="store_true")
    args = ap.parse_args()
    print(build(args.asm, args.v))
    sys.exit(0)
