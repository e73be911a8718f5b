"""Builds larder_amd/liblarder_moe.so for gfx950 with hipcc, in-tree.

    python3 -m larder_amd.build          # compile every .hip under larder_amd/csrc and link the library

Each source compiles to larder_amd/_build/<name>.o in parallel, then one link. Packed-FP32 instruction
selection is switched off (-Xclang -target-feature -Xclang -packed-fp32-ops) and floating-point contraction is off
(-ffp-contract=off) for every compile.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
SRC = PKG / "csrc"
OUT_DIR = PKG / "_build"
LIB = PKG / "liblarder_moe.so"
ARCH = os.environ.get("LMOE_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -ffp-contract=off: every multiply and add rounds on its own unless written as an explicit fmaf / builtin (the
# reference's CUDA prelude does the same with MUL/ADD _rn, gguf_cuda.py:4-20), so dequant and quantizer rounding
# follow ggml's exactly.
CFLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off", "-Xclang", "-target-feature",
          "-Xclang", "-packed-fp32-ops", "-Wall", "-Wno-unused-function", "-Wno-unused-variable"]

# Per-file extras. grouped.hip: MFMA accumulators in arch VGPRs. Left to its heuristics the compiler puts them in
# AGPRs with the untied MFMA form, and every K step then rotates them through ~130 accvgpr moves; in VGPRs they
# stay put and the kernel fits two workgroups a CU (237 VGPRs, no AGPRs).
FILE_FLAGS = {"grouped.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def sources():
    return sorted(SRC.glob("*.hip"))


def build(verbose=False):
    """Compile and link; returns the library path. Always recompiles (this is the 'does it build' check)."""
    OUT_DIR.mkdir(exist_ok=True)
    srcs = sources()
    objs = [OUT_DIR / (s.stem + ".o") for s in srcs]
    cmds = [[HIPCC, *CFLAGS, *FILE_FLAGS.get(s.name, []), "-c", str(s), "-o", str(o)] for s, o in zip(srcs, objs)]
    with ThreadPoolExecutor(max_workers=min(8, len(cmds))) as ex:
        for c, _ in zip(cmds, ex.map(_run, cmds)):
            if verbose:
                print(" ".join(c), flush=True)
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB, flush=True)
    return LIB


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
