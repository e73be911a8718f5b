#!/usr/bin/env python3
"""Writes tests/golden/dequant_q4.npz: input blocks and the reference's own dequantized float32 weights.

The block bit layouts (nibble order, the 6-bit scale/min packing of Q4_K) are conventions that no closed form
fixes, so they are pinned against the reference's own numpy restatement of ggml, ``gguf_ref.ref_dequant``
(/root/reference/gguf_ref.py:546-553, Q4_0 :345-351, Q4_K :253-276). This script imports that one pure-numpy
module from the read-only reference checkout (run here, in the build container, never on a GPU box) and
stores only data: the blocks fed in and the float32 weights it returned.

    python3 tests/golden/make_golden.py [/root/reference]

Blocks: random bytes with finite f16 scales (as gguf_ref.random_experts makes them, but drawn here), plus edge
blocks: d = 0, negative d, f16-subnormal d, the largest finite f16 d, +-inf and NaN d (refused by valid()), all-0x00 and all-0xFF nibbles, and blocks
from this build's own quantizers (oracle.gguf) on Gaussian weights.
"""
import importlib.util
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))


def load_ref(ref_root):
    spec = importlib.util.spec_from_file_location("gguf_ref", Path(ref_root) / "gguf_ref.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def blocks(rng, t, n):
    from oracle import gguf
    _, be, bb = gguf.TYPES[t]
    b = rng.integers(0, 256, (n, bb), dtype=np.uint8)
    for at in gguf.HALVES[t]:
        b[:, at:at + 2] = (rng.standard_normal((n, 1)) * 0.01).astype(np.float16).view(np.uint8)
    edge = []
    for d in (0.0, -0.013, 6.0e-8, -3.0e-6, 65504.0, 1.0, -1.0, np.inf, -np.inf, np.nan):
        for fill in (0x00, 0xFF, 0x5A, None):
            e = rng.integers(0, 256, bb, dtype=np.uint8) if fill is None else np.full(bb, fill, np.uint8)
            for at in gguf.HALVES[t]:
                e[at:at + 2] = np.array([d], np.float16).view(np.uint8)
            edge.append(e)
    if t == "Q4_K":
        # scale bytes with every top-two-bit pattern, so the 6-bit packing of sub-blocks 4..7 is exercised
        for v in (0x00, 0x3F, 0x40, 0x80, 0xC0, 0xFF):
            e = rng.integers(0, 256, bb, dtype=np.uint8)
            e[0:4] = np.array([0.02, 0.004], np.float16).view(np.uint8)
            e[4:16] = v
            edge.append(e)
    w = (rng.standard_normal((8, 512)) * 0.02).astype(np.float32)
    q = gguf.QUANTIZE[t](w).reshape(-1, bb)
    return np.concatenate([b, np.stack(edge), q], axis=0)


def main():
    ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    ref = load_ref(ref_root)
    rng = np.random.default_rng(20261201)
    out = {}
    for t in ("Q4_0", "Q4_K"):
        b = blocks(rng, t, 96)
        out[f"{t}_blocks"] = b
        out[f"{t}_want"] = ref.ref_dequant(b.reshape(-1), t).astype(np.float32)
        out[f"{t}_valid"] = np.array([bool(ref.valid(b[i], t)) for i in range(len(b))])
    np.savez_compressed(HERE / "dequant_q4.npz", **out)
    print("wrote", HERE / "dequant_q4.npz", {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
