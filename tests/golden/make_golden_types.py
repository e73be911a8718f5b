#!/usr/bin/env python3
"""Writes tests/golden/dequant_types.npz: Q4_1, Q5_K, Q6_K and Q8_0 input blocks and the reference's own
dequantized float32 weights, as make_golden.py does for Q4_0 and Q4_K.

The bit layouts (nibble and high-bit placement, Q5_K's fifth bit, Q6_K's ql/qh split and int8 scales) are
conventions no closed form fixes, so they are pinned against the reference's numpy restatement of ggml,
``gguf_ref.ref_dequant`` (/root/reference/gguf_ref.py:546-553; Q4_1 :345-351, Q5_K :261-276, Q6_K :392-401,
Q8_0 :354-355). This script imports that one pure-numpy module from the read-only reference checkout (run here, in
the build container, never on a GPU box) and stores only data: the blocks fed in and the weights it returned.

    python3 tests/golden/make_golden_types.py [/root/reference]

Blocks: random bytes with finite f16 scales, edge blocks (d = 0, negative, f16-subnormal, the largest finite f16,
+-inf and NaN; all-0x00, all-0xFF and mixed bytes), Q5_K / Q6_K blocks whose scale bytes take every high-bit
pattern, and blocks from this build's own quantizers (oracle.gguf) on Gaussian weights.
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
sys.path.insert(0, str(HERE))
from make_golden import load_ref   # noqa: E402

NEW = ("Q4_1", "Q5_K", "Q6_K", "Q8_0")


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
    if t == "Q5_K":
        for v in (0x00, 0x3F, 0x40, 0x80, 0xC0, 0xFF):
            e = rng.integers(0, 256, bb, dtype=np.uint8)
            e[0:4] = np.array([0.02, 0.004], np.float16).view(np.uint8)
            e[4:16] = v
            edge.append(e)
    if t == "Q6_K":
        for v in (0x00, 0x7F, 0x80, 0xFF, 0x01):
            e = rng.integers(0, 256, bb, dtype=np.uint8)
            e[192:208] = v
            e[208:210] = np.array([0.003], np.float16).view(np.uint8)
            edge.append(e)
    w = (rng.standard_normal((8, 512)) * 0.02).astype(np.float32)
    q = gguf.QUANTIZE[t](w).reshape(-1, bb)
    return np.concatenate([b, np.stack(edge), q], axis=0)


def main():
    ref = load_ref(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    rng = np.random.default_rng(20261202)
    out = {}
    for t in NEW:
        b = blocks(rng, t, 96)
        out[f"{t}_blocks"] = b
        out[f"{t}_want"] = ref.ref_dequant(b.reshape(-1), t).astype(np.float32)
        out[f"{t}_valid"] = np.array([bool(ref.valid(b[i], t)) for i in range(len(b))])
    np.savez_compressed(HERE / "dequant_types.npz", **out)
    print("wrote", HERE / "dequant_types.npz", {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
