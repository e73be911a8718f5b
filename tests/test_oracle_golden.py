"""The oracle's block decoding against vectors from the reference's own gguf_ref.ref_dequant
(tests/golden/make_golden.py and make_golden_types.py wrote them; gguf_ref.py:546-553, 564-581): bit for bit, NaN for NaN."""
from pathlib import Path

import numpy as np
import pytest

from oracle import gguf

GOLDEN = Path(__file__).resolve().parent / "golden" / "dequant_q4.npz"
GOLDEN_TYPES = Path(__file__).resolve().parent / "golden" / "dequant_types.npz"
ALL = [("Q4_0", GOLDEN), ("Q4_K", GOLDEN), ("Q4_1", GOLDEN_TYPES), ("Q5_K", GOLDEN_TYPES), ("Q6_K", GOLDEN_TYPES),
       ("Q8_0", GOLDEN_TYPES)]


@pytest.mark.parametrize("t,path", ALL)
def test_dequant_matches_reference_vectors(t, path):
    z = np.load(path)
    blocks, want = z[f"{t}_blocks"], z[f"{t}_want"]
    got = gguf.dequant(blocks.reshape(-1), t)
    assert got.dtype == np.float32 and got.shape == want.shape
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all(), f"{t}: {int((~same).sum())} weights differ from gguf_ref.ref_dequant"


@pytest.mark.parametrize("t,path", ALL)
def test_valid_matches_reference_vectors(t, path):
    z = np.load(path)
    blocks, want = z[f"{t}_blocks"], z[f"{t}_valid"]
    got = np.array([gguf.valid(b, t) for b in blocks])
    assert (got == want).all()
    assert not want.all() and want.any(), "the fixture holds both finite and non-finite scales"


def test_golden_covers_the_edge_blocks():
    z = np.load(GOLDEN)
    q = z["Q4_0_blocks"]
    d = q[:, 0:2].copy().view(np.float16)[:, 0]
    assert (d == 0).any() and (d < 0).any() and (np.abs(d.astype(np.float32)) < 6.1e-5).any()
    assert ((q[:, 2:] == 0xFF).all(axis=1)).any() and ((q[:, 2:] == 0x00).all(axis=1)).any()
    k = z["Q4_K_blocks"]
    # scale bytes with high bits set exercise sub-blocks 4..7's packing
    assert ((k[:, 4:16] & 0xC0) == 0xC0).all(axis=1).any()
