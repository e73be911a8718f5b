"""The CPU baseline (oracle/cpu_kern_port.cpp, a restatement of cpu_ext/cpu_kern.cpp's gather_qmm) against float64
numpy with the reference test's tolerance: f32 outputs within 1e-5 of the row's sum |x| |w|
(tests/test_cpu_kern.py:5-6, 39-46), on the gather shapes a MoE layer uses, and the lossless GGUF -> affine
conversion (Q4_0: scale d, bias -8 d; Q4_K: scale d sc, bias -dmin m)."""
import numpy as np
import pytest

from oracle import cpu_baseline as cb
from oracle import gguf, moe


def check(y, x64, w64):
    ref = x64 @ w64.T
    scale = np.abs(x64) @ np.abs(w64.T)
    assert (np.abs(y - ref) <= 1e-5 * scale + 1e-30).all(), float((np.abs(y - ref) / (scale + 1e-30)).max())


@pytest.mark.parametrize("t,N,K", [("Q4_0", 72, 512), ("Q4_0", 40, 2048), ("Q4_K", 64, 512), ("Q4_K", 24, 1024)])
@pytest.mark.parametrize("threads", [1, 4])
def test_gather_qmm_vs_float64(t, N, K, threads):
    cb.lib().ckp_set_threads(threads)
    rng = np.random.default_rng(N + K)
    E = 6
    w = gguf.random_experts(rng, E, N, K, t)
    A = cb.Affine(w, t, K)
    w64 = gguf.dequant_matrix(w, t).astype(np.float64)
    for rows in (1, 3, 17, 70):
        x = rng.standard_normal((rows, K)).astype(np.float32)
        idx = rng.integers(0, E, rows).astype(np.uint32)
        idx[0] = E + 1                                   # no such expert: zeros
        y = cb.gather_qmm(x, A, idx)
        assert (y[0] == 0).all()
        for r in range(1, rows):
            check(y[r:r + 1], x[r:r + 1].astype(np.float64), w64[idx[r]])


def test_affine_conversion_is_lossless():
    rng = np.random.default_rng(3)
    for t, K in (("Q4_0", 256), ("Q4_K", 512)):
        w = gguf.random_experts(rng, 2, 8, K, t)
        A = cb.Affine(w, t, K)
        q = np.stack([A.w & 15, A.w >> 4], axis=-1).reshape(2, 8, K).astype(np.float32)
        back = q * np.repeat(A.sc, 32, -1) + np.repeat(A.bi, 32, -1)
        assert (back == gguf.dequant_matrix(w, t)).all(), t


@pytest.mark.parametrize("t", ["Q4_0", "Q4_K"])
def test_cpu_layer_vs_oracle(t):
    cb.lib().ckp_set_threads(2)
    rng = np.random.default_rng(7)
    H, I, E, k = 512, 256, 8, 3
    w = tuple(gguf.random_experts(rng, E, r, c, t) for r, c in ((I, H), (I, H), (H, I)))
    G, U, D = cb.Affine(w[0], t, H), cb.Affine(w[1], t, H), cb.Affine(w[2], t, I)
    x = rng.standard_normal((4, H)).astype(np.float32)
    wr = (rng.standard_normal((E, H)) * 0.05).astype(np.float16)
    out = cb.moe_layer(x, wr, k, True, G, U, D, residual=x)
    lg = x @ wr.astype(np.float32).T
    _, _, want = moe.layer(x, lg, w, (t,) * 3, k, True, residual=x)
    assert moe.rel_l2(out, want) < 1e-5
