"""GPU parity of the trunk's 4-bit affine matmul (lmoe_qmv_rows: route_cuda.qmv_rows) against the CPU oracle
(oracle/qmv.py), bit for bit, at the reference test's shapes (tests/test_rows_cuda.py:46-66: the 35B's dense
shapes, g64 and g32, lm_head checked on a slice of its rows) and T = 1..20 rows (passes of 8 rows), plus a planted
bf16 fused multiply-add midpoint and the shared-expert MLP built on it (bf16 SwiGLU: within bf16 rounding)."""
import numpy as np
import pytest
import torch

from oracle import qmv

pytestmark = pytest.mark.gpu


def dev_bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda().bfloat16()


def weights(rng, N, K, G, scale=0.05):
    w = (rng.standard_normal((N, K)) * scale).astype(np.float32)
    wq, s, b = qmv.quantize_affine4(w, G)
    return wq, s, b


def to_dev(wq, s, b):
    return torch.from_numpy(wq.view(np.int32)).cuda(), dev_bf16(s), dev_bf16(b)


def host(t):
    return t.float().cpu().numpy()


SHAPES = [(2048, 8192, 64), (2048, 4096, 64), (2048, 32, 64), (4096, 2048, 64), (2048, 512, 64), (512, 2048, 64),
          (2560, 640, 32), (640, 2560, 32), (528, 40, 16), (1040, 33, 16)]


@pytest.mark.parametrize("K,N,G", SHAPES)
def test_qmv_rows_bit_exact(K, N, G):
    from larder_amd import trunk
    rng = np.random.default_rng(K + N + G)
    wq, s, b = weights(rng, N, K, G)
    W = to_dev(wq, s, b)
    x = qmv.bf16(rng.standard_normal((5, K)) * rng.uniform(0.3, 3.0))
    xd = dev_bf16(x)
    assert trunk.qmv_fits(xd, W[0], W[1], G, 4, "affine", W[2])
    # oracle on a slice of rows when N is large (rows are independent)
    n_chk = min(N, 256)
    for t in (1, 2, 3, 5):
        got = trunk.qmv_rows(xd[:t], W[0], W[1], W[2], G)
        again = trunk.qmv_rows(xd[:t], W[0], W[1], W[2], G)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), again.view(torch.int16))
        want = qmv.qmv_rows(x[:t], wq[:n_chk], s[:n_chk], b[:n_chk], G)
        assert (host(got)[:, :n_chk].view(np.uint32) == want.view(np.uint32)).all(), (K, N, G, t)


def test_qmv_rows_many_rows_and_lm_head_slice():
    """T = 20 (three passes of up to 8 rows), and the reference's lm_head shape 2048 -> 248320 on its first and
    last 128 rows."""
    from larder_amd import trunk
    rng = np.random.default_rng(9)
    K, N, G = 2048, 1024, 64
    wq, s, b = weights(rng, N, K, G)
    x = qmv.bf16(rng.standard_normal((20, K)))
    got = host(trunk.qmv_rows(dev_bf16(x), *to_dev(wq, s, b), G))
    want = qmv.qmv_rows(x, wq[:96], s[:96], b[:96], G)
    assert (got[:, :96] == want).all()
    N = 248320
    wq = rng.integers(0, 2 ** 32, (N, K // 8), dtype=np.uint64).astype(np.uint32)
    s = qmv.bf16(rng.uniform(0.001, 0.01, (N, K // G)))
    b = qmv.bf16(rng.uniform(-0.05, 0.0, (N, K // G)))
    x = qmv.bf16(rng.standard_normal((3, K)))
    got = host(trunk.qmv_rows(dev_bf16(x), *to_dev(wq, s, b), G))
    for sl in (slice(0, 128), slice(N - 128, N)):
        want = qmv.qmv_rows(x, wq[sl], s[sl], b[sl], G)
        assert (got[:, sl] == want).all()


def test_fma_midpoint_on_device():
    """Lane 0's slot 0 gets a tiny product at base 0 and a product exactly on a bf16 midpoint at base 512: one
    rounding goes toward the tiny term's sign (the oracle's fma_bf16), a double rounding would go to even."""
    from larder_amd import trunk
    K, G = 1024, 16
    # weight 1.0078125 (q 1, s 1.0078125, b 0) at elements 0 and 512; x[0] tiny, x[512] = 1.5078125 whose product
    # with 1.0078125 is 1.51959228515625: not a midpoint; search a pair that is
    found = None
    for xv in np.arange(1, 2, 1 / 128):
        for wv in np.arange(1, 2, 1 / 128):
            p = xv * wv
            ulp = 2.0 ** (np.frexp(p)[1] - 8)
            if p % ulp == ulp / 2:
                found = (float(xv), float(wv))
                break
        if found:
            break
    xv, wv = found
    for tiny in (2.0 ** -40, -(2.0 ** -40)):
        q = np.zeros((1, K), np.uint32)
        q[0, 0] = q[0, 512] = 1
        packed = np.zeros((1, K // 8), np.uint32)
        for j in range(8):
            packed |= q[:, j::8] << np.uint32(4 * j)
        s = np.full((1, K // G), wv, np.float32)
        b = np.zeros((1, K // G), np.float32)
        x = np.zeros((1, K), np.float32)
        x[0, 0], x[0, 512] = tiny / wv, xv
        x = qmv.bf16(x)
        want = qmv.qmv_rows(x, packed, s, b, G)
        got = host(trunk.qmv_rows(dev_bf16(x), *to_dev(packed, s, b), G))
        assert got[0, 0] == want[0, 0], (tiny, got, want)


def test_shared_expert_rows():
    from larder_amd import trunk
    rng = np.random.default_rng(4)
    H, I, G, T = 2048, 512, 64, 4
    gate, up, down = weights(rng, I, H, G), weights(rng, I, H, G), weights(rng, H, I, G)
    x = qmv.bf16(rng.standard_normal((T, H)))
    got = host(trunk.shared_expert_rows(dev_bf16(x), (*to_dev(*gate), G), (*to_dev(*up), G),
                                        (*to_dev(*down), G)))
    g = qmv.qmv_rows(x, *gate, G).astype(np.float64)
    u = qmv.qmv_rows(x, *up, G).astype(np.float64)
    h = qmv.bf16(g / (1 + np.exp(-g)) * u)
    want = qmv.qmv_rows(h, *down, G)
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < 1e-2, rel
