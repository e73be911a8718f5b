"""The qmv_rows oracle (oracle/qmv.py, the reference's route_cuda.qmv_rows, route_cuda.py:460-541) pinned without
the reference (MLX and CUDA are absent): exact small-integer cases, where every bf16 step is exact and the result
is the exact dot product rounded once (this pins the nibble order, the group indexing and the lane / slot / base
split, K past a multiple of 512 included); a hand-derived case where the bf16 slot accumulators lose what a
float32 accumulation keeps; and bf16 rounding against torch's."""
import numpy as np
import torch

from oracle import qmv


def pack(q):
    """int [N, K] 4-bit values -> uint32 [N, K / 8], element j of a word at bits 4j."""
    N, K = q.shape
    q = q.astype(np.uint32).reshape(N, K // 8, 8)
    out = np.zeros((N, K // 8), np.uint32)
    for j in range(8):
        out |= q[:, :, j] << np.uint32(4 * j)
    return out


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(50000) * np.exp(rng.uniform(-30, 30, 50000))).astype(np.float32)
    want = torch.from_numpy(x).bfloat16().float().numpy()
    assert (qmv.bf16(x) == want).all()
    assert list(qmv.bf16([257.0, 259.0, 1 + 2.0 ** -8, -(1 + 3 * 2.0 ** -8)])) == [256.0, 260.0, 1.0, -1.015625]


def test_unpack_order():
    w = np.array([[0x76543210, 0xFEDCBA98]], np.uint32)
    assert qmv.unpack4(w, 16).tolist() == [list(range(16))]


def test_exact_integer_cases():
    """Small integers keep every bf16 product and slot sum exact, so out = bf16(exact dot)."""
    rng = np.random.default_rng(1)
    for K, G, T in ((512, 32, 1), (1024, 64, 3), (528, 16, 2), (1040, 16, 1), (64, 32, 2)):
        N = 6
        q = rng.integers(0, 16, (N, K))
        s = rng.choice([0.5, 1.0, 2.0], (N, K // G)).astype(np.float32)
        b = rng.choice([-8.0, -4.0, 0.0, 2.0], (N, K // G)).astype(np.float32)
        x = rng.integers(-2, 3, (T, K)).astype(np.float32)
        w = pack(q)
        got = qmv.qmv_rows(x, w, s, b, G)
        wf = q * np.repeat(s, G, axis=1) + np.repeat(b, G, axis=1)
        exact = x.astype(np.float64) @ wf.T.astype(np.float64)
        assert (got == qmv.bf16(exact)).all(), (K, G, T)
        # a transposed nibble order or a shifted group gives another exact result
        wrong = pack(q[:, ::-1].copy())
        assert not (qmv.qmv_rows(x, wrong, s, b, G) == got).all()


def test_bf16_slot_accumulation():
    """K = 1536: lane 0's slot 0 takes elements 0, 512 and 1024. With weights 256, 1, 1 there and 0 elsewhere
    (x = 1), the bf16 slot sum is bf16(bf16(256 + 1) + 1) = 256, where the exact dot (and a float32 accumulation)
    gives 258 = bf16(258)."""
    K, G = 1536, 32
    q = np.zeros((1, K), np.int64)
    s = np.ones((1, K // G), np.float32)
    b = np.zeros((1, K // G), np.float32)
    q[0, 0], s[0, 0] = 8, 32.0          # 8 * 32 = 256
    q[0, 512] = 1
    q[0, 1024] = 1
    x = np.ones((1, K), np.float32)
    got = qmv.qmv_rows(x, pack(q), s, b, G)
    assert got[0, 0] == 256.0
    assert qmv.bf16(258.0) == 258.0


def test_weight_rounding_is_two_steps():
    """w = bf16(bf16(q s) + b), two roundings: q = 3, s = 1.0078125, b = -0.14453125 gives q s = 3.0234375 ->
    3.03125 (a tie, to even), + b = 2.88671875 -> 2.890625; one fused rounding would give bf16(2.87890625) =
    2.875."""
    K, G = 16, 16
    q = np.zeros((1, K), np.int64)
    q[0, 0] = 3
    s = np.full((1, 1), 1.0078125, np.float32)
    b = np.full((1, 1), -0.14453125, np.float32)
    x = np.zeros((1, K), np.float32)
    x[0, 0] = 1.0
    # every other weight is b (q = 0): x is 0 there
    assert qmv.qmv_rows(x, pack(q), s, b, G)[0, 0] == 2.890625


def test_random_close_to_exact():
    rng = np.random.default_rng(2)
    N, K, G = 32, 2048, 64
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    wq, s, b = qmv.quantize_affine4(w, G)
    x = qmv.bf16(rng.standard_normal((3, K)))
    got = qmv.qmv_rows(x, wq, s, b, G).astype(np.float64)
    exact = x.astype(np.float64) @ qmv.dequant_affine4(wq, s, b, G).T
    assert np.linalg.norm(got - exact) / np.linalg.norm(exact) < 2e-2
    # the quantizer's round trip
    back = qmv.dequant_affine4(wq, s, b, G)
    assert np.linalg.norm(back - w) / np.linalg.norm(w) < 0.12


def midpoint_products(rng, n):
    """bf16 pairs (x, w) in [1, 2) whose product lies exactly on a bf16 rounding midpoint."""
    out = []
    while len(out) < n:
        x = 1 + rng.integers(0, 128) / 128.0
        w = 1 + rng.integers(0, 128) / 128.0
        p = x * w
        _, e = np.frexp(p)
        ulp = 2.0 ** (e - 8)
        if p % ulp == ulp / 2:
            out.append((x, w, p))
    return out


def test_fma_single_rounding_at_midpoints():
    """x w exactly on a midpoint plus a tiny a: one rounding goes toward a's sign; rounding x w + a to float32 or
    float64 first would land on the midpoint and go to even."""
    rng = np.random.default_rng(5)
    for x, w, p in midpoint_products(rng, 20):
        _, e = np.frexp(p)
        ulp = 2.0 ** (e - 8)
        lo = np.floor(p / ulp) * ulp
        for a, want in ((2.0 ** -60, lo + ulp), (-(2.0 ** -60), lo), (0.0, float(qmv.bf16(p)))):
            assert qmv.fma_bf16(x, w, a) == want, (x, w, a)
        assert float(qmv.bf16(np.float32(p) + np.float32(2.0 ** -60))) == float(qmv.bf16(p))  # the double rounding
    # the rest of the time it is the plain rounding of the exact value
    x, w, a = (qmv.bf16(rng.standard_normal(20000)) for _ in range(3))
    assert (qmv.fma_bf16(x, w, a) == qmv.bf16(x.astype(np.float64) * w + a)).mean() > 0.999
