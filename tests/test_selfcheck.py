"""The load-time known-answer check (larder_amd.selfcheck) on the CPU: its recorded answers are the oracle's on its
fixed inputs, verify() passes them and refuses a wrong dequant bit pattern or an output off by more than the bar,
and a plausible mistake planted in the oracle changes the answers it would record (so a kernel with that mistake
fails the check). The check itself runs on the GPU in tests/test_gpu_mutants.py."""
import numpy as np
import pytest

from larder_amd import selfcheck as sc
from oracle import gguf, moe


def oracle_answers(t):
    x, w = sc.inputs(t)
    q = gguf.dequant_matrix(w[0], t)
    _, y = moe.gemv(x.astype(np.float16).astype(np.float32), w, np.array([0]), 1, (t,) * 3)
    return sc.digest(q), y[0]


@pytest.mark.parametrize("t", ["Q4_0", "Q4_K"])
def test_recorded_answers_are_the_oracles(t):
    x, w = sc.inputs(t)
    assert (x.astype(np.float16).astype(np.float32) == x).all()        # exact in f16
    for b in w:
        assert gguf.valid(b, t)
    dq, y = oracle_answers(t)
    assert dq == sc.EXPECT_DEQUANT[t]
    got, norm = sc.summary(t, y)
    want, wnorm = sc.EXPECT_Y[t]
    assert np.allclose(got, want, rtol=1e-6, atol=1e-9) and abs(norm - wnorm) <= 1e-6 * wnorm
    sc.verify(t, dq, [("oracle", y)])


@pytest.mark.parametrize("t", ["Q4_0", "Q4_K"])
def test_verify_refuses_wrong_answers(t):
    dq, y = oracle_answers(t)
    rng = np.random.default_rng(1)
    sc.verify(t, dq, [("close", y * (1 + 1e-4 * rng.standard_normal(y.shape)))])
    with pytest.raises(RuntimeError, match="dequant"):
        sc.verify(t, dq[:-1] + ("0" if dq[-1] != "0" else "1"), [("oracle", y)])
    with pytest.raises(RuntimeError, match="off the recorded answer"):
        sc.verify(t, dq, [("off", y * 1.01)])
    with pytest.raises(RuntimeError, match="off the recorded answer"):
        sc.verify(t, dq, [("ok", y), ("one row wrong", np.roll(y, 1))])


def test_planted_mistakes_change_the_answers(monkeypatch):
    """Each mistake, planted in the oracle, gives answers the check refuses."""
    q40, q4k = gguf._DQ["Q4_0"], gguf._DQ["Q4_K"]

    def offset7(b):  # q - 7 for q - 8
        return q40(b) + gguf._f16(b, 0)[:, None]

    def plus_min(b):  # + dmin * m for - dmin * m
        n = b.shape[0]
        _, m = gguf.scale_min_k4(b[:, 4:16])
        return q4k(b) + 2 * np.repeat(gguf._f16(b, 2)[:, None] * m, 32, axis=1).reshape(n, 256)

    for t, name, fn in (("Q4_0", "Q4_0", offset7), ("Q4_K", "Q4_K", plus_min)):
        with monkeypatch.context() as m:
            m.setitem(gguf._DQ, name, fn)
            dq, y = oracle_answers(t)
        with pytest.raises(RuntimeError):
            sc.verify(t, dq, [("mutant", y)])
    with monkeypatch.context() as m:     # SwiGLU without its sigmoid
        m.setattr(moe, "silu_mul", lambda g, u: (np.asarray(g, np.float32) * np.asarray(u, np.float32)))
        dq, y = oracle_answers("Q4_0")
    with pytest.raises(RuntimeError, match="off the recorded answer"):
        sc.verify("Q4_0", dq, [("mutant", y)])
