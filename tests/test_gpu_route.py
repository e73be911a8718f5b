"""GPU parity of the cache-biased route (lmoe_route_bias: route_cuda.route / bias_probs) against the CPU oracle
(oracle/route_bias.py), through the C ABI.

route() takes the gates as given, so the GPU and the oracle do the same arithmetic on the same T values: inds, ok
and rhs are compared bit for bit, on the reference test's workload (tests/test_route_cuda.py:44-63: E 512 k 10 and
E 256 k 8, T 1-5, fp32 and bf16 gates, bias 0 / 0.5 / 2, budget off / 0.2 / 0.01, rows with exact ties and rounded
rows, the residency table with quota and ring slots) plus fp16 and T up to 16, and at the budget's boundary (tau at
the float32 neighbours of (m_h - m_b) / m_h, where the order of the two k-gate sums decides, test_route_cuda.py
:120-152). bias_probs() computes the softmax itself; its gates can differ from the oracle's exact softmax by one ulp
of the dtype, so its picks are held exact where no two candidates lie within that ulp and its scores to it."""
import numpy as np
import pytest
import torch

from oracle import route_bias as rb

pytestmark = pytest.mark.gpu

TD = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def gates_of(rng, t, e, dt, i):
    """Router rows as the reference test makes them: softmax of broad normal logits, every 5th row with exact ties,
    every 7th rounded; returned as float32 holding dt values."""
    x = rng.normal(0, rng.uniform(0.5, 4.0), (t, e)).astype(np.float32)
    if i % 5 == 0:
        j = rng.integers(0, e, 6)
        x[:, j] = x[:, j[:1]]
    if i % 7 == 0:
        x = np.round(x * 4) / 4
    return rb.softmax_gates(x, dt)


def residency(rng, e):
    n = int(rng.integers(0, e // 3))
    held = rng.choice(e, n, replace=False)
    slot = np.full(e, -1, np.int32)
    slot[held] = rng.choice(4200, n, replace=False).astype(np.int32)
    return slot, 4000


def run_route(g, dt, mask, slot, lam, tau, k, lim=None, slots=True):
    from larder_amd import route
    gt = dev(g).to(TD[dt])
    out = route.route(gt, None if mask is None else dev(mask), dev(slot), lam, tau, k, lim=lim, slots=slots)
    torch.cuda.synchronize()
    return [host(o) for o in out]


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("e,k", [(512, 10), (256, 8), (128, 4), (60, 5)])
def test_route_matches_oracle(dt, e, k):
    rng = np.random.default_rng(e * 7 + k)
    n = 0
    for lam, tau in ((0.0, 0.0), (0.0, 0.2), (0.5, 0.0), (0.5, 0.2), (0.5, 0.01), (2.0, 0.2)):
        for i in range(6):
            t = 1 + i % 5 if i < 5 else 16
            g = gates_of(rng, t, e, dt, i)
            slot, lim = residency(rng, e)
            m = np.zeros(e, np.float32)
            m[rng.choice(e, int(rng.integers(0, e // 3)), replace=False)] = 1.0
            w_inds, w_ok, w_rhs = rb.route(g, dt, m, slot, lam, tau, k)
            inds, ok, rhs = run_route(g, dt, m, slot, lam, tau, k)
            assert (inds.astype(np.uint32) == w_inds).all(), (dt, e, k, lam, tau, i)
            assert bool(ok[0]) == w_ok and (rhs == w_rhs).all()
            (only,) = run_route(g, dt, m, slot, lam, tau, k, slots=False)
            assert (only.astype(np.uint32) == w_inds).all()
            t_inds, t_ok, t_rhs = rb.route(g, dt, None, slot, lam, tau, k, lim=lim)
            inds, ok, rhs = run_route(g, dt, None, slot, lam, tau, k, lim=lim)
            assert (inds.astype(np.uint32) == t_inds).all() and bool(ok[0]) == t_ok and (rhs == t_rhs).all()
            n += 1
    assert n == 36


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_route_budget_boundary(dt):
    """tau at the float32 neighbours of each row's budget ratio: the decision flips within them, and the GPU flips
    exactly where the oracle does."""
    rng = np.random.default_rng(11)
    e, k, lam = 512, 10, 0.5
    flips = 0
    for i in range(24):
        g = gates_of(rng, 1 + 2 * (i % 2), e, dt, i)
        m = np.zeros(e, np.float32)
        m[rng.choice(e, int(rng.integers(5, e // 3)), replace=False)] = 1.0
        slot = np.arange(e, dtype=np.int32)
        spread = rb.round_to(np.float32(g[0].max() - g[0].min()), dt)[()]
        ls = rb.round_to(np.float32(rb.round_to(np.float32(lam), dt)[()] * spread), dt)[()]
        rank = (g[0] + np.float32(ls) * m).astype(np.float32)
        mh = rb.row_reduce_sum(g[0][rb.topk_mlx(g[0], k)], dt)
        mb = rb.row_reduce_sum(g[0][rb.topk_mlx(rank, k)], dt)
        if mh <= mb:
            continue
        c = np.float32((mh - mb) / mh)
        picks = set()
        # float32 neighbours of the ratio, and for bf16 (where tau is rounded to bf16 first) bf16 neighbours
        step = [np.float32(c * (1 + j * 2.0 ** -8)) for j in (-2, -1, 1, 2)] if dt == "bf16" else []
        for tau in [np.nextafter(np.nextafter(c, 0), 0), np.nextafter(c, 0), c, np.nextafter(c, 1),
                    np.nextafter(np.nextafter(c, 1), 1)] + step:
            w_inds, _, _ = rb.route(g, dt, m, slot, lam, float(tau), k)
            inds, _, _ = run_route(g, dt, m, slot, lam, float(tau), k)
            assert (inds.astype(np.uint32) == w_inds).all(), (dt, i, float(tau))
            picks.add(w_inds[0].tobytes())
        flips += len(picks) > 1
    assert flips > 0  # the boundary was reached


def near_tie_ok(got, want, g, k, dt):
    """got == want, or every difference is between candidates whose oracle gates lie within one dt ulp of the
    k-th pick's gate (where the GPU's softmax rounding may order them otherwise)."""
    if (got == want).all():
        return True
    kth = g[want[0]]
    ulp = abs(float(rb.round_to(np.float32(kth * (1 + 2.0 ** (-7 if dt == 'bf16' else -10))), dt)) - float(kth))
    diff = set(got.tolist()) ^ set(want.tolist())
    return all(abs(float(g[i]) - float(kth)) <= 2 * ulp for i in diff)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("norm", [False, True])
def test_bias_probs_matches_oracle(dt, norm):
    from larder_amd import route
    rng = np.random.default_rng(21 + norm)
    e, k = 256, 8
    for lam, tau in ((0.5, 0.0), (0.5, 0.2), (2.0, 0.01)):
        for i in range(5):
            t = 1 + i
            lg = rb.round_to(rng.normal(0, rng.uniform(0.3, 6.0), (t, e)).astype(np.float32), dt)
            if i % 2 == 0:
                j = rng.integers(0, e, 12)
                lg[:, j] = lg[:, j[:1]]
            slot, lim = residency(rng, e)
            w_inds, w_sc = rb.bias_probs(lg, dt, slot, lam, tau, k, lim, norm)
            inds, sc = route.bias_probs(dev(lg).to(TD[dt]), dev(slot), lam, tau, k, lim, norm)
            torch.cuda.synchronize()
            inds, sc = host(inds).astype(np.uint32), host(sc.float())
            g = rb.softmax_gates(lg, dt)
            for r in range(t):
                assert near_tie_ok(inds[r], w_inds[r], g[r], k, dt), (dt, norm, lam, tau, i, r)
                if (inds[r] == w_inds[r]).all():
                    tol = 1e-6 if dt == "f32" else 2.0 ** -7
                    assert np.allclose(sc[r], w_sc[r], rtol=2 * tol, atol=1e-30), (dt, norm, i, r)


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("e,k", [(512, 10), (60, 5)])
def test_route_search_range_edges(dt, e, k):
    """The threshold search runs only over the bits where the keys differ: rows whose gates are all equal (no
    bit differs), take two or three values (a narrow range), or spread over one dt ulp, with and without the bias,
    against the oracle."""
    rng = np.random.default_rng(e + k)
    rows = [np.full(e, 1.0 / e), np.where(np.arange(e) % 3 == 0, 0.02, 0.001),
            np.choose(np.arange(e) % 3, [0.25, 0.125, 0.0625]), 0.01 * (1 + np.arange(e) % 2 * 2.0 ** -7)]
    for r in rows:
        g = np.asarray(torch.from_numpy(r[None].astype(np.float32)).to(TD[dt]).float().numpy())
        for lam, tau in ((0.0, 0.0), (0.5, 0.2), (2.0, 0.01)):
            slot, lim = residency(rng, e)
            m = np.zeros(e, np.float32)
            m[rng.choice(e, e // 4, replace=False)] = 1.0
            w_inds, w_ok, w_rhs = rb.route(g, dt, m, slot, lam, tau, k)
            inds, ok, rhs = run_route(g, dt, m, slot, lam, tau, k)
            assert (inds.astype(np.uint32) == w_inds).all(), (dt, e, k, lam, tau, r[:4])
            assert bool(ok[0]) == w_ok and (rhs == w_rhs).all()
