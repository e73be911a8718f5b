"""The cache-biased route oracle (oracle/route_bias.py) pinned against facts that do not come from its own
formulas: brute-force selections, the stable-sort tie rule, hand-derived reduction orders, the bias's and the
budget's limiting cases, and bf16 rounding of known bit patterns."""
import numpy as np

from oracle import route_bias as rb


def test_bf16_rounding_known_values():
    one = np.float32(1.0)
    ulp = np.float32(2.0 ** -7)
    # halfway between 1 and 1 + ulp rounds to even (1); just above halfway rounds up
    assert rb.round_to(np.float32(1.0 + 2.0 ** -8), "bf16") == one
    assert rb.round_to(np.float32(1.0 + 2.0 ** -8 + 2.0 ** -20), "bf16") == one + ulp
    # halfway between 1 + ulp and 1 + 2 ulp rounds to even (1 + 2 ulp)
    assert rb.round_to(np.float32(1.0 + 3 * 2.0 ** -8), "bf16") == np.float32(1.0 + 2 * 2.0 ** -7)
    assert rb.round_to(np.float32(-3.0), "bf16") == np.float32(-3.0)
    assert np.isnan(rb.round_to(np.float32(np.nan), "bf16"))
    assert rb.round_to(np.float32(1.0 + 2.0 ** -11), "f16") == one


def test_topk_mlx_against_a_stable_sort_brute_force():
    rng = np.random.default_rng(0)
    for _ in range(200):
        e = int(rng.integers(5, 40))
        k = int(rng.integers(1, e + 1))
        v = np.round(rng.normal(size=e) * 2).astype(np.float32)  # many exact ties
        pairs = sorted(range(e), key=lambda i: (float(v[i]), i))   # Python's sort is stable: ties by index
        assert rb.topk_mlx(v, k).tolist() == pairs[-k:]


def test_topk_mlx_ties_take_the_larger_index_and_come_ascending():
    v = np.array([1.0, 5.0, 1.0, 5.0, 3.0, 5.0], np.float32)
    assert rb.topk_mlx(v, 2).tolist() == [3, 5]
    assert rb.topk_mlx(v, 4).tolist() == [4, 1, 3, 5]


def test_budget_sum_orders_derived_by_hand():
    v = (np.arange(1, 11) * np.float32(0.1)).astype(np.float32)
    # bf16, k = 10: lane 0 adds positions 0-7, lane 1 positions 8-9, then xor 1 joins them
    a0 = np.float32(0.0)
    for x in v[:8]:
        a0 = rb.round_to(np.float32(a0 + x), "bf16")[()]
    a1 = rb.round_to(np.float32(rb.round_to(np.float32(0 + v[8]), "bf16") + v[9]), "bf16")[()]
    assert rb.row_reduce_sum(v, "bf16") == rb.round_to(np.float32(a0 + a1), "bf16")
    # f32, k = 10: lanes 0, 1, 2 hold positions 0-3, 4-7, 8-9; xor 2 joins 0 and 2, then xor 1 adds lane 1
    s = [np.float32(0.0)] * 3
    for lane in range(3):
        acc = np.float32(0.0)
        for x in v[4 * lane:4 * lane + 4]:
            acc = np.float32(acc + x)
        s[lane] = acc
    assert rb.row_reduce_sum(v, "f32") == np.float32(np.float32(s[0] + s[2]) + s[1])
    # k <= N: one lane, a plain sequential sum
    acc = np.float32(0.0)
    for x in v[:4]:
        acc = np.float32(acc + x)
    assert rb.row_reduce_sum(v[:4], "f32") == acc


def test_route_limiting_cases():
    rng = np.random.default_rng(1)
    e, k = 64, 6
    g = rb.softmax_gates(rng.normal(size=(3, e)).astype(np.float32), "f32")
    slot = np.arange(e, dtype=np.int32)
    # no bias: the plain top-k
    inds, ok, rhs = rb.route(g, "f32", np.ones(e, np.float32), slot, 0.0, 0.0, k)
    for r in range(3):
        assert inds[r].tolist() == rb.topk_mlx(g[r], k).tolist()
    assert ok and (rhs == inds).all()
    # a bias larger than any gap promotes the masked experts: the picks are the top k among them
    m = np.zeros(e, np.float32)
    held = rng.choice(e, 10, replace=False)
    m[held] = 1.0
    inds, _, _ = rb.route(g, "f32", m, slot, 4.0, 0.0, k)
    for r in range(3):
        sub = held[np.argsort(g[r][held], kind="stable")]
        assert sorted(inds[r].tolist()) == sorted(sub[-k:].tolist())
    # the budget at tau ~ 0 falls back to the honest picks whenever the bias moved mass; at tau 1 it never does
    honest = np.stack([rb.topk_mlx(row, k) for row in g])
    inds0, _, _ = rb.route(g, "f32", m, slot, 4.0, 1e-30, k)
    assert (inds0 == honest).all()
    inds1, _, _ = rb.route(g, "f32", m, slot, 4.0, 1.0, k)
    assert (inds1 == inds).all()


def test_table_mode_is_the_mask_it_implies_and_slots_map_through():
    rng = np.random.default_rng(2)
    e, k, lim = 128, 8, 4000
    g = rb.round_to(rb.softmax_gates(rng.normal(0, 2, size=(4, e)).astype(np.float32), "bf16"), "bf16")
    slot = np.full(e, -1, np.int32)
    held = rng.choice(e, 40, replace=False)
    slot[held] = rng.choice(4200, 40, replace=False)
    want = rb.route(g, "bf16", ((slot >= 0) & (slot < lim)).astype(np.float32), slot, 0.5, 0.2, k)
    got = rb.route(g, "bf16", None, slot, 0.5, 0.2, k, lim=lim)
    assert (want[0] == got[0]).all() and want[1] == got[1] and (want[2] == got[2]).all()
    assert (got[2] == np.maximum(slot[got[0].astype(np.int64)], 0)).all()
    assert got[1] == bool((slot[got[0].astype(np.int64)] >= 0).all())


def test_bias_probs_scores_are_the_picked_gates_renormalised():
    rng = np.random.default_rng(3)
    e, k = 256, 8
    lg = rb.round_to(rng.normal(0, 2, size=(2, e)).astype(np.float32), "bf16")
    slot = np.arange(e, dtype=np.int32)
    inds, sc = rb.bias_probs(lg, "bf16", slot, 0.5, 0.0, k, 64, False)
    g = rb.softmax_gates(lg, "bf16")
    assert (sc == np.take_along_axis(g, inds.astype(np.int64), axis=-1)).all()
    _, scn = rb.bias_probs(lg, "bf16", slot, 0.5, 0.0, k, 64, True)
    assert np.allclose(scn.sum(-1), 1.0, atol=2e-2)
