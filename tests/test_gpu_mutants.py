"""The parity bar refuses broken kernels. Plausible mistakes are planted in the oracle, on the CPU, never in a
kernel. For each, the answer of the mutated oracle is compared with the GPU's real outputs through the parity
tests' own bar (ids bit-exact, outputs within 2e-3 relative L2). Every mutant must fail that bar while the oracle
itself passes. So a kernel that made the same mistake would fail the parity tests: the mutant stands in for the
broken kernel (the reference's forced-mismatch test, tests/test_rows_cuda.py:279-302). Also: the load-time
known-answer self-check passes on the device and runs before the first launch."""
import numpy as np
import pytest
import torch

from oracle import gguf, moe

pytestmark = pytest.mark.gpu

BAR = 2e-3


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


# ---- mistakes, each planted in the oracle through a monkeypatch context ------------------------------------------

_Q40, _Q4K = gguf._DQ["Q4_0"], gguf._DQ["Q4_K"]
_SILU, _ROUTER = moe.silu_mul, moe.router


def q40_nibble_pairs(m):  # weights 2j, 2j + 1 from byte j (for j, j + 16)
    def wrong(b):
        qs = b[:, 2:18]
        q = np.stack([qs & 0xF, qs >> 4], axis=2).reshape(-1, 32).astype(np.int32)
        return (q - 8).astype(np.float32) * gguf._f16(b, 0)[:, None]
    m.setitem(gguf._DQ, "Q4_0", wrong)


def q40_offset(m):  # q - 7 for q - 8
    m.setitem(gguf._DQ, "Q4_0", lambda b: _Q40(b) + gguf._f16(b, 0)[:, None])


def q40_scale_bytes(m):  # the f16 scale read big-endian
    def wrong(b):
        b2 = b.copy()
        b2[:, 0], b2[:, 1] = b[:, 1], b[:, 0]
        return np.nan_to_num(_Q40(b2), nan=0.0, posinf=0.0, neginf=0.0)
    m.setitem(gguf._DQ, "Q4_0", wrong)


def q4k_min_sign(m):  # + dmin * m for - dmin * m
    def wrong(b):
        n = b.shape[0]
        _, mm = gguf.scale_min_k4(b[:, 4:16])
        return _Q4K(b) + 2 * np.repeat(gguf._f16(b, 2)[:, None] * mm, 32, axis=1).reshape(n, 256)
    m.setitem(gguf._DQ, "Q4_K", wrong)


def q4k_scale_packing(m):  # sub-blocks 4..7 take their high scale bits from the m bytes
    def wrong(s):
        s = s.astype(np.uint8)
        sc = np.concatenate([s[:, 0:4] & 63, (s[:, 8:12] & 0xF) | ((s[:, 4:8] >> 6) << 4)], axis=1)
        mm = np.concatenate([s[:, 4:8] & 63, (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)], axis=1)
        return sc.astype(np.float32), mm.astype(np.float32)
    m.setattr(gguf, "scale_min_k4", wrong)


def q4k_nibble_halves(m):  # sub-block 2c from the high nibbles, 2c + 1 from the low ones
    def wrong(b):
        n = b.shape[0]
        b2 = b.copy()
        b2[:, 16:144] = ((b[:, 16:144] & 0xF) << 4) | (b[:, 16:144] >> 4)
        return _Q4K(b2).reshape(n, 256)
    m.setitem(gguf._DQ, "Q4_K", wrong)


def swiglu_no_sigmoid(m):
    m.setattr(moe, "silu_mul", lambda g, u: (np.asarray(g, np.float32) * np.asarray(u, np.float32)))


def swiglu_on_up(m):  # silu(u) * g
    m.setattr(moe, "silu_mul", lambda g, u: _SILU(u, g))


def renorm_flipped(m):  # renormalise exactly when the layer does not, and the other way round
    m.setattr(moe, "router", lambda logits, k, norm: _ROUTER(logits, k, not norm))


def shared_gate_raw(m):  # the shared expert's gate logit used without its sigmoid
    m.setattr(moe, "sigmoid", lambda v: np.asarray(v, np.float32))


Q4_0_MUTANTS = [q40_nibble_pairs, q40_offset, q40_scale_bytes]
Q4_K_MUTANTS = [q4k_min_sign, q4k_scale_packing, q4k_nibble_halves]
ANY_MUTANTS = [swiglu_no_sigmoid, swiglu_on_up, renorm_flipped]


# ---- the GPU's outputs, computed once a case ---------------------------------------------------------------------

_CASES = {}


def _case(name):
    """(gpu ids, gpu out, oracle() -> (ids, out)) of one layer run on the device."""
    if name in _CASES:
        return _CASES[name]
    from larder_amd import grouped, layer as lay, workloads
    g = torch.Generator(device="cuda").manual_seed(41)
    if name == "cfg1_decode":   # Q4_0, E 60, top-4 without renorm, shared expert with a sigmoid gate
        cfg = workloads.CONFIGS[1]
        T = 2
    elif name == "q4k_decode":  # Q4_K at cfg2's shapes, 16 experts, top-8 renormalised
        cfg = dict(workloads.CONFIGS[2], E=16, types=("Q4_K",) * 3)
        T = 3
    else:                       # the grouped path: cfg4's shapes, 24 tokens
        cfg = workloads.CONFIGS[4]
        T = 24
    L = workloads.make_layer(cfg, g)
    x = torch.randn((T, cfg["H"]), generator=g, device="cuda").half()
    out = torch.empty((T, cfg["H"]), dtype=torch.float32, device="cuda")
    if name.endswith("_decode"):
        B = lay.DecodeBuffers(L, T)
        lay.decode(L, x, B, out)
    else:
        B = grouped.PrefillBuffers(L, T)
        grouped.prefill(L, x, B, out)
    torch.cuda.synchronize()
    xs = host(x.float())
    # routing pinned from x on both paths: the decode router's fixed order, which the prefill's exact pick reproduces
    lg = moe.router_logits_gemv(host(x), host(L.wr))
    w = tuple(host(b) for b in (L.wg, L.wu, L.wd))
    shared = dict(shared=tuple(host(b[0]) for b in L.shared), shared_gate_w=host(L.wsg.float())) if L.shared else {}

    def oracle():
        ids, _, want = moe.layer(xs, lg, w, cfg["types"], cfg["k"], cfg["norm"], **shared)
        return ids, want

    _CASES[name] = (host(B.ids).astype(np.uint32).reshape(T, -1)[:, :cfg["k"]], host(out), oracle, cfg)
    return _CASES[name]


def _passes(gpu_ids, gpu_out, ids, want):
    return np.array_equal(gpu_ids, ids) and moe.rel_l2(gpu_out, want) < BAR


CASES = [("cfg1_decode", Q4_0_MUTANTS + ANY_MUTANTS + [shared_gate_raw]),
         ("q4k_decode", Q4_K_MUTANTS + ANY_MUTANTS),
         ("cfg4_prefill", Q4_0_MUTANTS + ANY_MUTANTS)]


@pytest.mark.parametrize("name,mutant", [(c, mu) for c, ms in CASES for mu in ms],
                         ids=lambda v: v if isinstance(v, str) else v.__name__)
def test_bar_refuses_the_mutant(name, mutant, monkeypatch):
    gpu_ids, gpu_out, oracle, _ = _case(name)
    ids, want = oracle()
    assert _passes(gpu_ids, gpu_out, ids, want), f"{name}: the oracle itself must pass (rel L2 " \
                                                f"{moe.rel_l2(gpu_out, want):.2e})"
    with monkeypatch.context() as m:
        mutant(m)
        ids_m, want_m = oracle()
    assert not _passes(gpu_ids, gpu_out, ids_m, want_m), \
        f"{name}: a kernel with {mutant.__name__} would pass the bar (rel L2 {moe.rel_l2(gpu_out, want_m):.2e})"


def test_bar_refuses_the_other_tie_rule():
    """Ties to the larger index (MLX's order, the reference kernel's) would fail the ids check on tied rows."""
    from larder_amd import route
    rng = np.random.default_rng(3)
    E, k, T = 64, 8, 32
    lg = rng.integers(-4, 4, (T, E)).astype(np.float32)     # many ties
    ids, _ = route.topk(dev(lg), k, True)                     # best first
    gpu = host(ids).astype(np.uint32)
    assert np.array_equal(gpu, moe.topk_ids(lg, k))
    larger_first = np.stack([np.argsort(r, kind="stable")[::-1][:k] for r in lg]).astype(np.uint32)
    assert not np.array_equal(gpu, larger_first)


def test_self_check_on_the_device():
    """The known-answer check passes here, and it ran before this process's first launch on the device."""
    from larder_amd import _lib, selfcheck
    selfcheck.run()
    _lib.stream()
    assert _lib._CHECKED.get(torch.cuda.current_device()) is True
