"""The decode chain's run kernels (lmoe_gemv_gate_up_runs / lmoe_gemv_down_runs; the reference's gguf_gate_up_runs /
gguf_down_runs, gguf_cuda.py:33-152, driven by _gemv_runs and gated by _runs_ok, gguf_experts.py:600-607, 632-680):
rows of one slot each, a weight row read once a run of equal slots in a window of rows.
  * bit-equal to the chain (h and outputs) for sorted runs, unsorted slots, slots past the experts, windows of 1 to
    16 rows and row counts that leave a partial window, over the block-type mixes and dtypes the chain takes;
  * held to the oracle (2e-3 relative L2, h to 1e-5 on the x values the kernels see);
  * gemv() routes topk 1, more than one row through them once _runs_ok() passed, and through the chain with
    LMOE_GGUF_RUNS=0, for topk > 1, for one row, and when the check fails (a forced mismatch)."""
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


def same_bits(a, b):
    return a.shape == b.shape and bool(torch.equal(a.contiguous().view(torch.int32 if a.element_size() == 4 else
                                                                        torch.int16),
                                                   b.contiguous().view(torch.int32 if b.element_size() == 4 else
                                                                       torch.int16)))


# the first four and the last two run the register-resident chain and the run kernels that follow it
# (gguf_experts.fast_form: one Q4 type for gate and up, hidden 2048 / 4096, a width that is a multiple of 128 up to
# 8192; 4608 puts 72 units a row on the lanes, past one a lane); the rest the raw-activation chain and its run kernels
MIXES = [(("Q4_0",) * 3, 2048, 768), (("Q4_0",) * 3, 1344, 448), (("Q4_K",) * 3, 1024, 512),
         (("Q4_K",) * 3, 4096, 256), (("Q4_0", "Q4_K", "Q4_0"), 1024, 512), (("Q4_K", "Q4_0", "Q4_K"), 512, 512),
         (("Q4_K",) * 3, 2048, 512), (("Q4_0",) * 3, 4096, 1408), (("Q4_0",) * 3, 2048, 4608)]


def sorted_runs(rng, E, n_runs, longest):
    """Slots in runs of 1..longest equal ids (neighbouring runs may share an id), one run past the experts."""
    lens = rng.integers(1, longest + 1, n_runs)
    ids = rng.integers(0, E, n_runs)
    ids[n_runs // 2] = E + 1
    return np.repeat(ids, lens).astype(np.int32)


@pytest.mark.parametrize("types,H,I", MIXES)
@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16, torch.float32])
def test_runs_bit_equal_to_chain(types, H, I, xdt, monkeypatch):
    from larder_amd import gguf_experts as ge
    rng = np.random.default_rng(H * 5 + I)
    E = 5
    w = tuple(dev(gguf.random_experts(rng, E, r, c, t)) for (r, c), t in zip(((I, H), (I, H), (H, I)), types))
    cases = [sorted_runs(rng, E, 9, 12), rng.integers(0, E + 2, 37).astype(np.int32), np.full(21, 3, np.int32)]
    for slots in cases:
        n = slots.size
        x = dev(rng.standard_normal((n, H)).astype(np.float32)).to(xdt)
        sd = dev(slots)
        for odt in (torch.float32, torch.bfloat16):
            want = ge._chain(x, w, sd, 1, types, odt)
            for tr in (1, 3, 8, 16):
                monkeypatch.setenv("LMOE_GGUF_RUN_ROWS", str(tr))
                got = ge._gemv_runs(x, w, sd, types, odt)
                assert same_bits(got[0], want[0]), (slots[:8], tr, "h")
                assert same_bits(got[1], want[1]), (slots[:8], tr, "out")
        off = slots >= E
        assert (host(got[0])[off] == 0).all() and (host(got[1].float())[off] == 0).all()


@pytest.mark.parametrize("types,H,I", [MIXES[0], MIXES[2]])
def test_runs_vs_oracle(types, H, I):
    from larder_amd import gguf_experts as ge
    rng = np.random.default_rng(H + 3 * I)
    E = 6
    src = tuple(gguf.random_experts(rng, E, r, c, t) for (r, c), t in zip(((I, H), (I, H), (H, I)), types))
    slots = sorted_runs(rng, E, 7, 10)
    x = dev(rng.standard_normal((slots.size, H)).astype(np.float32)).half()
    h, y = ge._gemv_runs(x, tuple(dev(b) for b in src), dev(slots), types, torch.float32)
    hw, yw = moe.gemv(host(x.float()), src, slots, 1, types)
    assert moe.rel_l2(host(h), hw) < 1e-5
    assert moe.rel_l2(host(y), yw) < BAR


def test_gemv_dispatch(monkeypatch, capsys):
    """gemv() takes the run kernels for topk 1 and more than one row, once checked; the chain otherwise."""
    from larder_amd import gguf_experts as ge
    types, H, I = MIXES[0]
    rng = np.random.default_rng(11)
    E = 4
    src = tuple(gguf.random_experts(rng, E, r, c, t) for (r, c), t in zip(((I, H), (I, H), (H, I)), types))
    w = tuple(dev(b) for b in src)
    slots = np.sort(rng.integers(0, E, 24)).astype(np.int32)
    x = dev(rng.standard_normal((24, H)).astype(np.float32)).half()
    ran = []
    runs0, chain0 = ge._gemv_runs, ge._chain
    monkeypatch.setattr(ge, "_gemv_runs", lambda *a, **kw: ran.append("runs") or runs0(*a, **kw))
    monkeypatch.setattr(ge, "_chain", lambda *a, **kw: ran.append("chain") or chain0(*a, **kw))
    monkeypatch.setattr(ge, "_RUNS_OK", {})
    y = ge.gemv(x, w, dev(slots), 1, types, torch.float16)
    # the first call at this shape checks the run kernels against the chain, then uses them
    assert ran == ["chain", "runs", "runs"], ran
    assert "run kernels in use" in capsys.readouterr().out
    yw = moe.gemv(host(x.float()), src, slots, 1, types)[1]
    assert moe.rel_l2(host(y.float()), yw) < BAR
    for label, args, env in (("topk 2", (x[:12], w, dev(slots), 2), "1"), ("one row", (x[:1], w, dev(slots[:1]), 1), "1"),
                             ("knob off", (x, w, dev(slots), 1), "0")):
        ran.clear()
        monkeypatch.setenv("LMOE_GGUF_RUNS", env)
        ge.gemv(*args, types, torch.float16)
        assert ran == ["chain"], (label, ran)
    monkeypatch.setenv("LMOE_GGUF_RUNS", "1")
    ran.clear()
    ge.gemv(x, w, dev(slots), 1, types, torch.float16)
    assert ran == ["runs"]   # checked once a shape


def test_forced_mismatch_turns_the_runs_off(monkeypatch, capsys):
    """A run path whose output differs from the chain by one bit fails the check, and gemv() keeps the chain (the
    reference's forced-mismatch case, tests/test_rows_cuda.py:279-302)."""
    from larder_amd import gguf_experts as ge
    types, H, I = MIXES[2]
    runs0 = ge._gemv_runs

    def off_by_one_bit(*a, **kw):
        h, y = runs0(*a, **kw)
        y = y.clone()
        y.view(torch.int16).view(-1)[5] ^= 1
        return h, y

    monkeypatch.setattr(ge, "_RUNS_OK", {})
    monkeypatch.setattr(ge, "_gemv_runs", off_by_one_bit)
    assert not ge._runs_ok(H, I, types, torch.float16, torch.float16)
    assert "not used" in (out := capsys.readouterr().out) and "output is not bit-identical" in out
    rng = np.random.default_rng(2)
    w = tuple(dev(gguf.random_experts(rng, 3, r, c, t)) for (r, c), t in zip(((I, H), (I, H), (H, I)), types))
    x = dev(rng.standard_normal((6, H)).astype(np.float32)).half()
    ran = []
    chain0 = ge._chain
    monkeypatch.setattr(ge, "_chain", lambda *a, **kw: ran.append("chain") or chain0(*a, **kw))
    ge.gemv(x, w, dev(np.array([0, 0, 1, 1, 2, 2], np.int32)), 1, types, torch.float16)
    assert ran == ["chain"]


@pytest.mark.parametrize("types,H,I,topk", [(("Q4_0",) * 3, 2048, 768, 8), (("Q4_K",) * 3, 2048, 512, 10),
                                            (("Q4_0",) * 3, 4096, 1408, 4), (("Q4_K",) * 3, 4096, 256, 2)])
@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16, torch.float32])
def test_fast_chain_topk_vs_oracle(types, H, I, topk, xdt):
    """gemv() at topk > 1 on the register-resident chain (the form cfg2's and cfg5's decode rows take): every slot's
    unweighted output against the oracle, h to 1e-5 on the f16 values the kernels see (x is narrowed to f16 once),
    the outputs to 2e-3 against the oracle on x as given; slots past the experts give zero rows."""
    from larder_amd import gguf_experts as ge
    assert ge.fast_form(H, I, types)
    rng = np.random.default_rng(H + I + topk)
    E = 12
    src = tuple(gguf.random_experts(rng, E, r, c, t) for (r, c), t in zip(((I, H), (I, H), (H, I)), types))
    w = tuple(dev(b) for b in src)
    T = 3
    slots = np.stack([rng.permutation(E + 1)[:topk] for _ in range(T)]).reshape(-1).astype(np.int32)  # E: none
    x = dev(rng.standard_normal((T, H)).astype(np.float32)).to(xdt)
    h, y = ge._chain(x, w, dev(slots), topk, types, torch.float32)
    xs = host(x.float())
    hw16, _ = moe.gemv(host(x.half().float()), src, slots, topk, types)
    hw, yw = moe.gemv(xs, src, slots, topk, types)
    assert moe.rel_l2(host(h), hw16) < 1e-5
    assert moe.rel_l2(host(y), yw) < BAR
    off = slots >= E
    assert (host(h)[off] == 0).all() and (host(y)[off] == 0).all()
    # gemv() itself (no h asked for) gives the same bits
    assert same_bits(ge.gemv(x, w, dev(slots), topk, types, torch.float32), y)


@pytest.mark.parametrize("types,H,I", [(("Q4_0",) * 3, 2048, 768), (("Q4_K",) * 3, 2048, 512),
                                       (("Q4_0",) * 3, 2048, 1408), (("Q4_0",) * 3, 4096, 4608)])
def test_fast_chain_slot_bits_do_not_depend_on_the_call(types, H, I):
    """A slot's output is the same bits at topk 8 as at topk 1 with x repeated a slot, and alone: the chain's down
    sums each slot over its own lane group (16, 32 or 64 lanes), and gate/up is one workgroup row a slot."""
    from larder_amd import gguf_experts as ge
    rng = np.random.default_rng(I)
    E = 10
    w = tuple(dev(gguf.random_experts(rng, E, r, c, t)) for (r, c), t in zip(((I, H), (I, H), (H, I)), types))
    T, k = 2, 8
    slots = np.concatenate([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    x = dev(rng.standard_normal((T, H)).astype(np.float32)).half()
    h8, y8 = ge._chain(x, w, dev(slots), k, types, torch.float32)
    h1, y1 = ge._chain(x.repeat_interleave(k, 0), w, dev(slots), 1, types, torch.float32)
    assert same_bits(h8, h1) and same_bits(y8, y1)
    for s in (0, 5, 11):
        hs, ys = ge._chain(x[s // k:s // k + 1], w, dev(slots[s:s + 1]), 1, types, torch.float32)
        assert same_bits(hs[0], h8[s]) and same_bits(ys[0], y8[s])
