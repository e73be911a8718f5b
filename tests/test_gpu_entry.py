"""The drop-in entry larder_amd.gguf_experts.experts (the reference's gguf_experts.experts, gguf_experts.py:803-819,
called by StreamingSwitchGLU._experts, stream_fast.py:4569-4581) on the GPU, as its caller drives it:
  * experts packed from a GGUF file (gguf_pack.pack), placed by fill_slots into arena slots in a scrambled order,
    and handed over as one (gguf part, pad part) tuple a projection;
  * x (..., 1, H) broadcast against rhs (...) slot ids, the result rhs.shape + (1, H) in x's dtype;
  * without ``host`` the decode chain; with ``host`` the path dense_pays() picks, each forced once;
  * calibrate() measured into a temporary cache and read back from it.
Outputs are held to the oracle's fp32 dequant-then-matmul on the source tensors: 2e-3 relative L2 (f16 x), and
against the oracle rounded to bf16 for bf16 x."""
import numpy as np
import pytest
import torch

from oracle import gguf, moe
from test_gguf_pack import write_gguf

pytestmark = pytest.mark.gpu

BAR = 2e-3
E, S = 16, 24


def host(t):
    return t.detach().cpu().numpy()


def _bf16_round(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).float().numpy()


# the first two run the raw-activation chain, the third (cfg2's shape) the register-resident one
@pytest.fixture(scope="module", params=[(("Q4_0", "Q4_0", "Q4_0"), 1024, 256), (("Q4_K", "Q4_K", "Q6_K"), 1024, 512),
                                        (("Q4_0", "Q4_0", "Q4_0"), 2048, 768)])
def arena(request, tmp_path_factory):
    """(src experts per projection, bufs as (gguf, pad) tuples over arena slots, slot_of[expert], types, H)."""
    from larder_amd import gguf_pack as gp
    types, H, I = request.param
    d = tmp_path_factory.mktemp("entry")
    rng = np.random.default_rng(H + I)
    src = []
    for p, t in zip(("gate", "up", "down"), types):
        rows, cols = (I, H) if p != "down" else (H, I)
        src.append(gguf.random_experts(rng, E, rows, cols, t))
    tensors = [(f"blk.0.ffn_{p}_exps.weight", [w.shape[2] // gguf.TYPES[t][2] * gguf.TYPES[t][1], w.shape[1], E],
                gguf.TYPES[t][0], w.tobytes()) for p, t, w in zip(("gate", "up", "down"), types, src)]
    write_gguf(d / "m.gguf", [("general.alignment", 32)], tensors)
    gp.pack([d / "m.gguf"], d / "experts.bin", log=None)
    packed = gp.load_packed(d)
    slot_of = rng.permutation(S)[:E]                  # expert e lives in slot slot_of[e]
    order = rng.permutation(E)                        # filled in a scrambled order
    bufs = []
    for p in ("gate", "up", "down"):
        key = f"model.layers.0.mlp.switch_mlp.{p}_proj"
        m = packed["index"][key]
        part = m["parts"][0]
        g = torch.zeros((S,) + tuple(part["shape"]), dtype=torch.uint8, device="cuda")
        gp.fill_slots(packed, key, order, g, slot_of[order], chunk=5)
        pad = torch.zeros((S, m["stride"] - part["bytes"]), dtype=torch.uint8, device="cuda")
        bufs.append((g, pad))
    packed["fd"].close()
    return src, tuple(bufs), slot_of, types, H


def _want(src, x2, experts_of_rows, topk, types):
    _, y = moe.gemv(x2, tuple(src), experts_of_rows, topk, types)
    return y


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_experts_decode_form(arena, dtype):
    from larder_amd import gguf_experts as ge
    src, bufs, slot_of, types, H = arena
    rng = np.random.default_rng(7)
    T, k = 3, 4
    picks = rng.integers(0, E, (T, k))
    x = torch.from_numpy(rng.standard_normal((1, T, 1, H)).astype(np.float32)).cuda().to(dtype)
    rhs = torch.from_numpy(slot_of[picks].reshape(1, T, k).astype(np.int32)).cuda()
    y = ge.experts(x, bufs, rhs, "/".join(types))
    assert y.shape == (1, T, k, 1, H) and y.dtype == dtype
    want = _want(src, host(x.float()).reshape(T, H), picks.reshape(-1), k, types).reshape(1, T, k, 1, H)
    got = host(y.float())
    if dtype == torch.bfloat16:
        want = _bf16_round(want)
    assert moe.rel_l2(got, want) < BAR


def test_experts_host_form_takes_the_path_dense_pays_picks(arena, monkeypatch):
    from larder_amd import gguf_experts as ge
    src, bufs, slot_of, types, H = arena
    rng = np.random.default_rng(8)
    R = 40
    picks = rng.integers(0, E, R)
    x = torch.from_numpy(rng.standard_normal((R, 1, H)).astype(np.float32)).cuda().half()
    rhs = torch.from_numpy(slot_of[picks].reshape(1, R).astype(np.int32)).cuda()
    host_slots = slot_of[picks].reshape(1, R)
    ran = []
    dense0, gemv0 = ge.dense, ge.gemv
    monkeypatch.setattr(ge, "dense", lambda *a, **kw: ran.append("dense") or dense0(*a, **kw))
    monkeypatch.setattr(ge, "gemv", lambda *a, **kw: ran.append("gemv") or gemv0(*a, **kw))
    want = _want(src, host(x.float()).reshape(R, H), picks, 1, types).reshape(1, R, 1, H)
    outs = {}
    for label, cost in (("chain", None), ("dense", [1.0, 1.0, 0.0, 0.0, 0.0]), ("chain", [0.0, 0.0, 1.0, 1.0, 1.0])):
        monkeypatch.setattr(ge, "_COST", cost)
        ran.clear()
        y = ge.experts(x, bufs, rhs, types, host=host_slots)
        assert ran == (["dense"] if label == "dense" else ["gemv"]), (label, ran)
        assert y.shape == (1, R, 1, H) and y.dtype == torch.float16
        assert moe.rel_l2(host(y.float()), want) < BAR
        outs.setdefault(label, host(y.float()))
    assert moe.rel_l2(outs["dense"], outs["chain"]) < BAR
    # without host the decode chain runs whatever the fit says
    monkeypatch.setattr(ge, "_COST", [1.0, 1.0, 0.0, 0.0, 0.0])
    ran.clear()
    ge.experts(x, bufs, rhs, types)
    assert ran == ["gemv"]
    # LMOE_DENSE overrides the fit either way
    for env, cost, path in (("0", [1.0, 1.0, 0.0, 0.0, 0.0], "gemv"), ("1", [0.0, 0.0, 1.0, 1.0, 1.0], "dense")):
        monkeypatch.setenv("LMOE_DENSE", env)
        monkeypatch.setattr(ge, "_COST", cost)
        ran.clear()
        y = ge.experts(x, bufs, rhs, types, host=host_slots)
        assert ran == [path], (env, ran)
        assert moe.rel_l2(host(y.float()), want) < BAR
    monkeypatch.delenv("LMOE_DENSE")
    with pytest.raises(ValueError, match="one row of x per slot"):
        ge.experts(x[:5], bufs, rhs, types, host=host_slots)


def test_calibrate_on_the_device(arena, monkeypatch, tmp_path):
    from larder_amd import gguf_experts as ge
    src, bufs, slot_of, types, H = arena
    I = bufs[0][0].shape[1]
    monkeypatch.setenv("LMOE_CACHE", str(tmp_path))
    monkeypatch.setattr(ge, "_COST", None)
    cost = ge.calibrate(H, I, types)
    assert len(cost) == 5 and all(c >= 0.0 for c in cost)
    assert len(list(tmp_path.glob("dense-switch-*.json"))) == 1
    # one row goes through the chain; thousands of rows over a few experts through the grouped path
    assert not ge.dense_pays(1, 1)
    assert ge.dense_pays(8, 8192)

    def no_measure(*a):
        raise AssertionError("the second call must read the cache")

    monkeypatch.setattr(ge, "_measure", no_measure)
    assert ge.calibrate(H, I, "/".join(types)) == cost
