"""Experts packed from a GGUF file and loaded into HBM by larder_amd.gguf_pack feed the expert kernels: the device
buffers hold the GGUF bytes exactly, and the decode chain and the grouped path on them agree with the CPU oracle
run on the source tensors (2e-3 relative L2, the north star's bar). Arena-slot filling (fill_slots: experts into
chosen slots of a smaller buffer, in any order) is checked byte for byte."""
import numpy as np
import pytest
import torch

from oracle import gguf, moe
from test_gguf_pack import write_gguf

pytestmark = pytest.mark.gpu

BAR = 2e-3


def host(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("types,H,I", [(("Q4_0", "Q4_0", "Q4_0"), 2048, 768), (("Q4_K", "Q4_K", "Q4_K"), 1024, 512),
                                       (("Q4_K", "Q4_K", "Q4_0"), 1024, 256), (("Q4_K", "Q4_K", "Q6_K"), 1024, 512),
                                       (("Q8_0", "Q8_0", "Q5_K"), 1024, 256)])
def test_packed_layer_through_kernels(tmp_path, types, H, I):
    from larder_amd import gguf_experts as ge, gguf_pack as gp
    rng = np.random.default_rng(H + I)
    E = 16
    src = []
    for p, t in zip(("gate", "up", "down"), types):
        rows, cols = (I, H) if p != "down" else (H, I)
        w = gguf.random_experts(rng, E, rows, cols, t)
        src.append(w)
    tensors = [(f"blk.0.ffn_{p}_exps.weight", [w.shape[2] // gguf.TYPES[t][2] * gguf.TYPES[t][1], w.shape[1], E],
                gguf.TYPES[t][0], w.tobytes()) for p, t, w in zip(("gate", "up", "down"), types, src)]
    write_gguf(tmp_path / "m.gguf", [("general.alignment", 32)], tensors)
    gp.pack([tmp_path / "m.gguf"], tmp_path / "experts.bin", log=None)
    packed = gp.load_packed(tmp_path)
    bufs, ts = gp.load_layer(packed, 0)
    assert ts == "/".join(types)
    for b, w in zip(bufs, src):
        assert b.shape == w.shape and (host(b) == w).all()

    # the decode chain: 3 tokens x top-4
    topk, T = 4, 3
    slots = rng.integers(0, E, T * topk).astype(np.int32)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).cuda().half()
    y = ge.gemv(x, bufs, torch.from_numpy(slots).cuda(), topk, ts, torch.float32)
    _, yw = moe.gemv(host(x.float()), tuple(src), slots, topk, types)
    assert moe.rel_l2(host(y), yw) < BAR

    # the grouped path: 96 rows, one slot a row
    R = 96
    rows = rng.integers(0, E, R).astype(np.int32)
    xr = torch.from_numpy(rng.standard_normal((R, H)).astype(np.float32)).cuda().half()
    yd = ge.dense(xr, bufs, torch.from_numpy(rows), ts, torch.float32)
    _, ydw = moe.gemv(host(xr.float()), tuple(src), rows, 1, types)
    assert moe.rel_l2(host(yd), ydw) < BAR

    # arena slots: experts 9, 2, 2, 15 into slots 3, 0, 5, 1 of a 6-slot buffer
    key = "model.layers.0.mlp.switch_mlp.down_proj"
    arena = torch.zeros((6,) + tuple(bufs[2].shape[1:]), dtype=torch.uint8, device="cuda")
    gp.fill_slots(packed, key, [9, 2, 2, 15], arena, [3, 0, 5, 1], chunk=3)
    a = host(arena)
    for e, s in zip([9, 2, 2, 15], [3, 0, 5, 1]):
        assert (a[s] == src[2][e]).all()
    assert (a[[2, 4]] == 0).all()
    with pytest.raises(ValueError, match="slots outside"):
        gp.fill_slots(packed, key, [1], arena, [6])
    packed["fd"].close()
