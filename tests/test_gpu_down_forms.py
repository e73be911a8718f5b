"""The two-wavefront down kernel's equivalent forms give the same bits: its h units as one run through LDS (the
default) or one lane's own loads each (LMOE_DOWN_HL=0). Through the decode stack of each configuration, eagerly."""

import pytest
import torch

from larder_amd import layer as lay, workloads

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cfgid,dtype", [(2, torch.float16), (5, torch.bfloat16), (1, torch.bfloat16)])
def test_down_forms_same_bits(cfgid, dtype, monkeypatch):
    print(f"down forms cfg{cfgid} {dtype}", flush=True)
    cfg = workloads.CONFIGS[cfgid]
    g = torch.Generator(device="cuda").manual_seed(10 + cfgid)
    layers = [workloads.make_layer(cfg, g) for _ in range(2)]
    st = lay.DecodeStack(layers, 1, dtype=dtype)
    outs = {}
    for name, env in (("default", {}), ("per-lane h", {"LMOE_DOWN_HL": "0"})):
        monkeypatch.delenv("LMOE_DOWN_HL", raising=False)
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        res = []
        for seed in range(3):
            x = torch.randn((1, cfg["H"]), generator=torch.Generator(device="cuda").manual_seed(seed),
                            device="cuda").to(dtype)
            st.x_in.copy_(x)
            res.append(st.step().clone())
        torch.cuda.synchronize()
        outs[name] = res
    for name, res in outs.items():
        for a, b in zip(res, outs["default"]):
            assert torch.equal(a, b), name
