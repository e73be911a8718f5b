"""The decode kernels' stamping forms (lmoe_timeline_*, larder_amd.timeline): the same bits as the unstamped kernels,
eagerly and replayed from a captured graph, one listed launch per router / gate/up / down, and every workgroup's
stamps in phase order."""
import numpy as np
import pytest
import torch

from larder_amd import layer as lay, timeline, workloads

pytestmark = pytest.mark.gpu


def check_stamps(stamps, launches, nl):
    assert [name for name, _, _ in launches] == ["router", "gate_up", "down"] * nl
    for name, r0, n in launches:
        rows = stamps[r0:r0 + n]
        assert (rows[:, 0] != 0).all(), name
        assert (rows[:, 4] != 0).all(), name  # every workgroup of these shapes reaches its end
        if name == "gate_up":
            assert (rows[:, 1:4] != 0).all()
        if name == "down":
            assert (rows[:, [1, 3]] != 0).all()
        for row in rows:
            v = row[:5][row[:5] != 0]
            assert (np.diff(v) >= 0).all(), (name, row)
        assert (rows[:, 5:] == 0).all()


@pytest.mark.parametrize("cfgid,dtype", [(2, torch.float16), (5, torch.bfloat16), (1, torch.bfloat16)])
def test_stamping_forms_same_bits_and_phase_order(cfgid, dtype):
    print(f"timeline cfg{cfgid} {dtype}", flush=True)
    cfg = workloads.CONFIGS[cfgid]
    g = torch.Generator(device="cuda").manual_seed(cfgid)
    nl = 2
    layers = [workloads.make_layer(cfg, g) for _ in range(nl)]
    st = lay.DecodeStack(layers, 1, dtype=dtype)
    x = torch.randn((1, cfg["H"]), generator=g, device="cuda").to(dtype)
    st.x_in.copy_(x)
    want = st.step().clone()
    with timeline.Timeline(nl * 4096) as tl:
        st.x_in.copy_(x)
        got = st.step().clone()
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    check_stamps(tl.buf.cpu().numpy(), tl.launches, nl)

    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with timeline.Timeline(nl * 4096) as tg:
        with torch.cuda.stream(s), torch.cuda.graph(graph, stream=s):
            st.step()
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(3):
        tg.buf.zero_()
        st.x_in.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(st.x_out, want), rep
        check_stamps(tg.buf.cpu().numpy(), tg.launches, nl)
    assert timeline.clock_khz() > 0
