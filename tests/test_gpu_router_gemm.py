"""The prefill router GEMM (lmoe_router_gemm): logits of x [T, H] against the router weight [E, H] (and the shared
expert's gate row) on the matrix cores, through the C ABI, against an fp64 product of the same f16 operands.
f16 x f16 products are exact in fp32, so only the fp32 summation differs: 1e-5 relative L2 and a per-element
bound of 1e-5 of the row's |x| . |w| scale. Shapes cover partial tiles (T not a multiple of 64, E + gate not a
multiple of 128), each K split the picker makes (1 to 8), the cfg5 router (2048 x 4096 x 513) and T = 1."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,H,E,ng", [(1, 2048, 128, 0), (63, 1024, 60, 1), (150, 2048, 60, 1), (200, 2048, 32, 0),
                                      (2048, 4096, 512, 1), (4096, 2048, 128, 0), (130, 4096, 257, 0),
                                      (8192, 2048, 512, 0)])
def test_router_gemm_vs_fp64(T, H, E, ng):
    from larder_amd import _lib, grouped
    from larder_amd._lib import call, ptr, stream
    rng = np.random.default_rng(T + H + E)
    x = rng.standard_normal((T, H)).astype(np.float16)
    w = (rng.standard_normal((E + ng, H)) * 0.02).astype(np.float16)
    xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    xh = grouped.as_gemm_f16(xd)
    wk = grouped.as_gemm_f16(wd)
    ks = _lib.lib().lmoe_router_gemm_ksplit(T, H, E + ng)
    nws = _lib.lib().lmoe_router_gemm_workspace_bytes(T, H, E + ng)
    assert (nws > 0) == (ks > 1)
    ws = torch.empty(max(nws // 4, 1), dtype=torch.float32, device="cuda")
    lg = torch.full((T, E), float("nan"), dtype=torch.float32, device="cuda")
    gate = torch.full((T,), float("nan"), dtype=torch.float32, device="cuda")
    call("lmoe_router_gemm", ptr(xh), T, H, ptr(wk), E, ng, ptr(ws), ptr(lg), ptr(gate) if ng else None, stream())
    torch.cuda.synchronize()
    want = x.astype(np.float64) @ w.astype(np.float64).T
    got = lg.cpu().numpy()
    scale = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    assert np.isfinite(got).all()
    assert np.linalg.norm(got - want[:, :E]) / np.linalg.norm(want[:, :E]) < 1e-5
    assert (np.abs(got - want[:, :E]) <= 1e-5 * scale[:, :E] + 1e-30).all()
    if ng:
        gg = gate.cpu().numpy()
        assert (np.abs(gg - want[:, E]) <= 1e-5 * scale[:, E] + 1e-30).all()


def test_router_gemm_split_picker():
    """The split keeps at least 4 K steps a slice, divides the K steps, and reaches ~512 workgroups when it can."""
    from larder_amd import _lib
    L = _lib.lib()
    assert L.lmoe_router_gemm_ksplit(2048, 4096, 513) == 4
    assert L.lmoe_router_gemm_ksplit(8192, 2048, 128) == 4
    assert L.lmoe_router_gemm_ksplit(8192, 2048, 512) == 1
    assert L.lmoe_router_gemm_ksplit(150, 2048, 61) == 8
    assert L.lmoe_router_gemm_ksplit(1, 256, 8) == 1
    assert L.lmoe_router_gemm_workspace_bytes(8192, 2048, 512) == 0
    assert L.lmoe_router_gemm_workspace_bytes(2048, 4096, 513) == 4 * 2048 * 640 * 4
