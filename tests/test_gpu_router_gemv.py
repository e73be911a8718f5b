"""The per-layer router GEMV (lmoe_router_gemv, k_router_gemv) bit for bit against the oracle's restatement of its
fixed summation order (oracle.moe.router_logits_gemv, itself pinned by test_oracle_router_order.py), at 1 to 16
tokens, 1 to 4 items a thread (H 1,024 to 8,192), f16 and bf16 x and weights, with and without the shared expert's
gate row. Every token's x goes through the kernel's own loads (the first token's with the weights, later tokens' in
the token loop), so this pins both."""
import numpy as np
import pytest
import torch

from oracle import moe

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,H,E,xdt,wdt,shared", [
    (1, 2048, 128, torch.float16, torch.float16, False),   # cfg2's shape
    (3, 2048, 60, torch.bfloat16, torch.bfloat16, True),   # cfg1's, a shared gate row
    (16, 4096, 512, torch.bfloat16, torch.float16, True),  # cfg5's, the most tokens
    (5, 8192, 64, torch.float16, torch.bfloat16, False),   # four items a thread
    (2, 1024, 9, torch.float16, torch.float16, False),     # fewer items than threads
])
def test_router_gemv_logits_bit_exact(T, H, E, xdt, wdt, shared):
    from larder_amd import _lib
    print(f"router gemv T{T} H{H} E{E} {xdt} {wdt} shared={shared}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(T * 1000 + E)
    x = torch.randn((T, H), generator=g, device="cuda").to(xdt)
    wr = (torch.randn((E, H), generator=g, device="cuda") * 0.05).to(wdt)
    wsg = (torch.randn((H,), generator=g, device="cuda") * 0.05).to(wdt) if shared else None
    rows = E + (1 if shared else 0)
    logits = torch.full((T, rows), float("nan"), device="cuda")
    _lib.call("lmoe_router_gemv", _lib.ptr(x), _lib.dcode(xdt), _lib.ptr(wr), _lib.ptr(wsg), _lib.dcode(wdt), T, H,
              E, _lib.ptr(logits), None, _lib.Q4_0, _lib.stream())
    torch.cuda.synchronize()
    w_all = wr.float().cpu().numpy()
    if shared:
        w_all = np.concatenate([w_all, wsg.float().cpu().numpy()[None]], axis=0)
    want = moe.router_logits_gemv(x.float().cpu().numpy(), w_all)
    got = logits.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), np.abs(got - want).max()
