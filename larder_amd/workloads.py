"""Synthetic workloads of the five benchmark configurations, built directly on the GPU.

Weights are Gaussian N(0, 0.02^2) drawn with torch's seeded CUDA generator and quantized on the device
(lmoe_quantize_q4_0 / lmoe_quantize_q4_k), activations Gaussian N(0, 1). Shapes:

  cfg1  H 2048, E 60, top-4, softmax without renormalisation, I 1408, shared expert Is 5632 with a sigmoid gate
  cfg2  48 layers of H 2048, E 128, top-8 renormalised, I 768, no shared expert; batch-1 decode
  cfg3  one cfg2 layer, 8192 tokens, logits N(0,1) + per-expert bias N(0,1) (skewed groups); bf16 activations
  cfg4  one cfg2 layer, 64 sequences x 1 token, logits N(0,1) + a Zipf(1.1) log-prior (ragged groups 0..~40)
  cfg5  H 4096, E 512, top-10, I 512, shared Is 512, Q4_K
"""
import torch

from ._lib import F32, call, ptr, row_bytes, stream
from .layer import MoELayer

CONFIGS = {
    1: dict(H=2048, E=60, k=4, I=1408, norm=False, Is=5632, types=("Q4_0",) * 3),
    2: dict(H=2048, E=128, k=8, I=768, norm=True, Is=0, types=("Q4_0",) * 3, layers=48),
    3: dict(H=2048, E=128, k=8, I=768, norm=True, Is=0, types=("Q4_0",) * 3, T=8192),
    4: dict(H=2048, E=128, k=8, I=768, norm=True, Is=0, types=("Q4_0",) * 3, T=64),
    5: dict(H=4096, E=512, k=10, I=512, norm=True, Is=512, types=("Q4_K",) * 3),
}


def quantized_experts(t, n, rows, cols, gen, std=0.02, chunk_rows=1 << 18):
    """n experts [n, rows, row bytes] in ggml type t (Q4_0 or Q4_K) quantized on the device from N(0, std^2) float32
    weights drawn on the GPU (lmoe_quantize_q4_0 / lmoe_quantize_q4_k)."""
    fn = {"Q4_0": "lmoe_quantize_q4_0", "Q4_K": "lmoe_quantize_q4_k"}[t]
    out = torch.empty((n, rows, row_bytes(t, cols)), dtype=torch.uint8, device="cuda")
    flat = out.view(n * rows, -1)
    total = n * rows
    for r0 in range(0, total, chunk_rows):
        r1 = min(total, r0 + chunk_rows)
        w = torch.randn((r1 - r0, cols), generator=gen, device="cuda", dtype=torch.float32) * std
        call(fn, ptr(w), F32, r1 - r0, cols, ptr(flat[r0:r1]), stream())
        del w
    return out


# byte offsets of each block type's f16 scale fields
SCALE_AT = {"Q4_0": (0,), "Q4_K": (0, 2), "Q4_1": (0, 2), "Q8_0": (0,), "Q5_K": (0, 2), "Q6_K": (208,)}


def random_blocks(t, n, rows, cols, gen, scale=1e-3):
    """n experts [n, rows, row bytes] of ggml type t as random blocks with finite f16 scales in [0, scale), made on
    the device: timing inputs for the types without a device quantizer (the kernels' time does not depend on the
    values)."""
    rb = row_bytes(t, cols)
    from ._lib import TYPES
    _, be, bb = TYPES[t]
    nb = cols // be
    b = torch.randint(0, 256, (n, rows, nb, bb), generator=gen, device="cuda", dtype=torch.uint8)
    for at in SCALE_AT[t]:
        d = (torch.rand((n, rows, nb, 1), generator=gen, device="cuda") * scale).to(torch.float16)
        b[..., at:at + 2] = d.view(torch.uint8).reshape(n, rows, nb, 2)
    return b.reshape(n, rows, rb).contiguous()


def q4_0_experts(n, rows, cols, gen, std=0.02, chunk_rows=1 << 18):
    """n experts [n, rows, cols / 32 * 18] uint8 quantized from N(0, std^2) float32 weights drawn on the GPU."""
    return quantized_experts("Q4_0", n, rows, cols, gen, std, chunk_rows)


def router_weight(E, H, gen, std=0.02, dtype=torch.float16):
    return (torch.randn((E, H), generator=gen, device="cuda", dtype=torch.float32) * std).to(dtype)


def make_layer(cfg, gen, with_router=True):
    """One MoE layer of configuration ``cfg`` (a CONFIGS entry) with its weights quantized on the device."""
    H, E, I, Is = cfg["H"], cfg["E"], cfg["I"], cfg["Is"]
    tg, tu, td = cfg["types"]
    wg = quantized_experts(tg, E, I, H, gen)
    wu = quantized_experts(tu, E, I, H, gen)
    wd = quantized_experts(td, E, H, I, gen)
    wr = router_weight(E, H, gen) if with_router else None
    shared = wsg = None
    if Is:
        shared = (quantized_experts(tg, 1, Is, H, gen), quantized_experts(tu, 1, Is, H, gen),
                  quantized_experts(td, 1, H, Is, gen))
        wsg = router_weight(1, H, gen).reshape(H)
    return MoELayer(wg, wu, wd, cfg["types"], cfg["k"], cfg["norm"], wr=wr, shared=shared, wsg=wsg)


def skewed_logits(T, E, gen, bias_std=1.0):
    """cfg3 router logits: N(0, 1) per (token, expert) plus a per-expert bias N(0, bias_std^2)."""
    bias = torch.randn((E,), generator=gen, device="cuda") * bias_std
    return torch.randn((T, E), generator=gen, device="cuda") + bias


def zipf_logits(T, E, gen, s=1.1, scale=0.5):
    """cfg4 router logits: N(0, 1) plus scale * log of a Zipf(s) prior over a random permutation of the experts.
    scale 0.5 makes the busiest expert of a 64-token step take ~41 rows (of 512) and ~102 experts get rows, the
    ragged 0..~40 groups cfg4 is quoted on; the plain log-prior (scale 1) gave ~62 rows and 52 experts."""
    rank = torch.randperm(E, generator=gen, device="cuda").to(torch.float32) + 1.0
    prior = -s * torch.log(rank)
    prior = prior - torch.logsumexp(prior, 0)
    return torch.randn((T, E), generator=gen, device="cuda") + scale * prior


def decode_bytes(cfg, n_unique):
    """Algorithmic HBM bytes of one decode pass of one layer touching n_unique routed experts (weights only;
    activations add T * H * (in + out) bytes)."""
    H, I, Is, E = cfg["H"], cfg["I"], cfg["Is"], cfg["E"]
    expert = 2 * I * row_bytes(cfg["types"][0], H) + H * row_bytes(cfg["types"][2], I)
    shared = (2 * Is * row_bytes(cfg["types"][0], H) + H * row_bytes(cfg["types"][2], Is)) if Is else 0
    router = E * H * 2 + (H * 2 if Is else 0)
    return n_unique * expert + shared + router


def expert_flops(cfg, rows):
    """2 * rows * 3 * H * I: the routed experts' GEMM flops for ``rows`` (token, k) rows."""
    return 2 * rows * 3 * cfg["H"] * cfg["I"]


