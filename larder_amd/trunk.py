"""The steps beside the routed experts on T rows: the trunk's 4-bit affine matmul and the shared expert built on it.

    qmv_fits(x, w, scales, group_size, bits, mode, biases)   route_cuda.py:516-522
    qmv_rows(x, w, scales, biases, group_size)               route_cuda.py:525-541 (lmoe_qmv_rows)
    shared_expert_rows(x, gate, up, down)                    mlx_lm's shared_expert MLP on qmv_rows projections

qmv_rows gives every row of x the bits of the reference's kernel (MLX 0.32.4's one-row qmv arithmetic: bf16
weights, bf16 fused multiply-add slots, a float32 slot sum and lane butterfly), reading the weights once a pass.
Weights are MLX's affine 4-bit layout as torch tensors on the GPU: w uint32 / int32 [N, K / 8], scales and biases
bfloat16 [N, K / G].
"""
import torch

from ._lib import call, ptr, stream

__all__ = ["qmv_fits", "qmv_rows", "shared_expert_rows"]


def qmv_fits(x, w, scales, group_size, bits, mode, biases):
    """Whether qmv_rows serves this product (route_cuda.py:516-522): 4-bit affine with biases, bf16 x, scales and
    biases, a 2-D packed weight, K a multiple of 16 and of the group size, the group size a multiple of 16."""
    k = x.shape[-1]
    return (bits == 4 and mode == "affine" and biases is not None and x.dtype == torch.bfloat16
            and scales.dtype == torch.bfloat16 and biases.dtype == torch.bfloat16
            and w.dtype in (torch.int32, torch.uint32) and w.dim() == 2 and k % 16 == 0 and k % group_size == 0
            and group_size % 16 == 0 and w.shape[-1] * 8 == k)


def qmv_rows(x, w, scales, biases, group_size):
    """x [..., T, K] bf16 times the 4-bit affine weight (transposed) -> [..., T, N] bf16, each row bit-equal to the
    reference's one-row pass (route_cuda.py:525-541)."""
    if not qmv_fits(x, w, scales, group_size, 4, "affine", biases):
        raise ValueError("qmv_rows: bf16 x, 4-bit affine uint32 weights with bf16 scales and biases, K a multiple of "
                         "16 and of the group size")
    K = x.shape[-1]
    N = w.shape[0]
    x2 = x.reshape(-1, K).contiguous()
    out = torch.empty((x2.shape[0], N), dtype=torch.bfloat16, device=x.device)
    call("lmoe_qmv_rows", ptr(x2), x2.shape[0], ptr(w.contiguous()), ptr(scales.contiguous()),
         ptr(biases.contiguous()), N, K, group_size, ptr(out), stream())
    return out.reshape(x.shape[:-1] + (N,))


def shared_expert_rows(x, gate, up, down):
    """mlx_lm's shared-expert MLP, down(silu(gate(x)) * up(x)), for x [..., T, H] bf16 with each projection a
    (w, scales, biases, group_size) 4-bit affine weight run through qmv_rows; the SwiGLU rounds once to bf16
    (lmoe_swiglu_bf16). The sigmoid-gated add to the routed output is route.tail's."""
    g = qmv_rows(x, *gate)
    u = qmv_rows(x, *up)
    h = torch.empty_like(g)
    call("lmoe_swiglu_bf16", ptr(g), ptr(u), g.numel(), ptr(h), stream())
    return qmv_rows(h, *down)
