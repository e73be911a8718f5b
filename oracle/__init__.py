"""CPU oracle for the routed-expert MoE layer over GGUF Q4_0 / Q4_K blocks.

TEST INFRASTRUCTURE ONLY. Nothing in the product path (``larder_amd``) imports, links or runs anything under
``oracle/``; only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use it, and only
as the checker (or, for ``cpu_baseline``, as the thing timed beside the GPU).

Modules:
  gguf.py            numpy restatement of ggml's Q4_0 / Q4_K block formats (dequant) plus this build's own
                     deterministic quantizers for Gaussian weights.
  moe.py             router softmax / top-k (ties to the lowest expert index), stable per-expert grouping, SwiGLU,
                     weighted combine, sigmoid-gated shared expert, and the fp32 dequant-then-matmul layer.
  cpu_kern_port.cpp  C++ restatement of the reference CPU kernel (cpu_ext/cpu_kern.cpp gather_qmm) with a C ABI,
                     used as the timed CPU baseline; built by oracle/Makefile into oracle/build/.
"""
