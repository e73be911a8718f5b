"""The C ABI: the in-tree library loads, exports every entry point include/larder_moe.h declares, and refuses bad
arguments with a negative code and a reason before it touches the GPU (so these run without one)."""
import ctypes
import re
from pathlib import Path

import pytest

from larder_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "larder_moe.h"


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(lmoe_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported(built_lib):
    names = declared()
    assert len(names) >= 12
    for n in names:
        assert hasattr(built_lib, n), f"{n} is declared in larder_moe.h but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature in larder_amd/_lib.py"


def test_no_undeclared_signatures():
    assert set(_lib.SIGNATURES) == set(declared())


def test_abi_version(built_lib):
    assert built_lib.lmoe_abi_version() == _lib.ABI_VERSION


def test_refusals_without_a_gpu(built_lib):
    L = built_lib
    p = ctypes.c_void_p(16)   # never dereferenced: every call below is refused during argument checks
    rc = L.lmoe_router_topk(p, 7, 1, 128, 8, 1, p, p, None)
    assert rc == _lib.EINVAL and b"dtype" in L.lmoe_error()
    rc = L.lmoe_router_topk(p, _lib.F32, 1, 2000, 8, 1, p, p, None)
    assert rc == _lib.ESHAPE and b"experts" in L.lmoe_error()
    rc = L.lmoe_router_topk(p, _lib.F32, 1, 128, 33, 1, p, p, None)
    assert rc == _lib.ESHAPE and b"top-k" in L.lmoe_error()
    rc = L.lmoe_gemv_gate_up(p, _lib.F16, p, 8, 8, p, p, 9, 9, 128, 2048, 768, p, None)
    assert rc == _lib.ETYPE and b"types 9/9" in L.lmoe_error()
    # the types beyond Q4_0 / Q4_K: the general chain only, their own row-length and alignment rules
    rc = L.lmoe_gemv_gate_up_prepped(p, p, p, 8, 8, p, p, 14, 14, 128, 2048, 768, p, None, 14, None)
    assert rc == _lib.ETYPE and b"general chain" in L.lmoe_error()
    rc = L.lmoe_gemv_gate_up(p, _lib.F16, p, 8, 8, p, p, 14, 14, 128, 2048 + 32, 768, p, None)
    assert rc == _lib.ESHAPE and b"256" in L.lmoe_error()
    rc = L.lmoe_gemv_gate_up(p, _lib.F16, p, 8, 8, ctypes.c_void_p(18), p, 13, 13, 128, 2048, 768, p, None)
    assert rc == _lib.EALIGN and b"16-byte" in L.lmoe_error()
    # prepared h feeds Q4_0 / Q4_K / Q6_K / Q8_0 downs only: a Q5_K down (13) is refused before any launch
    rc = L.lmoe_gemv_down_combine_prepped(p, 0, p, p, 1, 8, p, 13, 128, 768, 2048, None, None, 0, None, 0, p,
                                          _lib.F16, None)
    assert rc == _lib.ETYPE and b"general chain" in L.lmoe_error()
    rc = L.lmoe_dequant_gemm_f16(p, 9, 4, 16, 64, p, None)
    assert rc == _lib.ETYPE
    rc = L.lmoe_dequant_gemm_f16(p, 8, 4, 16, 48, p, None)
    assert rc == _lib.ESHAPE
    rc = L.lmoe_grouped_gate_up_f16w(p, _lib.F32, 64, 1, p, p, p, p, 4, 128, p, p, 8, 2048, 768, p, None)
    assert rc == _lib.EINVAL and b"float16" in L.lmoe_error()
    rc = L.lmoe_grouped_gate_up_f16w(p, _lib.F16, 64, 1, p, p, p, p, 4, 128, p, p, 8, 2048, 100, p, None)
    assert rc == _lib.ESHAPE
    rc = L.lmoe_grouped_gate_up_f16w(p, _lib.F16, 64, 1, p, p, p, p, 4, 32, p, p, 8, 2048, 768, p, None)
    assert rc == _lib.ESHAPE and b"tile rows" in L.lmoe_error()
    rc = L.lmoe_grouped_down_f16w(p, p, p, p, 4, 128, p, 8, 768, 2000, p, _lib.F16, None)
    assert rc == _lib.ESHAPE
    rc = L.lmoe_gemv_gate_up(p, _lib.F16, p, 8, 8, p, p, _lib.Q4_0, _lib.Q4_0, 128, 2000, 768, p, None)
    assert rc == _lib.ESHAPE
    rc = L.lmoe_gemv_gate_up(p, _lib.F16, p, 8, 8, p, p, _lib.Q4_K, _lib.Q4_K, 128, 2048 + 64, 768, p, None)
    assert rc == _lib.ESHAPE and b"256" in L.lmoe_error()
    rc = L.lmoe_gemv_gate_up(p, _lib.F16, p, 8, 8, ctypes.c_void_p(18), p, _lib.Q4_0, _lib.Q4_0, 128, 2048, 768, p,
                             None)
    assert rc == _lib.EALIGN
    rc = L.lmoe_gemv_down_combine(p, p, p, 1, 40, p, _lib.Q4_0, 128, 768, 2048, None, None, 0, None, 0, p,
                                  _lib.F16, None)
    assert rc == _lib.ESHAPE
    rc = L.lmoe_group_rows(p, 10, 2000, 128, p, p, p, p, None, None, p, None)
    assert rc == _lib.ESHAPE
    rc = L.lmoe_dequant(p, 9, 4, 16, 64, p, 1, p, _lib.F32, None)
    assert rc == _lib.ETYPE
    rc = L.lmoe_quantize_q4_0(p, _lib.F32, 4, 33, p, None)
    assert rc == _lib.ESHAPE
    assert L.lmoe_max_tiles(65536, 128, 128) == 512 + 128
    # the run kernels: Q4_0 / Q4_K only, a window of at least one row, aligned rows
    rc = L.lmoe_gemv_gate_up_runs(p, _lib.F16, p, 8, 8, p, p, 14, 14, 128, 2048, 768, p, None)
    assert rc == _lib.ETYPE and b"run kernels" in L.lmoe_error()
    rc = L.lmoe_gemv_gate_up_runs(p, _lib.F16, p, 8, 0, p, p, _lib.Q4_0, _lib.Q4_0, 128, 2048, 768, p, None)
    assert rc == _lib.ESHAPE and b"window 0" in L.lmoe_error()
    rc = L.lmoe_gemv_gate_up_runs(ctypes.c_void_p(18), _lib.F16, p, 8, 8, p, p, _lib.Q4_0, _lib.Q4_0, 128, 2048, 768,
                                  p, None)
    assert rc == _lib.EALIGN
    rc = L.lmoe_gemv_gate_up_runs(p, _lib.F16, p, 0, 8, p, p, _lib.Q4_0, _lib.Q4_0, 128, 2048, 768, p, None)
    assert rc == 0   # no rows: nothing to launch
    rc = L.lmoe_gemv_down_runs(p, p, 8, 8, p, 8, 128, 768, 2048, p, _lib.F16, None)
    assert rc == _lib.ETYPE and b"run kernels" in L.lmoe_error()
    rc = L.lmoe_gemv_down_runs(p, p, 8, 8, p, _lib.Q4_K, 128, 640, 2048, p, _lib.F16, None)
    assert rc == _lib.ESHAPE and b"256" in L.lmoe_error()
    rc = L.lmoe_gemv_down_runs(p, p, 8, 8, p, _lib.Q4_0, 128, 768, 2048, p, 9, None)
    assert rc == _lib.EINVAL
    # the stream layout: Q4 only, rows a multiple of 128; the Q4_K GEMM on it only at 64-row tiles
    assert L.lmoe_stream_bytes(_lib.Q4_0, 4, 256, 512) == 4 * 256 * 16 * 18
    assert L.lmoe_stream_bytes(_lib.Q4_K, 4, 256, 512) == 4 * 256 * 2 * 144
    assert L.lmoe_stream_bytes(_lib.Q4_0, 4, 200, 512) == 0 and L.lmoe_stream_bytes(14, 4, 256, 512) == 0
    assert L.lmoe_stream_bytes(_lib.Q4_K, 4, 256, 320) == 0
    rc = L.lmoe_stream_repack(p, 14, 4, 256, 512, p, None)
    assert rc == _lib.ETYPE
    rc = L.lmoe_stream_repack(p, _lib.Q4_0, 4, 200, 512, p, None)
    assert rc == _lib.ESHAPE and b"128" in L.lmoe_error()
    rc = L.lmoe_grouped_gate_up_sl(p, _lib.F16, 64, 1, p, p, p, p, 4, 128, 1, None, p, p, _lib.Q4_K, _lib.Q4_K, 8,
                                   1024, 512, p, None)
    assert rc == _lib.ESHAPE and b"64-row" in L.lmoe_error()
    rc = L.lmoe_grouped_down_sl(p, 64, p, p, p, 4, 32, 1, None, p, _lib.Q4_K, 8, 512, 1024, p, _lib.F16, None)
    assert rc == _lib.ESHAPE and b"64-row" in L.lmoe_error()
    # the top-k and the K-order conversion in one launch: the top-k's limits and the conversion's
    rc = L.lmoe_topk_and_gemm_f16(p, _lib.F32, 4, 2000, 8, 1, p, p, p, _lib.F16, 4096, p, None)
    assert rc == _lib.ESHAPE and b"experts" in L.lmoe_error()
    rc = L.lmoe_topk_and_gemm_f16(p, _lib.F32, 4, 128, 8, 1, p, p, p, _lib.F16, 4016, p, None)
    assert rc == _lib.ESHAPE and b"multiple of 32" in L.lmoe_error()
    rc = L.lmoe_topk_and_gemm_f16(p, _lib.F32, 4, 128, 8, 1, p, p, ctypes.c_void_p(18), _lib.F16, 4096, p, None)
    assert rc == _lib.EALIGN
    # the prefill router GEMM with its top-k: the top-k's limits, and shared slices only with the gate row
    rc = L.lmoe_router_gemm_topk(p, 64, 2048, p, 128, 0, p, p, None, 33, 1, 0, p, p, None)
    assert rc == _lib.ESHAPE and b"top-k 33" in L.lmoe_error()
    rc = L.lmoe_router_gemm_topk(p, 64, 2048, p, 128, 0, p, p, None, 8, 1, 1, p, p, None)
    assert rc == _lib.EINVAL and b"gate row" in L.lmoe_error()
    # the drop-in chain's register-resident form: hidden 2048 / 4096, one Q4 type, h or its prepared rows asked for;
    # its down: a width that is a multiple of 128 up to 8192
    rc = L.lmoe_gemv_chain_gate_up(p, _lib.F16, p, 8, 8, p, p, _lib.Q4_0, 128, 1024, 768, p, p, _lib.Q4_0, None)
    assert rc == _lib.ESHAPE and b"hidden 2048 or 4096" in L.lmoe_error()
    rc = L.lmoe_gemv_chain_gate_up(p, _lib.F16, p, 8, 8, p, p, 14, 128, 2048, 768, p, p, _lib.Q4_0, None)
    assert rc == _lib.ETYPE
    rc = L.lmoe_gemv_chain_gate_up(p, _lib.F16, p, 8, 8, p, p, _lib.Q4_0, 128, 2048, 768, None, None, _lib.Q4_0, None)
    assert rc == _lib.EINVAL and b"neither h" in L.lmoe_error()
    rc = L.lmoe_gemv_chain_down(p, p, 8, p, _lib.Q4_0, 128, 704, 2048, p, _lib.F16, None)
    assert rc == _lib.ESHAPE and b"multiple of 128" in L.lmoe_error()
    rc = L.lmoe_gemv_down_runs_prepped(p, p, 8, 4, p, _lib.Q4_0, 128, 704, 2048, p, _lib.F16, None)
    assert rc == _lib.ESHAPE and b"multiple of 128" in L.lmoe_error()
    rc = L.lmoe_gemv_gate_up_runs_prepped(p, p, 8, 4, p, p, _lib.Q4_K, 128, 2048, 767, p, None, _lib.Q4_K, None)
    assert rc == _lib.ESHAPE and b"even width" in L.lmoe_error()


def test_grouped_refusals_without_a_gpu(built_lib):
    L = built_lib
    p = ctypes.c_void_p(16)   # never dereferenced: refused during argument checks
    z = None
    assert L.lmoe_grouped_gate_up(p, 1, 4, 1, p, p, p, p, 4, p, p, 3, 3, 4, 512, 256, p, z) == _lib.ETYPE
    assert L.lmoe_grouped_gate_up(p, 1, 4, 1, p, p, p, p, 4, p, p, 2, 12, 4, 512, 256, p, z) == _lib.ETYPE
    assert b"share one type" in L.lmoe_error()
    assert L.lmoe_grouped_gate_up(p, 1, 4, 1, p, p, p, p, 4, p, p, 12, 12, 4, 512 + 64, 256, p, z) == _lib.ESHAPE
    assert L.lmoe_grouped_gate_up(p, 1, 4, 1, p, p, p, p, 4, p, p, 2, 2, 4, 512, 256 + 32, p, z) == _lib.ESHAPE
    assert L.lmoe_grouped_gate_up(p, 9, 4, 1, p, p, p, p, 4, p, p, 2, 2, 4, 512, 256, p, z) == _lib.EINVAL
    assert L.lmoe_grouped_gate_up(p, 2, 4, 1, p, p, p, p, 4, p, p, 2, 2, 4, 512, 256, p, z) == _lib.EINVAL
    assert b"lmoe_to_gemm_f16" in L.lmoe_error()
    assert L.lmoe_grouped_gate_up(p, 1, 4, 1, p, p, p, p, 4, p, p, 2, 2, 4, 576, 200, p, z) == _lib.ESHAPE
    assert L.lmoe_grouped_gate_up(p, 1, 4, 1, p, p, p, p, 4, p, p, 2, 2, 4, 512, 256, z, z) == _lib.EINVAL
    assert L.lmoe_grouped_gate_up(ctypes.c_void_p(8), 1, 4, 1, p, p, p, p, 4, p, p, 2, 2, 4, 512, 256, p, z) == \
        _lib.EALIGN
    assert L.lmoe_grouped_down(p, p, p, p, 4, p, 2, 4, 256, 512 + 64, p, 1, z) == _lib.ESHAPE
    assert L.lmoe_grouped_down(p, p, p, p, 4, p, 2, 4, 256 + 32, 512, p, 1, z) == _lib.ESHAPE
    assert L.lmoe_grouped_down(p, p, p, p, 4, p, 2, 4, 256, 512, p, 2, z) == _lib.EINVAL
    assert L.lmoe_grouped_down(p, p, p, p, 4, p, 5, 4, 256, 512, p, 1, z) == _lib.ETYPE
    assert L.lmoe_grouped_down(p, p, p, p, 4, p, 2, 4, 320, 600, p, 1, z) == _lib.ESHAPE
    assert L.lmoe_to_f16(p, 7, 10, p, z) == _lib.EINVAL
    assert L.lmoe_to_f16(p, 0, -1, p, z) == _lib.ESHAPE
    assert L.lmoe_to_gemm_f16(p, 0, 48, p, z) == _lib.ESHAPE  # not a multiple of 32
    f = ctypes.c_float
    assert L.lmoe_route_bias(p, 0, 17, 256, 8, p, p, 10, f(0.5), f(0.0), 0, 0, p, None, None, None, z) == _lib.ESHAPE
    assert L.lmoe_route_bias(p, 0, 2, 256, 33, p, p, 10, f(0.5), f(0.0), 0, 0, p, None, None, None, z) == _lib.ESHAPE
    assert L.lmoe_route_bias(p, 0, 2, 256, 8, None, None, 10, f(0.5), f(0.0), 0, 0, p, None, None, None, z) == \
        _lib.EINVAL
    assert L.lmoe_route_bias(p, 0, 2, 256, 8, p, p, 10, f(-1.0), f(0.0), 0, 0, p, None, None, None, z) == _lib.EINVAL
    assert L.lmoe_route_bias(p, 0, 2, 256, 8, p, None, 10, f(0.5), f(0.0), 0, 0, p, p, p, None, z) == _lib.EINVAL
    assert L.lmoe_to_gemm_f16(ctypes.c_void_p(8), 0, 64, p, z) == _lib.EALIGN
    assert L.lmoe_grouped_tile_rows() == 128


def test_python_refuses_unsupported_types():
    with pytest.raises(ValueError, match="IQ4_XS"):
        _lib.qcode("IQ4_XS")
    assert [_lib.qcode(t) for t in ("Q4_0", "Q4_1", "Q8_0", "Q4_K", "Q5_K", "Q6_K")] == [2, 3, 8, 12, 13, 14]


def test_gemm_k_order_index():
    """kperm_index against the order written out by hand: inside a 32-wide block, positions 0..31 hold natural
    columns 0-3, 16-19, 4-7, 20-23, 8-11, 24-27, 12-15, 28-31."""
    from larder_amd import grouped
    block = [0, 1, 2, 3, 16, 17, 18, 19, 4, 5, 6, 7, 20, 21, 22, 23, 8, 9, 10, 11, 24, 25, 26, 27,
             12, 13, 14, 15, 28, 29, 30, 31]
    pos = grouped.kperm_index(96, "cpu").tolist()
    for j in range(96):
        assert 32 * (j // 32) + block[pos[j] % 32] == j
    assert sorted(pos) == list(range(96))


def test_grouped_launch_choices(built_lib):
    """lmoe_grouped_pick_tile_rows / pick_ksplit / workspace_bytes (host functions, no GPU): the configurations'
    choices, and split-K slices that divide K into at least 8 steps each (4 two-unit steps) with a workspace that
    holds them."""
    from larder_amd import grouped
    q = _lib.qcode
    pick = lambda R, E, ts: built_lib.lmoe_grouped_pick_tile_rows(R, E, *(q(t) for t in ts))  # noqa: E731
    assert pick(8192 * 8, 128, ("Q4_0",) * 3) == 128      # cfg3 prefill
    assert pick(64 * 8, 128, ("Q4_0",) * 3) == 32         # cfg4 batched decode
    assert pick(2048 * 10, 512, ("Q4_K",) * 3) == 64      # cfg5 prefill: the direct-copy Q4_K kernel
    assert pick(64, 512, ("Q4_K",) * 3) == 64             # few rows, Q4_K
    assert pick(64, 128, ("Q4_K", "Q4_K", "Q6_K")) == 64   # Q4_K gate/up, f16 down
    assert pick(64, 128, ("Q4_0", "Q4_0", "Q6_K")) == 128  # Q4_0 gate/up, f16 down
    for ts in (("Q8_0",) * 3, ("Q4_0", "Q4_K", "Q4_0"), ("Q6_K", "Q6_K", "Q4_K")):
        assert pick(2048 * 8, 128, ts) == 64              # gate/up on f16 weights
    assert grouped.pick_tile_rows(512, 128, ("Q4_0",) * 3) == 32
    for R, E, bm, K in ((512, 128, 32, 2048), (512, 128, 32, 768), (80, 60, 32, 5632), (512, 128, 32, 256),
                        (512, 128, 128, 2048), (4096, 128, 32, 2048), (16, 4, 32, 192)):
        ks = built_lib.lmoe_grouped_pick_ksplit(R, E, bm, K)
        if bm != 32 or R >= 16 * E:
            assert ks == 1
        else:
            assert ks == 1 or (ks in (2, 3, 4) and (K // 64) % (2 * ks) == 0 and K // 64 // ks >= 8)
    assert built_lib.lmoe_grouped_pick_ksplit(512, 128, 32, 2048) == 4   # 32 steps: 4 slices of 8
    assert built_lib.lmoe_grouped_pick_ksplit(512, 128, 32, 768) == 1    # 12 steps: no slice of 8
    assert built_lib.lmoe_grouped_pick_ksplit(512, 128, 32, 1024) == 2   # 16 steps: 2 slices of 8
    assert built_lib.lmoe_grouped_pick_ksplit(512, 128, 32, 256) == 1    # 4 steps
    R, E, H, I = 512, 128, 2048, 768
    ku, kd = built_lib.lmoe_grouped_pick_ksplit(R, E, 32, H), built_lib.lmoe_grouped_pick_ksplit(R, E, 32, I)
    assert built_lib.lmoe_grouped_workspace_bytes(R, E, 32, H, I) == 4 * max(ku * R * 2 * I, kd * R * H)
    assert built_lib.lmoe_grouped_workspace_bytes(R, E, 128, H, I) == 0
    assert grouped.splitk_floats(R, E, 32, H, I) * 4 == built_lib.lmoe_grouped_workspace_bytes(R, E, 32, H, I)


def test_tile_and_split_knobs(built_lib, monkeypatch):
    """LMOE_TILE_ROWS / LMOE_KSPLIT override the pickers on every call when the value is one the GEMMs take for the
    types, and are ignored otherwise; the split-K workspace follows the forced split."""
    q = _lib.qcode
    pick = lambda R, E, ts: built_lib.lmoe_grouped_pick_tile_rows(R, E, *(q(t) for t in ts))  # noqa: E731
    q40, q4k, mix = ("Q4_0",) * 3, ("Q4_K",) * 3, ("Q4_K", "Q4_K", "Q6_K")
    for v, want in (("64", 64), ("128", 128), ("32", 32), ("48", 128), ("", 128)):
        monkeypatch.setenv("LMOE_TILE_ROWS", v)
        assert pick(8192 * 8, 128, q40) == want, v
    monkeypatch.setenv("LMOE_TILE_ROWS", "32")
    assert pick(2048 * 10, 512, q4k) == 32                  # Q4_K has 32-row tiles too
    assert pick(64, 128, mix) == 64                          # an f16-weight down has none: the rule
    monkeypatch.setenv("LMOE_TILE_ROWS", "128")
    assert pick(64, 128, mix) == 128
    monkeypatch.delenv("LMOE_TILE_ROWS")
    ks = built_lib.lmoe_grouped_pick_ksplit
    assert ks(8192 * 8, 128, 32, 2048) == 1                 # the rule: enough rows an expert
    monkeypatch.setenv("LMOE_KSPLIT", "2")
    assert ks(8192 * 8, 128, 32, 2048) == 1                 # more than 65,535 rows: not taken
    assert ks(4096, 128, 32, 2048) == 2
    assert ks(4096, 128, 128, 2048) == 1                    # split-K only on 32-row tiles
    # both GEMMs split in 2 (gate/up over H = 2048, down over I = 768): the larger slice set, down's
    assert built_lib.lmoe_grouped_workspace_bytes(4096, 128, 32, 2048, 768) == 2 * 4096 * max(2 * 768, 2048) * 4
    monkeypatch.setenv("LMOE_KSPLIT", "3")
    assert ks(4096, 128, 32, 2048) == 1                     # 32 K steps do not split in 3: the rule
    assert ks(512, 128, 32, 768) == 3                       # 12 K steps split in 3
    monkeypatch.setenv("LMOE_KSPLIT", "1")
    assert ks(512, 128, 32, 2048) == 1                      # the rule would split in 4


def test_dense_knob(monkeypatch):
    """LMOE_DENSE forces experts()'s switch either way, else dense_pays decides."""
    from larder_amd import gguf_experts as ge
    for v, rule, want in (("1", False, True), ("0", True, False), ("", True, True), ("", False, False),
                          ("2", True, True)):
        monkeypatch.setenv("LMOE_DENSE", v)
        assert ge._dense_knob(lambda r=rule: r) is want
