"""The no-allocation grouping (lmoe_group_rows_noalloc) against the workspace form (lmoe_group_rows), through the C
ABI: bit-exact counts, offsets, order, inverse and work list, on two calls in a row (the second smaller, so what the
first left in the shared scratch must not leak into it), plus the refusal past the scratch's size."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import moe

pytestmark = pytest.mark.gpu


def _group(fn, ids, E, bm, ws=None):
    from larder_amd import _lib
    R = ids.numel()
    u32 = dict(dtype=torch.int32, device="cuda")
    counts = torch.full((E,), -1, **u32)
    offsets = torch.full((E + 1,), -1, **u32)
    order = torch.full((max(R, 1),), -1, **u32)
    inv = torch.full((max(R, 1),), -1, **u32)
    mt = _lib.lib().lmoe_max_tiles(R, E, bm)
    tiles = torch.full((mt,), -1, **u32)
    n_tiles = torch.full((1,), -1, **u32)
    args = [_lib.ptr(ids), R, E, bm, _lib.ptr(counts), _lib.ptr(offsets), _lib.ptr(order), _lib.ptr(inv),
            _lib.ptr(tiles), _lib.ptr(n_tiles)]
    if ws is not None:
        args.append(_lib.ptr(ws))
    _lib.call(fn, *args, _lib.stream())
    torch.cuda.synchronize()
    n = int(n_tiles.item())
    return [t.cpu().numpy() for t in (counts, offsets, order[:R], inv[:R])] + [tiles[:n].cpu().numpy()]


@pytest.mark.parametrize("first,second", [((65536, 128, 128), (5000, 128, 32)), ((300000, 128, 128), (700, 60, 32)),
                                          ((60000, 1024, 128), (4096, 512, 128))])
def test_group_rows_noalloc_matches_workspace_form(first, second):
    from larder_amd import _lib
    for i, (R, E, bm) in enumerate((first, second)):
        print(f"no-alloc grouping: call {i} R {R} E {E} bm {bm}", flush=True)
        rng = np.random.default_rng(R + E)
        ids_np = rng.integers(0, E + 3, R).astype(np.int32)   # a few ids past the experts
        ids_np[: R // 7] = rng.integers(0, 4, R // 7)          # a skewed head
        ids = torch.from_numpy(ids_np).cuda()
        ws = torch.empty(_lib.lib().lmoe_group_workspace_bytes(R, E), dtype=torch.uint8, device="cuda")
        want = _group("lmoe_group_rows", ids, E, bm, ws)
        got = _group("lmoe_group_rows_noalloc", ids, E, bm)
        for w, g in zip(want, got):
            assert np.array_equal(w, g)
        counts, offsets, order, inv = moe.group_rows(ids_np.astype(np.uint32), E)
        assert np.array_equal(got[0].astype(np.uint32), counts)
        assert np.array_equal(got[2].astype(np.uint32), order)


def test_group_rows_noalloc_refuses_past_its_scratch():
    from larder_amd import _lib
    ids = torch.zeros(1, dtype=torch.int32, device="cuda")
    u = torch.zeros(2048, dtype=torch.int32, device="cuda")
    R = 1 << 20                   # (4097 chunks + 1) x 129 buckets x 4 bytes > 1 MiB
    rc = _lib.lib().lmoe_group_rows_noalloc(_lib.ptr(ids), R, 128, 128, _lib.ptr(u), _lib.ptr(u), _lib.ptr(u),
                                            _lib.ptr(u), None, None, _lib.stream())
    assert rc == _lib.EWORKSPACE
    assert b"scratch" in _lib.lib().lmoe_error()
