"""The wavefront top-k's algorithm (larder_amd/csrc/lmoe_common.h, topk_wave) emulated on the CPU
(tests/emul/topk_wave.cpp: 64 lanes as loops, ballots as masks): its one-bit threshold search (which stops once
exactly k keys are at or above the prefix) and a two-bits-a-step form both give the oracle's picks (lowest index
first among equal logits) on the tie-heavy rows the GPU tests use (test_gpu_decode.tie_logits), in float32, float16
and bfloat16, and the compaction writes exactly k picks, so it never reaches past the 32-pick LDS area. So does
rank_pick_wave (one rank's pick without the compaction), rank by rank. This is the CPU check a faster top-k must pass
before it runs on a GPU."""
import shutil
import subprocess

import numpy as np
import pytest
import torch

from oracle import moe

SRC = __file__.rsplit("/", 1)[0] + "/emul/topk_wave.cpp"


def tie_logits(rng, T, E):
    lg = rng.normal(0, 1.0, (T, E)).astype(np.float32) * rng.uniform(0.5, 4.0)
    for r in range(T):
        if r % 5 == 0:
            j = rng.integers(0, E, 6)
            lg[r, j] = lg[r, j[0]]
        if r % 7 == 0:
            lg[r] = np.round(lg[r] * 2) / 2
        if r % 13 == 0:
            lg[r] = 0.25
    return lg


@pytest.fixture(scope="module")
def emul(tmp_path_factory):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no g++")
    exe = tmp_path_factory.mktemp("emul") / "topk_wave"
    subprocess.run([cxx, "-O2", "-std=c++17", "-o", str(exe), SRC], check=True)
    return str(exe)


def negative_tie_rows(rng, T, E):
    """All-negative rows in steps of 0.5: the k-th largest key is negative (its low bits set) and tied."""
    return (-np.round(np.abs(rng.normal(0, 2.0, (T, E))) * 2) / 2 - 0.5).astype(np.float32)


def run_emul(exe, lg, k, slip=0):
    T, E = lg.shape
    lines = [f"{T} {E} {k}"] + [" ".join(f"{b:08x}" for b in row.view(np.uint32)) for row in lg]
    out = subprocess.run([exe, str(slip)], input="\n".join(lines) + "\n", capture_output=True, text=True,
                         check=True).stdout.strip().splitlines()
    assert len(out) == T
    return [[p.split() for p in line.split("|")] for line in out]


def rows_for(E, k, dtype):
    rng = np.random.default_rng(E * 7 + k)
    lg = np.concatenate([tie_logits(rng, 67, E), negative_tie_rows(rng, 16, E)])
    return torch.from_numpy(lg).to(dtype).float().numpy()        # the values the kernel sees for this dtype


@pytest.mark.parametrize("E,k", [(60, 4), (128, 8), (512, 10), (1024, 32), (9, 9)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_wave_topk_emulation_matches_oracle(emul, E, k, dtype):
    lg = rows_for(E, k, dtype)
    want, _ = moe.router(lg, k, False)
    for r, forms in enumerate(run_emul(emul, lg, k)):
        for name, f in zip(("one-bit", "two-bit", "rank pick"), forms):
            assert f[0] == "ok" and int(f[1]) == k, (name, r, f)
            assert [int(v) for v in f[2:]] == [int(v) for v in want[r]], (name, r)


@pytest.mark.parametrize("slip", [2, 3])
def test_emulation_catches_planted_slips(emul, slip):
    """Slips planted in the two-bit search on the CPU (2: candidates tried low to high; 3: the loop one step short,
    leaving the threshold's two low bits clear) give wrong picks and more than k of them, the overrun that runs past
    a 32-pick LDS area when k = 32. (A '>' for '>=' in the candidate test gives the right picks: the keys above a
    threshold just under the k-th are still exactly the top k.)"""
    wrong = over = 0
    for E, k in [(128, 8), (1024, 32)]:
        for dtype in (torch.float32, torch.bfloat16):
            lg = rows_for(E, k, dtype)
            want, _ = moe.router(lg, k, False)
            for r, forms in enumerate(run_emul(emul, lg, k, slip)):
                f = forms[1]
                wrong += f[0] != "ok" or [int(v) for v in f[2:]] != [int(v) for v in want[r]]
                over += int(f[1]) > k
    assert wrong > 0 and over > 0


def test_emulation_catches_an_early_stop_slip(emul):
    """The one-bit search stops only at a prefix with exactly k keys at or above it. Stopping at the first prefix
    with at least k (slip 4, planted on the CPU) keeps a threshold too low: more than k picks and wrong ids."""
    wrong = over = 0
    for E, k in [(128, 8), (512, 10)]:
        lg = rows_for(E, k, torch.float32)
        want, _ = moe.router(lg, k, False)
        for r, forms in enumerate(run_emul(emul, lg, k, 4)):
            f = forms[0]
            wrong += f[0] != "ok" or [int(v) for v in f[2:]] != [int(v) for v in want[r]]
            over += int(f[1]) > k
    assert wrong > 0 and over > 0


@pytest.mark.parametrize("slip", [5, 6])
def test_emulation_catches_rank_pick_slips(emul, slip):
    """rank_pick_wave (one rank's pick, no compaction) on the tie-heavy rows: a slip planted on the CPU (5: the lowest
    index among the smallest keys when the search stops early; 6: the keys above the threshold not counted when it
    runs to the end) gives wrong ids."""
    wrong = 0
    for E, k in [(128, 8), (512, 10), (60, 4)]:
        for dtype in (torch.float32, torch.bfloat16):
            lg = rows_for(E, k, dtype)
            want, _ = moe.router(lg, k, False)
            for r, forms in enumerate(run_emul(emul, lg, k, slip)):
                wrong += [int(v) for v in forms[2][2:]] != [int(v) for v in want[r]]
    assert wrong > 0
