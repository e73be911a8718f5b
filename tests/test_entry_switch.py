"""The drop-in entry's path switch on the CPU (larder_amd.gguf_experts: dense_pays and calibrate's cache), with the
device key and the measurement replaced so that no GPU is needed. The reference's rule (gguf_experts.py:797-800):
the dense path pays when its fixed + per-expert + per-row cost is below the chain's fixed + per-row cost; with no
fit, every pass takes the chain."""
import json

import pytest

from larder_amd import gguf_experts as ge


def test_dense_pays_rule(monkeypatch):
    monkeypatch.setattr(ge, "_COST", None)
    assert not ge.dense_pays(1, 10_000)                      # no fit: the chain
    # chain 10 us + 2 us a row; dense 50 us + 1 us an expert + 0.1 us a row
    monkeypatch.setattr(ge, "_COST", [10e-6, 2e-6, 50e-6, 1e-6, 0.1e-6])
    # p rows over u experts: dense 50 + u + 0.1 p against chain 10 + 2 p
    assert not ge.dense_pays(4, 10)                          # 55 vs 30
    assert ge.dense_pays(4, 40)                              # 58 vs 90
    assert not ge.dense_pays(100, 40)                        # 154 vs 90
    assert ge.dense_pays(100, 100)                           # 160 vs 210


def test_calibrate_caches_by_device_and_shape(monkeypatch, tmp_path):
    monkeypatch.setenv("LMOE_CACHE", str(tmp_path))
    monkeypatch.setattr(ge, "_device_key", lambda: ["gfx950", 256, "7.0", "src"])
    calls = []

    def fake_measure(hid, inter, types):
        calls.append((hid, inter, types))
        return [1e-5, 2e-6, 4e-5, 1e-6, 1e-7]

    monkeypatch.setattr(ge, "_measure", fake_measure)
    checked = []
    monkeypatch.setattr(ge, "_runs_ok", lambda *a: checked.append(a) or True)
    cost = ge.calibrate(2048, 768, "Q4_0/Q4_0/Q4_0")
    assert cost == [1e-5, 2e-6, 4e-5, 1e-6, 1e-7] and ge._COST == cost and len(calls) == 1
    # the run kernels are checked at load (gguf_experts.py:791-792), at the reference's bf16 -> bf16
    import torch
    assert checked == [(2048, 768, ("Q4_0",) * 3, torch.bfloat16, torch.bfloat16)]
    files = list(tmp_path.glob("dense-switch-*.json"))
    assert len(files) == 1 and json.loads(files[0].read_text())["cost"] == cost
    # the second call reads the cache
    assert ge.calibrate(2048, 768, ("Q4_0", "Q4_0", "Q4_0")) == cost and len(calls) == 1
    # another shape, or another device, is measured again
    ge.calibrate(2048, 512, "Q4_0/Q4_0/Q4_0")
    monkeypatch.setattr(ge, "_device_key", lambda: ["gfx950", 304, "7.0", "src"])
    ge.calibrate(2048, 768, "Q4_0/Q4_0/Q4_0")
    assert len(calls) == 3 and len(list(tmp_path.glob("dense-switch-*.json"))) == 3
    # a damaged cache file is measured over
    for f in tmp_path.glob("dense-switch-*.json"):
        f.write_text("{")
    ge.calibrate(2048, 768, "Q4_0/Q4_0/Q4_0")
    assert len(calls) == 4
    # every load asks (the check itself runs once a key); LMOE_GGUF_RUNS=0 skips it
    assert len(checked) == 5
    monkeypatch.setenv("LMOE_GGUF_RUNS", "0")
    ge.calibrate(2048, 768, "Q4_0/Q4_0/Q4_0")
    assert len(checked) == 5


def test_calibrate_unwritable_cache_still_fits(monkeypatch, tmp_path, capsys):
    blocker = tmp_path / "file"
    blocker.write_text("")
    monkeypatch.setenv("LMOE_CACHE", str(blocker / "sub"))      # a directory under a file: cannot be created
    monkeypatch.setattr(ge, "_device_key", lambda: ["gfx950", 256, "7.0", "src"])
    monkeypatch.setattr(ge, "_measure", lambda h, i, t: [0.0, 1e-6, 0.0, 0.0, 0.0])
    monkeypatch.setattr(ge, "_runs_ok", lambda *a: True)
    assert ge.calibrate(1024, 256, "Q4_K/Q4_K/Q4_K") == [0.0, 1e-6, 0.0, 0.0, 0.0]
    assert "not cached" in capsys.readouterr().out


def test_entry_refuses_unknown_types():
    with pytest.raises(ValueError):
        ge._types("Q4_0/Q4_0/IQ2_XS")
    with pytest.raises(ValueError):
        ge._types(("Q4_0", "Q4_0"))
