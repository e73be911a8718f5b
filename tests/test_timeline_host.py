"""larder_amd.timeline's host side on synthetic stamps (no GPU): per-layer phase times from the layer's first router
workgroup start, unreached phases dropped, and a launch order that is not router / gate/up / down refused."""
import numpy as np
import pytest

from larder_amd import timeline


def test_layer_phases_and_summary():
    khz = 100_000  # 100 ticks a microsecond
    st = np.zeros((14, 8), dtype=np.int64)
    launches = []
    row = 0
    for l in range(2):
        base = 10_000 + 5_000 * l
        for name, n in (("router", 3), ("gate_up", 2), ("down", 2)):
            launches.append((name, row, n))
            for w in range(n):
                off = {"router": 0, "gate_up": 400, "down": 900}[name] + 10 * w
                st[row + w, 0] = base + off
                st[row + w, 4] = base + off + 300
                if name != "router":
                    st[row + w, 1] = base + off + 100
                    st[row + w, 3] = base + off + 200
                if name == "gate_up":
                    st[row + w, 2] = base + off + 150
            row += n
    res = timeline.layer_phases(st, launches, khz)
    assert len(res["router"]["start"]) == 2
    np.testing.assert_allclose(res["router"]["start"][1], [0.0, 0.1, 0.2])
    np.testing.assert_allclose(res["gate_up"]["top-k done"][0], [5.5, 5.6])
    assert res["router"]["inputs in"][0].size == 0  # not stamped by the router
    s = timeline.summary(res)
    assert s["down"]["end"] == {"first": 12.0, "median": 12.05, "last": 12.1}
    assert "inputs in" not in s["router"]
    with pytest.raises(ValueError):
        timeline.layer_phases(st, launches[1:] + launches[:1], khz)
