"""npu_amd.profiler keeps the reference's interface (npu/profiler.py:21-78): enable /
disable / reset / report(total_label) on PROF and ``with profile(name)``."""
import time

import pytest

from npu_amd import profiler as P


def test_disabled_records_nothing(capsys):
    P.PROF.reset()
    P.PROF.disable()
    with P.profile("moe.block"):
        pass
    assert P.PROF.summary() == {}
    P.PROF.report()
    assert "no regions" in capsys.readouterr().out


def test_regions_nest_and_report(capsys):
    P.PROF.reset()
    P.PROF.enable()
    try:
        for _ in range(3):
            with P.profile("total"):
                with P.profile("moe.block"):
                    time.sleep(0.002)
                with P.profile("moe.shared"):
                    pass
    finally:
        P.PROF.disable()
    s = P.PROF.summary()
    assert set(s) == {"total", "moe.block", "moe.shared"}
    assert all(r["calls"] == 3 for r in s.values())
    assert s["total"]["host_ms"] >= s["moe.block"]["host_ms"] >= 6.0
    P.PROF.report(total_label="total")
    lines = capsys.readouterr().out.splitlines()
    assert lines[1].startswith("total") and lines[1].rstrip().endswith("100.0%")
    assert [ln.split()[0] for ln in lines[1:]] == ["total", "moe.block", "moe.shared"]
    P.PROF.reset()
    assert P.PROF.summary() == {}


@pytest.mark.gpu
def test_device_time_recorded(gpu):
    """On a GPU every region also holds the device time of the work it enqueued."""
    import torch
    x = torch.randn(2048, 2048, device=gpu)
    P.PROF.reset()
    P.PROF.enable()
    try:
        for _ in range(2):
            with P.profile("mm"):
                y = x @ x
    finally:
        P.PROF.disable()
    s = P.PROF.summary()
    assert s["mm"]["calls"] == 2 and s["mm"]["device_ms"] is not None and s["mm"]["device_ms"] > 0
    assert torch.isfinite(y).all()
    P.PROF.reset()
