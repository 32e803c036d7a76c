"""Timed regions for the MoE drop-in, under the reference's profiler interface.

Interface kept (``npu/profiler.py:21-78``, used by ``qwen/test_npu_generate5.py:224-392``
and ``bench_chatbot.py:216-241``): ``PROF.enabled``, ``PROF.enable()``,
``PROF.disable()``, ``PROF.reset()``, ``PROF.report(total_label=...)`` and
``with profile(name): ...``.

Each region records its host wall time and, when a GPU is present and the current
stream is not being captured, a pair of timing events on the current stream around
the work enqueued inside it.  No region synchronises: the events are resolved in
``summary()`` / ``report()``, which wait for the last of them.  The device column
therefore measures the GPU work of a region (launches are asynchronous, so the host
column mostly measures the enqueue), and nesting is allowed.  Disabled, ``profile``
returns one shared no-op context and records nothing.
"""
from __future__ import annotations

import contextlib
import time
from dataclasses import dataclass, field

import torch

_OFF = contextlib.nullcontext()


@dataclass
class RegionStats:
    calls: int = 0
    host_ns: int = 0
    device_ms: float = 0.0
    device_calls: int = 0
    events: list = field(default_factory=list)      # (start, end) event pairs not yet resolved

    def resolve(self) -> None:
        for a, b in self.events:
            b.synchronize()
            self.device_ms += a.elapsed_time(b)
            self.device_calls += 1
        self.events.clear()


class Profiler:
    """Named regions with host and device times (see the module docstring)."""

    def __init__(self) -> None:
        self.enabled = False
        self._regions: dict[str, RegionStats] = {}

    def enable(self) -> None:
        self.enabled = True

    def disable(self) -> None:
        self.enabled = False

    def reset(self) -> None:
        self._regions = {}

    def region(self, name: str):
        return self._span(name) if self.enabled else _OFF

    @contextlib.contextmanager
    def _span(self, name: str):
        st = self._regions.setdefault(name, RegionStats())
        ev = None
        if torch.cuda.is_available() and not torch.cuda.is_current_stream_capturing():
            ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            ev[0].record()
        t0 = time.perf_counter_ns()
        try:
            yield st
        finally:
            st.host_ns += time.perf_counter_ns() - t0
            st.calls += 1
            if ev is not None:
                ev[1].record()
                st.events.append(ev)

    def summary(self) -> dict[str, dict[str, float]]:
        """{name: {calls, host_ms, device_ms (None without events)}}, after resolving events."""
        out = {}
        for name, st in self._regions.items():
            st.resolve()
            out[name] = {"calls": st.calls, "host_ms": st.host_ns / 1e6,
                         "device_ms": st.device_ms if st.device_calls else None}
        return out

    def report(self, total_label: str = "total") -> None:
        """Print one line per region, longest first.  The share column is relative to the
        region named ``total_label`` when there is one, else to the sum of all regions."""
        rows = self.summary()
        if not rows:
            print("profile: no regions recorded")
            return

        def t(r):
            return r["device_ms"] if r["device_ms"] is not None else r["host_ms"]
        base = t(rows[total_label]) if total_label in rows else sum(t(r) for r in rows.values())
        w = max(24, max(len(n) for n in rows) + 2)
        print(f"{'region':<{w}}{'calls':>7}{'host ms':>11}{'device ms':>11}{'ms/call':>10}{'share':>8}")
        for name, r in sorted(rows.items(), key=lambda kv: -t(kv[1])):
            dev = f"{r['device_ms']:>11.3f}" if r["device_ms"] is not None else f"{'-':>11}"
            share = 100.0 * t(r) / base if base else 0.0
            print(f"{name:<{w}}{r['calls']:>7d}{r['host_ms']:>11.3f}{dev}{t(r) / r['calls']:>10.4f}{share:>7.1f}%")


PROF = Profiler()


def profile(name: str):
    """``with profile("moe.block"): ...`` times the region when ``PROF`` is enabled."""
    return PROF.region(name)
