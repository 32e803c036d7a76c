"""Per-op wall-clock profiler with the reference's API (``npu/profiler.py:21-78``).

``PROF.enable()``, ``with profile("moe.shared"): ...``, ``PROF.report()``,
``PROF.reset()``.  Disabled, ``profile(name)`` returns a shared no-op context
manager.  Because GPU work is asynchronous, host wall-clock around a launch
measures the enqueue only; ``PROF.sync = True`` makes each timed region
synchronise the current device stream on exit so the time covers the GPU work
(use ``rocprofv3 --kernel-trace`` for per-kernel times).
"""
from __future__ import annotations

import time
from collections import defaultdict


class _Profiler:
    __slots__ = ("enabled", "sync", "_ns", "_cnt")

    def __init__(self) -> None:
        self.enabled = False
        self.sync = False
        self._ns: dict[str, int] = defaultdict(int)
        self._cnt: dict[str, int] = defaultdict(int)

    def enable(self) -> None:
        self.enabled = True

    def disable(self) -> None:
        self.enabled = False

    def reset(self) -> None:
        self._ns.clear()
        self._cnt.clear()

    def add(self, name: str, ns: int) -> None:
        self._ns[name] += ns
        self._cnt[name] += 1

    def totals(self) -> dict[str, tuple[int, int]]:
        return {k: (self._ns[k], self._cnt[k]) for k in self._ns}

    def report(self, total_label: str = "total") -> None:
        if not self._ns:
            print("[profiler] no samples recorded")
            return
        total = self._ns.get(total_label, sum(self._ns.values()))
        print(f"{'op':<28} {'total_ms':>10} {'calls':>7} {'ms/call':>10} {'%':>6}")
        for name, ns in sorted(self._ns.items(), key=lambda kv: -kv[1]):
            c = self._cnt[name]
            pct = 100.0 * ns / total if total else 0.0
            print(f"{name:<28} {ns / 1e6:>10.3f} {c:>7d} {ns / 1e6 / c:>10.4f} {pct:>5.1f}%")


PROF = _Profiler()


class _Timer:
    __slots__ = ("name", "t0")

    def __init__(self, name: str) -> None:
        self.name = name

    def __enter__(self):
        self.t0 = time.perf_counter_ns()
        return self

    def __exit__(self, *exc):
        if PROF.sync:
            import torch
            if torch.cuda.is_available():
                torch.cuda.current_stream().synchronize()
        PROF.add(self.name, time.perf_counter_ns() - self.t0)
        return False


class _Noop:
    __slots__ = ()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


_NOOP = _Noop()


def profile(name: str):
    return _Timer(name) if PROF.enabled else _NOOP
