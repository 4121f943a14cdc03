"""Per-launch device timing of the C-ABI entry points.

While a ``KernelTimer`` is active, every wrapper in ``sparseforge_amd``
brackets its C-ABI call with a pair of HIP events recorded on the stream the
call launches on (torch's current stream of the tensors' device) and tags it
with the algorithmic work of that launch (FLOPs or bytes).  ``summary()``
synchronises once and reports, per entry point, the launch count, total and
average device time and the achieved rate.  This is the equivalent of the
reference's ``torch.profiler.record_function`` regions
(legacy/main_llama.py:2019, :2139, :2168), narrowed to the hot-path kernels.

When no timer is active the hooks cost one attribute read per call.
"""
from __future__ import annotations

import contextlib
from dataclasses import dataclass, field

import torch

_active: "KernelTimer | None" = None


@dataclass
class _Rec:
    name: str
    work: float
    unit: str
    ev0: torch.cuda.Event
    ev1: torch.cuda.Event


@dataclass
class KernelStats:
    name: str
    unit: str
    launches: int = 0
    total_ms: float = 0.0
    total_work: float = 0.0

    @property
    def avg_ms(self) -> float:
        return self.total_ms / max(self.launches, 1)

    @property
    def rate(self) -> float:
        """Work per second (FLOP/s or B/s) over the device time of the launches."""
        return self.total_work / (self.total_ms * 1e-3) if self.total_ms > 0 else 0.0


@dataclass
class KernelTimer:
    records: list = field(default_factory=list)

    def begin(self, name: str, work: float, unit: str, device: torch.device) -> _Rec:
        s = torch.cuda.current_stream(device)
        r = _Rec(name, float(work), unit, torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        r.ev0.record(s)
        self.records.append(r)
        return r

    @staticmethod
    def end(rec: _Rec, device: torch.device) -> None:
        rec.ev1.record(torch.cuda.current_stream(device))

    def summary(self) -> dict:
        torch.cuda.synchronize()
        out: dict[str, KernelStats] = {}
        for r in self.records:
            st = out.setdefault(r.name, KernelStats(r.name, r.unit))
            st.launches += 1
            st.total_ms += r.ev0.elapsed_time(r.ev1)
            st.total_work += r.work
        return out


@contextlib.contextmanager
def kernel_timer():
    """Activate a KernelTimer for the enclosed region (not re-entrant)."""
    global _active
    if _active is not None:
        raise RuntimeError("a KernelTimer is already active")
    t = KernelTimer()
    _active = t
    try:
        yield t
    finally:
        _active = None


@contextlib.contextmanager
def region(name: str, work: float, unit: str, device: torch.device):
    """Bracket one C-ABI launch; a no-op unless a KernelTimer is active."""
    t = _active
    if t is None:
        yield
        return
    rec = t.begin(name, work, unit, device)
    try:
        yield
    finally:
        t.end(rec, device)
