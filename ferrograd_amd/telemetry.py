"""Device memory telemetry: the mirror of the gpu_telemetry monitor the
reference's example harness uses (crates/ferrograd/examples/
matmul_chain3.rs:145-171) over the C ABI.

    monitor = GpuMonitor.start(ctx, interval_s=0.01)
    ...                                   # work on the device
    telemetry = monitor.stop()
    for sample in telemetry.samples:
        for heap in sample.heaps:         # one heap: the device's memory
            heap.usage, heap.budget       # bytes
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import List, Optional

from ._lib import call


@dataclass
class Heap:
    usage: Optional[int]
    budget: Optional[int]


@dataclass
class Sample:
    time_s: float
    heaps: List[Heap] = field(default_factory=list)


@dataclass
class Telemetry:
    samples: List[Sample]

    def average_usage(self) -> int:
        u = [h.usage for s in self.samples for h in s.heaps if h.usage is not None]
        return sum(u) // len(u) if u else 0

    def max_budget(self) -> int:
        b = [h.budget for s in self.samples for h in s.heaps if h.budget is not None]
        return max(b) if b else 0


class GpuMonitor:
    """GpuMonitor::start(interval) / stop() (gpu_telemetry 0.2)."""

    def __init__(self, handle):
        self.handle = handle

    @staticmethod
    def start(ctx, interval_s: float = 0.01) -> "GpuMonitor":
        h = ctypes.c_void_p()
        call("fg_monitor_start", getattr(ctx, "ctx", ctx).handle,
             max(100, int(round(interval_s * 1e6))), ctypes.byref(h))
        return GpuMonitor(h)

    def stop(self) -> Telemetry:
        n = ctypes.c_int()
        try:
            call("fg_monitor_stop", self.handle, ctypes.byref(n))
            out = []
            t, u, b = ctypes.c_double(), ctypes.c_uint64(), ctypes.c_uint64()
            for i in range(n.value):
                call("fg_monitor_sample", self.handle, i, ctypes.byref(t), ctypes.byref(u),
                     ctypes.byref(b))
                out.append(Sample(t.value, [Heap(u.value, b.value)]))
            return Telemetry(out)
        finally:
            call("fg_monitor_destroy", self.handle)
            self.handle = None
