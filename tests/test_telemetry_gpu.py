"""Device memory telemetry (fg_monitor_*): samples arrive at the requested
interval and see an allocation made while the monitor runs."""
import time

import pytest

pytestmark = pytest.mark.gpu


def test_monitor_sees_an_allocation(gpu_ctx):
    import torch

    from ferrograd_amd.telemetry import GpuMonitor

    torch.cuda.synchronize()
    mon = GpuMonitor.start(gpu_ctx, 0.002)
    time.sleep(0.05)
    x = torch.empty(2 * 1024 ** 3, dtype=torch.uint8, device="cuda")  # 2 GiB
    x.fill_(1)
    torch.cuda.synchronize()
    time.sleep(0.05)
    tel = mon.stop()
    del x
    n = len(tel.samples)
    assert n >= 10
    times = [s.time_s for s in tel.samples]
    assert times == sorted(times)
    used = [s.heaps[0].usage for s in tel.samples]
    budget = tel.max_budget()
    assert budget > 64 * 1024 ** 3  # an MI355X has 288 GB
    assert all(0 < u <= budget for u in used)
    assert max(used) - min(used) >= int(1.9 * 1024 ** 3)
    assert 0 < tel.average_usage() <= budget
