"""The bench's timing events: HIP events created without the system-scope fence time a launch
like default (torch) events do."""
import pytest
import torch

from peco_amd import _native

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_fenceless_events_time_like_torch_events(announce):
    announce("fenceless and torch events around the same matrix products")
    a = torch.randn(4096, 4096, device=DEV)
    b = torch.randn(4096, 4096, device=DEV)
    torch.cuda.synchronize()
    ref0, ref1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    timer = _native.LaunchTimer()
    stream = torch.cuda.current_stream().cuda_stream
    ref0.record()
    timer.start(stream)
    for _ in range(20):
        a = a @ b * 1e-2
    timer.stop(stream)
    ref1.record()
    torch.cuda.synchronize()
    (ms,) = timer.elapsed_ms()
    ref = ref0.elapsed_time(ref1)
    assert 0.0 < ms <= ref * 1.05 and ms >= 0.8 * ref, (ms, ref)
    assert len(timer) == 0  # the pairs are released once read
    start, end = _native.FencelessEvent(), _native.FencelessEvent()
    start.record()
    a = a @ b
    end.record()
    torch.cuda.synchronize()
    assert start.elapsed_time(end) > 0.0
