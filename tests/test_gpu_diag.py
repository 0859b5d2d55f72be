"""GPU checks of the measurement aids (no counterpart in the reference):
lisaq_timestamp (the device clock, stream-ordered) and lisaq_read_stream
(a read-only stream that writes nothing for a buffer of ones)."""
import pytest

from lisa_amd import _lib

pytestmark = pytest.mark.gpu


def test_timestamps_bracket_a_read_stream(dev):
    """Two stamps around a 64 MB read: increasing, and the interval at least
    what HBM can deliver (64 MB at 8 TB/s = 8 us = 800 ticks of 100 MHz) and
    well under a second; the sink of a buffer of ones stays untouched."""
    import torch

    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    stamps = torch.zeros(2, dtype=torch.int64, device=dev)
    buf = torch.ones(64 << 20, dtype=torch.uint8, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    _lib.check(lib.lisaq_timestamp(st, stamps.data_ptr()))
    _lib.check(lib.lisaq_read_stream(st, buf.data_ptr(), buf.numel(), 4, sink.data_ptr()))
    _lib.check(lib.lisaq_timestamp(st, stamps.data_ptr() + 8))
    torch.cuda.synchronize()
    t0, t1 = stamps.cpu().tolist()
    assert 800 <= t1 - t0 < 100_000_000, (t0, t1)
    assert not sink.any()


def test_timestamp_rejects_unaligned(dev):
    import torch

    lib = _lib.load()
    stamps = torch.zeros(2, dtype=torch.int64, device=dev)
    rc = lib.lisaq_timestamp(torch.cuda.current_stream().cuda_stream, stamps.data_ptr() + 4)
    assert rc == _lib.EINVAL_LAYOUT
