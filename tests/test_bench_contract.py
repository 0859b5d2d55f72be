"""bench.py pieces that run without a GPU: the algorithmic byte count of the
headline metric and the cpu_baseline record (on a small shape)."""
import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_headline_bytes_per_call():
    b = _bench()
    # packed W 44,564,480 + scales/biases 5,570,560 + x 10,240 + y 34,816
    assert b.qmv_bytes(1, 17408, 5120, 4, 64) == 50_180_096
    # 2-bit: W halves, scales/biases unchanged
    assert b.qmv_bytes(1, 17408, 5120, 2, 64) == 22_282_240 + 5_570_560 + 10_240 + 34_816


def test_cpu_baseline_record():
    pytest.importorskip("numpy")
    b = _bench()
    rec = b.cpu_baseline(1, 256, 1024, 4, 64, 0.2)
    for key in ("value", "unit", "cores", "kind", "sample", "us_per_call", "materialize"):
        assert key in rec, key
    assert rec["kind"] == "port" and rec["unit"] == "GB/s" and rec["cores"] >= 1
    assert rec["value"] > 0 and rec["materialize"]["value"] > 0 and rec["materialize"]["calls"] >= 2
