"""bench.py's contract on the CPU: one GPU only, and the committed traffic
record it reports is readable and close to the algorithmic bytes."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def test_traffic_record_is_read():
    sys.path.insert(0, ROOT)
    import bench
    t = bench.vocab_traffic()
    assert isinstance(t, int)
    assert 1.0 <= t / bench.VOCAB_BYTES < 1.1
