"""bench.py's command-line contract without a GPU: every workload name parses, and a run on more
than one GPU is refused with exit status 2 before anything touches a device."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_workload_names_parse():
    sys.path.insert(0, ROOT)
    import bench
    for wl in ("cfg1", "cfg2", "cfg3", "cfg5", "op", "noncausal", "linear"):
        old = sys.argv
        sys.argv = ["bench.py", "--workload", wl]
        try:
            assert bench.parse().workload == wl
        finally:
            sys.argv = old


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "measures one GPU" in r.stderr
