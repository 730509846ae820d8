"""bench.py's command-line contract that needs no GPU."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    # this build measures one GPU: --gpus N > 1 exits with status 2 and says so
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], cwd=ROOT,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2, r.stderr
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_guarded_section_records_its_error():
    # a secondary section that raises leaves an error entry, not a missing line
    sys.path.insert(0, ROOT)
    import bench

    assert bench.guarded(lambda: {"us": 1.0}) == {"us": 1.0}
    r = bench.guarded(lambda: 1 / 0)
    assert r == {"error": "ZeroDivisionError: division by zero"}
