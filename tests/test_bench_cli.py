"""bench.py and __graft_entry__.py compile, and the bench refuses more than
one GPU with a message (no GPU touched), as the driver's contract asks."""
import os
import py_compile
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_entry_points_compile():
    for f in ("bench.py", "__graft_entry__.py"):
        py_compile.compile(os.path.join(ROOT, f), doraise=True)


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2, r.stderr
    assert "one GPU only" in r.stderr
