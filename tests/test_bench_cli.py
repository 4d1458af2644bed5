"""bench.py's command-line contract that needs no GPU: one GPU only, a JSON error line
and a nonzero exit for --gpus above 1 (no figure at several GPUs is produced)."""
import json
import os
import subprocess
import sys

from conftest import ROOT


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    line = r.stdout.strip().splitlines()[-1]
    assert "one GPU" in json.loads(line)["error"]
