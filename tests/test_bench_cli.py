"""bench.py's contract on the CPU: one GPU only (--gpus above 1 exits with a
message before touching a device), and the roofline traffic of every bench
config comes from a committed rocprofv3 summary under profiles/."""
from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)
import bench  # noqa: E402


@pytest.mark.parametrize("argv,env", [(["--gpus", "2"], {}), ([], {"WORLD_SIZE": "4"})])
def test_more_than_one_gpu_exits_with_a_message(argv, env):
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), *argv], capture_output=True, text=True,
                       timeout=120, env={**os.environ, **env})
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


@pytest.mark.parametrize("cfg", [2, 3, 4, 5, 6, 7, 8, 9, 10, 11])
def test_traffic_comes_from_a_committed_profile(cfg):
    t = bench.measured_traffic(cfg)
    assert isinstance(t, int) and t > 0
