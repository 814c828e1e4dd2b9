"""bench.py's command line without a GPU: the multi-GPU request is refused
before anything touches a device, and the configurations it measures are
BASELINE.json's."""

import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_configs_match_baseline():
    sys.path.insert(0, ROOT)
    import bench
    with open(os.path.join(ROOT, "BASELINE.json")) as f:
        configs = json.load(f)["configs"]
    # configs[1..3]: bs1 512 -> 256; bs8 1024 -> 512; bs32 4096 -> 256
    assert bench.CONFIGS["c2"][:3] == (1, 512, 256) and "batch 1, 512 prompt tokens" in configs[1]
    assert bench.CONFIGS["c3"][:3] == (8, 1024, 512) and "Batch 8" in configs[2] and "512 greedy" in configs[2]
    assert bench.CONFIGS["c4"][:3] == (32, 4096, 256) and "Batch 32" in configs[3] and "4096 tokens" in configs[3]
