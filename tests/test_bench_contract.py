"""bench.py's contract on the CPU: more than one GPU is refused with a message (this build measures
one GPU), the configs named by BASELINE.json exist, and every committed traffic summary the bench
line cites parses and names an existing rocprofv3 summary."""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300, cwd=ROOT)
    assert r.returncode != 0
    assert "gpus 1" in r.stderr
    assert r.stdout.strip() == ""  # no bench line


def test_configs_and_traffic_files():
    sys.path.insert(0, str(ROOT))
    import bench

    for name in ("tiny", "mixtral", "deepseek", "qwen3_fp8", "qwen3_bwd"):
        assert name in bench.CONFIGS
    files = sorted((ROOT / "profiles").glob("traffic_*.json"))
    assert files
    for f in files:
        d = json.loads(f.read_text())
        assert isinstance(d["bytes_per_launch"], int) and d["bytes_per_launch"] > 0
        assert (ROOT / "profiles" / d["source"]).exists(), d["source"]
        nbytes, kernel = bench._traffic(f.stem[len("traffic_"):])
        assert nbytes == d["bytes_per_launch"] and kernel == d["kernel"]
    assert bench._traffic("no_such_config") == (None, None)
