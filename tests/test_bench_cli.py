"""The bench.py driver contract on the CPU: more than one GPU is refused with one JSON line, and
the documented flags parse (no GPU is touched by either)."""

import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_exits_with_a_message():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                          text=True, timeout=120, cwd=ROOT)
    assert proc.returncode == 2
    line = json.loads(proc.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"] and line["n_gpus_requested"] == 2


def test_documented_flags_parse():
    sys.path.insert(0, str(ROOT))
    try:
        import bench
    finally:
        sys.path.remove(str(ROOT))
    argv = sys.argv
    try:
        sys.argv = ["bench.py", "--steps", "3", "--warmup", "1", "--serial", "--no-cpu-baseline",
                    "--no-kernel-timing", "--no-layer-step", "--no-attention-configs", "--no-gemm-tuning"]
        args = bench.parse()
    finally:
        sys.argv = argv
    assert (args.steps, args.warmup, args.gpus) == (3, 1, 1)
    assert args.serial and args.no_attention_configs and args.no_layer_step
