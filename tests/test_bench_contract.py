"""bench.py's offline pieces: its kernel names match the committed traffic summary (the roofline's `traffic` comes
from there), and --gpus above 1 is refused without touching a GPU."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_dominant_kernel_is_in_the_traffic_summary():
    import bench

    tk = json.load(open(bench.TRAFFIC_FILE))["kernels"]
    hit = [v for k, v in tk.items() if bench.KERNELS["dot"][0] in k]
    assert len(hit) == 1 and hit[0]["traffic_bytes"] > 0


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode != 0 and "one GPU" in (r.stdout + r.stderr)
