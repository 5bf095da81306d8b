"""bench.py's one-GPU contract, on the CPU: more than one GPU is refused with a message before anything touches a
device, and the traffic summary it quotes is keyed to the step's launch shapes."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_multi_gpu_is_refused():
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, cwd=ROOT, timeout=120)
    assert p.returncode == 2 and "one GPU" in p.stderr and not p.stdout.strip()


def test_traffic_summary_matches_the_step():
    sys.path.insert(0, ROOT)
    import bench
    names = ["gdn.qkv|gdn.z", "gdn.out", "attn.q|attn.k|attn.v", "attn.o", "mlp.gate+mlp.up", "mlp.down"]
    t = bench._traffic("tq_gemv_kernel", 4, 1, names)
    with open(os.path.join(ROOT, "profiles", "gemv_traffic_config1.json")) as f:
        summary = json.load(f)
    assert t == summary["hbm_bytes_per_launch"]
    assert bench._traffic("tq_gemv_kernel", 4, 1, names[:-1]) is None      # another launch list: no figure
    assert bench._traffic("tq_gemv_kernel", 5, 1, names) is None
