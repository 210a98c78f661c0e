"""bench.py's contract on the CPU: one GPU only (any --gpus above 1 exits with
status 2 and says why), the headline's algorithmic bytes, and the HBM traffic
figure it reports read from the committed rocprofv3 summary."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_headline_bytes_and_traffic():
    import bench
    # 8 KV heads x 32768 tokens x (K + V) x (48 code bytes + 4 f16 scales)
    assert bench.c3_bytes() == 8 * 32768 * 2 * (48 + 8) == 29_360_128
    with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
        rec = json.load(f)["kernels"]["stream_decode_kernel_c3"]
    t = bench.traffic("stream_decode_kernel_c3")
    assert t == rec["hbm_bytes_per_launch"]
    # every byte of the algorithmic figure is read once; the excess (query,
    # partials, merge) stays a few per cent
    assert 1.0 <= t / bench.c3_bytes() < 1.1
    assert bench.traffic("no_such_kernel") is None
