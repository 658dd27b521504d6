"""CPU checks of bench.py's command-line contract that need no GPU: a run for
more than one GPU stops with a message before touching a device (this build
measures one GPU), and the kernel-source hash that gates the committed HBM
traffic record is stable and covers every file the decode GEMV is built from."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], cwd=ROOT,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)
    assert not r.stdout.strip().startswith("{")          # no JSON line for a run that did not happen


def test_traffic_record_is_tied_to_the_kernel_sources():
    sys.path.insert(0, ROOT)
    import bench
    h = bench.kernel_source_hash()
    assert h == bench.kernel_source_hash() and len(h) == 16
    with open(os.path.join(ROOT, "profiles", "gemv_17408x5120_traffic.json")) as f:
        rec = json.load(f)
    for k in ("source_sha256", "bytes_per_launch", "read_bytes", "write_bytes", "algorithmic_bytes"):
        assert k in rec, k
    assert rec["bytes_per_launch"] == rec["read_bytes"] + rec["write_bytes"]
    assert rec["algorithmic_bytes"] == 23750272
    # the committed record was measured on the committed sources
    t, why = bench.load_traffic(os.path.join(ROOT, "profiles", "gemv_17408x5120_traffic.json"))
    assert t is not None, why
