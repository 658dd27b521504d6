"""CPU: the caller-side shape predicate (include/bonsai_p40_dispatch.h),
compiled with gcc and run on the reference's dispatch cases."""
import os
import subprocess
import tempfile

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_dispatch_predicate_cases():
    src = os.path.join(ROOT, "tests", "host", "test_dispatch.c")
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "t")
        subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", src, "-o", exe], check=True)
        r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout
    assert "0 failed" in r.stdout
