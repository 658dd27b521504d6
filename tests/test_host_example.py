"""The C++ host program of tests/host/example_decode.cpp: it includes
include/bonsai_p40.h and links libbonsai_p40.so as a reference host does
(docs/INTEGRATION.md:257-263 of the reference).  Built in-tree by
`make -C p40-kernel_amd` (the build step), run here."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "host", "example_decode")


def _exe():
    if not os.path.exists(EXE):
        subprocess.run(["make", "-C", os.path.join(ROOT, "p40-kernel_amd"), "example"], check=True)
    return EXE


def test_host_program_argument_checks():
    """Links and runs without a device: invalid arguments return 1, empty
    work 0, out-of-scope entry points 2."""
    r = subprocess.run([_exe(), "--args-only"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "args-only: 0 failed" in r.stdout


@pytest.mark.gpu
def test_host_program_on_device():
    """One layer input through RMSNorm + FWHT + Q8_1 then a GEMV, and through
    the fused single-launch entry point: bit-identical, from plain C++."""
    assert os.path.exists(EXE), "build tests/host/example_decode first (make -C p40-kernel_amd)"
    print("[case] C++ host program on the device", flush=True)
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "device: 0 failed" in r.stdout
