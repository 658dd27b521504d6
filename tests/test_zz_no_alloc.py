"""The allocation-free FFN gate/up launch (bonsai_p40_ffn_gate_up_swiglu_noalloc,
the library's static per-GPU scratch in place of a workspace) against the
workspace form: the same Q8_1 bytes, on two calls in a row, the second with a
smaller n_ff (the scratch keeps the first call's contents)."""
import os
import subprocess
import sys

import numpy as np
import pytest

import bonsai_p40 as B
from oracle import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def run_pair(n_ff, n_embd, rms, seed):
    Wg = dev(O.gen_weights(seed, n_ff, n_embd))
    Wu = dev(O.gen_weights(seed + 1, n_ff, n_embd))
    x = dev(O.gen_normal(seed + 2, n_embd) * 2)
    nw = dev(O.gen_normal(seed + 3, n_embd) * 0.1 + 1) if rms else None
    hs = dev(np.where(O.gen_normal(seed + 4, n_ff) > 0, 1.0, -1.0).astype(np.float32))
    ws = torch.zeros(B.ffn_workspace_bytes(n_ff), dtype=torch.uint8, device="cuda")
    ref = torch.zeros(B.q8_bytes(n_ff), dtype=torch.uint8, device="cuda")
    B.ffn_gate_up_swiglu(Wg, Wu, x, nw, None, hs, ref, n_ff, n_embd, 1e-6, ws)
    got = torch.full((B.q8_bytes(n_ff),), 0xAB, dtype=torch.uint8, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    B.ffn_gate_up_swiglu_noalloc(Wg, Wu, x, nw, None, hs, got, n_ff, n_embd, 1e-6, status)
    np.testing.assert_array_equal(host(got), host(ref))
    assert int(host(status)[0]) == 0


def test_noalloc_matches_workspace_form_two_calls():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    B.lib()
    print("[case] noalloc ffn 17408x5120 (RMSNorm), then 4096x6144", flush=True)
    run_pair(17408, 5120, True, 8100)
    run_pair(4096, 6144, False, 8200)


def test_noalloc_rejects_sizes_beyond_its_scratch():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    f = B.lib().bonsai_p40_ffn_gate_up_swiglu_noalloc
    import ctypes as C
    assert f(16, 16, 16, None, None, None, 16, B.FFN_NOALLOC_MAX_NFF + 1024, 5120, C.c_float(1e-6), None, None) == 1


# The child's first call into the noalloc entry point is inside a graph
# capture (the scratch address is looked up there), then the graph is
# replayed with eager work between replays, and every replay must equal the
# workspace form.
_CHILD = r"""
import os, sys
sys.path[:0] = [os.environ["P40_ROOT"], os.path.join(os.environ["P40_ROOT"], "p40-kernel_amd")]
import numpy as np, torch
import bonsai_p40 as B
from oracle import oracle as O
n_ff, n_embd = 4096, 5120
dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
Wg, Wu = dev(O.gen_weights(8300, n_ff, n_embd)), dev(O.gen_weights(8301, n_ff, n_embd))
x = dev(O.gen_normal(8302, n_embd))
got = torch.full((B.q8_bytes(n_ff),), 0xAB, dtype=torch.uint8, device="cuda")
status = torch.zeros(1, dtype=torch.int32, device="cuda")
torch.cuda.synchronize()
s = torch.cuda.Stream()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):
    B.ffn_gate_up_swiglu_noalloc(Wg, Wu, x, None, None, None, got, n_ff, n_embd, 1e-6, status)
ws = torch.zeros(B.ffn_workspace_bytes(n_ff), dtype=torch.uint8, device="cuda")
ref = torch.zeros(B.q8_bytes(n_ff), dtype=torch.uint8, device="cuda")
B.ffn_gate_up_swiglu(Wg, Wu, x, None, None, None, ref, n_ff, n_embd, 1e-6, ws)
torch.cuda.synchronize()
for rep in range(3):
    got.fill_(0xAB)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(got, ref), f"replay {rep} differs from the workspace form"
    B.ffn_gate_up_swiglu(Wg, Wu, x * 2, None, None, None, ref, n_ff, n_embd, 1e-6, ws)
    B.ffn_gate_up_swiglu(Wg, Wu, x, None, None, None, ref, n_ff, n_embd, 1e-6, ws)
    torch.cuda.synchronize()
assert int(status.item()) == 0
print("child ok", flush=True)
"""


def test_noalloc_first_call_inside_graph_capture():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    print("[case] noalloc ffn 4096x5120: first call inside a graph capture (child process)", flush=True)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, P40_ROOT=root)
    r = subprocess.run([sys.executable, "-c", _CHILD], env=env, capture_output=True, text=True, timeout=180)
    assert r.returncode == 0 and "child ok" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
