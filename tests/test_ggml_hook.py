"""The ggml-hip hook (include/bonsai_p40_ggml.h): the gfx950 counterparts of
the reference fork's bonsai_p40_should_use / bonsai_p40_mul_mat
(integrations/prismml/bonsai-p40.diff:245-302).

CPU: the opt-in switch, the type / column checks and the shape predicate
decide before any device work (the reference's dispatch cases,
tests/test_p40.cpp:653-698, through the tensor views).  GPU: the op the hook
takes equals the reference hook's two launches (quant_activations + gemv) bit
for bit on the model widths, is within the GEMV tolerance of the oracle on a
width without the one-launch kernel (scratch path), and declines without a
scratch there."""
import os
import subprocess

import numpy as np
import pytest

import bonsai_p40 as B
from oracle import oracle as O

F32, PQ2 = B.GGML_TYPE_F32, B.GGML_TYPE_PQ2_0
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GLUE = os.path.join(ROOT, "tests", "host", "ggml_glue")


def _glue():
    if not os.path.exists(GLUE):
        subprocess.run(["make", "-C", os.path.join(ROOT, "p40-kernel_amd"), "example"], check=True)
    return GLUE


def _env(enable: bool):
    env = {k: v for k, v in os.environ.items() if k != "BONSAI_P40"}
    if enable:
        env["BONSAI_P40"] = "1"
    return env


def test_fork_glue_compiles_and_declines_without_device():
    """tests/host/ggml_glue.cpp: the glue a fork adds (tensor views, the
    should_use gate, the mul_mat call), built with g++ against the header and
    the library; with the path switched off and on shapes the predicate
    rejects it declines without touching the device."""
    r = subprocess.run([_glue(), "--args-only"], capture_output=True, text=True, timeout=120, env=_env(False))
    assert r.returncode == 0, r.stdout + r.stderr
    assert "args-only: 0 failed" in r.stdout


def views(n_out, n_in, W=0, x=0, y=0, n_tok=1, w_nb1=None, w_ne2=1):
    """src0 (PQ2_0 [n_out][n_in]), src1 (F32 [n_tok][n_in]), dst (F32 [n_tok][n_out])."""
    nb1 = w_nb1 if w_nb1 is not None else n_in // 128 * 34
    src0 = B.ggml_tensor(PQ2, [n_in, n_out, w_ne2], [34, nb1], W)
    src1 = B.ggml_tensor(F32, [n_in, n_tok], [4, 4 * n_in], x)
    dst = B.ggml_tensor(F32, [n_out, n_tok], [4, 4 * n_out], y)
    return src0, src1, dst


def test_should_use_is_opt_in(knobs):
    knobs.unset("BONSAI_P40")
    assert not B.ggml_should_use(PQ2, 0, 1)
    knobs.set("BONSAI_P40", 0)
    assert not B.ggml_should_use(PQ2, 0, 1)


def test_should_use_type_and_columns(knobs):
    knobs.set("BONSAI_P40", 1)
    assert not B.ggml_should_use(F32, 0, 1)          # not PQ2_0
    assert not B.ggml_should_use(42, 0, 1)           # Q2_0
    assert not B.ggml_should_use(PQ2, 0, 8)          # a batch: stock path
    assert not B.ggml_should_use(PQ2, -1, 1)         # no such device
    assert not B.ggml_should_use(PQ2, 1 << 20, 1)


@pytest.mark.parametrize("case", ["3d_weights", "batch", "non_contiguous", "n_in_128", "too_wide", "f16_weights",
                                  "null"])
def test_mul_mat_declines_outside_the_predicate(case):
    """Shapes the reference predicate rejects are declined before any device
    work (null data pointers are never touched)."""
    if case == "3d_weights":
        v = views(17408, 5120, w_ne2=4)
    elif case == "batch":
        v = views(17408, 5120, n_tok=4)
    elif case == "non_contiguous":
        v = views(17408, 5120, w_nb1=4096)
    elif case == "n_in_128":
        v = views(64, 5121)
    elif case == "too_wide":
        v = views(64, 65536)
    elif case == "f16_weights":
        v = views(64, 5120)
        v[0].type = 1
    else:
        v = views(64, 5120)                          # valid shape, null data
    assert not B.ggml_mul_mat(*v, stream=0)


@pytest.mark.gpu
def test_should_use_on_gfx950(knobs):
    import torch
    knobs.set("BONSAI_P40", 1)
    assert B.ggml_should_use(PQ2, torch.cuda.current_device(), 1)


@pytest.mark.gpu
@pytest.mark.parametrize("n_out,n_in", [(17408, 5120), (5120, 17408), (1024, 5120), (300, 3072)])
def test_mul_mat_one_launch_equals_reference_hook_sequence(n_out, n_in):
    """Widths with n_in % 1024 == 0: one launch, no scratch; y bit-identical
    to quant_activations + gemv (the reference hook's launches) on the model
    widths, within the GEMV tolerance of the oracle everywhere."""
    import torch
    from test_gpu_parity import case, dev, host, normwise
    case(f"ggml hook one launch {n_out}x{n_in}")
    W = dev(O.gen_weights(3100 + n_in, n_out, n_in))
    x = O.gen_normal(3101 + n_out, n_in) * 2
    y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    assert B.ggml_mul_mat(*views(n_out, n_in, W, dev(x), y))
    xq = torch.zeros(n_in // 32 * 36, dtype=torch.uint8, device="cuda")
    B.quant_activations(dev(x), xq, n_in)
    y2 = torch.zeros(n_out, dtype=torch.float32, device="cuda")
    B.gemv(W, xq, y2, n_out, n_in)
    ref = O.gemv(host(W), O.quantize_q8_1(x, True), n_out, n_in)
    assert normwise(host(y), ref) <= 1e-5
    if n_in in (5120, 17408):
        np.testing.assert_array_equal(host(y).view(np.uint32), host(y2).view(np.uint32))


@pytest.mark.gpu
def test_mul_mat_scratch_path():
    """n_in = 5248 (41 blocks, not a multiple of 1024): the reference's two
    launches through the caller's scratch; declined without one."""
    import torch
    from test_gpu_parity import case, dev, host, normwise
    case("ggml hook scratch path 700x5248")
    n_out, n_in = 700, 5248
    W = dev(O.gen_weights(3200, n_out, n_in))
    x = O.gen_normal(3201, n_in)
    y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    assert not B.ggml_mul_mat(*views(n_out, n_in, W, dev(x), y))
    need = n_in // 32 * 36
    scratch = torch.zeros(need, dtype=torch.uint8, device="cuda")
    assert not B.ggml_mul_mat(*views(n_out, n_in, W, dev(x), y), scratch, need - 4)
    assert B.ggml_mul_mat(*views(n_out, n_in, W, dev(x), y), scratch, need)
    ref = O.gemv(host(W), O.quantize_q8_1(x, True), n_out, n_in)
    assert normwise(host(y), ref) <= 1e-5
    np.testing.assert_array_equal(host(scratch), O.quantize_q8_1(x, True))


@pytest.mark.gpu
def test_fork_glue_on_device():
    """The C++ glue takes a 17408x5120 op on the gfx950 with BONSAI_P40=1, and
    its output equals quant_activations + gemv bit for bit."""
    assert os.path.exists(GLUE), "build tests/host/ggml_glue first (make -C p40-kernel_amd)"
    print("[case] C++ ggml glue on the device", flush=True)
    r = subprocess.run([GLUE], capture_output=True, text=True, timeout=120, env=_env(True))
    assert r.returncode == 0, r.stdout + r.stderr
    assert "device: 0 failed" in r.stdout
