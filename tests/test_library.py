"""CPU tests of the native boundary: libbonsai_p40.so loads, exports every
symbol include/bonsai_p40.h declares, and the argument checks that run before
any device work return the reference's codes (1 = invalid, 0 = no-op)."""
import ctypes as C
import os
import re

import pytest

import bonsai_p40 as B

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols(headers=("bonsai_p40.h", "bonsai_p40_ggml.h")):
    text = "".join(open(os.path.join(ROOT, "include", h)).read() for h in headers)
    return sorted(set(re.findall(r"^(?:int|int64_t)\s+(bonsai_p40_\w+)\s*\(", text, re.M)))


def test_every_header_is_scanned():
    """The export check covers every header of include/ that declares entry points."""
    for h in os.listdir(os.path.join(ROOT, "include")):
        found = header_symbols((h,))
        assert not found or h in ("bonsai_p40.h", "bonsai_p40_ggml.h"), h


def test_library_exports_every_header_symbol():
    L = B.lib()
    syms = header_symbols()
    assert len(syms) >= 13
    for s in syms:
        assert hasattr(L, s), s
    assert set(syms) == set(B.SIGNATURES)


def test_reference_symbol_set_is_kept():
    ref = ["bonsai_p40_gemv", "bonsai_p40_quant_activations", "bonsai_p40_gemm",
           "bonsai_p40_repack", "bonsai_p40_gemv_repack", "bonsai_p40_fwht",
           "bonsai_p40_rmsnorm", "bonsai_p40_gdn_step", "bonsai_p40_attn"]
    assert set(ref) <= set(header_symbols(("bonsai_p40.h",)))


NULL = None


@pytest.mark.parametrize("name,args,rc", [
    ("bonsai_p40_gemv", (NULL, NULL, NULL, 16, 100), 1),        # n_in % 128
    ("bonsai_p40_gemv", (NULL, NULL, NULL, 16, 0), 1),          # n_in <= 0
    ("bonsai_p40_gemv", (NULL, NULL, NULL, 0, 128), 0),         # empty no-op
    ("bonsai_p40_gemv", (NULL, 2, NULL, 16, 128), 1),           # misaligned xq
    ("bonsai_p40_chunk_dots", (NULL, NULL, NULL, 16, 96), 1),
    ("bonsai_p40_quant_activations", (NULL, NULL, 33), 1),
    ("bonsai_p40_quant_activations", (NULL, NULL, 0), 1),
    ("bonsai_p40_gemm", (NULL, NULL, NULL, 16, 96, 4), 1),
    ("bonsai_p40_gemm", (NULL, NULL, NULL, 0, 128, 4), 0),
    ("bonsai_p40_gemm", (NULL, NULL, NULL, 16, 128, 0), 0),
    ("bonsai_p40_gemm_ws", (NULL, NULL, NULL, 16, 96, 4, NULL, 0), 1),      # as bonsai_p40_gemm
    ("bonsai_p40_gemm_ws", (NULL, NULL, NULL, 0, 128, 4, NULL, 0), 0),
    ("bonsai_p40_repack", (NULL, NULL, 4, 128 * 12), 1),        # nb % 8
    ("bonsai_p40_repack", (NULL, NULL, 0, 1024), 1),
    ("bonsai_p40_gemv_repack", (NULL, NULL, NULL, 4, 128 * 4), 1),
    ("bonsai_p40_fwht", (NULL, NULL, 1000), 1),
    ("bonsai_p40_fwht", (NULL, NULL, 0), 1),
    ("bonsai_p40_fwht_quant", (NULL, NULL, NULL, 512), 1),
    ("bonsai_p40_quant_tokens", (NULL, NULL, NULL, 1000, 2, 1), 1),
    ("bonsai_p40_quant_tokens", (NULL, NULL, NULL, 1024, 0, 1), 1),
    ("bonsai_p40_swiglu_fwht_quant", (NULL, NULL, NULL, NULL, 100), 1),
    ("bonsai_p40_fwht_gemv", (NULL, 16, NULL, NULL, 16, 1000), 1),    # n_in % 1024
    ("bonsai_p40_fwht_gemv", (NULL, NULL, NULL, NULL, 16, 1024), 1),  # x NULL
    ("bonsai_p40_fwht_gemv", (NULL, 16, NULL, NULL, 0, 1024), 0),     # empty no-op
    ("bonsai_p40_quant_gemv", (NULL, 16, NULL, 16, 1000), 1),          # n_in % 1024
    ("bonsai_p40_quant_gemv", (NULL, NULL, NULL, 16, 1024), 1),        # x NULL
    ("bonsai_p40_quant_gemv", (NULL, 16, NULL, 0, 1024), 0),           # empty no-op
    ("bonsai_p40_launch_probe", (0, 64, 16), 1),
    ("bonsai_p40_launch_probe", (1, 2048, 16), 1),
    ("bonsai_p40_launch_probe", (1, 64, NULL), 1),
    ("bonsai_p40_overlap_probe", (4, 1, 1, 1, 16), 1),                 # no mode 4
    ("bonsai_p40_unit_dma_probe", (16, 16, 4096, 16), 1),              # not a GEMV width it models
    ("bonsai_p40_unit_dma_probe", (16, 0, 5120, 16), 1),               # no rows
    ("bonsai_p40_unit_dma_probe", (18, 16, 5120, 16), 1),              # W alignment
    ("bonsai_p40_gemv_group", (NULL, NULL, NULL, 1, NULL, 128), 1),   # NULL arrays
    ("bonsai_p40_fwht_gemv_group", (NULL, NULL, NULL, 1, 16, NULL, 1024), 1),
    ("bonsai_p40_rmsnorm_fwht_quant", (16, 16, NULL, 16, 1000, 1, C.c_float(1e-6)), 1),   # n % 1024
    ("bonsai_p40_rmsnorm_fwht_quant", (16, NULL, NULL, 16, 1024, 1, C.c_float(1e-6)), 1),  # w NULL
    ("bonsai_p40_rmsnorm_fwht_quant", (16, 16, NULL, 18, 1024, 1, C.c_float(1e-6)), 1),    # xq align
    ("bonsai_p40_rmsnorm_fwht_quant", (16, 16, NULL, 16, 1024, 0, C.c_float(1e-6)), 0),    # no tokens
    ("bonsai_p40_rmsnorm", (NULL, NULL, NULL, 0, 64, C.c_float(1e-6)), 0),
    ("bonsai_p40_rmsnorm", (NULL, NULL, NULL, 4, 0, C.c_float(1e-6)), 1),
])
def test_argument_checks(name, args, rc):
    fn = getattr(B.lib(), name)
    assert fn(*args, None) == rc


def test_group_argument_checks():
    L = B.lib()
    W = (C.c_void_p * 5)(*([16] * 5))
    y = (C.c_void_p * 5)(*([16] * 5))
    n = (C.c_int64 * 5)(*([0] * 5))
    Wp, yp, np_ = (C.cast(a, C.c_void_p) for a in (W, y, n))
    assert L.bonsai_p40_gemv_group(Wp, yp, np_, 0, None, 128, None) == 1         # n_mat < 1
    assert L.bonsai_p40_gemv_group(Wp, yp, np_, 5, None, 128, None) == 1         # n_mat > 4
    assert L.bonsai_p40_gemv_group(Wp, yp, np_, 3, None, 128, None) == 0         # all empty
    assert L.bonsai_p40_gemv_group(Wp, yp, np_, 3, None, 100, None) == 1         # n_in % 128
    assert L.bonsai_p40_fwht_gemv_group(Wp, yp, np_, 2, 16, None, 1024, None) == 0
    assert L.bonsai_p40_fwht_gemv_group(Wp, yp, np_, 2, 16, None, 2000, None) == 1
    assert L.bonsai_p40_rmsnorm_fwht_gemv_group(Wp, yp, np_, 2, 16, 16, None, 1024, C.c_float(1e-6), None) == 0
    assert L.bonsai_p40_rmsnorm_fwht_gemv_group(Wp, yp, np_, 2, 16, None, None, 1024, C.c_float(1e-6), None) == 1
    assert L.bonsai_p40_rmsnorm_fwht_gemv_group(Wp, yp, np_, 2, 16, 16, None, 1000, C.c_float(1e-6), None) == 1
    n[1] = 1 << 30
    assert L.bonsai_p40_gemv_group(Wp, yp, np_, 2, None, 128, None) == 1         # too many rows


def test_out_of_scope_entries_report_not_implemented():
    L = B.lib()
    assert L.bonsai_p40_gdn_step(*([None] * 7), 16, 48, 128, 128, None) == 2
    assert L.bonsai_p40_attn(*([None] * 4), 4, 24, 4, 256, C.c_float(0.0625), None) == 2


def _gpu_visible():
    if os.path.exists("/dev/kfd"):
        return True
    try:
        import torch
        return torch.cuda.device_count() > 0      # counts without initialising the device
    except Exception:
        return False


A = 4096          # a 16-byte aligned placeholder address (never dereferenced: the check returns first)
EPS = C.c_float(1e-6)

# (entry, valid arguments, positions of the pointers that the work needs)
NULL_CASES = [
    ("bonsai_p40_gemv", (A, A, A, 16, 128), (0, 1, 2)),
    ("bonsai_p40_chunk_dots", (A, A, A, 16, 128), (0, 1, 2)),
    ("bonsai_p40_quant_activations", (A, A, 64), (0, 1)),
    ("bonsai_p40_fwht_quant", (A, NULL, A, 1024), (0, 2)),
    ("bonsai_p40_quant_tokens", (A, NULL, A, 1024, 2, 1), (0, 2)),
    ("bonsai_p40_rmsnorm_fwht_quant", (A, A, NULL, A, 1024, 1, EPS), (0, 1, 3)),
    ("bonsai_p40_swiglu_fwht_quant", (A, A, NULL, A, 1024), (0, 1, 3)),
    ("bonsai_p40_gemm", (A, A, A, 16, 128, 4), (0, 1, 2)),
    ("bonsai_p40_gemm_ws", (A, A, A, 16, 128, 4, NULL, 0), (0, 1, 2)),
    ("bonsai_p40_repack", (A, A, 4, 1024), (0, 1)),
    ("bonsai_p40_gemv_repack", (A, A, A, 4, 1024), (0, 1, 2)),
    ("bonsai_p40_fwht", (A, NULL, 1024), (0,)),
    ("bonsai_p40_fwht_gemv", (A, A, NULL, A, 16, 1024), (0, 1, 3)),
    ("bonsai_p40_quant_gemv", (A, A, A, 16, 1024), (0, 1, 2)),
    ("bonsai_p40_rmsnorm", (A, A, A, 4, 64, EPS), (0, 1, 2)),
    ("bonsai_p40_quantize_pq2_0", (A, A, 128), (0, 1)),
    ("bonsai_p40_dequantize_pq2_0", (A, A, 128), (0, 1)),
    ("bonsai_p40_stream_read", (A, 1024, A, 1), (0, 2)),
    ("bonsai_p40_unit_dma_probe", (A, 1024, 5120, A), (0, 3)),
]


@pytest.mark.skipif(_gpu_visible(), reason="passes placeholder pointers: only where no GPU can run them")
@pytest.mark.parametrize("name,args,ptrs", NULL_CASES, ids=[c[0] for c in NULL_CASES])
def test_null_device_pointers_are_invalid(name, args, ptrs):
    """A NULL pointer that the work would read or write returns 1 before any
    launch (the reference would launch with it); the empty no-ops keep
    returning 0 before that check."""
    fn = getattr(B.lib(), name)
    for k in ptrs:
        bad = list(args)
        bad[k] = NULL
        assert fn(*bad, None) == 1, (name, k)


@pytest.mark.skipif(_gpu_visible(), reason="passes placeholder pointers: only where no GPU can run them")
def test_null_pointers_in_groups_are_invalid():
    L = B.lib()
    for fn, extra in ((L.bonsai_p40_gemv_group, (A, 128)),
                      (L.bonsai_p40_fwht_gemv_group, (A, NULL, 1024)),
                      (L.bonsai_p40_rmsnorm_fwht_gemv_group, (A, A, NULL, 1024, EPS))):
        for hole in ("W", "y"):
            W = (C.c_void_p * 2)(A, A)
            y = (C.c_void_p * 2)(A, A)
            (W if hole == "W" else y)[1] = None
            n = (C.c_int64 * 2)(16, 16)
            assert fn(W, y, n, 2, *extra, None) == 1, (fn, hole)
        W = (C.c_void_p * 1)(A)
        y = (C.c_void_p * 1)(A)
        n = (C.c_int64 * 1)(16)
        assert fn(W, y, n, 1, *((NULL,) + extra[1:]), None) == 1


LIMIT_CASES = [
    ("gemv: n_out >= 2^30", "bonsai_p40_gemv", (A, A, A, 1 << 30, 128)),
    ("gemv: n_in / 128 > 2^24", "bonsai_p40_gemv", (A, A, A, 16, 128 * ((1 << 24) + 1))),
    ("gemv_repack: W not 8-byte aligned", "bonsai_p40_gemv_repack", (A + 4, A, A, 4, 1024)),
    ("gemm: W not 2-byte aligned", "bonsai_p40_gemm", (A + 1, A, A, 16, 128, 4)),
    ("gemm_ws: workspace not 16-byte aligned", "bonsai_p40_gemm_ws", (A, A, A, 4096, 5120, 512, A + 4, 1 << 30)),
    ("gemm_ws: workspace too small", "bonsai_p40_gemm_ws", (A, A, A, 4096, 5120, 512, A, 512 * 160 * 68 - 1)),
    ("fwht_quant: xq not 4-byte aligned", "bonsai_p40_fwht_quant", (A, NULL, A + 2, 1024)),
    ("quant_tokens: more than 65535 tokens", "bonsai_p40_quant_tokens", (A, NULL, A, 1024, 65536, 1)),
    ("quant_tokens: n * n_tok > 2^40", "bonsai_p40_quant_tokens", (A, NULL, A, 1 << 30, 2048, 0)),
    ("quant_tokens: signs without the rotation", "bonsai_p40_quant_tokens", (A, A, A, 1024, 2, 0)),
]


@pytest.mark.skipif(_gpu_visible(), reason="passes placeholder pointers: only where no GPU can run them")
@pytest.mark.parametrize("what,name,args", LIMIT_CASES, ids=[c[0] for c in LIMIT_CASES])
def test_documented_limits_are_invalid(what, name, args):
    """The size and alignment limits the header states return 1 before any
    launch."""
    assert getattr(B.lib(), name)(*args, None) == 1, what


@pytest.mark.skipif(_gpu_visible(), reason="passes placeholder pointers: only where no GPU can run them")
def test_concurrent_calls_from_host_threads():
    """Eight host threads call the launch paths (per-device property caches,
    once-per-device kernel attributes, the tuning table and its reload) at
    the same time.  Without a device every launch reports the runtime's
    error; the calls must neither crash nor disagree with a serial call."""
    import threading
    L = B.lib()
    calls = [
        lambda: L.bonsai_p40_gemv(4096, 8192, 16384, 17408, 5120, None),
        lambda: L.bonsai_p40_gemv(4096, 8192, 16384, 300, 3072, None),
        lambda: L.bonsai_p40_gemm(4096, 8192, 16384, 256, 5120, 8, None),
        lambda: L.bonsai_p40_gemm(4096, 8192, 16384, 4096, 5120, 512, None),
        lambda: L.bonsai_p40_gemv_repack(4096, 8192, 16384, 256, 5120, None),
        lambda: L.bonsai_p40_reload_tuning(),
    ]
    serial = [c() for c in calls]
    assert serial[-1] == 0 and all(rc != 0 for rc in serial[:-1])
    out, errors = [], []

    def worker(i):
        try:
            for k in range(40):
                j = (i + k) % len(calls)
                out.append((j, calls[j]()))
        except Exception as e:  # pragma: no cover - reported below
            errors.append(e)

    ts = [threading.Thread(target=worker, args=(i,)) for i in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors
    assert len(out) == 8 * 40
    assert all(rc == serial[j] for j, rc in out)


def test_ffn_gate_up_swiglu_argument_checks():
    f = B.lib().bonsai_p40_ffn_gate_up_swiglu
    args = [16, 16, 16, None, None, None, 16, 17408, 5120, C.c_float(1e-6)]
    assert f(*args, None, None, None) == 1                      # no workspace
    assert f(*args, 24, None, None) == 1                        # workspace not 16-byte aligned
    bad = list(args)
    bad[7] = 1000                                               # n_ff % 1024
    assert f(*bad, 32, None, None) == 1
    bad = list(args)
    bad[8] = 5000                                               # n_embd % 1024
    assert f(*bad, 32, None, None) == 1
    bad = list(args)
    bad[6] = 18                                                 # hq not 4-byte aligned
    assert f(*bad, 32, None, None) == 1
    bad = list(args)
    bad[2] = None                                               # no x
    assert f(*bad, 32, None, None) == 1


def test_chain_plan_argument_checks():
    """Invalid decode-chain steps are rejected (rc 1) before anything touches
    a device; the run entry point checks its pointers."""
    L = B.lib()
    ok = dict(W=[16], y=[16], n_out=[64], n_in=5120, x=16)
    bad_steps = [
        B.chain_step(7, **ok),                                              # unknown kind
        B.chain_step(B.CHAIN_Q8, W=[16], y=[16], n_out=[64], n_in=5000, x=16),   # n_in % 1024
        B.chain_step(B.CHAIN_Q8, W=[16], y=[16], n_out=[64], n_in=7168, x=16),   # width not supported
        B.chain_step(B.CHAIN_FWHT, W=[16], y=[16], n_out=[64], n_in=17408, x=16),  # fused prologue at 17408
        B.chain_step(B.CHAIN_Q8, W=[24], y=[16], n_out=[64], n_in=5120, x=16),   # W not 16-byte aligned
        B.chain_step(B.CHAIN_FWHT, W=[16], y=[16], n_out=[64], n_in=5120, x=20),  # fp32 x not 16-byte aligned
        B.chain_step(B.CHAIN_Q8, W=[16], y=[16], n_out=[0], n_in=5120, x=16),    # empty matrix
        B.chain_step(B.CHAIN_Q8, W=[], y=[], n_out=[], n_in=5120, x=16),         # no matrix
        B.chain_step(B.CHAIN_Q8, W=[16] * 4, y=[16] * 4, n_out=[8] * 4, n_in=5120, x=None),  # no input
        B.chain_step(B.CHAIN_RMSNORM_FWHT, **ok),                           # no norm weights
        B.chain_step(B.CHAIN_SWIGLU, n_in=17408, x=16, x2=None, q_out=16),  # no up rows
        B.chain_step(B.CHAIN_SWIGLU, n_in=17408, x=16, x2=16, q_out=18),    # q_out not 4-byte aligned
    ]
    for i, s in enumerate(bad_steps):
        arr = (B.ChainStep * 1)(s)
        assert L.bonsai_p40_chain_plan(C.cast(arr, C.c_void_p), 1, 256) == 1, i
    arr = (B.ChainStep * 1)(B.chain_step(B.CHAIN_Q8, **ok))
    assert L.bonsai_p40_chain_plan(None, 1, 256) == 1
    assert L.bonsai_p40_chain_plan(C.cast(arr, C.c_void_p), 0, 256) == 1
    assert L.bonsai_p40_chain_plan(C.cast(arr, C.c_void_p), 1, None) == 1
    assert L.bonsai_p40_chain_plan(C.cast(arr, C.c_void_p), 1, 264) == 1     # plan not 16-byte aligned
    assert L.bonsai_p40_chain_plan_bytes(0) == 0
    assert L.bonsai_p40_chain_plan_bytes(3) > 0
    assert L.bonsai_p40_chain_run(None, 1, 256, None, None) == 1
    assert L.bonsai_p40_chain_run(256, 1, None, None, None) == 1
    assert L.bonsai_p40_chain_run(256, 0, 256, None, None) == 1


def test_gemm_workspace_bytes():
    """68 bytes per Q8_1 block of X (its q bytes as f16 and d as fp32); 0 for
    an empty or invalid shape and where the converted activation would reach
    2 GiB."""
    L = B.lib()
    assert B.gemm_workspace_bytes(5120, 2048) == 2048 * 160 * 68
    assert B.gemm_workspace_bytes(17408, 512) == 512 * 544 * 68
    assert L.bonsai_p40_gemm_workspace_bytes(5120, 0) == 0
    assert L.bonsai_p40_gemm_workspace_bytes(100, 16) == 0
    assert L.bonsai_p40_gemm_workspace_bytes(17408, 65536) == 0       # 65536 * 544 * 64 >= 2^31
