"""The FFN gate/up launch with its SwiGLU glue (bonsai_p40_ffn_gate_up_swiglu):
gate and up GEMVs from the fp32 layer input, then, inside the same launch,
SwiGLU -> FWHT -> Q8_1 of their outputs (src/ops.h:27-31) for the down
projection.  Its Q8_1 bytes must equal the separate launches'
(bonsai_p40_rmsnorm_fwht_gemv_group / bonsai_p40_fwht_gemv_group, then
bonsai_p40_swiglu_fwht_quant), the chain must match the oracle stage-wise,
and the workspace must be back to zero after every call (each block's
finaliser clears the row words it consumed)."""
import numpy as np
import pytest

import bonsai_p40 as B
from oracle import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    B.lib()   # fail loudly if the native library is missing
    yield
    torch.cuda.synchronize()


def case(msg):
    print(f"[case] {msg}", flush=True)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def signs(seed, n):
    return np.where(O.gen_normal(seed, n) > 0, 1.0, -1.0).astype(np.float32)


def separate(Wg, Wu, x, nw, xs, hs, n_ff, n_embd, eps):
    """The same chain as two launches: grouped fused GEMV, then the glue."""
    g = torch.empty(n_ff, dtype=torch.float32, device="cuda")
    u = torch.empty(n_ff, dtype=torch.float32, device="cuda")
    if nw is None:
        B.fwht_gemv_group([Wg, Wu], x, xs, [g, u], [n_ff, n_ff], n_embd)
    else:
        B.rmsnorm_fwht_gemv_group([Wg, Wu], x, nw, xs, [g, u], [n_ff, n_ff], n_embd, eps)
    hq = torch.zeros(B.q8_bytes(n_ff), dtype=torch.uint8, device="cuda")
    B.swiglu_fwht_quant(g, u, hs, hq, n_ff)
    return host(hq), host(g), host(u)


def fused_width(n_embd, rms):
    """Widths with a one-launch kernel (the others run the grouped GEMV and
    the glue as two launches, leaving plain fp32 rows in the workspace)."""
    return n_embd // 128 in ({8, 40, 48} if rms else {8, 40, 48, 80, 96, 136})


CASES = [
    # n_ff, n_embd, rms, x_signs, h_signs
    (17408, 5120, True, False, False),        # the model's FFN, as a layer runs it
    (17408, 5120, False, True, True),
    (17408, 5120, True, True, True),
    (1024, 5120, True, False, True),          # one block: a single finalising workgroup
    (5120, 6144, False, False, False),
    (3072, 1024, True, True, False),
    (2048, 17408, False, False, False),       # widest input rows
    (4096, 2048, True, False, False),         # no streaming kernel: grouped GEMV + glue launches
]


@pytest.mark.parametrize("n_ff,n_embd,rms,xsg,hsg", CASES)
def test_ffn_gate_up_swiglu_equals_separate_launches(n_ff, n_embd, rms, xsg, hsg):
    case(f"ffn_gate_up_swiglu n_ff={n_ff} n_embd={n_embd} rms={rms} x_signs={xsg} h_signs={hsg}")
    Wg = dev(O.gen_weights(6000 + n_ff, n_ff, n_embd))
    Wu = dev(O.gen_weights(6001 + n_ff, n_ff, n_embd))
    x_np = O.gen_normal(6002 + n_embd, n_embd) * 2
    nw_np = O.gen_normal(6003 + n_embd, n_embd) * 0.1 + 1
    x = dev(x_np)
    nw = dev(nw_np) if rms else None
    xs = dev(signs(6004 + n_embd, n_embd)) if xsg else None
    hs = dev(signs(6005 + n_ff, n_ff)) if hsg else None
    eps = 1e-6
    ref_hq, ref_g, ref_u = separate(Wg, Wu, x, nw, xs, hs, n_ff, n_embd, eps)
    ws = torch.zeros(B.ffn_workspace_bytes(n_ff), dtype=torch.uint8, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    fused = fused_width(n_embd, rms)
    for rep in range(3):                                # each call leaves the workspace ready
        hq = torch.full((B.q8_bytes(n_ff),), 0xAB, dtype=torch.uint8, device="cuda")
        B.ffn_gate_up_swiglu(Wg, Wu, x, nw, xs, hs, hq, n_ff, n_embd, eps, ws, status)
        np.testing.assert_array_equal(host(hq), ref_hq)
        w = host(ws)
        assert not np.any(w[:B.FFN_SYNC_BYTES].view(np.uint32)), "sync words not zero after the call"
        gu = w[B.FFN_SYNC_BYTES:].view(np.uint32)
        if fused:
            assert not np.any(gu), "row words not cleared by the finalisers"
        else:
            np.testing.assert_array_equal(gu[:n_ff], ref_g.view(np.uint32))
            np.testing.assert_array_equal(gu[n_ff:], ref_u.view(np.uint32))
        assert int(host(status)[0]) == 0


@pytest.mark.parametrize("n_ff,n_embd", [(17408, 5120), (5120, 6144), (1024, 5120), (3072, 1024)])
def test_ffn_single_wave_finaliser(n_ff, n_embd, knobs):
    """With the four-wave quads switched off (BONSAI_FFN_QUAD=0) each block is
    finalised by one wave: the same bytes, the workspace back to zero."""
    case(f"ffn_gate_up_swiglu single-wave finaliser n_ff={n_ff} n_embd={n_embd}")
    knobs.set("BONSAI_FFN_QUAD", "0")
    Wg = dev(O.gen_weights(6200 + n_ff, n_ff, n_embd))
    Wu = dev(O.gen_weights(6201 + n_ff, n_ff, n_embd))
    x = dev(O.gen_normal(6202 + n_embd, n_embd) * 2)
    nw = dev(O.gen_normal(6203 + n_embd, n_embd) * 0.1 + 1)
    hs = dev(signs(6204 + n_ff, n_ff))
    ref_hq, _, _ = separate(Wg, Wu, x, nw, None, hs, n_ff, n_embd, 1e-6)
    ws = torch.zeros(B.ffn_workspace_bytes(n_ff), dtype=torch.uint8, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    for rep in range(2):
        hq = torch.full((B.q8_bytes(n_ff),), 0xAB, dtype=torch.uint8, device="cuda")
        B.ffn_gate_up_swiglu(Wg, Wu, x, nw, None, hs, hq, n_ff, n_embd, 1e-6, ws, status)
        np.testing.assert_array_equal(host(hq), ref_hq)
        assert not np.any(host(ws).view(np.uint32))
        assert int(host(status)[0]) == 0


def test_ffn_gate_up_swiglu_against_oracle_chain():
    """Config 1 through the fused launch and the down GEMV, stage-wise against
    the oracle: gate/up (from the separate grouped launch, whose hq the fused
    launch equals byte for byte) within the GEMV tolerance of the oracle on
    the device's own Q8_1 input, hq within one q step (device and glibc expf
    differ in the last ulp), y_down within the GEMV tolerance of the oracle
    on the device's hq."""
    n_ff, n_embd = 17408, 5120
    case("ffn_gate_up_swiglu config 1 against the oracle chain")
    Wg_np = O.gen_weights(6100, n_ff, n_embd)
    Wu_np = O.gen_weights(6101, n_ff, n_embd)
    Wd_np = O.gen_weights(6102, n_embd, n_ff)
    x_np = O.gen_normal(6103, n_embd)
    ws = torch.zeros(B.ffn_workspace_bytes(n_ff), dtype=torch.uint8, device="cuda")
    hq = torch.zeros(B.q8_bytes(n_ff), dtype=torch.uint8, device="cuda")
    Wg, Wu, x = dev(Wg_np), dev(Wu_np), dev(x_np)
    B.ffn_gate_up_swiglu(Wg, Wu, x, None, None, None, hq, n_ff, n_embd, 0.0, ws)
    sep_hq, g_dev, u_dev = separate(Wg, Wu, x, None, None, None, n_ff, n_embd, 0.0)
    np.testing.assert_array_equal(host(hq), sep_hq)
    y = torch.empty(n_embd, dtype=torch.float32, device="cuda")
    B.gemv(dev(Wd_np), hq, y, n_embd, n_ff)
    xq = O.quantize_q8_1(O.fwht(x_np), True)
    gu = np.concatenate([g_dev, u_dev])
    g_ref = O.gemv(Wg_np, xq, n_ff, n_embd, nthreads=16)
    u_ref = O.gemv(Wu_np, xq, n_ff, n_embd, nthreads=16)
    for got, ref in ((gu[:n_ff], g_ref), (gu[n_ff:], u_ref)):
        assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))
    hq_np = host(hq)
    _, _, q1 = O.q81_fields(hq_np)
    _, _, q2 = O.q81_fields(O.quantize_q8_1(O.fwht(O.swiglu(gu[:n_ff], gu[n_ff:])), True))
    assert np.max(np.abs(q1.astype(int) - q2.astype(int))) <= 1
    assert np.mean(q1 != q2) < 0.01
    y_ref = O.gemv(Wd_np, hq_np, n_embd, n_ff, nthreads=16)
    assert np.max(np.abs(host(y) - y_ref)) <= 1e-5 * np.max(np.abs(y_ref))
