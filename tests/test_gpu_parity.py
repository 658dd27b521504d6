"""GPU parity tests: the HIP path (through the C ABI) against the CPU oracle.

Bars (from the reference host code, src/pq2_0.h, src/fwht.h, tests/test_p40.cpp):
  * Q8_1 bytes, repacked bytes, int32 chunk dots, FWHT fp32 bits: exact;
  * fp32 GEMV/GEMM outputs: max |dy| <= 1e-5 * max |y_ref| (normwise; the
    device sums chunks in a different order than the host's sequential loop);
  * chains containing expf (SwiGLU): 1e-4 normwise, since device and glibc
    expf differ in the last ulp.
"""
import os
import sys

import numpy as np
import pytest

import bonsai_p40 as B
from oracle import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-5


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    B.lib()   # fail loudly if the native library is missing
    yield
    torch.cuda.synchronize()


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def normwise(got, ref):
    scale = max(float(np.max(np.abs(ref))), 1e-30)
    return float(np.max(np.abs(got.astype(np.float64) - ref.astype(np.float64)))) / scale


def offset_copy(a: np.ndarray, offset: int):
    """Device copy of a byte array starting `offset` bytes past a 256-B boundary."""
    buf = torch.zeros(a.size + 64, dtype=torch.uint8, device="cuda")
    buf[offset:offset + a.size] = dev(a)
    return buf, buf.data_ptr() + offset


# ------------------------------------------------------------------ FWHT
def test_fwht_fixture_bits(golden):
    case("fwht n=2048 fixture, signs None / length-n")
    x = dev(golden["f3_in"])
    B.fwht(x, None, 2048)
    assert np.array_equal(bits(host(x)), bits(golden["f3_out"]))
    x = dev(golden["f3_in"])
    B.fwht_signs_n(x, None, 2048)
    assert np.array_equal(bits(host(x)), bits(golden["f3_out"]))
    x = dev(golden["f3_in"])
    B.fwht_signs_n(x, dev(golden["f3_signs"]), 2048)
    assert np.array_equal(bits(host(x)), bits(golden["f3_out_signed"]))


@pytest.mark.parametrize("n,offset", [(5120, 0), (17408, 0), (17408, 1), (1024, 3)])
def test_fwht_seeded_bits(n, offset):
    """Both sign meanings: bonsai_p40_fwht reuses signs[0..1023] for every
    block (the reference device kernel, elementwise_p40.cu:23) and equals the
    host fwht_blocks with that vector tiled; bonsai_p40_fwht_signs_n reads a
    length-n vector (src/fwht.h:38-42).  The 1024-entry buffer is followed by
    NaN guards, which a read past its end would carry into the result."""
    case(f"fwht n={n} float offset={offset}")
    x = O.gen_normal(300 + n, n)
    s = np.where(O.gen_normal(301 + n, n) > 0, 1.0, -1.0).astype(np.float32)
    buf = torch.zeros(n + 8, dtype=torch.float32, device="cuda")
    buf[offset:offset + n] = dev(x)
    B.fwht_signs_n(buf.data_ptr() + 4 * offset, dev(s), n)
    assert np.array_equal(bits(host(buf)[offset:offset + n]), bits(O.fwht(x, s)))
    s1 = torch.full((1024 + 64,), float("nan"), dtype=torch.float32, device="cuda")
    s1[:1024] = dev(s[:1024])
    buf[offset:offset + n] = dev(x)
    B.fwht(buf.data_ptr() + 4 * offset, s1, n)
    assert np.array_equal(bits(host(buf)[offset:offset + n]), bits(O.fwht(x, np.tile(s[:1024], n // 1024))))


# ------------------------------------------------------------- quantisers
@pytest.mark.parametrize("name", ["seeded", "special", "k32"])
def test_quant_activations_fixture(golden, name):
    case(f"quant_activations fixture {name}")
    x = golden[f"f2_{name}_in"]
    q = torch.zeros(x.size // 32 * 36, dtype=torch.uint8, device="cuda")
    B.quant_activations(dev(x), q, x.size)
    np.testing.assert_array_equal(host(q), golden[f"f2_{name}_perm"])


@pytest.mark.parametrize("n", [32, 96, 5120, 17408, 32768])
def test_quant_activations_seeded(n):
    case(f"quant_activations n={n}")
    x = O.gen_normal(400 + n, n) * 2.5
    q = torch.zeros(n // 32 * 36, dtype=torch.uint8, device="cuda")
    B.quant_activations(dev(x), q, n)
    np.testing.assert_array_equal(host(q), O.quantize_q8_1(x, True))


@pytest.mark.parametrize("n,signed", [(5120, False), (5120, True), (17408, True), (6144, False)])
def test_fwht_quant_bytes(n, signed):
    case(f"fwht_quant n={n} signed={signed}")
    x = O.gen_normal(500 + n, n)
    s = np.where(O.gen_normal(501 + n, n) > 0, 1.0, -1.0).astype(np.float32) if signed else None
    q = torch.zeros(n // 32 * 36, dtype=torch.uint8, device="cuda")
    B.fwht_quant(dev(x), None if s is None else dev(s), q, n)
    np.testing.assert_array_equal(host(q), O.quantize_q8_1(O.fwht(x, s), True))


@pytest.mark.parametrize("n,n_tok,rotate", [(1024, 5, True), (5120, 64, True), (256, 5, False),
                                            (5120, 3, False)])
def test_quant_tokens_chunk_major(n, n_tok, rotate):
    case(f"quant_tokens n={n} n_tok={n_tok} rotate={rotate}")
    X = O.gen_normal(600 + n + n_tok, n * n_tok).reshape(n_tok, n)
    q = torch.zeros(n // 32 * n_tok * 36, dtype=torch.uint8, device="cuda")
    B.quant_tokens(dev(X), None, q, n, n_tok, rotate)
    Xr = np.stack([O.fwht(X[t]) for t in range(n_tok)]) if rotate else X
    np.testing.assert_array_equal(host(q), O.quantize_chunk_major(Xr))


def test_swiglu_fwht_quant_fixture(golden):
    case("swiglu_fwht_quant n=2048 fixture")
    q = torch.zeros(2048 // 32 * 36, dtype=torch.uint8, device="cuda")
    B.swiglu_fwht_quant(dev(golden["f7_gate"]), dev(golden["f7_up"]), None, q, 2048)
    got = host(q)
    ref = golden["f7_hq"]
    d1, s1, q1 = O.q81_fields(got)
    d2, s2, q2 = O.q81_fields(ref)
    # device expf may differ from glibc in the last ulp: q bytes may move by 1
    assert np.max(np.abs(q1.astype(int) - q2.astype(int))) <= 1
    assert np.mean(q1 != q2) < 0.01
    assert np.max(np.abs(d1.astype(int) - d2.astype(int))) <= 1


@pytest.mark.parametrize("n,signed,offset", [(17408, True, 0), (5120, False, 1), (1024, True, 0)])
def test_swiglu_fwht_quant_seeded(n, signed, offset):
    """Against the oracle chain (glibc expf): q within one step, rare."""
    case(f"swiglu_fwht_quant n={n} signed={signed} float offset={offset}")
    g = O.gen_normal(2600 + n, n) * 2
    u = O.gen_normal(2601 + n, n)
    sg = np.where(O.gen_normal(2602 + n, n) > 0, 1.0, -1.0).astype(np.float32) if signed else None
    gb = torch.zeros(n + 4, dtype=torch.float32, device="cuda")
    ub = torch.zeros(n + 4, dtype=torch.float32, device="cuda")
    gb[offset:offset + n] = dev(g)
    ub[offset:offset + n] = dev(u)
    q = torch.zeros(n // 32 * 36, dtype=torch.uint8, device="cuda")
    B.swiglu_fwht_quant(gb.data_ptr() + 4 * offset, ub.data_ptr() + 4 * offset,
                        None if sg is None else dev(sg), q, n)
    d1, s1, q1 = O.q81_fields(host(q))
    d2, s2, q2 = O.q81_fields(O.quantize_q8_1(O.fwht(O.swiglu(g, u), sg), True))
    assert np.max(np.abs(q1.astype(int) - q2.astype(int))) <= 1
    assert np.mean(q1 != q2) < 0.01
    assert np.max(np.abs(d1.astype(int) - d2.astype(int))) <= 1


# --------------------------------------------------------- chunk dots / GEMV
SHAPES = [
    (8, 5120), (5, 5120), (1, 5120), (64, 17408), (33, 6144), (7, 1024), (9, 10240),
    (6, 12288), (3, 384), (4, 128), (17, 2048),
]


def make(n_out, n_in, seed, p3=0.001):
    W = O.gen_weights(seed, n_out, n_in, p3)
    xq = O.quantize_q8_1(O.fwht(O.gen_normal(seed + 1, n_in)) if n_in % 1024 == 0
                         else O.gen_normal(seed + 1, n_in), True)
    return W, xq


@pytest.mark.parametrize("k", [5120, 17408])
def test_chunk_dots_fixture(golden, k):
    case(f"chunk_dots fixture k={k}")
    out = torch.zeros((8, k // 32), dtype=torch.int32, device="cuda")
    B.chunk_dots(dev(golden[f"f4_{k}_W"]), dev(golden[f"f4_{k}_xq"]), out, 8, k)
    np.testing.assert_array_equal(host(out), golden[f"f4_{k}_sumi"])


@pytest.mark.parametrize("n_out,n_in", SHAPES)
@pytest.mark.parametrize("w_offset", [0, 2])
def test_chunk_dots_exact(n_out, n_in, w_offset):
    case(f"chunk_dots {n_out}x{n_in} W offset {w_offset}")
    W, xq = make(n_out, n_in, 700 + n_out + n_in, 0.05)
    buf, wp = offset_copy(W, w_offset)
    out = torch.full((n_out, n_in // 32), -999999, dtype=torch.int32, device="cuda")
    B.chunk_dots(wp, dev(xq), out, n_out, n_in)
    np.testing.assert_array_equal(host(out), O.chunk_dots(W, xq, n_out, n_in))


@pytest.mark.parametrize("k", [5120, 17408])
def test_gemv_fixture(golden, k):
    case(f"gemv fixture k={k}")
    y = torch.zeros(8, dtype=torch.float32, device="cuda")
    B.gemv(dev(golden[f"f4_{k}_W"]), dev(golden[f"f4_{k}_xq"]), y, 8, k)
    assert normwise(host(y), golden[f"f4_{k}_y"]) <= TOL


@pytest.mark.parametrize("n_out,n_in", SHAPES)
@pytest.mark.parametrize("w_offset", [0, 2])
def test_gemv_matches_oracle(n_out, n_in, w_offset):
    case(f"gemv {n_out}x{n_in} W offset {w_offset}")
    W, xq = make(n_out, n_in, 800 + n_out + n_in)
    buf, wp = offset_copy(W, w_offset)
    y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    B.gemv(wp, dev(xq), y, n_out, n_in)
    assert normwise(host(y), O.gemv(W, xq, n_out, n_in)) <= TOL


@pytest.mark.parametrize("n_out,n_in", [(17408, 5120), (5120, 17408), (6144, 5120), (1024, 5120),
                                        (5120, 6144), (17407, 5120), (5120, 5120)])
def test_gemv_model_shapes(n_out, n_in):
    case(f"gemv model shape {n_out}x{n_in}")
    W, xq = make(n_out, n_in, 900 + n_in)
    y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    Wd = dev(W)
    B.gemv(Wd, dev(xq), y, n_out, n_in)
    ref = O.gemv(W, xq, n_out, n_in, nthreads=16)
    got = host(y)
    assert np.all(np.isfinite(got))
    assert normwise(got, ref) <= TOL
    # the same weights twice in a row give identical output (no state)
    B.gemv(Wd, dev(xq), y, n_out, n_in)
    assert np.array_equal(bits(host(y)), bits(got))


def test_gemv_code3_and_extremes():
    case("gemv all-code-3 rows, saturated activations")
    n_out, n_in = 6, 2048
    W = O.gen_weights(950, n_out, n_in, 1.0)            # every code is 3 (+2)
    x = np.zeros(n_in, np.float32)
    x[::7] = 1e4
    x[1::7] = -1e4
    xq = O.quantize_q8_1(x, True)
    y = torch.zeros(n_out, dtype=torch.float32, device="cuda")
    B.gemv(dev(W), dev(xq), y, n_out, n_in)
    assert normwise(host(y), O.gemv(W, xq, n_out, n_in)) <= TOL
    out = torch.zeros((n_out, n_in // 32), dtype=torch.int32, device="cuda")
    B.chunk_dots(dev(W), dev(xq), out, n_out, n_in)
    np.testing.assert_array_equal(host(out), O.chunk_dots(W, xq, n_out, n_in))


# ------------------------------------------------------- fused FWHT + GEMV
ROT_WIDTHS = (8, 40, 48, 80, 96, 136)     # n_in / 128 of the streaming kernel


@pytest.mark.parametrize("n_out,n_in,signed", [
    (17408, 5120, False), (6144, 5120, True), (1024, 5120, False), (5120, 6144, True),
    (5120, 17408, False), (5120, 17408, True), (17407, 5120, True), (333, 1024, False),
    (97, 10240, True), (100, 12288, True), (77, 2048, True), (64, 3072, False), (1, 5120, False)])
def test_fwht_gemv(n_out, n_in, signed):
    case(f"fwht_gemv {n_out}x{n_in} signed={signed}")
    W = O.gen_weights(1600 + n_out + n_in, n_out, n_in)
    x = O.gen_normal(1601 + n_in, n_in)
    s = np.where(O.gen_normal(1602 + n_in, n_in) > 0, 1.0, -1.0).astype(np.float32) if signed else None
    Wd, xd = dev(W), dev(x)
    sd = None if s is None else dev(s)
    y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    B.fwht_gemv(Wd, xd, sd, y, n_out, n_in)
    got = host(y)
    xq_ref = O.quantize_q8_1(O.fwht(x, s), True)
    assert np.all(np.isfinite(got))
    assert normwise(got, O.gemv(W, xq_ref, n_out, n_in, nthreads=16)) <= TOL
    np.testing.assert_array_equal(bits(host(xd)), bits(x))          # x is not modified
    # the separate pre-pass + GEMV: same Q8_1 bytes, and on the streaming
    # widths the same kernel arithmetic, so the same bits
    q = torch.zeros(n_in // 32 * 36, dtype=torch.uint8, device="cuda")
    B.fwht_quant(xd, sd, q, n_in)
    y2 = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    B.gemv(Wd, q, y2, n_out, n_in)
    if n_in // 128 in ROT_WIDTHS and not (signed and n_in == 17408):
        np.testing.assert_array_equal(bits(got), bits(host(y2)))
    # a second call in a row gives the same bits (no state)
    B.fwht_gemv(Wd, xd, sd, y, n_out, n_in)
    np.testing.assert_array_equal(bits(host(y)), bits(got))


@pytest.mark.parametrize("n_out,n_in", [
    (17408, 5120), (6144, 5120), (1024, 5120), (5120, 6144), (5120, 17408), (17407, 5120),
    (333, 1024), (97, 10240), (100, 12288), (77, 2048), (64, 3072), (1, 5120)])
def test_quant_gemv(n_out, n_in):
    """y = W . Q8_1(x) in one launch: within the GEMV tolerance of the oracle,
    x unchanged, and on the streaming widths bit-identical to
    quant_activations + gemv (the reference hook's two launches)."""
    case(f"quant_gemv {n_out}x{n_in}")
    W = O.gen_weights(1650 + n_out + n_in, n_out, n_in)
    x = O.gen_normal(1651 + n_in, n_in) * 1.5
    Wd, xd = dev(W), dev(x)
    y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    B.quant_gemv(Wd, xd, y, n_out, n_in)
    got = host(y)
    xq_ref = O.quantize_q8_1(x, True)
    assert np.all(np.isfinite(got))
    assert normwise(got, O.gemv(W, xq_ref, n_out, n_in, nthreads=16)) <= TOL
    np.testing.assert_array_equal(bits(host(xd)), bits(x))
    q = torch.zeros(n_in // 32 * 36, dtype=torch.uint8, device="cuda")
    B.quant_activations(xd, q, n_in)
    np.testing.assert_array_equal(host(q), xq_ref)
    y2 = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    B.gemv(Wd, q, y2, n_out, n_in)
    if n_in // 128 in ROT_WIDTHS:
        np.testing.assert_array_equal(bits(got), bits(host(y2)))


@pytest.mark.parametrize("x_offset", [4, 8])
def test_quant_gemv_unaligned_x(x_offset):
    """x off a 16-byte boundary takes the generic kernel: same tolerance."""
    case(f"quant_gemv unaligned x offset {x_offset}")
    n_out, n_in = 300, 5120
    W = O.gen_weights(1750, n_out, n_in)
    x = O.gen_normal(1751, n_in)
    buf, xp = offset_copy(x.view(np.uint8), x_offset)
    y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    B.quant_gemv(dev(W), xp, y, n_out, n_in)
    assert normwise(host(y), O.gemv(W, O.quantize_q8_1(x, True), n_out, n_in)) <= TOL


GROUPS = [
    (5120, (6144, 1024, 1024)),               # q, k, v
    (5120, (17408, 17408)),                   # gate, up
    (5120, (17407, 3, 0, 1001)),              # ragged: partial 2-row units, an empty matrix
    (6144, (5120, 7)),
    (17408, (5120, 100, 33)),
    (2048, (64, 300)),                        # no streaming kernel: one launch per matrix
]


@pytest.mark.parametrize("n_in,n_outs", GROUPS)
def test_gemv_group(n_in, n_outs):
    case(f"gemv_group n_in={n_in} n_outs={n_outs}")
    Ws = [O.gen_weights(1800 + m + n_in, max(r, 1), n_in) for m, r in enumerate(n_outs)]
    xq = O.quantize_q8_1(O.fwht(O.gen_normal(1810 + n_in, n_in)), True)
    Wd = [dev(W) for W in Ws]
    xd = dev(xq)
    ys = [torch.full((max(r, 1),), float("nan"), dtype=torch.float32, device="cuda") for r in n_outs]
    B.gemv_group(Wd, xd, ys, n_outs, n_in)
    for W, Wdm, y, r in zip(Ws, Wd, ys, n_outs):
        got = host(y)
        if r == 0:
            assert np.isnan(got).all()        # skipped: untouched
            continue
        assert normwise(got, O.gemv(W, xq, r, n_in, nthreads=16)) <= TOL
        y1 = torch.full((r,), float("nan"), dtype=torch.float32, device="cuda")
        B.gemv(Wdm, xd, y1, r, n_in)
        np.testing.assert_array_equal(bits(got), bits(host(y1)))


@pytest.mark.parametrize("n_in,n_outs", GROUPS)
@pytest.mark.parametrize("signed", [False, True])
def test_fwht_gemv_group(n_in, n_outs, signed):
    case(f"fwht_gemv_group n_in={n_in} n_outs={n_outs} signed={signed}")
    Ws = [O.gen_weights(1900 + m + n_in, max(r, 1), n_in) for m, r in enumerate(n_outs)]
    x = O.gen_normal(1910 + n_in, n_in)
    s = np.where(O.gen_normal(1911 + n_in, n_in) > 0, 1.0, -1.0).astype(np.float32) if signed else None
    xq = O.quantize_q8_1(O.fwht(x, s), True)
    Wd = [dev(W) for W in Ws]
    xd = dev(x)
    sd = None if s is None else dev(s)
    ys = [torch.full((max(r, 1),), float("nan"), dtype=torch.float32, device="cuda") for r in n_outs]
    B.fwht_gemv_group(Wd, xd, sd, ys, n_outs, n_in)
    for W, Wdm, y, r in zip(Ws, Wd, ys, n_outs):
        got = host(y)
        if r == 0:
            assert np.isnan(got).all()
            continue
        assert normwise(got, O.gemv(W, xq, r, n_in, nthreads=16)) <= TOL
        y1 = torch.full((r,), float("nan"), dtype=torch.float32, device="cuda")
        B.fwht_gemv(Wdm, xd, sd, y1, r, n_in)
        np.testing.assert_array_equal(bits(got), bits(host(y1)))


RMS_GROUPS = [
    (5120, (6144, 1024, 1024), True),         # q, k, v after the attention norm
    (5120, (17408, 17408), False),            # gate, up after the FFN norm
    (5120, (17407, 3, 0, 1001), True),        # ragged
    (6144, (5120, 7), False),
    (1024, (300, 64), True),
    (2048, (64, 300), True),                  # no streaming kernel: generic fused kernel
    (17408, (100, 33), False),                # no RMS streaming instance: generic fused kernel
]


@pytest.mark.parametrize("n_in,n_outs,signed", RMS_GROUPS)
def test_rmsnorm_fwht_gemv_group(n_in, n_outs, signed):
    """Bit-identical to the fused RMSNorm pre-pass followed by the grouped
    GEMV (both scale with an fp64 sum of squares), and within the fp32
    tolerance of the oracle chain with that scale."""
    case(f"rmsnorm_fwht_gemv_group n_in={n_in} n_outs={n_outs} signed={signed}")
    Ws = [O.gen_weights(2400 + m + n_in, max(r, 1), n_in) for m, r in enumerate(n_outs)]
    x = O.gen_normal(2410 + n_in, n_in) * 4
    nw = O.gen_normal(2411 + n_in, n_in) * 0.1 + 1
    s = np.where(O.gen_normal(2412 + n_in, n_in) > 0, 1.0, -1.0).astype(np.float32) if signed else None
    eps = 1e-6
    Wd = [dev(W) for W in Ws]
    xd, nwd = dev(x), dev(nw)
    sd = None if s is None else dev(s)
    ys = [torch.full((max(r, 1),), float("nan"), dtype=torch.float32, device="cuda") for r in n_outs]
    B.rmsnorm_fwht_gemv_group(Wd, xd, nwd, sd, ys, n_outs, n_in, eps)
    xq = torch.zeros(n_in // 32 * 36, dtype=torch.uint8, device="cuda")
    B.rmsnorm_fwht_quant(xd, nwd, sd, xq, n_in, 1, eps)
    rs = rms_scale_fp64(x, eps)
    xq_o = O.quantize_q8_1(O.fwht(((x * rs).astype(np.float32) * nw).astype(np.float32), s), True)
    np.testing.assert_array_equal(host(xq), xq_o)
    for W, Wdm, y, r in zip(Ws, Wd, ys, n_outs):
        got = host(y)
        if r == 0:
            assert np.isnan(got).all()
            continue
        assert normwise(got, O.gemv(W, xq_o, r, n_in, nthreads=16)) <= TOL
        y1 = torch.full((r,), float("nan"), dtype=torch.float32, device="cuda")
        B.gemv(Wdm, xq, y1, r, n_in)
        np.testing.assert_array_equal(bits(got), bits(host(y1)))


def test_rmsnorm_fwht_gemv_group_unaligned_x():
    """x 4 bytes past a 16-byte boundary: the generic fused kernel (its own
    fp32 summation order), within the tolerance of the oracle GEMV on the
    same Q8_1 activation."""
    case("rmsnorm_fwht_gemv_group unaligned x 5120")
    n_in, r = 5120, 500
    W = O.gen_weights(2500, r, n_in)
    x = O.gen_normal(2501, n_in + 1)
    nw = O.gen_normal(2502, n_in) * 0.1 + 1
    xbuf = dev(x)
    xv = xbuf[1:]
    y = torch.full((r,), float("nan"), dtype=torch.float32, device="cuda")
    B.rmsnorm_fwht_gemv_group([dev(W)], xv, dev(nw), None, [y], [r], n_in, 1e-6)
    rs = rms_scale_fp64(x[1:], 1e-6)
    xq_o = O.quantize_q8_1(O.fwht(((x[1:] * rs).astype(np.float32) * nw).astype(np.float32)), True)
    assert normwise(host(y), O.gemv(W, xq_o, r, n_in, nthreads=16)) <= TOL


@pytest.mark.parametrize("x_offset", [4, 8])
def test_fwht_gemv_unaligned_x(x_offset):
    case(f"fwht_gemv unaligned x offset {x_offset}")
    n_out, n_in = 300, 5120
    W = O.gen_weights(1700, n_out, n_in)
    x = O.gen_normal(1701, n_in)
    buf, xp = offset_copy(x.view(np.uint8), x_offset)
    y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    B.fwht_gemv(dev(W), xp, None, y, n_out, n_in)
    ref = O.gemv(W, O.quantize_q8_1(O.fwht(x), True), n_out, n_in)
    assert normwise(host(y), ref) <= TOL


# ------------------------------------------------------------------ repack
@pytest.mark.parametrize("n_out,n_in", [(8, 5120), (33, 17408), (5, 1024), (16, 6144)])
def test_repack_bytes_and_gemv_repack(n_out, n_in):
    case(f"repack + gemv_repack {n_out}x{n_in}")
    W = O.gen_weights(1000 + n_in, n_out, n_in, 0.01)
    Wr = torch.zeros(W.size, dtype=torch.uint8, device="cuda")
    B.repack(dev(W), Wr, n_out, n_in)
    Wr_h = host(Wr)
    np.testing.assert_array_equal(Wr_h, O.repack(W, n_out, n_in))
    x = O.fwht(O.gen_normal(1001 + n_in, n_in)) * 1.7
    y = torch.zeros(n_out, dtype=torch.float32, device="cuda")
    B.gemv_repack(Wr, dev(x), y, n_out, n_in)
    assert normwise(host(y), O.gemv_repack(Wr_h, x, n_out, n_in)) <= TOL


@pytest.mark.parametrize("n_out,n_in", [(17408, 5120), (5120, 17408), (6144, 5120), (17407, 5120),
                                        (1023, 6144), (3, 1024), (100, 10240), (77, 12288)])
def test_gemv_repack_streaming(n_out, n_in):
    """The repacked-layout GEMV on the streaming kernel: against the oracle,
    and bit-identical to bonsai_p40_gemv on the original layout with the
    activation quantised by bonsai_p40_quant_activations (same chunk walk,
    same quantiser, same sums)."""
    case(f"gemv_repack streaming {n_out}x{n_in}")
    W = O.gen_weights(1700 + n_out + n_in, n_out, n_in)
    Wd = dev(W)
    Wr = torch.zeros(W.size, dtype=torch.uint8, device="cuda")
    B.repack(Wd, Wr, n_out, n_in)
    x = O.gen_normal(1701 + n_in, n_in) * 1.3
    xd = dev(x)
    y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    B.gemv_repack(Wr, xd, y, n_out, n_in)
    got = host(y)
    assert np.all(np.isfinite(got))
    assert normwise(got, O.gemv(W, O.quantize_q8_1(x, True), n_out, n_in, nthreads=16)) <= TOL
    q = torch.zeros(n_in // 32 * 36, dtype=torch.uint8, device="cuda")
    B.quant_activations(xd, q, n_in)
    y2 = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    B.gemv(Wd, q, y2, n_out, n_in)
    np.testing.assert_array_equal(bits(got), bits(host(y2)))


def test_repack_fixture(golden):
    case("repack fixture 8x5120")
    Wr = torch.zeros(golden["f4_5120_W"].size, dtype=torch.uint8, device="cuda")
    B.repack(dev(golden["f4_5120_W"]), Wr, 8, 5120)
    np.testing.assert_array_equal(host(Wr), golden["f5_Wr"])


# -------------------------------------------------------------------- GEMM
@pytest.mark.parametrize("tag", ["64x256x5", "32x1024x8"])
def test_gemm_fixture(golden, tag):
    case(f"gemm fixture {tag}")
    n_out, n_in, n_tok = map(int, tag.split("x"))
    Y = torch.zeros(n_out * n_tok, dtype=torch.float32, device="cuda")
    B.gemm(dev(golden[f"f6_{tag}_W"]), dev(golden[f"f6_{tag}_Xq"]), Y, n_out, n_in, n_tok)
    assert normwise(host(Y), golden[f"f6_{tag}_Y"]) <= TOL


@pytest.mark.parametrize("n_out,n_in,n_tok", [(96, 1024, 1), (130, 2048, 2), (64, 5120, 4),
                                              (200, 1024, 8), (70, 2048, 13), (17, 17408, 5),
                                              (300, 6144, 16), (70, 1024, 37), (128, 5120, 128),
                                              (33, 384, 65), (40, 384, 3), (50, 1152, 6)])
def test_gemm_matches_oracle(n_out, n_in, n_tok):
    case(f"gemm {n_out}x{n_in}x{n_tok}")
    W = O.gen_weights(1100 + n_out, n_out, n_in, 0.01)
    X = O.gen_normal(1101 + n_tok, n_tok * n_in).reshape(n_tok, n_in)
    Xq = O.quantize_chunk_major(X)
    Y = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
    B.gemm(dev(W), dev(Xq), Y, n_out, n_in, n_tok)
    assert normwise(host(Y), O.gemm(W, Xq, n_out, n_in, n_tok, nthreads=16)) <= TOL


@pytest.mark.parametrize("n_out,n_in,n_tok", [(17408, 5120, 512), (5120, 17408, 512),
                                              (17408, 5120, 2048), (5120, 17408, 2048)])
def test_gemm_prefill_shapes_row_sample(n_out, n_in, n_tok):
    """Config 4: both prefill shapes at M = 512 and 2048 against the oracle
    on the first and last rows and on rows either side of the split launch
    (at M = 2048 the rows of the full 128-token-tile rounds and the rest run
    as two launches)."""
    case(f"gemm prefill {n_out}x{n_in}x{n_tok} (oracle on a row sample)")
    W = O.gen_weights(1200 + n_in, n_out, n_in)
    X = np.stack([O.fwht(O.gen_normal(1201 + t, n_in)) for t in range(n_tok)])
    Xq = O.quantize_chunk_major(X)
    Y = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
    B.gemm(dev(W), dev(Xq), Y, n_out, n_in, n_tok)
    got = host(Y)
    assert np.all(np.isfinite(got))
    cut = 16384 if n_out == 17408 else 4096
    rows = np.r_[0:64, cut - 32:cut + 32, n_out - 64:n_out]
    rb = n_in // 128 * 34
    Ws = np.concatenate([W[r * rb:(r + 1) * rb] for r in rows])
    ref = O.gemm(Ws, Xq, rows.size, n_in, n_tok, nthreads=16)
    assert normwise(got[rows], ref) <= TOL


@pytest.mark.parametrize("n_out,n_in,n_tok", [
    (17408, 5120, 2), (6144, 5120, 3), (1025, 5120, 4), (5120, 6144, 2), (77, 6144, 4),
    (6144, 5120, 2), (4096, 5120, 2), (4095, 5120, 2), (2048, 5120, 2), (34816, 5120, 2),
    (2048, 6144, 2), (6144, 6144, 2), (1024, 6144, 2),
    (333, 1024, 3), (64, 10240, 2), (31, 12288, 2), (17407, 5120, 2), (5120, 17408, 2),
    (301, 17408, 3), (100, 17408, 4), (257, 12288, 4), (5120, 17408, 4)])
def test_gemm_small_batch_streaming(n_out, n_in, n_tok, knobs):
    """With the block-diagonal kernel switched off: 2 tokens run on the
    streaming GEMV kernel with per-token planes (3 on the widths without a
    4x4x4 kernel), 3..4 on the 4x4x4 MFMA kernel (4 on the other widths on
    the 16x16 MFMA kernel): against the oracle, and against one GEMV per
    token (bit-identical for 2 tokens, where the unit shape and the
    arithmetic are the GEMV's)."""
    knobs.set("BONSAI_GEMM_BD", "0")
    case(f"gemm small batch {n_out}x{n_in}x{n_tok}")
    W = O.gen_weights(1400 + n_out + n_tok, n_out, n_in)
    X = np.stack([O.fwht(O.gen_normal(1401 + t + n_in, n_in)) for t in range(n_tok)])
    Xq = O.quantize_chunk_major(X)
    Wd = dev(W)
    Y = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
    B.gemm(Wd, dev(Xq), Y, n_out, n_in, n_tok)
    got = host(Y)
    assert np.all(np.isfinite(got))
    assert normwise(got, O.gemm(W, Xq, n_out, n_in, n_tok, nthreads=16)) <= TOL
    same_units = n_tok == 2
    for t in range(n_tok):
        y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
        B.gemv(Wd, dev(O.quantize_q8_1(X[t], True)), y, n_out, n_in)
        if same_units:
            np.testing.assert_array_equal(bits(got[:, t]), bits(host(y)))
        else:
            assert normwise(got[:, t], host(y)) <= 2 * TOL


@pytest.mark.parametrize("n_out,n_in,n_tok", [
    (17408, 5120, 4), (17408, 5120, 3), (6144, 5120, 4), (5121, 6144, 3), (33, 1024, 4),
    (17407, 5120, 4), (1026, 6144, 4), (7, 5120, 3), (4095, 5120, 4), (4096, 5120, 3)])
def test_gemm_small_batch_mfma4(n_out, n_in, n_tok, knobs):
    """3..4 tokens on the 4x4x4 MFMA streaming kernel (4- and 8-wave
    workgroups either side of 4096 rows; the block-diagonal kernel switched
    off): against the oracle and against one GEMV per token."""
    knobs.set("BONSAI_GEMM_BD", "0")
    case(f"gemm small batch (mfma4) {n_out}x{n_in}x{n_tok}")
    W = O.gen_weights(1600 + n_out + n_tok, n_out, n_in)
    X = np.stack([O.fwht(O.gen_normal(1601 + t + n_in, n_in)) for t in range(n_tok)])
    Xq = O.quantize_chunk_major(X)
    Wd = dev(W)
    Y = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
    B.gemm(Wd, dev(Xq), Y, n_out, n_in, n_tok)
    got = host(Y)
    assert np.all(np.isfinite(got))
    assert normwise(got, O.gemm(W, Xq, n_out, n_in, n_tok, nthreads=16)) <= TOL
    for t in range(n_tok):
        y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
        B.gemv(Wd, dev(O.quantize_q8_1(X[t], True)), y, n_out, n_in)
        assert normwise(got[:, t], host(y)) <= 2 * TOL


@pytest.mark.parametrize("cfg", ["auto", "1", "2", "3", "4", "5"])
@pytest.mark.parametrize("n_out,n_in,n_tok", [
    (17408, 5120, 8), (5120, 17408, 4), (6144, 5120, 5), (1000, 6144, 6), (77, 2048, 7),
    (33, 17408, 3), (5121, 12288, 8), (17, 10240, 4), (17408, 5120, 3), (5120, 6144, 8),
    (5120, 17408, 8), (17407, 5120, 6), (12289, 5120, 7)])
def test_gemm_small_batch_block_diagonal(n_out, n_in, n_tok, cfg, knobs):
    """3..8 tokens on the block-diagonal 16x16x64 MFMA kernel in each of its
    workgroup shapes (16 or 32 rows, K split 2, 4 or 8 ways) and through the
    default choice: against the oracle and against one GEMV per token."""
    if cfg == "auto":
        knobs.unset("BONSAI_GEMM_BD")
    else:
        knobs.set("BONSAI_GEMM_BD", cfg)
    case(f"gemm small batch (block-diagonal cfg {cfg}) {n_out}x{n_in}x{n_tok}")
    W = O.gen_weights(1900 + n_out + n_tok, n_out, n_in)
    X = np.stack([O.fwht(O.gen_normal(1901 + t + n_in, n_in)) for t in range(n_tok)])
    Xq = O.quantize_chunk_major(X)
    Wd = dev(W)
    Y = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
    B.gemm(Wd, dev(Xq), Y, n_out, n_in, n_tok)
    got = host(Y)
    assert np.all(np.isfinite(got))
    assert normwise(got, O.gemm(W, Xq, n_out, n_in, n_tok, nthreads=16)) <= TOL
    for t in range(n_tok):
        y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
        B.gemv(Wd, dev(O.quantize_q8_1(X[t], True)), y, n_out, n_in)
        assert normwise(got[:, t], host(y)) <= 2 * TOL


@pytest.mark.parametrize("xl", ["0", "1", "2", "3"])
@pytest.mark.parametrize("n_out,n_in", [(17408, 5120), (5120, 17408), (6144, 5120), (1000, 5120)])
def test_gemv_xcd_unit_numbering(n_out, n_in, xl, knobs):
    """Every XCD grouping of the unit numbering (2^xl consecutive units per
    XCD) covers each unit once: against the oracle and bit-identical to the
    plain numbering (the unit shape and the arithmetic do not change)."""
    case(f"gemv {n_out}x{n_in} XCD group 2^{xl}")
    W, xq = make(n_out, n_in, 3100 + n_out + n_in)
    Wd, xd = dev(W), dev(xq)
    knobs.set("BONSAI_GEMV_XCD_LOG2M", xl)
    y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    B.gemv(Wd, xd, y, n_out, n_in)
    got = host(y)
    assert normwise(got, O.gemv(W, xq, n_out, n_in, nthreads=16)) <= TOL
    knobs.set("BONSAI_GEMV_XCD_LOG2M", "0")
    y0 = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    B.gemv(Wd, xd, y0, n_out, n_in)
    np.testing.assert_array_equal(bits(got), bits(host(y0)))


# rows of 5120 columns: 2-row units over 2048 waves (one 8-wave workgroup per
# CU), so the last round holds T = 1..4 units per workgroup on these shapes;
# 17407 rows end in a one-row unit inside the tail, 17000 rows leave a last
# round that is not a whole number per workgroup (no shared tail)
@pytest.mark.parametrize("xl", ["0", "3"])
@pytest.mark.parametrize("n_out", [16896, 17407, 17408, 17920, 18432, 17000])
def test_gemv_shared_tail(n_out, xl, knobs):
    """The shared tail (the last round's units dealt slot by slot over every
    wave of the workgroup) is bit-identical to one wave per unit, and both
    match the oracle."""
    n_in = 5120
    case(f"gemv {n_out}x{n_in} shared tail, XCD group 2^{xl}")
    W, xq = make(n_out, n_in, 3300 + n_out)
    Wd, xd = dev(W), dev(xq)
    knobs.set("BONSAI_GEMV_XCD_LOG2M", xl)
    out = {}
    for tail in ("1", "0"):
        knobs.set("BONSAI_GEMV_TAIL", tail)
        y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
        B.gemv(Wd, xd, y, n_out, n_in)
        out[tail] = host(y)
    np.testing.assert_array_equal(bits(out["1"]), bits(out["0"]))
    assert normwise(out["1"], O.gemv(W, xq, n_out, n_in, nthreads=16)) <= TOL


@pytest.mark.parametrize("kind", ["group_gate_up", "group_qkv", "fwht", "rms_group"])
def test_gemv_shared_tail_fused_and_grouped(kind, knobs):
    """The shared tail in the grouped (gate+up: T = 4; q/k/v on 6-wave
    workgroups: T = 2), fused-rotation and RMSNorm-fused launches: bit-identical
    to one wave per unit."""
    n_in = 5120
    n_outs = {"group_gate_up": [17408, 17408], "group_qkv": [5120, 1024, 1024]}.get(kind, [17408])
    case(f"shared tail {kind} {n_outs}x{n_in}")
    Ws = [O.gen_weights(3400 + i, n, n_in) for i, n in enumerate(n_outs)]
    Wd = [dev(W) for W in Ws]
    x = O.gen_normal(3410, n_in)
    xq = dev(O.quantize_q8_1(O.fwht(x), True))
    signs = dev(np.where(O.gen_normal(3411, n_in) < 0, -1.0, 1.0).astype(np.float32))
    nw = dev(O.gen_normal(3412, n_in) * 0.1 + 1)
    out = {}
    for tail in ("1", "0"):
        knobs.set("BONSAI_GEMV_TAIL", tail)
        ys = [torch.full((n,), float("nan"), dtype=torch.float32, device="cuda") for n in n_outs]
        if kind.startswith("group"):
            B.gemv_group(Wd, xq, ys, n_outs, n_in)
        elif kind == "fwht":
            B.fwht_gemv(Wd[0], dev(x), signs, ys[0], n_outs[0], n_in)
        else:
            B.rmsnorm_fwht_gemv_group(Wd, dev(x), nw, signs, ys, n_outs, n_in, 1e-6)
        out[tail] = [host(y) for y in ys]
    for a, b in zip(out["1"], out["0"]):
        assert not np.isnan(a).any()
        np.testing.assert_array_equal(bits(a), bits(b))
    if kind.startswith("group"):
        xqh = O.quantize_q8_1(O.fwht(x), True)
        for W, n, got in zip(Ws, n_outs, out["1"]):
            assert normwise(got, O.gemv(W, xqh, n, n_in, nthreads=16)) <= TOL


def test_gemm_subnormal_and_zero_block_scales():
    """Blocks whose fp16 scale is subnormal or zero (the prefill kernel
    multiplies the scale into its f16 operand)."""
    case("gemm 200x2048x64 with subnormal / zero block scales")
    n_out, n_in, n_tok = 200, 2048, 64
    W = O.gen_weights(1500, n_out, n_in).copy()
    nb = n_in // 128
    rng = np.random.default_rng(3)
    for r in range(n_out):
        for b in rng.choice(nb, 3, replace=False):
            off = (r * nb + b) * 34
            W[off:off + 2] = np.frombuffer(np.uint16(rng.integers(0, 1024)).tobytes(), np.uint8)
    X = O.gen_normal(1501, n_tok * n_in).reshape(n_tok, n_in)
    Xq = O.quantize_chunk_major(X)
    Y = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
    B.gemm(dev(W), dev(Xq), Y, n_out, n_in, n_tok)
    assert normwise(host(Y), O.gemm(W, Xq, n_out, n_in, n_tok, nthreads=16)) <= TOL


@pytest.mark.parametrize("waves", ["16", "8"])
def test_gemm_large_block_scales_with_code3(waves, knobs):
    """Blocks whose fp16 scale has |d| >= 32768 and that hold code 3 (value
    2d, past the fp16 range): the prefill kernel stages d / 2 for them and
    doubles their chunk sums; both workgroup shapes, and the GEMV on the same
    weights."""
    knobs.set("BONSAI_GEMM_F16_WAVES", waves)
    case(f"gemm 200x2048x64 with |d| >= 32768 and code 3 ({waves} waves)")
    n_out, n_in, n_tok = 200, 2048, 64
    W = O.gen_weights(1700, n_out, n_in).copy()
    nb = n_in // 128
    rng = np.random.default_rng(17)
    for r in range(n_out):
        for b in rng.choice(nb, 3 if r % 5 else 0, replace=False):
            off = (r * nb + b) * 34
            bits = np.uint16(rng.integers(0x7800, 0x7C00) | (0x8000 if rng.random() < 0.5 else 0))
            W[off:off + 2] = np.frombuffer(bits.tobytes(), np.uint8)
            W[off + 2:off + 34] = rng.integers(0, 256, 32, dtype=np.uint8)
    _, codes = O.pq2_fields(W)
    assert np.any(codes == 3)
    X = O.gen_normal(1701, n_tok * n_in).reshape(n_tok, n_in)
    Xq = O.quantize_chunk_major(X)
    Y = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
    Wd = dev(W)
    B.gemm(Wd, dev(Xq), Y, n_out, n_in, n_tok)
    got = host(Y)
    assert np.all(np.isfinite(got))
    assert normwise(got, O.gemm(W, Xq, n_out, n_in, n_tok, nthreads=16)) <= TOL
    xq = O.quantize_q8_1(X[0], True)
    y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    B.gemv(Wd, dev(xq), y, n_out, n_in)
    assert normwise(host(y), O.gemv(W, xq, n_out, n_in)) <= TOL


@pytest.mark.parametrize("bn", ["64", "128"])
@pytest.mark.parametrize("n_out,n_in,n_tok", [(1000, 5120, 200), (300, 6144, 77), (129, 1024, 130)])
def test_gemm_token_tile(bn, n_out, n_in, n_tok, knobs):
    """Both token tiles of the prefill kernel on ragged shapes (partial row
    and token tiles), against the oracle."""
    knobs.set("BONSAI_GEMM_F16_BN", bn)
    case(f"gemm {n_out}x{n_in}x{n_tok} token tile {bn}")
    W = O.gen_weights(2800 + n_out, n_out, n_in)
    X = O.gen_normal(2801 + n_tok, n_tok * n_in).reshape(n_tok, n_in)
    Xq = O.quantize_chunk_major(X)
    Y = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
    B.gemm(dev(W), dev(Xq), Y, n_out, n_in, n_tok)
    got = host(Y)
    assert np.all(np.isfinite(got))
    assert normwise(got, O.gemm(W, Xq, n_out, n_in, n_tok, nthreads=16)) <= TOL


@pytest.mark.parametrize("n_out,n_in,n_tok", [(17408, 5120, 512), (5120, 17408, 1024), (17408, 5120, 300)])
def test_gemm_split_last_round(n_out, n_in, n_tok, knobs):
    """Where the 128-token tiles leave a part-filled last round, the rows of
    the full rounds and the remaining rows run as two launches (128- and
    64-token tiles): y is bit-identical to the single launch, and the rows
    either side of the split match the oracle."""
    case(f"gemm {n_out}x{n_in}x{n_tok} split last round")
    W = O.gen_weights(3300 + n_out, n_out, n_in)
    X = np.stack([O.fwht(O.gen_normal(3301 + t, n_in)) for t in range(n_tok)])
    Xq = O.quantize_chunk_major(X)
    Wd, Xd = dev(W), dev(Xq)
    got = {}
    for split in ("1", "0"):
        knobs.set("BONSAI_GEMM_F16_SPLIT", split)
        Y = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
        B.gemm(Wd, Xd, Y, n_out, n_in, n_tok)
        got[split] = host(Y)
    assert np.all(np.isfinite(got["1"]))
    np.testing.assert_array_equal(bits(got["1"]), bits(got["0"]))
    cut = 16384 if n_out == 17408 else 4096
    rows = np.r_[cut - 40:cut + 40]
    rb = n_in // 128 * 34
    Ws = np.concatenate([W[r * rb:(r + 1) * rb] for r in rows])
    ref = O.gemm(Ws, Xq, rows.size, n_in, n_tok, nthreads=16)
    assert normwise(got["1"][rows], ref) <= TOL


@pytest.mark.parametrize("mi", ["8", "5"])
@pytest.mark.parametrize("n_out,n_in,n_tok", [(1000, 5120, 300), (300, 1024, 77), (257, 2048, 513),
                                              (999, 6144, 1000), (40, 256, 17), (161, 17408, 260)])
def test_gemm_wide_kernel(mi, n_out, n_in, n_tok, knobs):
    """The wide prefill kernel (256- or 160-row tiles, 256 tokens) forced on
    ragged shapes: partial row and token tiles, two blocks per row up to 136.
    Bit-identical to the 128-row kernel (both add the chunks' products in K
    order with the same FMA), and against the oracle."""
    case(f"gemm wide kernel {n_out}x{n_in}x{n_tok} ({mi} x 32 rows)")
    W = O.gen_weights(3400 + n_out, n_out, n_in)
    X = np.stack([O.gen_normal(3401 + t, n_in) for t in range(n_tok)])
    if n_in % 1024 == 0:
        X = np.stack([O.fwht(x) for x in X])
    Xq = O.quantize_chunk_major(X)
    Wd, Xd = dev(W), dev(Xq)
    got = {}
    knobs.set("BONSAI_GEMM_WIDE_MI", mi)
    for wide in ("2", "0"):
        knobs.set("BONSAI_GEMM_WIDE", wide)
        Y = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
        B.gemm(Wd, Xd, Y, n_out, n_in, n_tok)
        got[wide] = host(Y)
    assert np.all(np.isfinite(got["2"]))
    np.testing.assert_array_equal(bits(got["2"]), bits(got["0"]))
    assert normwise(got["2"], O.gemm(W, Xq, n_out, n_in, n_tok, nthreads=16)) <= TOL


@pytest.mark.parametrize("n_out,n_in,n_tok", [(17408, 5120, 768), (17408, 5120, 512), (6144, 5120, 2048),
                                              (5120, 6144, 2048), (17408, 5120, 384)])
def test_gemm_default_dispatch_single_round(n_out, n_in, n_tok, knobs):
    """Shapes whose wide tiles fill less than one round of the CUs: the
    default dispatch (one round of 256-row tiles at 17408x5120 M = 768 and
    6144x5120 M = 2048, of 160-row tiles at 17408x5120 M = 512 and
    5120x6144 M = 2048, the LDS kernel at M = 384) is bit-identical to the LDS
    kernel alone and matches the oracle on a row sample."""
    case(f"gemm default dispatch {n_out}x{n_in}x{n_tok}")
    W = O.gen_weights(3600 + n_out + n_tok, n_out, n_in)
    X = np.stack([O.fwht(O.gen_normal(3601 + t, n_in)) for t in range(n_tok)])
    Xq = O.quantize_chunk_major(X)
    Wd, Xd = dev(W), dev(Xq)
    got = {}
    for wide in ("1", "0"):
        knobs.set("BONSAI_GEMM_WIDE", wide)
        Y = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
        B.gemm(Wd, Xd, Y, n_out, n_in, n_tok)
        got[wide] = host(Y)
    assert np.all(np.isfinite(got["1"]))
    np.testing.assert_array_equal(bits(got["1"]), bits(got["0"]))
    rows = np.r_[0:48, n_out // 2 - 24:n_out // 2 + 24, n_out - 48:n_out]
    rb = n_in // 128 * 34
    Ws = np.concatenate([W[r * rb:(r + 1) * rb] for r in rows])
    assert normwise(got["1"][rows], O.gemm(Ws, Xq, rows.size, n_in, n_tok, nthreads=16)) <= TOL


@pytest.mark.parametrize("mi", ["8", "5"])
def test_gemm_wide_kernel_edge_scales(mi, knobs):
    """The wide kernel on blocks with subnormal or zero scales and on blocks
    with |d| >= 32768 holding code 3 (staged as d / 2, a second pass adds the
    other half): against the oracle and bit-identical to the 128-row kernel."""
    case(f"gemm wide kernel 300x2048x300 edge scales ({mi} x 32 rows)")
    n_out, n_in, n_tok = 300, 2048, 300
    W = O.gen_weights(3500, n_out, n_in).copy()
    nb = n_in // 128
    rng = np.random.default_rng(35)
    for r in range(n_out):
        for b in rng.choice(nb, 3, replace=False):
            off = (r * nb + b) * 34
            if r % 3 == 0:
                bits16 = np.uint16(rng.integers(0x7800, 0x7C00) | (0x8000 if rng.random() < 0.5 else 0))
                W[off + 2:off + 34] = rng.integers(0, 256, 32, dtype=np.uint8)
            else:
                bits16 = np.uint16(rng.integers(0, 1024))
            W[off:off + 2] = np.frombuffer(bits16.tobytes(), np.uint8)
    X = O.gen_normal(3501, n_tok * n_in).reshape(n_tok, n_in)
    Xq = O.quantize_chunk_major(X)
    Wd, Xd = dev(W), dev(Xq)
    got = {}
    knobs.set("BONSAI_GEMM_WIDE_MI", mi)
    for wide in ("2", "0"):
        knobs.set("BONSAI_GEMM_WIDE", wide)
        Y = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
        B.gemm(Wd, Xd, Y, n_out, n_in, n_tok)
        got[wide] = host(Y)
    assert np.all(np.isfinite(got["2"]))
    np.testing.assert_array_equal(bits(got["2"]), bits(got["0"]))
    assert normwise(got["2"], O.gemm(W, Xq, n_out, n_in, n_tok, nthreads=16)) <= TOL


def _gemm_pair(Wd, Xd, n_out, n_in, n_tok, dirty=True):
    """Y from bonsai_p40_gemm and from bonsai_p40_gemm_ws (workspace filled
    with 0xFF first, so that nothing stale can pass for converted data)."""
    Y0 = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
    B.gemm(Wd, Xd, Y0, n_out, n_in, n_tok)
    nws = B.gemm_workspace_bytes(n_in, n_tok)
    ws = torch.full((max(nws, 16),), 255 if dirty else 0, dtype=torch.uint8, device="cuda")
    Y1 = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
    B.gemm_ws(Wd, Xd, Y1, n_out, n_in, n_tok, ws)
    return host(Y0), host(Y1)


@pytest.mark.parametrize("mi", ["8", "5"])
@pytest.mark.parametrize("n_out,n_in,n_tok", [(8200, 5120, 300), (8192, 1024, 77), (8193, 2048, 513),
                                              (8211, 6144, 1000), (8192, 256, 17), (8192, 17408, 260)])
def test_gemm_ws_wide_kernel(mi, n_out, n_in, n_tok, knobs):
    """bonsai_p40_gemm_ws with the wide kernel forced on ragged shapes
    (partial row and token tiles): the activation converted once into the
    workspace and DMA'd into the tiles gives Y bit-identical to
    bonsai_p40_gemm's staged conversion."""
    case(f"gemm_ws wide kernel {n_out}x{n_in}x{n_tok} ({mi} x 32 rows)")
    W = O.gen_weights(3700 + n_out, n_out, n_in)
    X = np.stack([O.gen_normal(3701 + t, n_in) for t in range(n_tok)])
    Xq = O.quantize_chunk_major(X)
    knobs.set("BONSAI_GEMM_WIDE_MI", mi)
    knobs.set("BONSAI_GEMM_WIDE", "2")
    y0, y1 = _gemm_pair(dev(W), dev(Xq), n_out, n_in, n_tok)
    assert np.all(np.isfinite(y1))
    np.testing.assert_array_equal(bits(y1), bits(y0))
    rows = np.r_[0:64, n_out - 64:n_out]
    rb = n_in // 128 * 34
    Ws = np.concatenate([W[r * rb:(r + 1) * rb] for r in rows])
    assert normwise(y1[rows], O.gemm(Ws, Xq, rows.size, n_in, n_tok, nthreads=16)) <= TOL


@pytest.mark.parametrize("mi", ["8", "5"])
def test_gemm_ws_edge_scales(mi, knobs):
    """The workspace path on subnormal, zero and |d| >= 32768 block scales
    (the second pass over the big blocks restarts the activation DMA):
    bit-identical to bonsai_p40_gemm."""
    case(f"gemm_ws wide kernel 8200x2048x300 edge scales ({mi} x 32 rows)")
    n_out, n_in, n_tok = 8200, 2048, 300
    W = O.gen_weights(3500, n_out, n_in).copy()
    nb = n_in // 128
    rng = np.random.default_rng(36)
    for r in range(n_out):
        for b in rng.choice(nb, 3, replace=False):
            off = (r * nb + b) * 34
            if r % 3 == 0:
                bits16 = np.uint16(rng.integers(0x7800, 0x7C00) | (0x8000 if rng.random() < 0.5 else 0))
                W[off + 2:off + 34] = rng.integers(0, 256, 32, dtype=np.uint8)
            else:
                bits16 = np.uint16(rng.integers(0, 1024))
            W[off:off + 2] = np.frombuffer(bits16.tobytes(), np.uint8)
    X = O.gen_normal(3502, n_tok * n_in).reshape(n_tok, n_in)
    Xq = O.quantize_chunk_major(X)
    knobs.set("BONSAI_GEMM_WIDE_MI", mi)
    knobs.set("BONSAI_GEMM_WIDE", "2")
    y0, y1 = _gemm_pair(dev(W), dev(Xq), n_out, n_in, n_tok)
    assert np.all(np.isfinite(y1))
    np.testing.assert_array_equal(bits(y1), bits(y0))


@pytest.mark.parametrize("n_out,n_in,n_tok", [(17408, 5120, 2048), (5120, 17408, 2048), (17408, 5120, 512),
                                              (6144, 5120, 2048), (17408, 5120, 384), (4096, 5120, 16)])
def test_gemm_ws_default_dispatch(n_out, n_in, n_tok):
    """The default dispatch with a workspace on the prefill shapes (wide
    tiles and the 128-row kernel for the rows they leave, one round of
    160-row tiles, the LDS kernel alone at M = 384, the small-batch path at
    16 tokens): bit-identical to bonsai_p40_gemm, called twice on one
    workspace, and a NULL workspace runs bonsai_p40_gemm."""
    case(f"gemm_ws default dispatch {n_out}x{n_in}x{n_tok}")
    W = O.gen_weights(3800 + n_tok, n_out, n_in)
    X = np.stack([O.fwht(O.gen_normal(3801 + t, n_in)) for t in range(n_tok)])
    Xq = O.quantize_chunk_major(X)
    Wd, Xd = dev(W), dev(Xq)
    y0, y1 = _gemm_pair(Wd, Xd, n_out, n_in, n_tok)
    assert np.all(np.isfinite(y1))
    np.testing.assert_array_equal(bits(y1), bits(y0))
    y0b, y1b = _gemm_pair(Wd, Xd, n_out, n_in, n_tok, dirty=False)
    np.testing.assert_array_equal(bits(y1b), bits(y0))
    Y2 = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
    B.gemm_ws(Wd, Xd, Y2, n_out, n_in, n_tok, None, 0)
    np.testing.assert_array_equal(bits(host(Y2)), bits(y0))


def test_gemm_equals_gemv_per_token():
    case("gemm n_tok=3 equals three gemv")
    n_out, n_in, n_tok = 300, 5120, 3
    W = O.gen_weights(1300, n_out, n_in)
    X = np.stack([O.fwht(O.gen_normal(1301 + t, n_in)) for t in range(n_tok)])
    Xq = O.quantize_chunk_major(X)
    Y = torch.zeros((n_out, n_tok), dtype=torch.float32, device="cuda")
    Wd = dev(W)
    B.gemm(Wd, dev(Xq), Y, n_out, n_in, n_tok)
    got = host(Y)
    for t in range(n_tok):
        xq = O.quantize_q8_1(X[t], True)
        y = torch.zeros(n_out, dtype=torch.float32, device="cuda")
        B.gemv(Wd, dev(xq), y, n_out, n_in)
        assert normwise(got[:, t], host(y)) <= 2 * TOL


# -------------------------------------------------------- config-1 FFN chain
def test_ffn_chain_config1():
    case("FFN chain gate/up 17408x5120 -> swiglu_fwht_quant -> down 5120x17408")
    n_embd, n_ff = 5120, 17408
    Wg = O.gen_weights(1400, n_ff, n_embd)
    Wu = O.gen_weights(1401, n_ff, n_embd)
    Wd = O.gen_weights(1402, n_embd, n_ff)
    x = O.gen_normal(1403, n_embd)
    xq = torch.zeros(n_embd // 32 * 36, dtype=torch.uint8, device="cuda")
    B.fwht_quant(dev(x), None, xq, n_embd)
    g = torch.zeros(n_ff, dtype=torch.float32, device="cuda")
    u = torch.zeros(n_ff, dtype=torch.float32, device="cuda")
    B.gemv(dev(Wg), xq, g, n_ff, n_embd)
    B.gemv(dev(Wu), xq, u, n_ff, n_embd)
    hq = torch.zeros(n_ff // 32 * 36, dtype=torch.uint8, device="cuda")
    B.swiglu_fwht_quant(g, u, None, hq, n_ff)
    y = torch.zeros(n_embd, dtype=torch.float32, device="cuda")
    B.gemv(dev(Wd), hq, y, n_embd, n_ff)
    # oracle chain, stage by stage: each GPU stage is compared with the oracle
    # applied to the GPU's own input of that stage
    xq_o = O.quantize_q8_1(O.fwht(x), True)
    assert np.array_equal(host(xq), xq_o)
    g_h, u_h = host(g), host(u)
    assert normwise(g_h, O.gemv(Wg, xq_o, n_ff, n_embd, 16)) <= TOL
    assert normwise(u_h, O.gemv(Wu, xq_o, n_ff, n_embd, 16)) <= TOL
    hq_h = host(hq)
    hq_o = O.quantize_q8_1(O.fwht(O.swiglu(g_h, u_h)), True)
    _, _, q1 = O.q81_fields(hq_h)
    _, _, q2 = O.q81_fields(hq_o)
    assert np.max(np.abs(q1.astype(int) - q2.astype(int))) <= 1     # device vs glibc expf ulps
    assert np.mean(q1 != q2) < 1e-3
    assert normwise(host(y), O.gemv(Wd, hq_h, n_embd, n_ff, 16)) <= TOL
    # end to end against the all-oracle chain: the Q8_1 re-quantisation of h
    # turns 1e-6 differences in g, u into occasional +-1 steps of q, so the
    # bound here is the quantisation noise level, not the fp32 tolerance
    hq_full = O.quantize_q8_1(O.fwht(O.swiglu(O.gemv(Wg, xq_o, n_ff, n_embd, 16),
                                                O.gemv(Wu, xq_o, n_ff, n_embd, 16))), True)
    assert normwise(host(y), O.gemv(Wd, hq_full, n_embd, n_ff, 16)) <= 2e-3


# ------------------------------------------- RMSNorm -> FWHT -> Q8_1 pre-pass
FWHT_ROWS = np.array([(((l ^ (l >> 2)) & 1) | ((((l >> 1) ^ (l >> 2)) & 1) << 1) |
                       ((((l >> 2) ^ (l >> 3)) & 1) << 2) | (l & 0x38)) for l in range(64)])


def rms_sumsq_canonical(x: np.ndarray) -> float:
    """The kernels' one summation order of the fp64 sum of squares: per
    1024-block, lane l adds the (exact) squares of its 16 elements
    16 row(l) + r in order, the 64 lane sums meet in a balanced tree in lane
    order (the DPP moves and readlanes of the wave sum), and the block sums
    are added in block order."""
    tot = 0.0
    for b in range(x.size // 1024):
        lanes = x[1024 * b:1024 * (b + 1)].astype(np.float64).reshape(64, 16)[FWHT_ROWS]
        s = np.zeros(64)
        for r in range(16):
            s = s + lanes[:, r] * lanes[:, r]
        while s.size > 1:
            s = s[0::2] + s[1::2]
        tot = tot + s[0]
    return tot


def rms_scale_fp64(x: np.ndarray, eps: float) -> np.float32:
    """The fused kernels' scale: the canonical fp64 sum of squares, then
    1 / sqrtf(float(ss / n) + eps) in fp32 (each step correctly rounded)."""
    m = np.float32(rms_sumsq_canonical(x) / x.size)
    return np.float32(1.0) / np.sqrt(np.float32(m + np.float32(eps)))


def test_rms_sum_order_is_one_order():
    """Every normalising path adds the squares in the same order, so they
    agree byte for byte even on a row whose fp64 sum of squares depends on
    the order (values over 24 decades): the per-block pre-pass (few
    tokens), the per-token pre-pass (many tokens), the grouped GEMV with the
    norm inside (its y equals the GEMV of the pre-pass output) and the
    emulation of the canonical order."""
    case("rms sum order: per-block, per-token, fused GEMV, n=5120")
    n, eps = 5120, 1e-6
    g = O.gen_normal(2900, n)
    x = (g * np.power(10.0, (O.gen_normal(2901, n) * 4).clip(-12, 12))).astype(np.float32)
    x64 = x.astype(np.float64) ** 2
    assert np.sum(x64) != rms_sumsq_canonical(x) or np.sum(x64[::-1]) != rms_sumsq_canonical(x)
    w = O.gen_normal(2902, n) * 0.1 + 1
    xq1 = torch.zeros(n // 32 * 36, dtype=torch.uint8, device="cuda")
    B.rmsnorm_fwht_quant(dev(x), dev(w), None, xq1, n, 1, eps)                 # per-block kernel
    n_tok = 1000                                                               # per-token kernel
    X = np.tile(x, (n_tok, 1))
    xqn = torch.zeros(n // 32 * 36 * n_tok, dtype=torch.uint8, device="cuda")
    B.rmsnorm_fwht_quant(dev(X), dev(w), None, xqn, n, n_tok, eps)
    got_n = host(xqn).reshape(n // 32, n_tok, 36)[:, 0, :].reshape(-1)
    s = rms_scale_fp64(x, eps)
    exp = O.quantize_q8_1(O.fwht(((x * s).astype(np.float32) * w).astype(np.float32)), True)
    np.testing.assert_array_equal(host(xq1), exp)
    np.testing.assert_array_equal(got_n, exp)
    W = O.gen_weights(2903, 1024, n)
    y_fused = torch.zeros(1024, dtype=torch.float32, device="cuda")
    B.rmsnorm_fwht_gemv_group([dev(W)], dev(x), dev(w), None, [y_fused], [1024], n, eps)
    y_two = torch.zeros(1024, dtype=torch.float32, device="cuda")
    B.gemv_group([dev(W)], xq1, [y_two], [1024], n)
    np.testing.assert_array_equal(host(y_fused).view(np.uint32), host(y_two).view(np.uint32))


def chunk_major(blocks):
    """Token-major Q8_1 rows -> chunk-major (block (c, t) at c * n_tok + t)."""
    B_ = np.stack([b.reshape(-1, 36) for b in blocks], axis=1)
    return B_.reshape(-1)


@pytest.mark.parametrize("n,n_tok,use_signs", [
    (1024, 1, False), (5120, 1, False), (5120, 1, True), (17408, 1, True),
    (5120, 3, True), (17408, 2, False), (32768, 1, False),
    (1024, 4100, False), (2048, 2100, True)])      # the last two: one workgroup per token
def test_rmsnorm_fwht_quant_bit_exact(n, n_tok, use_signs):
    """Byte-exact against the host FWHT and quantiser applied to
    (x * s) * w with the kernel's fp64-sum scale s."""
    case(f"rmsnorm_fwht_quant n={n} n_tok={n_tok} signs={use_signs}")
    X = (O.gen_normal(2100 + n + n_tok, n_tok * n) * 2.5).reshape(n_tok, n)
    w = O.gen_normal(2101 + n, n) * 0.1 + 1
    signs = (np.where(O.gen_normal(2102 + n, n) < 0, -1, 1)).astype(np.float32) if use_signs else None
    eps = 1e-6
    xq = torch.full((n // 32 * 36 * n_tok,), 0xAB, dtype=torch.uint8, device="cuda")
    B.rmsnorm_fwht_quant(dev(X), dev(w), dev(signs) if use_signs else None, xq, n, n_tok, eps)
    s = np.array([rms_scale_fp64(X[t], eps) for t in range(n_tok)], np.float32)
    Y = ((X * s[:, None]).astype(np.float32) * w).astype(np.float32)
    if use_signs:
        Y = (Y * signs).astype(np.float32)
    q = O.quantize_q8_1(O.fwht(Y.reshape(-1)), True)          # blocks are independent
    exp = q.reshape(n_tok, n // 32, 36).transpose(1, 0, 2).reshape(-1)
    np.testing.assert_array_equal(host(xq), exp)


@pytest.mark.parametrize("n,n_tok", [(5120, 1), (1024, 4100)])
def test_rmsnorm_fwht_quant_unaligned(n, n_tok):
    """x and w one float past a 16-byte boundary (scalar loads), per-block and
    per-token kernels: byte-exact against the same emulation."""
    case(f"rmsnorm_fwht_quant unaligned n={n} n_tok={n_tok}")
    X = (O.gen_normal(2700 + n, n_tok * n) * 2).reshape(n_tok, n)
    w = O.gen_normal(2701 + n, n) * 0.1 + 1
    xb = torch.zeros(n_tok * n + 4, dtype=torch.float32, device="cuda")
    wb = torch.zeros(n + 4, dtype=torch.float32, device="cuda")
    xb[1:1 + n_tok * n] = dev(X.reshape(-1))
    wb[1:1 + n] = dev(w)
    xq = torch.full((n // 32 * 36 * n_tok,), 0xAB, dtype=torch.uint8, device="cuda")
    B.rmsnorm_fwht_quant(xb.data_ptr() + 4, wb.data_ptr() + 4, None, xq, n, n_tok, 1e-6)
    s = np.array([rms_scale_fp64(X[t], 1e-6) for t in range(n_tok)], np.float32)
    Y = ((X * s[:, None]).astype(np.float32) * w).astype(np.float32)
    q = O.quantize_q8_1(O.fwht(Y.reshape(-1)), True)
    exp = q.reshape(n_tok, n // 32, 36).transpose(1, 0, 2).reshape(-1)
    np.testing.assert_array_equal(host(xq), exp)


def test_rmsnorm_fwht_quant_against_reference_order():
    """Against the reference's own chain (sequential fp32 sum of squares,
    src/ops.h:13-22): the scales differ by that sum's rounding, so a few q
    move by one step; d and every other byte agree."""
    case("rmsnorm_fwht_quant vs sequential-sum chain, 4 x 17408")
    n, n_tok, eps = 17408, 4, 1e-6
    X = (O.gen_normal(2200, n_tok * n) * 1.5).reshape(n_tok, n)
    w = O.gen_normal(2201, n) * 0.1 + 1
    xq = torch.zeros(n // 32 * 36 * n_tok, dtype=torch.uint8, device="cuda")
    B.rmsnorm_fwht_quant(dev(X), dev(w), None, xq, n, n_tok, eps)
    ref = chunk_major([O.quantize_q8_1(O.fwht(O.rmsnorm(X[t], w, eps)), True) for t in range(n_tok)])
    d_g, s_g, q_g = O.q81_fields(host(xq))
    d_r, s_r, q_r = O.q81_fields(ref)
    assert np.max(np.abs(d_g.astype(np.int32) - d_r.astype(np.int32))) <= 1        # fp16 ulps
    dq = np.abs(q_g.astype(np.int32) - q_r.astype(np.int32))
    assert dq.max() <= 1 and np.count_nonzero(dq) <= 1e-3 * dq.size
    assert np.max(np.abs(s_g.astype(np.int32) - s_r.astype(np.int32))) <= 32


def test_rmsnorm_fwht_quant_feeds_gemv():
    """One token through the fused pre-pass then the GEMV equals the GEMV of
    the emulated Q8_1 bit for bit."""
    case("rmsnorm_fwht_quant -> gemv 6144x5120")
    n_out, n = 6144, 5120
    x = O.gen_normal(2300, n) * 3
    w = O.gen_normal(2301, n) * 0.1 + 1
    W = O.gen_weights(2302, n_out, n)
    xq = torch.zeros(n // 32 * 36, dtype=torch.uint8, device="cuda")
    B.rmsnorm_fwht_quant(dev(x), dev(w), None, xq, n, 1, 1e-6)
    y = torch.zeros(n_out, dtype=torch.float32, device="cuda")
    B.gemv(dev(W), xq, y, n_out, n)
    s = rms_scale_fp64(x, 1e-6)
    xq_e = O.quantize_q8_1(O.fwht(((x * s).astype(np.float32) * w).astype(np.float32)), True)
    y2 = torch.zeros(n_out, dtype=torch.float32, device="cuda")
    B.gemv(dev(W), dev(xq_e), y2, n_out, n)
    np.testing.assert_array_equal(host(y).view(np.uint32), host(y2).view(np.uint32))


# ----------------------------------------------------------------- rmsnorm
def test_rmsnorm():
    case("rmsnorm 3x5120")
    n_rows, n = 3, 5120
    x = O.gen_normal(1500, n_rows * n).reshape(n_rows, n)
    w = O.gen_normal(1501, n) * 0.1 + 1
    y = torch.zeros((n_rows, n), dtype=torch.float32, device="cuda")
    B.rmsnorm(dev(x), dev(w), y, n_rows, n, 1e-6)
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(host(y), ref, rtol=2e-6, atol=1e-6)


# ------------------------------------------------------------------ probes
@pytest.mark.parametrize("n_out,n_in", [(17408, 5120), (5120, 17408), (300, 5120), (7, 17408)])
def test_unit_dma_probe_runs(n_out, n_in):
    """The GEMV's DMA-only skeleton runs to completion on the GEMV's shapes
    (full grid and a grid smaller than the CU count) and leaves its sink
    untouched."""
    case(f"unit_dma_probe {n_out}x{n_in}")
    W = torch.randint(0, 256, (n_out * (n_in // 128) * 34,), dtype=torch.uint8, device="cuda")
    sink = torch.zeros(4096, dtype=torch.int32, device="cuda")
    for _ in range(3):
        B.unit_dma_probe(W, n_out, n_in, sink)
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0
