"""Rows far wider than the model's, through the C ABI.

Widths past the shape-specialised kernels take the runtime-shaped streaming
kernel while its unit fits (up to 17 sixteen-byte pieces per lane: 65536
columns), then the wave-per-row kernel.  The fused FWHT / Q8_1 GEMVs stage
the whole Q8_1 activation (36 bytes per 32 columns) in a workgroup's LDS less
1 KiB for their partial sums: 144384 columns fit MI355X's 160 KiB, 145408 do
not, and that call must return 1 and launch nothing.  The quantisers, the
int32 chunk dots, the GEMV, the fused and RMSNorm-fused GEMVs and the GEMM
(2 ... 40 tokens) are checked at these widths: bytes and int32 dots exactly,
fp32 outputs within 1e-5 of the oracle.  The chunk-major token quantiser is
checked at its token limit (65535, one grid row per token)."""
import numpy as np
import pytest

import bonsai_p40 as B
from oracle import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-5
N_OUT = 333
WIDTHS = [32768, 65536, 130048, 144384, 145408, 262144]
FUSED_MAX = 144384


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


def rel_err(got, ref):
    return float(np.max(np.abs(got.astype(np.float64) - ref.astype(np.float64)))) / max(float(np.max(np.abs(ref))), 1e-30)


def fused_fits(n_in):
    props = torch.cuda.get_device_properties(0)
    return n_in // 32 * 36 <= props.shared_memory_per_block - 1024


def test_fused_width_limit_matches_the_device():
    """The documented limit is the device's: on MI355X 144384 columns fit."""
    assert fused_fits(FUSED_MAX) and not fused_fits(FUSED_MAX + 1024)


@pytest.mark.parametrize("n_in", WIDTHS)
def test_wide_quantisers_and_chunk_dots(n_in):
    case(f"wide rows: quantisers and int32 chunk dots, {N_OUT}x{n_in}")
    x = O.gen_normal(10_000 + n_in % 997, n_in)
    xq = torch.empty(B.q8_bytes(n_in), dtype=torch.uint8, device="cuda")
    B.quant_activations(dev(x), xq, n_in)
    ref_q = O.quantize_q8_1(x, True)
    assert np.array_equal(host(xq), ref_q)
    B.fwht_quant(dev(x), None, xq, n_in)
    assert np.array_equal(host(xq), O.quantize_q8_1(O.fwht(x), True))
    W = O.gen_weights(10_100 + n_in % 991, N_OUT, n_in, p3=0.01)
    out = torch.empty(N_OUT * n_in // 32, dtype=torch.int32, device="cuda")
    B.chunk_dots(dev(W), dev(ref_q), out, N_OUT, n_in)
    assert np.array_equal(host(out).reshape(-1), O.chunk_dots(W, ref_q, N_OUT, n_in).reshape(-1))


@pytest.mark.parametrize("n_in", WIDTHS)
def test_wide_gemv_and_fused(n_in):
    case(f"wide rows: GEMV, fused FWHT GEMV, one-launch Q8_1 GEMV, {N_OUT}x{n_in}")
    W = O.gen_weights(10_200 + n_in % 983, N_OUT, n_in)
    Wd = dev(W)
    x = O.gen_normal(10_300 + n_in % 977, n_in)
    xq = O.quantize_q8_1(O.fwht(x), True)
    y = torch.full((N_OUT,), float("nan"), dtype=torch.float32, device="cuda")
    B.gemv(Wd, dev(xq), y, N_OUT, n_in)
    ref = O.gemv(W, xq, N_OUT, n_in, nthreads=16)
    assert rel_err(host(y), ref) <= TOL
    xd = dev(x.astype(np.float32))
    if n_in <= FUSED_MAX:
        y.fill_(float("nan"))
        B.fwht_gemv(Wd, xd, None, y, N_OUT, n_in)
        assert rel_err(host(y), ref) <= TOL
        y.fill_(float("nan"))
        B.quant_gemv(Wd, xd, y, N_OUT, n_in)
        assert rel_err(host(y), O.gemv(W, O.quantize_q8_1(x, True), N_OUT, n_in, nthreads=16)) <= TOL
    else:
        # the activation does not fit in LDS: invalid argument, nothing launched
        y.fill_(7.0)
        assert B.call("bonsai_p40_fwht_gemv", Wd, xd, None, y, N_OUT, n_in) == 1
        assert B.call("bonsai_p40_quant_gemv", Wd, xd, y, N_OUT, n_in) == 1
        with pytest.raises(B.BonsaiError, match="returned 1"):
            B.fwht_gemv_group([Wd], xd, None, [y], [N_OUT], n_in)
        with pytest.raises(B.BonsaiError, match="returned 1"):
            B.rmsnorm_fwht_gemv_group([Wd], xd, xd, None, [y], [N_OUT], n_in, 1e-6)
        assert bool((y == 7.0).all()), "a rejected call wrote its output"


@pytest.mark.parametrize("n_in", [65536, FUSED_MAX])
def test_wide_rmsnorm_fused_group(n_in):
    """The RMSNorm-fused grouped GEMV quantises the same Q8_1 as the device
    pre-pass (the sum of squares is added in one order everywhere)."""
    case(f"wide rows: RMSNorm-fused grouped GEMV, 2 x {N_OUT}x{n_in}")
    Ws = [O.gen_weights(10_400 + k, N_OUT, n_in) for k in range(2)]
    x = O.gen_normal(10_410, n_in) * 3
    nw = O.gen_normal(10_411, n_in) * 0.1 + 1
    xd, nwd = dev(x.astype(np.float32)), dev(nw.astype(np.float32))
    xq = torch.empty(B.q8_bytes(n_in), dtype=torch.uint8, device="cuda")
    B.rmsnorm_fwht_quant(xd, nwd, None, xq, n_in, 1, 1e-6)
    xq_h = host(xq)
    ys = [torch.full((N_OUT,), float("nan"), dtype=torch.float32, device="cuda") for _ in range(2)]
    B.rmsnorm_fwht_gemv_group([dev(W) for W in Ws], xd, nwd, None, ys, [N_OUT, N_OUT], n_in, 1e-6)
    for W, y in zip(Ws, ys):
        assert rel_err(host(y), O.gemv(W, xq_h, N_OUT, n_in, nthreads=16)) <= TOL


@pytest.mark.parametrize("n_in,n_tok", [(32768, t) for t in (2, 3, 6, 16, 40)] +
                         [(FUSED_MAX, t) for t in (2, 6, 16, 40)] + [(262144, 8)])
def test_wide_gemm(n_in, n_tok):
    case(f"wide rows: GEMM {N_OUT}x{n_in}, {n_tok} tokens")
    W = O.gen_weights(10_500 + n_in % 971 + n_tok, N_OUT, n_in)
    X = np.stack([O.fwht(O.gen_normal(10_600 + t, n_in)) for t in range(n_tok)])
    Xq = O.quantize_chunk_major(X)
    Y = torch.full((N_OUT, n_tok), float("nan"), dtype=torch.float32, device="cuda")
    B.gemm(dev(W), dev(Xq), Y, N_OUT, n_in, n_tok)
    got = host(Y)
    assert np.all(np.isfinite(got))
    ref = O.gemm(W, Xq, N_OUT, n_in, n_tok, nthreads=16).reshape(N_OUT, n_tok)
    assert rel_err(got, ref) <= TOL


@pytest.mark.parametrize("rotate", [1, 0])
def test_token_quantiser_at_its_token_limit(rotate):
    """bonsai_p40_quant_tokens runs one grid row per token: 65535 tokens are
    the most it takes (bytes exact), 65536 return 1 and write nothing."""
    n, n_tok = 1024, 65535
    case(f"chunk-major token quantiser, {n_tok} tokens of {n}, rotate={rotate}")
    X = O.gen_normal(10_700 + rotate, n * n_tok).reshape(n_tok, n)
    Xd = dev(X.astype(np.float32))
    Xq = torch.empty(B.q8_bytes(n, n_tok), dtype=torch.uint8, device="cuda")
    B.quant_tokens(Xd, None, Xq, n, n_tok, bool(rotate))
    ref = O.quantize_chunk_major(O.fwht(X.ravel()).reshape(n_tok, n) if rotate else X)
    assert np.array_equal(host(Xq), ref)
    big = torch.zeros((n_tok + 1) * n, dtype=torch.float32, device="cuda")
    out = torch.full((B.q8_bytes(n, n_tok + 1),), 0x5A, dtype=torch.uint8, device="cuda")
    assert B.call("bonsai_p40_quant_tokens", big, None, out, n, n_tok + 1, rotate) == 1
    assert bool((out == 0x5A).all()), "a rejected call wrote its output"
