"""GPU tests whose expected values are exact integers or exact bytes.

* Integer chunk dots through the public GEMV/GEMM entry points: every block
  scale is fp16 1.0 and every activation chunk holds a +-127, so the Q8_1
  scale is exactly 1.0 and q equals the integer input.  Y[r, t] is then the
  sum of the int32 chunk dots sum_k (code - 1) * q (src/pq2_0.h:149-172,
  tests/test_p40.cpp:449-470), an integer below 2^24, which every kernel must
  return exactly whatever its summation order.  The expected values come from
  a float64 product of the un-permuted codes and inputs (exact for integers
  this size), not from the oracle's restatement.  Each kernel the dispatcher
  can pick is reached (decode GEMV and its fallbacks, the 2..16-token
  streaming and MFMA kernels, the f16-MFMA prefill tile GEMM with both token
  tiles and the split last round at M = 2048, the int8-MFMA tile GEMMs).
* The Q8_1 scale encode on exact fp16 ties (amax / 127 halfway between two
  fp16 values): bytes equal the host's ties-away encode.
* The reference ternary quantiser / dequantiser on the device against the F9
  fixture and the oracle.
"""
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


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def unit_scale_weights(seed, n_out, n_in, p3=0.05):
    """PQ2_0 weights with every block scale fp16 1.0 (codes as generated,
    with a share of code 3)."""
    W = O.gen_weights(seed, n_out, n_in, p3).copy()
    blk = W.reshape(-1, 34)
    blk[:, 0] = 0x00
    blk[:, 1] = 0x3C
    return W


def integer_tokens(seed, n_tok, n_in):
    """[n_tok, n_in] integers in [-127, 127], each 32-chunk holding a +-127:
    the Q8_1 scale is 127 / 127 = 1 and q = x exactly."""
    rng = np.random.default_rng(seed)
    X = rng.integers(-127, 128, size=(n_tok, n_in)).astype(np.float32)
    pos = rng.integers(0, 32, size=(n_tok, n_in // 32))
    sgn = np.where(rng.random((n_tok, n_in // 32)) < 0.5, 127.0, -127.0).astype(np.float32)
    Xc = X.reshape(n_tok, n_in // 32, 32)
    np.put_along_axis(Xc, pos[..., None], sgn[..., None], axis=2)
    return X


def exact_product(W, X, rows, n_in):
    """sum_k (code[r, k] - 1) * X[t, k] for the given rows, float64 (exact)."""
    nb = n_in // 128
    rb = nb * 34
    Ws = np.concatenate([W[r * rb:(r + 1) * rb] for r in rows])
    _, codes = O.pq2_fields(Ws)
    C = codes.reshape(len(rows), n_in).astype(np.float64) - 1.0
    return C @ X.astype(np.float64).T


def check_exact(got, W, X, rows, n_in):
    ref = exact_product(W, X, rows, n_in)
    assert np.max(np.abs(ref)) < 2 ** 24
    g = got[rows]
    if not np.array_equal(g.astype(np.float64), ref):
        bad = np.argwhere(g.astype(np.float64) != ref)
        r, t = bad[0]
        raise AssertionError(f"{len(bad)} outputs differ; first row {rows[r]} token {t}: "
                             f"got {g[r, t]!r}, exact {ref[r, t]!r}")


def run_gemm(W, X, n_out, n_in, n_tok, w_offset=0, x_offset=0):
    Xq = O.quantize_chunk_major(X)
    d, _, _ = O.q81_fields(Xq)
    assert np.all(d == 0x3C00)                       # every activation scale is exactly 1
    wbuf = torch.zeros(W.size + 64, dtype=torch.uint8, device="cuda")
    wbuf[w_offset:w_offset + W.size] = dev(W)
    xbuf = torch.zeros(Xq.size + 64, dtype=torch.uint8, device="cuda")
    xbuf[x_offset:x_offset + Xq.size] = dev(Xq)
    Y = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
    B.gemm(wbuf.data_ptr() + w_offset, xbuf.data_ptr() + x_offset, Y, n_out, n_in, n_tok)
    return host(Y)


def sample_rows(n_out, cuts=()):
    rows = set(range(min(48, n_out))) | set(range(max(0, n_out - 48), n_out))
    for c in cuts:
        rows |= set(range(max(0, c - 40), min(n_out, c + 40)))
    return np.array(sorted(rows))


# (n_out, n_in, n_tok, env, w_offset, x_offset): each row reaches one kernel
EXACT_CASES = [
    # decode GEMV: streaming kernel on the model widths, generic widths, 2-byte offset W
    (17408, 5120, 1, {}, 0, 0),
    (5120, 17408, 1, {}, 0, 0),
    (5120, 5120, 1, {}, 0, 0),
    (1024, 5120, 1, {}, 0, 0),
    (300, 3072, 1, {}, 0, 0),
    (77, 384, 1, {}, 0, 0),
    (65, 5120, 1, {}, 2, 0),
    # 2 tokens: per-token planes on the streaming kernel
    (17408, 5120, 2, {}, 0, 0),
    (5120, 17408, 2, {}, 0, 0),
    # 3..8 tokens: block-diagonal 16x16x64 int8 MFMA (default), every shape
    (17408, 5120, 3, {}, 0, 0),
    (5120, 17408, 8, {}, 0, 0),
    (17408, 5120, 8, {"BONSAI_GEMM_BD": "2"}, 0, 0),
    (1000, 6144, 5, {"BONSAI_GEMM_BD": "3"}, 0, 0),
    (333, 5120, 7, {"BONSAI_GEMM_BD": "4"}, 0, 0),
    # 3..4 tokens without it: the 4x4x4 MFMA streaming kernel
    (17408, 5120, 4, {"BONSAI_GEMM_BD": "0"}, 0, 0),
    (6144, 5120, 3, {"BONSAI_GEMM_BD": "0"}, 0, 0),
    # 5..16 tokens: the streamed 16x16x32 int8 MFMA kernel
    (17408, 5120, 13, {}, 0, 0),
    (5120, 17408, 16, {}, 0, 0),
    (300, 5120, 9, {"BONSAI_GEMM_SMALL_CFG": "3"}, 0, 0),
    # <= 16 tokens with an unaligned X: the skinny kernel
    (200, 5120, 6, {"BONSAI_GEMM_BD": "0"}, 0, 4),
    # f16-MFMA prefill tile GEMM: 64- and 128-token tiles, ragged edges
    (1000, 5120, 17, {}, 0, 0),
    (300, 6144, 77, {"BONSAI_GEMM_F16_BN": "128"}, 0, 0),
    (129, 1024, 130, {"BONSAI_GEMM_F16_BN": "64"}, 0, 0),
    (17408, 5120, 512, {}, 0, 0),
    (5120, 17408, 512, {}, 0, 0),
    # the f16 tile GEMM on an odd block count (zero-scale padding step) and a
    # 2-byte offset W
    (70, 384, 65, {}, 0, 0),
    (90, 1024, 40, {}, 2, 0),
    # the int8-MFMA tile GEMMs: 2-byte loads (odd block count, offset W) and
    # both aligned tile shapes
    (70, 384, 65, {"BONSAI_GEMM_KERNEL": "1"}, 0, 0),
    (90, 1024, 40, {"BONSAI_GEMM_KERNEL": "1"}, 2, 0),
    (256, 5120, 20, {"BONSAI_GEMM_KERNEL": "1"}, 0, 0),
    (256, 5120, 100, {"BONSAI_GEMM_KERNEL": "1"}, 0, 0),
]


@pytest.mark.parametrize("n_out,n_in,n_tok,env,w_offset,x_offset", EXACT_CASES)
def test_integer_chunk_dots_exact(n_out, n_in, n_tok, env, w_offset, x_offset, knobs):
    for k, v in env.items():
        knobs.set(k, v)
    case(f"exact integer gemm {n_out}x{n_in}x{n_tok} env={env} W+{w_offset} X+{x_offset}")
    W = unit_scale_weights(5000 + n_out + n_tok, n_out, n_in)
    X = integer_tokens(5001 + n_in + n_tok, n_tok, n_in)
    got = run_gemm(W, X, n_out, n_in, n_tok, w_offset, x_offset)
    assert np.all(np.isfinite(got))
    check_exact(got, W, X, sample_rows(n_out), n_in)


@pytest.mark.parametrize("n_out,n_in", [(17408, 5120), (5120, 17408)])
def test_integer_chunk_dots_exact_prefill_2048(n_out, n_in):
    """Config 4 at M = 2048 (the split two-launch path of the prefill GEMM):
    exact sums on rows either side of the split and at both ends."""
    n_tok = 2048
    case(f"exact integer gemm prefill {n_out}x{n_in}x{n_tok}")
    W = unit_scale_weights(5100 + n_out, n_out, n_in)
    X = integer_tokens(5101 + n_in, n_tok, n_in)
    got = run_gemm(W, X, n_out, n_in, n_tok)
    assert np.all(np.isfinite(got))
    cut = 16384 if n_out == 17408 else 4096
    check_exact(got, W, X, sample_rows(n_out, (cut,)), n_in)


# ------------------------------------------------------------- fp16 ties
def tie_chunks(seed):
    """32-element chunks whose amax / 127 is exactly halfway between two fp16
    values (normal binades and the subnormal range), with random signs and
    random other elements."""
    rng = np.random.default_rng(seed)
    ds = []
    for e in range(-14, 16):
        for m in rng.choice(1023, 6, replace=False):
            ds.append((1.0 + (2 * int(m) + 1) / 2048.0) * 2.0 ** e)
    for k in rng.choice(1023, 40, replace=False):
        ds.append((int(k) + 0.5) * 2.0 ** -24)
    ds = np.array(ds, np.float64)
    amax = (ds * 127.0).astype(np.float32)
    assert np.all(amax.astype(np.float64) == ds * 127.0)              # exact in fp32
    assert np.all((amax / np.float32(127.0)).astype(np.float64) == ds)  # the device's d
    X = (rng.random((ds.size, 32)) * 2 - 1).astype(np.float32) * amax[:, None]
    pos = rng.integers(0, 32, ds.size)
    X[np.arange(ds.size), pos] = np.where(rng.random(ds.size) < 0.5, amax, -amax)
    return X.ravel(), amax / np.float32(127.0)


def test_q8_1_scale_fp16_ties():
    case("Q8_1 quantisers on exact fp16 ties of amax/127")
    x, d = tie_chunks(77)
    n = x.size
    away = np.array([O.f32_to_f16(v) for v in d], np.uint16)
    rne = d.astype(np.float16).view(np.uint16)
    assert np.sum(away != rne) >= 100                 # the ties-away branch is exercised
    ref = O.quantize_q8_1(x, True)
    dref, _, _ = O.q81_fields(ref)
    assert np.array_equal(dref, away)
    q = torch.zeros(n // 32 * 36, dtype=torch.uint8, device="cuda")
    B.quant_activations(dev(x), q, n)
    np.testing.assert_array_equal(host(q), ref)
    # chunk-major token quantiser, several token rows
    n_tok, k = 4, 32 * 64
    xs = np.resize(x, n_tok * k).reshape(n_tok, k)
    Xq = torch.zeros(k // 32 * n_tok * 36, dtype=torch.uint8, device="cuda")
    B.quant_tokens(dev(xs), None, Xq, k, n_tok, False)
    np.testing.assert_array_equal(host(Xq), O.quantize_chunk_major(xs))


# ------------------------------------------- ternary quantiser / dequantiser
def test_quantize_pq2_0_fixture(golden):
    case("quantize_pq2_0 / dequantize_pq2_0 F9 fixture")
    x = golden["f9_x"]
    w = torch.zeros(x.size // 128 * 34, dtype=torch.uint8, device="cuda")
    B.quantize_pq2_0(dev(x), w, x.size)
    np.testing.assert_array_equal(host(w), golden["f9_w"])
    wd = golden["f9_wd"]
    y = torch.full((wd.size // 34 * 128,), float("nan"), dtype=torch.float32, device="cuda")
    B.dequantize_pq2_0(dev(wd), y, y.numel())
    np.testing.assert_array_equal(bits(host(y)), bits(golden["f9_deq"]))


@pytest.mark.parametrize("n,w_offset", [(17408 * 128, 0), (1000 * 128, 2), (128, 0)])
def test_quantize_pq2_0_seeded(n, w_offset):
    case(f"quantize_pq2_0 n={n} W offset {w_offset}")
    x = O.gen_normal(5200 + n, n, 0.02)
    x[::997] *= 40.0                                   # a few large weights per block set
    wbuf = torch.zeros(n // 128 * 34 + 64, dtype=torch.uint8, device="cuda")
    wp = wbuf.data_ptr() + w_offset
    B.quantize_pq2_0(dev(x), wp, n)
    got = host(wbuf)[w_offset:w_offset + n // 128 * 34]
    ref = O.quantize_pq2_0(x)
    np.testing.assert_array_equal(got, ref)
    y = torch.full((n,), float("nan"), dtype=torch.float32, device="cuda")
    B.dequantize_pq2_0(wp, y, n)
    np.testing.assert_array_equal(bits(host(y)), bits(O.dequantize_pq2_0(ref, n)))
