"""Weight matrices of 2 GiB and more, through the C ABI.

Past 2 GiB the streaming GEMV kernels can no longer give the DMA a buffer
descriptor whose range is the matrix: they switch to 64-bit addresses and clamp a
trailing unit's pieces to the end of W themselves.  The small-batch kernels
for 3..16 tokens address W with unsigned 32-bit per-lane offsets, which must
hold up to 4 GiB.  From 4 GiB on, those kernels are skipped and the others
(per-token planes, 4x4x4 MFMA, the skinny kernel, the prefill tile GEMM) use
64-bit offsets.

The matrices are filled on the device (random code bytes, random finite fp16
block scales), so only a row sample goes to the host: the first rows, rows on
both sides of the 2 GiB and 4 GiB byte boundaries, the middle, the last rows
(an odd row count, so the last unit is partial) and seeded random rows.  Those
rows are checked against the oracle at the fp32 tolerance of the path (1e-5 of
the sample's max |y|), and every output must be finite (written)."""
import numpy as np
import pytest

import bonsai_p40 as B
from oracle import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-5
GIB = 1 << 30


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    B.lib()   # fail loudly if the native library is missing
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def case(msg):
    print(f"[case] {msg}", flush=True)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def device_weights(seed, n_out, n_in):
    """PQ2_0 rows made on the device: random code bytes, fp16 block scales in
    [0.001, 0.05)."""
    nb = n_in // 128
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    W = torch.randint(0, 256, (n_out * nb * 34,), dtype=torch.uint8, device="cuda", generator=g)
    scales = (torch.rand(n_out, nb, device="cuda", generator=g) * 0.049 + 0.001).half()
    W.view(n_out, nb, 34)[:, :, 0:2] = scales.view(torch.uint8).view(n_out, nb, 2)
    del scales
    torch.cuda.synchronize()
    return W


def sample_rows(n_out, rs, seed):
    rows = set(range(32)) | set(range(n_out - 33, n_out)) | set(range(n_out // 2 - 16, n_out // 2 + 16))
    for edge in (2 * GIB, 4 * GIB):
        b = edge // rs
        if b < n_out:
            rows |= set(range(max(0, b - 24), min(n_out, b + 24)))
    rng = np.random.default_rng(seed)
    rows |= set(int(r) for r in rng.integers(0, n_out, 64))
    return np.array(sorted(rows), dtype=np.int64)


def host_rows(W, n_out, rs, rows):
    return W.view(n_out, rs)[torch.from_numpy(rows).cuda()].cpu().numpy().ravel()


def rel_err(got, ref):
    return float(np.max(np.abs(got.astype(np.float64) - ref.astype(np.float64)))) / max(float(np.max(np.abs(ref))), 1e-30)


# (n_out, n_in): 5120-column rows just past 2 GiB, 17408-column rows just past
# 2 GiB, and 5120-column rows past 4 GiB; odd row counts
SHAPES = {"2g_5120": (1_600_001, 5120), "2g_17408": (470_001, 17408), "4g_5120": (3_200_001, 5120)}


@pytest.fixture(scope="module")
def mats():
    cache = {}

    def get(key):
        if key not in cache:
            cache.clear()                     # one large matrix at a time
            torch.cuda.empty_cache()
            n_out, n_in = SHAPES[key]
            cache[key] = device_weights(9700 + len(key) + n_out % 97, n_out, n_in)
        return cache[key]
    yield get
    cache.clear()
    torch.cuda.empty_cache()


def check_gemv_rows(y, W, n_out, n_in, xq, seed):
    rs = 34 * (n_in // 128)
    assert bool(torch.isfinite(y).all()), "an output was not written"
    rows = sample_rows(n_out, rs, seed)
    ref = O.gemv(host_rows(W, n_out, rs, rows), xq, len(rows), n_in, nthreads=16)
    got = y[torch.from_numpy(rows).cuda()].cpu().numpy()
    err = rel_err(got, ref)
    assert err <= TOL, f"sampled rows: rel err {err:.3g}"


@pytest.mark.parametrize("key", ["2g_5120", "2g_17408", "4g_5120"])
def test_gemv_large_matrix(mats, key):
    n_out, n_in = SHAPES[key]
    rs = 34 * (n_in // 128)
    assert n_out * rs >= 2 * GIB
    case(f"large GEMV {n_out}x{n_in} ({n_out * rs / GIB:.2f} GiB)")
    W = mats(key)
    assert W.numel() == n_out * rs
    x = O.gen_normal(9801, n_in)
    xq = O.quantize_q8_1(O.fwht(x), True)
    y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    B.gemv(W, dev(xq), y, n_out, n_in)
    check_gemv_rows(y, W, n_out, n_in, xq, 9802)
    if n_in % 1024 == 0:
        # the fused FWHT + Q8_1 + GEMV and the one-launch Q8_1 + GEMV stream the same units
        case(f"large fused FWHT GEMV {n_out}x{n_in}")
        y.fill_(float("nan"))
        B.fwht_gemv(W, dev(x.astype(np.float32)), None, y, n_out, n_in)
        check_gemv_rows(y, W, n_out, n_in, xq, 9803)
        case(f"large one-launch Q8_1 GEMV {n_out}x{n_in}")
        y.fill_(float("nan"))
        B.quant_gemv(W, dev(x.astype(np.float32)), y, n_out, n_in)
        check_gemv_rows(y, W, n_out, n_in, O.quantize_q8_1(x, True), 9804)


@pytest.mark.parametrize("key,n_tok", [("2g_5120", t) for t in (2, 3, 4, 6, 8, 12, 64)] +
                         [("4g_5120", t) for t in (2, 3, 8, 16, 40)] + [("2g_17408", 2), ("2g_17408", 8)])
def test_gemm_large_matrix(mats, key, n_tok):
    n_out, n_in = SHAPES[key]
    rs = 34 * (n_in // 128)
    case(f"large GEMM {n_out}x{n_in} ({n_out * rs / GIB:.2f} GiB), {n_tok} tokens")
    W = mats(key)
    assert W.numel() == n_out * rs
    X = np.stack([O.fwht(O.gen_normal(9900 + t, n_in)) for t in range(n_tok)])
    Xq = O.quantize_chunk_major(X)
    assert Xq.size == (n_in // 32) * n_tok * 36
    Y = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
    B.gemm(W, dev(Xq), Y, n_out, n_in, n_tok)
    assert bool(torch.isfinite(Y).all()), "an output was not written"
    rows = sample_rows(n_out, rs, 9950 + n_tok)
    ref = O.gemm(host_rows(W, n_out, rs, rows), Xq, len(rows), n_in, n_tok, nthreads=16)
    got = Y[torch.from_numpy(rows).cuda()].cpu().numpy()
    err = rel_err(got, ref.reshape(len(rows), n_tok))
    assert err <= TOL, f"sampled rows: rel err {err:.3g}"
