"""Seeded random shapes through the GEMV, one-launch, fused and GEMM entry
points against the oracle: widths with and without a streaming kernel, row
counts from 1 up, 2..257 tokens, so that every dispatch boundary is crossed
by some case.  Bar: the fp32 tolerance of the path (1e-5), measured against
max |y| where enough outputs make that representative, else against the
largest row's sum of |contributions| (a lone output can cancel to far below
its terms, and then its relative error says nothing about the kernel)."""
import random

import numpy as np
import pytest

import bonsai_p40 as B
from oracle import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-5
WIDTHS = [128, 256, 640, 1024, 1152, 2048, 3072, 5120, 6144, 10240, 17408]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def contribution_scale(W, xq, n_out, n_in):
    """max over rows of sum over chunks |dw * da * chunk dot| (the reference's terms)."""
    nb = n_in // 128
    dots = O.chunk_dots(W, xq, n_out, n_in).astype(np.float64).reshape(n_out, n_in // 32)
    dw = W.reshape(n_out, nb, 34)[:, :, :2].copy().view(np.float16).astype(np.float64).reshape(n_out, nb)
    da = xq.reshape(n_in // 32, 36)[:, :2].copy().view(np.float16).astype(np.float64).ravel()
    return float(np.abs(dots * np.repeat(dw, 4, axis=1) * da[None, :]).sum(axis=1).max())


def rel_err(got, ref, scale=None):
    s = scale if scale is not None else max(float(np.max(np.abs(ref))), 1e-30)
    return float(np.max(np.abs(got.astype(np.float64) - ref.astype(np.float64)))) / max(s, 1e-30)


def cases(seed, n):
    rng = random.Random(seed)
    out = []
    while len(out) < n:
        kind = rng.choice(["gemv", "quant_gemv", "fwht_gemv", "gemm"])
        n_in = rng.choice(WIDTHS if kind in ("gemv", "gemm") else [w for w in WIDTHS if w % 1024 == 0])
        n_out = rng.choice([1, 7, 64, 129, 333, 1024, 2047, 4096, 6144, rng.randint(1, 9000)])
        n_tok = rng.choice([2, 3, 4, 5, 8, 11, 16, 17, 64, 130]) if kind == "gemm" else 1
        if n_out * n_in * n_tok > 6144 * 5120 * 8:
            continue
        out.append((kind, n_out, n_in, n_tok, rng.randint(0, 1 << 30)))
    return out


@pytest.mark.parametrize("kind,n_out,n_in,n_tok,seed", cases(20261202, 64))
def test_random_shape(kind, n_out, n_in, n_tok, seed):
    print(f"case {kind} {n_out}x{n_in} tokens {n_tok} seed {seed}", flush=True)
    W = O.gen_weights(seed, n_out, n_in)
    if kind == "gemm":
        X = np.stack([O.fwht(O.gen_normal(seed + 2 + t, n_in)) if n_in % 1024 == 0
                      else O.gen_normal(seed + 2 + t, n_in) for t in range(n_tok)])
        Xq = O.quantize_chunk_major(X)
        Y = torch.full((n_out, n_tok), float("nan"), dtype=torch.float32, device="cuda")
        B.gemm(dev(W), dev(Xq), Y, n_out, n_in, n_tok)
        got = host(Y)
        assert np.all(np.isfinite(got))
        ref = O.gemm(W, Xq, n_out, n_in, n_tok, nthreads=16)
        scale = None
        if n_out * n_tok < 64:
            scale = max(contribution_scale(W, O.quantize_q8_1(X[t], True), n_out, n_in) for t in range(n_tok))
        assert rel_err(got, ref, scale) <= TOL
        return
    x = O.gen_normal(seed + 1, n_in)
    y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    if kind == "gemv":
        xq = O.quantize_q8_1(x, True)
        B.gemv(dev(W), dev(xq), y, n_out, n_in)
    elif kind == "quant_gemv":
        xq = O.quantize_q8_1(x, True)
        B.quant_gemv(dev(W), dev(x), y, n_out, n_in)
    else:
        xq = O.quantize_q8_1(O.fwht(x), True)
        B.fwht_gemv(dev(W), dev(x), None, y, n_out, n_in)
    got = host(y)
    assert np.all(np.isfinite(got))
    ref = O.gemv(W, xq, n_out, n_in, nthreads=16)
    scale = contribution_scale(W, xq, n_out, n_in) if n_out < 64 else None
    assert rel_err(got, ref, scale) <= TOL
