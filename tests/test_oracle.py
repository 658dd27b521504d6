"""CPU tests: pin the oracle (oracle/pq2_oracle.c) before it is trusted.

Each oracle function is checked against (a) the golden fixtures written from
the reference's own compiled host code (tests/golden/golden.npz), (b) the live
compiled reference oracle/_ref where it was built, and (c) what the
mathematics fixes independently of any restatement: the naive Sylvester
matrix, brute-force integer dots over the un-permuted layout, a
double-precision dequantised GEMM, involutions and round trips.
"""
import numpy as np
import pytest

from oracle import oracle as O

HAS_REF = O.ref() is not None


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


# ---------------------------------------------------------------- fp16 (F1)
def test_f16_encode_edge_cases(golden):
    got = np.array([O.f32_to_f16(float(v)) for v in golden["f1_in"]], np.uint16)
    np.testing.assert_array_equal(got, golden["f1_out"])


def test_f16_encode_exhaustive_hash(golden):
    # all 2^32 float bit patterns, hashed (FNV-1a over the 16-bit codes)
    h = O.lib().orc_f16_encode_hash(0, 1 << 32, 1)
    assert h == int(golden["f1_hash_all"][0])


def test_f16_decode_all_patterns(golden):
    got = np.array([O.f16_to_f32(h) for h in range(65536)], np.float32)
    np.testing.assert_array_equal(bits(got), bits(golden["f1_decode_all"]))


def test_f16_ties_round_away():
    # 1 + 2^-11 is halfway between 1 and 1 + 2^-10: host rounds away (up)
    assert O.f32_to_f16(1.0 + 2.0 ** -11) == 0x3C01
    assert O.f32_to_f16(-(1.0 + 2.0 ** -11)) == 0xBC01
    assert O.f32_to_f16(65520.0) == 0x7C00          # rounds up into inf


# ---------------------------------------------------------------- Q8_1 (F2)
@pytest.mark.parametrize("name", ["seeded", "special", "k32"])
def test_q8_1_fixtures(golden, name):
    x = golden[f"f2_{name}_in"]
    np.testing.assert_array_equal(O.quantize_q8_1(x, True), golden[f"f2_{name}_perm"])
    np.testing.assert_array_equal(O.quantize_q8_1(x, False), golden[f"f2_{name}_plain"])


def test_q8_1_permutation_is_involution_and_fields():
    x = O.gen_normal(5, 1024) * 3
    qp, qn = O.quantize_q8_1(x, True), O.quantize_q8_1(x, False)
    j = np.arange(32)
    perm = 16 * (j >> 4) + 4 * (j & 3) + ((j >> 2) & 3)
    assert np.array_equal(perm[perm], j)                       # involution
    dp, sp, qsp = O.q81_fields(qp)
    dn, sn, qsn = O.q81_fields(qn)
    assert np.array_equal(qsp, qsn[:, perm])
    assert np.array_equal(sp, qsn.astype(np.int32).sum(1))     # s = raw sum of q
    # amax element maps to +-127 and d = fp16(amax / 127)
    xc = x.reshape(-1, 32)
    amax = np.abs(xc).max(1)
    assert np.all(np.abs(qsn.astype(int)).max(1) == 127)
    assert np.array_equal(dn, np.array([O.f32_to_f16(np.float32(a) / np.float32(127)) for a in amax]))


# ---------------------------------------------------------------- FWHT (F3)
def test_fwht_fixture_bits(golden):
    assert np.array_equal(bits(O.fwht(golden["f3_in"])), bits(golden["f3_out"]))
    assert np.array_equal(bits(O.fwht(golden["f3_in"], golden["f3_signs"])),
                          bits(golden["f3_out_signed"]))


def test_fwht_equals_sylvester_matrix():
    x = O.gen_normal(7, 1024)
    i = np.arange(1024)
    pc = np.vectorize(lambda v: bin(v).count("1"))(i[:, None] & i[None, :]) & 1
    H = np.where(pc == 1, -1.0, 1.0) / 32.0
    np.testing.assert_allclose(O.fwht(x), H @ x.astype(np.float64), rtol=0, atol=2e-6)
    y = O.fwht(O.fwht(x))                                      # orthonormal involution
    np.testing.assert_allclose(y, x, rtol=0, atol=1e-5)


def test_fwht_signs_per_block():
    # signs are a length-n vector: block b uses signs[1024b:1024b+1024]
    x = O.gen_normal(8, 2048)
    s = np.where(O.gen_normal(9, 2048) > 0, 1.0, -1.0).astype(np.float32)
    a = O.fwht(x, s)
    b = O.fwht(x * s)
    assert np.array_equal(bits(a), bits(b))


# -------------------------------------------------------- chunk dot (F4)
@pytest.mark.parametrize("k", [5120, 17408])
def test_chunk_dots_fixture(golden, k):
    W, xq = golden[f"f4_{k}_W"], golden[f"f4_{k}_xq"]
    got = O.chunk_dots(W, xq, 8, k)
    np.testing.assert_array_equal(got, golden[f"f4_{k}_sumi"])


@pytest.mark.parametrize("k", [5120, 17408])
def test_row_dot_fixture_bits(golden, k):
    y = O.gemv(golden[f"f4_{k}_W"], golden[f"f4_{k}_xq"], 8, k)
    assert np.array_equal(bits(y), bits(golden[f"f4_{k}_y"]))


def test_chunk_dot_brute_force_plain_layout():
    # sum (code-1) * q over the UN-permuted activation must equal the
    # permuted dp4a formulation for every chunk (src/pq2_0.h:149-177)
    n_out, k = 4, 1024
    W = O.gen_weights(11, n_out, k, 0.05)
    x = O.gen_normal(12, k) * 2
    qp, qn = O.quantize_q8_1(x, True), O.quantize_q8_1(x, False)
    _, codes = O.pq2_fields(W)
    codes = codes.reshape(n_out, k).astype(np.int64)
    _, _, qs = O.q81_fields(qn)
    q = qs.reshape(-1).astype(np.int64)
    brute = ((codes - 1) * q[None, :]).reshape(n_out, k // 32, 32).sum(-1)
    np.testing.assert_array_equal(O.chunk_dots(W, qp, n_out, k), brute)


def test_gemv_double_precision_reference():
    n_out, k = 16, 2048
    W = O.gen_weights(13, n_out, k)
    xq = O.quantize_q8_1(O.fwht(O.gen_normal(14, k)), True)
    dw, codes = O.pq2_fields(W)
    dwf = np.array([O.f16_to_f32(h) for h in dw], np.float64).reshape(n_out, k // 128)
    da, _, _ = O.q81_fields(xq)
    daf = np.array([O.f16_to_f32(h) for h in da], np.float64)
    S = O.chunk_dots(W, xq, n_out, k).astype(np.float64)
    ref = (S * np.repeat(dwf, 4, axis=1) * daf[None, :]).sum(1)
    y = O.gemv(W, xq, n_out, k)
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))


# ------------------------------------------------------------ repack (F5)
def test_repack_fixture_and_round_trip(golden):
    W = golden["f4_5120_W"]
    Wr = O.repack(W, 8, 5120)
    np.testing.assert_array_equal(Wr, golden["f5_Wr"])
    np.testing.assert_array_equal(O.unpack(Wr, 8, 5120), W)
    y = np.array([O.lib().orc_repack_row_dot(O._p(Wr[r * 1360:], O._u8p),
                                            O._p(golden["f4_5120_xq"], O._u8p), 40)
                  for r in range(8)], np.float32)
    assert np.array_equal(bits(y), bits(golden["f5_y"]))


def test_repack_rejects_bad_widths():
    W = O.gen_weights(15, 2, 128 * 12)
    with pytest.raises(ValueError):
        O.repack(W, 2, 128 * 12)


# -------------------------------------------------------------- GEMM (F6)
@pytest.mark.parametrize("tag", ["64x256x5", "32x1024x8"])
def test_gemm_fixture(golden, tag):
    n_out, n_in, n_tok = map(int, tag.split("x"))
    W, X, Xq, Y = (golden[f"f6_{tag}_{s}"] for s in ("W", "X", "Xq", "Y"))
    np.testing.assert_array_equal(O.quantize_chunk_major(X), Xq)
    got = O.gemm(W, Xq, n_out, n_in, n_tok)
    assert np.array_equal(bits(got.ravel()), bits(Y))


def test_gemm_vs_dequantised_double():
    n_out, n_in, n_tok = 24, 512, 6
    W = O.gen_weights(16, n_out, n_in, 0.01)
    X = O.gen_normal(17, n_tok * n_in).reshape(n_tok, n_in)
    Xq = O.quantize_chunk_major(X)
    wd = np.stack([O.dequantize_pq2_0(W[r * (n_in // 128) * 34:], n_in) for r in range(n_out)]).astype(np.float64)
    blk = Xq.reshape(n_in // 32, n_tok, 36)
    xd = np.zeros((n_in, n_tok))
    j = np.arange(32)
    perm = 16 * (j >> 4) + 4 * (j & 3) + ((j >> 2) & 3)
    for c in range(n_in // 32):
        for t in range(n_tok):
            d, _, qs = O.q81_fields(blk[c, t].copy())
            xd[c * 32 + perm, t] = qs[0].astype(np.float64) * O.f16_to_f32(d[0])
    ref = wd @ xd
    got = O.gemm(W, Xq, n_out, n_in, n_tok)
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))


# ------------------------------------------------------------ SwiGLU (F7)
def test_swiglu_chain(golden):
    h = O.swiglu(golden["f7_gate"], golden["f7_up"])
    np.testing.assert_allclose(h, golden["f7_h"], rtol=2e-6, atol=1e-7)
    assert np.array_equal(O.quantize_q8_1(O.fwht(golden["f7_h"]), True), golden["f7_hq"])


# ------------------------------------------------------------ RMSNorm (F8)
@pytest.mark.parametrize("n", [3072, 1024])
def test_rmsnorm_fixture(golden, n):
    x, w, eps = golden[f"f8_{n}_x"], golden[f"f8_{n}_w"], float(golden[f"f8_{n}_eps"])
    y = O.rmsnorm(x, w, eps)
    np.testing.assert_array_equal(y.view(np.uint32), golden[f"f8_{n}_y"].view(np.uint32))
    assert np.array_equal(O.quantize_q8_1(O.fwht(y), True), golden[f"f8_{n}_yq"])


def test_rmsnorm_closed_form_and_planted_mistakes():
    """Against the float64 formula; a missing eps, a sum over n-1 elements
    or a mean taken as the plain sum must each fail the same check."""
    n, eps = 4096, 1e-2
    x = O.gen_normal(901, n) * 0.05                  # mean(x^2) ~ eps: eps matters
    w = O.gen_normal(902, n) * 0.1 + 1
    x64 = x.astype(np.float64)
    exact = x64 / np.sqrt((x64 ** 2).mean() + eps) * w
    tol = lambda y: np.max(np.abs(y - exact)) / np.max(np.abs(exact))   # noqa: E731
    assert tol(O.rmsnorm(x, w, eps)) < 1e-5
    assert tol(x64 / np.sqrt((x64 ** 2).mean()) * w) > 1e-3
    assert tol(x64 / np.sqrt((x64[:-16] ** 2).sum() / n + eps) * w) > 1e-5
    assert tol(x64 / np.sqrt((x64 ** 2).sum() + eps) * w) > 1e-3


# ------------------------------- ternary quantiser / dequantiser / dot (F9)
def test_quantize_pq2_0_fixture(golden):
    """Bytes of quantize_row_pq2_0 (src/pq2_0.h:74-90) on weight-like and
    edge-case blocks: +-0.5 products (lroundf ties), zero blocks, an fp16-tie
    scale, subnormal and overflowing scales."""
    np.testing.assert_array_equal(O.quantize_pq2_0(golden["f9_x"]), golden["f9_w"])


def test_quantize_pq2_0_closed_form():
    """Independent of the restatement: d = fp16(amax) rounded half away,
    code = clamp(round_half_away(x / amax) + 1, 0, 3) with the reciprocal
    taken once in fp32; planted mistakes (RNE rounding, no +1 bias, d =
    amax / 2) must fail the same comparison."""
    x = np.concatenate([O.gen_normal(17, 4096, 0.02),
                        np.repeat(np.float32([2.0, 1.0, -1.0, 0.5]), 32)])
    w = O.quantize_pq2_0(x)
    d, codes = O.pq2_fields(w)
    xb = x.reshape(-1, 128)
    amax = np.max(np.abs(xb), axis=1)
    assert np.array_equal(d, [O.f32_to_f16(a) for a in amax])
    inv = np.where(amax > 0, np.float32(1.0) / amax, np.float32(0)).astype(np.float32)
    prod = (xb * inv[:, None]).astype(np.float32)
    away = np.trunc(prod + np.copysign(0.5, prod)).astype(np.int64)   # exact for |prod| <= 1
    ref = np.clip(away + 1, 0, 3)
    assert np.array_equal(codes, ref)
    assert np.any(prod == 0.5) and np.any(prod == -0.5)               # the tie cases are present
    assert not np.array_equal(codes, np.clip(np.rint(prod).astype(np.int64) + 1, 0, 3))
    assert not np.array_equal(codes, np.clip(away, 0, 3))
    half = [O.f32_to_f16(a / 2) for a in amax]
    assert not np.array_equal(d, half)


def test_dequantize_pq2_0_fixture_and_closed_form(golden):
    """dequantize_row_pq2_0 (src/pq2_0.h:62-71) bit patterns, incl. code 3
    (+2d) rows, and the value rule (code - 1) * d from the decoded fields."""
    wd = golden["f9_wd"]
    y = O.dequantize_pq2_0(wd, wd.size // 34 * 128)
    np.testing.assert_array_equal(bits(y), bits(golden["f9_deq"]))
    d, codes = O.pq2_fields(wd)
    assert np.any(codes == 3)
    dv = np.array([O.f16_to_f32(h) for h in d], np.float32)
    ref = (codes.astype(np.float32) - 1) * dv[:, None]
    np.testing.assert_array_equal(bits(y), bits(ref.ravel()))
    assert not np.array_equal(bits(y), bits((codes.astype(np.float32) * dv[:, None]).ravel()))


def test_pq2_0_dot_f32_fixture_and_closed_form(golden):
    """pq2_0_dot_f32 (src/pq2_0.h:134-142) bit patterns, and within fp32
    rounding of the double-precision dot of the dequantised block; a
    dropped "- 1" or a missing scale must fail the same check."""
    wd, a = golden["f9_wd"], golden["f9_a"]
    got = O.pq2_0_dot_f32(wd, a)
    np.testing.assert_array_equal(bits(got), bits(golden["f9_dot"]))
    d, codes = O.pq2_fields(wd)
    dv = np.array([O.f16_to_f32(h) for h in d], np.float64)
    a2 = a.reshape(-1, 128).astype(np.float64)
    exact = ((codes.astype(np.float64) - 1) * a2).sum(axis=1) * dv
    fin = np.isfinite(exact)
    scale = np.abs(codes - 1.0) @ np.ones(128) * np.max(np.abs(a2), axis=1) * np.abs(dv) + 1e-30
    err = np.abs(got[fin] - exact[fin]) / scale[fin]
    assert np.max(err) < 1e-6
    no_bias = (codes.astype(np.float64) * a2).sum(axis=1) * dv
    assert np.max(np.abs(no_bias[fin] - exact[fin]) / scale[fin]) > 1e-3
    no_scale = ((codes.astype(np.float64) - 1) * a2).sum(axis=1)
    assert np.max(np.abs(no_scale[fin] - exact[fin]) / scale[fin]) > 1e-3


# ------------------------------------------------- planted-mistake checks
def test_checks_detect_planted_mistakes(golden):
    """The fixture comparisons must fail for plausible oracle mistakes."""
    k = 5120
    W, xq, sumi = golden[f"f4_{k}_W"], golden[f"f4_{k}_xq"], golden[f"f4_{k}_sumi"]
    got = O.chunk_dots(W, xq, 8, k)
    d, s, _ = O.q81_fields(xq)
    dropped_bias = got + s[None, :].astype(np.int32)         # forgot "- s"
    assert not np.array_equal(dropped_bias, sumi)
    unpermuted = O.chunk_dots(W, O.quantize_q8_1(O.fwht(O.gen_normal(1105, k)), False), 8, k)
    assert not np.array_equal(unpermuted, sumi)
    rne = np.array([np.float16(v).view(np.uint16) for v in golden["f1_in"]], np.uint16)
    assert not np.array_equal(rne, golden["f1_out"])        # RNE != host ties-away


# ------------------------------------------------ live compiled reference
@pytest.mark.skipif(not HAS_REF, reason="oracle/_ref not built (no reference tree)")
def test_live_reference_agrees_on_seeded_configs():
    R = O.ref()
    for k, n_out, seed in ((5120, 32, 201), (17408, 8, 202), (6144, 16, 203)):
        W = O.gen_weights(seed, n_out, k)
        x = O.gen_normal(seed + 1, k)
        xr = np.array(x)
        R.ref_fwht_blocks(O._p(xr, O._f32p), None, k)
        assert np.array_equal(bits(O.fwht(x)), bits(xr))
        q = O.quantize_q8_1(xr, True)
        qr = np.empty_like(q)
        R.ref_quantize_q8_1(O._p(xr, O._f32p), O._p(qr, O._u8p), k, 1)
        assert np.array_equal(q, qr)
        yr = np.empty(n_out, np.float32)
        R.ref_gemv(O._p(W, O._u8p), O._p(q, O._u8p), O._p(yr, O._f32p), n_out, k)
        assert np.array_equal(bits(O.gemv(W, q, n_out, k)), bits(yr))
